"""torch.library operators under the reference's names, backed by libmoc_amd.so.

Registered (schema as in the reference, plus a fake kernel each so the ops
trace under torch.compile):

  moc_native::optimized_global_topk_bf16(Tensor scores, int k) -> Tensor[]
  moc_native::optimized_global_selected_up_silu_bf16(x, topk_vals, topk_idx, up_weight)
  moc_native::optimized_global_selected_down_bf16(sparse_z, topk_idx, down_weight_t)
  moc_native::optimized_global_after_gate_bf16(x, gate_scores, up_weight, down_weight_t, k)
      (moc/inference/cuda/optimized_global_moc_ext.cpp:88-100)
  moc::optimized_global_topk_bf16 / _selected_up_silu_bf16 / _selected_down_bf16
      (moc/inference/optimized_global_moc_ops.py:165-244)
  moc::fused_grouped_top2_up_silu(x, gate_weight, up_weight) -> (idx, sparse_z)
  moc::selected_grouped_down(sparse_z, idx, w_down_t) -> Tensor
      (moc/inference/triton_grouped_moc_ops.py:26-143)

The argument checks raise the reference's messages.  The Top-K ops return
the selection in the order of the reference's stable descending radix sort
(optimized_global_moc_ext.cu:39-83): value descending, ties to the lower
channel index.  One documented difference: -0.0 and +0.0 rank equal here
(the reference's key encoding puts -0.0 below +0.0).
"""
from __future__ import annotations

import torch

from . import kernels as K

_REGISTERED = False


def _check_topk(scores: torch.Tensor, k: int) -> None:
    if not scores.is_cuda:
        raise RuntimeError("scores must be CUDA")
    if scores.dim() != 2:
        raise RuntimeError("scores must be [B, I]")
    if scores.dtype != torch.bfloat16:
        raise RuntimeError("scores must be BF16")
    if not (0 < k <= scores.shape[1]):
        raise RuntimeError("invalid k")


def value_order(vals: torch.Tensor, idx: torch.Tensor):
    """(vals, idx) of a selection in ascending channel order -> the same
    pairs ordered by value descending, equal values by ascending channel (a
    stable sort keeps the channel order among equal values).  The sort key
    is vals + 0.0 in f32, which turns -0.0 into +0.0, so the two zeros rank
    equal whatever the sort's key encoding; NaN sorts above +inf."""
    keys = vals.float() + 0.0
    order = torch.sort(keys, dim=-1, descending=True, stable=True).indices
    return torch.gather(vals, -1, order), torch.gather(idx, -1, order)


def _topk_impl(scores: torch.Tensor, k: int):
    _check_topk(scores, k)
    vals, idx, _ = K.topk_rows(scores.contiguous(), int(k), idx_dtype=torch.int64)
    return value_order(vals, idx)


def _up_impl(x, topk_vals, topk_idx, up_weight):
    for t, n in ((x, "x"), (topk_vals, "topk_vals"), (up_weight, "w_up")):
        if t.dtype != torch.bfloat16:
            raise RuntimeError(f"{n} must be BF16")
    if topk_idx.dtype != torch.int64:
        raise RuntimeError("idx must be int64")
    return K.selected_up_silu(x, topk_vals, topk_idx, up_weight)


def _down_impl(sparse_z, topk_idx, down_weight_t):
    if sparse_z.dtype != torch.bfloat16:
        raise RuntimeError("sparse_z must be BF16")
    if down_weight_t.dtype != torch.bfloat16:
        raise RuntimeError("w_down_t must be BF16")
    if topk_idx.dtype != torch.int64:
        raise RuntimeError("idx must be int64")
    return K.selected_down(sparse_z, topk_idx, down_weight_t)


def _after_gate_impl(x, gate_scores, up_weight, down_weight_t, k):
    for t, n in ((x, "x"), (gate_scores, "gate_scores"), (up_weight, "up_weight"),
                 (down_weight_t, "down_weight_t")):
        if t.dtype != torch.bfloat16:
            raise RuntimeError(f"{n} must be BF16")
    if not (0 < k <= gate_scores.shape[1]):
        raise RuntimeError("invalid k")
    return K.global_after_gate(x, gate_scores, up_weight, down_weight_t, int(k))


def register() -> None:
    """Register all operators once (idempotent)."""
    global _REGISTERED
    if _REGISTERED:
        return

    # ---- moc_native:: (C++ dispatcher names of the reference extension)
    @torch.library.custom_op("moc_native::optimized_global_topk_bf16", mutates_args=())
    def native_topk(scores: torch.Tensor, k: int) -> list[torch.Tensor]:
        v, i = _topk_impl(scores, k)
        return [v, i]

    @native_topk.register_fake
    def _(scores, k):
        b = scores.shape[0]
        return [scores.new_empty(b, k), scores.new_empty(b, k, dtype=torch.int64)]

    @torch.library.custom_op("moc_native::optimized_global_selected_up_silu_bf16", mutates_args=())
    def native_up(x: torch.Tensor, topk_vals: torch.Tensor, topk_idx: torch.Tensor,
                  up_weight: torch.Tensor) -> torch.Tensor:
        return _up_impl(x, topk_vals, topk_idx, up_weight)

    @native_up.register_fake
    def _(x, topk_vals, topk_idx, up_weight):
        return torch.empty_like(topk_vals, dtype=x.dtype)

    @torch.library.custom_op("moc_native::optimized_global_selected_down_bf16", mutates_args=())
    def native_down(sparse_z: torch.Tensor, topk_idx: torch.Tensor,
                    down_weight_t: torch.Tensor) -> torch.Tensor:
        return _down_impl(sparse_z, topk_idx, down_weight_t)

    @native_down.register_fake
    def _(sparse_z, topk_idx, down_weight_t):
        return sparse_z.new_empty(sparse_z.shape[0], down_weight_t.shape[1])

    @torch.library.custom_op("moc_native::optimized_global_after_gate_bf16", mutates_args=())
    def native_after_gate(x: torch.Tensor, gate_scores: torch.Tensor, up_weight: torch.Tensor,
                          down_weight_t: torch.Tensor, k: int) -> torch.Tensor:
        return _after_gate_impl(x, gate_scores, up_weight, down_weight_t, k)

    @native_after_gate.register_fake
    def _(x, gate_scores, up_weight, down_weight_t, k):
        return x.new_empty(x.shape[0], down_weight_t.shape[1])

    # ---- moc:: (Python custom_op duplicates of the reference)
    @torch.library.custom_op("moc::optimized_global_topk_bf16", mutates_args=())
    def moc_topk(scores: torch.Tensor, k: int) -> tuple[torch.Tensor, torch.Tensor]:
        return _topk_impl(scores, k)

    @moc_topk.register_fake
    def _(scores, k):
        b = scores.shape[0]
        return scores.new_empty(b, k), scores.new_empty(b, k, dtype=torch.int64)

    @torch.library.custom_op("moc::optimized_global_selected_up_silu_bf16", mutates_args=())
    def moc_up(x: torch.Tensor, topk_vals: torch.Tensor, topk_idx: torch.Tensor,
               up_weight: torch.Tensor) -> torch.Tensor:
        return _up_impl(x, topk_vals, topk_idx, up_weight)

    @moc_up.register_fake
    def _(x, topk_vals, topk_idx, up_weight):
        return torch.empty_like(topk_vals, dtype=x.dtype)

    @torch.library.custom_op("moc::optimized_global_selected_down_bf16", mutates_args=())
    def moc_down(sparse_z: torch.Tensor, topk_idx: torch.Tensor,
                 down_weight_t: torch.Tensor) -> torch.Tensor:
        return _down_impl(sparse_z, topk_idx, down_weight_t)

    @moc_down.register_fake
    def _(sparse_z, topk_idx, down_weight_t):
        return sparse_z.new_empty(sparse_z.shape[0], down_weight_t.shape[1])

    @torch.library.custom_op("moc::fused_grouped_top2_up_silu", mutates_args=())
    def grouped_up(x: torch.Tensor, gate_weight: torch.Tensor,
                   up_weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        if not (x.is_cuda and gate_weight.is_cuda and up_weight.is_cuda):
            raise ValueError("inputs must be CUDA")
        if x.dtype != gate_weight.dtype or x.dtype != up_weight.dtype:
            raise ValueError("dtype mismatch")
        return K.grouped_top2_up_silu(x, gate_weight, up_weight)

    @grouped_up.register_fake
    def _(x, gate_weight, up_weight):
        k = (gate_weight.shape[0] // 8) * 2
        return x.new_empty(x.shape[0], k, dtype=torch.int64), x.new_empty(x.shape[0], k)

    @torch.library.custom_op("moc::selected_grouped_down", mutates_args=())
    def grouped_down(sparse_z: torch.Tensor, idx: torch.Tensor,
                     w_down_t: torch.Tensor) -> torch.Tensor:
        return K.selected_grouped_down(sparse_z, idx, w_down_t)

    @grouped_down.register_fake
    def _(sparse_z, idx, w_down_t):
        return sparse_z.new_empty(sparse_z.shape[0], w_down_t.shape[1])

    _REGISTERED = True
