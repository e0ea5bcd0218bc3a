"""MoC 2:8 kernels as Python callables (moc/inference/triton_fused_ffn_kernels.py).

  fused_gate_top2of8_selected_up_silu[_into]  <- :159-221, :428-472
  selected_down_from_sparse_z[_into]          <- :270-301, :475-499
  selected_down_from_sparse_z_splitk          <- :373-418 (same result; the
      split over k is internal to the gfx950 kernel)

Block-size keyword arguments of the reference are accepted and ignored: the
gfx950 kernels pick their own tiling.  The `_into` forms write into caller
buffers, so a HIP graph capture of them allocates nothing.
"""
from __future__ import annotations

import torch

from .. import kernels as K


def fused_gate_top2of8_selected_up_silu(x, gate_weight, up_weight, grouped_b: int = 8,
                                        BLOCK_B: int = 16, BLOCK_G: int = 16, BLOCK_H: int = 64):
    if grouped_b != 8:
        raise ValueError(f"only grouped_b=8 is supported, got {grouped_b}")
    if x.dim() != 2 or gate_weight.dim() != 2 or up_weight.dim() != 2:
        raise ValueError("x, gate_weight, up_weight must all be 2D")
    if not (x.is_cuda and gate_weight.is_cuda and up_weight.is_cuda):
        raise ValueError("inputs must be CUDA")
    if not (x.dtype == gate_weight.dtype == up_weight.dtype):
        raise ValueError(
            f"dtype mismatch: x={x.dtype}, gate={gate_weight.dtype}, up={up_weight.dtype}")
    if gate_weight.shape[1] != x.shape[1] or up_weight.shape[1] != x.shape[1]:
        raise ValueError(
            f"H mismatch: x={x.shape}, gate={gate_weight.shape}, up={up_weight.shape}")
    if gate_weight.shape[0] != up_weight.shape[0]:
        raise ValueError(f"gate I={gate_weight.shape[0]} != up I={up_weight.shape[0]}")
    if gate_weight.shape[0] % 8 != 0:
        raise ValueError(f"intermediate I={gate_weight.shape[0]} must be divisible by 8")
    return K.grouped_top2_up_silu(x, gate_weight, up_weight)


def fused_gate_top2of8_selected_up_silu_into(x, gate_weight, up_weight, topk_idx_out,
                                             sparse_z_out, grouped_b: int = 8, BLOCK_B: int = 16,
                                             BLOCK_G: int = 16, BLOCK_H: int = 64) -> None:
    if grouped_b != 8:
        raise ValueError(f"only grouped_b=8 is supported, got {grouped_b}")
    b = x.shape[0]
    inter = gate_weight.shape[0]
    if inter % 8 != 0:
        raise ValueError(f"intermediate I={inter} must be divisible by 8")
    k = inter // 4
    if tuple(topk_idx_out.shape) != (b, k) or tuple(sparse_z_out.shape) != (b, k):
        raise ValueError(
            f"out shapes must be ({b},{k}); got idx={tuple(topk_idx_out.shape)}, "
            f"sz={tuple(sparse_z_out.shape)}")
    K.grouped_top2_up_silu(x, gate_weight, up_weight, idx_out=topk_idx_out, sz_out=sparse_z_out)


def selected_down_from_sparse_z(sparse_z, idx, w_down_t, BLOCK_K: int = 64, BLOCK_H: int = 32):
    if not (sparse_z.is_cuda and idx.is_cuda and w_down_t.is_cuda):
        raise ValueError("inputs must be CUDA")
    if sparse_z.dtype != torch.bfloat16 or w_down_t.dtype != torch.bfloat16 or idx.dtype != torch.int64:
        raise ValueError("sparse_z/w_down_t must be bf16 and idx int64")
    return K.selected_grouped_down(sparse_z, idx, w_down_t)


def selected_down_from_sparse_z_splitk(sparse_z, idx, w_down_t, BLOCK_K: int = 64,
                                       BLOCK_H: int = 32, SPLITS: int = 4):
    return selected_down_from_sparse_z(sparse_z, idx, w_down_t)


def selected_down_from_sparse_z_into(sparse_z, idx, w_down_t, out, BLOCK_K: int = 128,
                                     BLOCK_H: int = 16, workspace=None) -> None:
    b = sparse_z.shape[0]
    h = w_down_t.shape[1]
    if tuple(out.shape) != (b, h):
        raise ValueError(f"out shape must be ({b},{h}); got {tuple(out.shape)}")
    K.selected_grouped_down(sparse_z, idx, w_down_t, out=out, workspace=workspace)
