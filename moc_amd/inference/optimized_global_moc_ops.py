"""Global-MoC operators and graph runner (moc/inference/optimized_global_moc_ops.py).

load_optimized_global_moc_extension() loads libmoc_amd.so (built in-tree by
`python -m moc_amd.build`; no JIT compile at first use), registers the
moc_native:: and moc:: operators and returns the extension object whose
methods the reference's callers use (optimized_global_moc_ext.cpp:78-86).
make_optimized_global_moc_graph_runner() captures the decode path - gate
GEMV, Top-K, selected Up * SiLU, selected Down - in a HIP graph, replayed
per call (reference :106-162).
"""
from __future__ import annotations

import torch

from .. import _native, kernels as K, ops


class OptimizedGlobalMoCExtension:
    """The methods of the reference's pybind module
    (optimized_global_moc_ext.cpp:25-86), on the gfx950 kernels.

    cub_topk_bf16_512x11 returns [values, int64 indices] ordered as the
    reference's stable descending radix sort emits them: value descending,
    ties to the lower channel index (-0.0 and +0.0 rank equal here).  The
    reference's I <= 5632 limit of its one-CTA sort is lifted (I <= 16384).
    The checks raise RuntimeError with the reference's TORCH_CHECK messages.
    """

    def __init__(self, lib):
        self.lib = lib

    @staticmethod
    def _rows_contiguous(w: torch.Tensor) -> bool:
        """W_down^T may come with padded rows (the module's decode layout,
        InferenceMoCSwiGLUFFN._down_weight_t): unit column stride suffices."""
        return w.dim() == 2 and w.stride(1) == 1 and w.stride(0) >= w.shape[1]

    @staticmethod
    def _require(cond: bool, msg: str) -> None:
        if not cond:
            raise RuntimeError(msg)

    def cub_topk_bf16_512x11(self, scores: torch.Tensor, k: int):
        r = self._require
        r(scores.is_cuda, "scores must be CUDA")
        r(scores.dim() == 2, "scores must be [B, I]")
        r(scores.dtype == torch.bfloat16, "scores must be BF16")
        r(scores.is_contiguous(), "scores must be contiguous")
        r(0 < k <= scores.shape[1], "invalid k")
        vals, idx, _ = K.topk_rows(scores, int(k), idx_dtype=torch.int64)
        return list(ops.value_order(vals, idx))

    def selected_up_silu_bf16(self, x, topk_vals, idx, w_up):
        r = self._require
        r(x.is_cuda and topk_vals.is_cuda and idx.is_cuda and w_up.is_cuda, "all tensors must be CUDA")
        r(x.dtype == torch.bfloat16, "x must be BF16")
        r(topk_vals.dtype == torch.bfloat16, "topk_vals must be BF16")
        r(w_up.dtype == torch.bfloat16, "w_up must be BF16")
        r(idx.dtype == torch.int64, "idx must be int64")
        r(x.is_contiguous() and topk_vals.is_contiguous() and idx.is_contiguous()
          and w_up.is_contiguous(), "inputs must be contiguous")
        return K.selected_up_silu(x, topk_vals, idx, w_up)

    def selected_down_bf16_h32_k16(self, sparse_z, idx, w_down_t):
        r = self._require
        r(sparse_z.is_cuda and idx.is_cuda and w_down_t.is_cuda, "all tensors must be CUDA")
        r(sparse_z.dtype == torch.bfloat16, "sparse_z must be BF16")
        r(w_down_t.dtype == torch.bfloat16, "w_down_t must be BF16")
        r(idx.dtype == torch.int64, "idx must be int64")
        r(sparse_z.is_contiguous() and idx.is_contiguous() and self._rows_contiguous(w_down_t),
          "inputs must be contiguous")
        return K.selected_down(sparse_z, idx, w_down_t)

    def optimized_global_after_gate_bf16(self, x, gate_scores, up_weight, down_weight_t, k: int):
        r = self._require
        r(x.is_cuda and gate_scores.is_cuda and up_weight.is_cuda and down_weight_t.is_cuda,
          "all tensors must be CUDA")
        for t, n in ((x, "x"), (gate_scores, "gate_scores"), (up_weight, "up_weight"),
                     (down_weight_t, "down_weight_t")):
            r(t.dtype == torch.bfloat16, f"{n} must be BF16")
        r(x.is_contiguous() and gate_scores.is_contiguous() and up_weight.is_contiguous()
          and self._rows_contiguous(down_weight_t), "inputs must be contiguous")
        r(0 < k <= gate_scores.shape[1], "invalid k")
        return K.global_after_gate(x, gate_scores, up_weight, down_weight_t, int(k))


_EXT: OptimizedGlobalMoCExtension | None = None


def load_optimized_global_moc_extension(build_dir=None) -> OptimizedGlobalMoCExtension:
    """Load the gfx950 library (once), register the ops and return the
    extension object.  build_dir is accepted for the reference's signature;
    the library is built in-tree ahead of time."""
    global _EXT
    if _EXT is None:
        lib = _native.load()
        ops.register()
        _EXT = OptimizedGlobalMoCExtension(lib)
    return _EXT


def ensure_native_ops_ready() -> None:
    load_optimized_global_moc_extension()


def make_optimized_global_moc_graph_runner(module, batch_size: int = 1):
    """Capture the global-MoC decode path for a fixed batch size in a HIP graph."""
    load_optimized_global_moc_extension()
    if module.config.grouped:
        raise ValueError("optimized global MoC graph runner requires ungrouped MoC")
    module._ensure_down_weight_t()
    hidden = module.config.hidden_size
    inter = module.config.intermediate_size
    k = module.config.k
    device = module.gate_proj.weight.device
    dtype = module.gate_proj.weight.dtype
    x_buf = torch.zeros(batch_size, hidden, device=device, dtype=dtype)
    gate_buf = torch.empty(batch_size, inter, device=device, dtype=dtype)
    y_buf = torch.empty(batch_size, hidden, device=device, dtype=dtype)
    up_w = module.up_proj.weight.contiguous()
    down_t = module._down_weight_t  # [inter, hidden] rows at the module's padded pitch
    gate_w = module.gate_proj.weight.contiguous()
    if batch_size <= 16 and dtype == torch.bfloat16:
        # gate GEMV (+ dense U from 4 tokens on, same launch) and the
        # after-gate kernel through the one layer entry
        ws = K.global_decode_workspace(batch_size, inter, k, hidden, device)

        def path():
            K.global_decode(x_buf, gate_w, up_w, down_t, k, workspace=ws, out=y_buf)
    else:
        ws = K.global_after_gate_workspace(batch_size, inter, k, hidden, device)

        def path():
            K.gemv(x_buf, gate_w, out=gate_buf)
            K.global_after_gate(x_buf, gate_buf, up_w, down_t, k, workspace=ws, out=y_buf)

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(3):
            path()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        path()

    def runner(x_in: torch.Tensor) -> torch.Tensor:
        x_2d, original_shape = module._flatten_decode_input(x_in)
        if x_2d.shape[0] != batch_size:
            raise ValueError(f"runner built for batch_size={batch_size}, got {x_2d.shape[0]}")
        x_buf.copy_(x_2d)
        graph.replay()
        return module._restore_output_shape(y_buf, original_shape)

    runner.graph = graph
    # the graph's buffers live as long as the runner (a freed one would be
    # handed to other tensors while replays still use it; the workspace
    # carries the after-gate kernel's zeroed arrival counters between replays)
    runner.buffers = (x_buf, gate_buf, y_buf, ws, up_w, down_t, gate_w)
    return runner


def optimized_global_topk_bf16(scores: torch.Tensor, k: int):
    ensure_native_ops_ready()
    return torch.ops.moc.optimized_global_topk_bf16(scores, k)


def optimized_global_selected_up_silu_bf16(x, topk_vals, topk_idx, up_weight):
    ensure_native_ops_ready()
    return torch.ops.moc.optimized_global_selected_up_silu_bf16(x, topk_vals, topk_idx, up_weight)


def optimized_global_selected_down_bf16(sparse_z, topk_idx, down_weight_t):
    ensure_native_ops_ready()
    return torch.ops.moc.optimized_global_selected_down_bf16(sparse_z, topk_idx, down_weight_t)
