"""Global-MoC operators and graph runner (moc/inference/optimized_global_moc_ops.py).

load_optimized_global_moc_extension() loads libmoc_amd.so (built in-tree by
`python -m moc_amd.build`; no JIT compile at first use) and registers the
moc_native:: and moc:: operators.  make_optimized_global_moc_graph_runner()
captures the decode path - gate GEMV, Top-K, selected Up * SiLU, selected
Down - in a HIP graph, replayed per call (reference :106-162).
"""
from __future__ import annotations

import torch

from .. import _native, kernels as K, ops


def load_optimized_global_moc_extension(build_dir=None):
    """Load the gfx950 library and register the ops; returns the ctypes handle."""
    lib = _native.load()
    ops.register()
    return lib


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
    ws = K.global_after_gate_workspace(batch_size, inter, k, hidden, device)
    up_w = module.up_proj.weight.contiguous()
    down_t = module._down_weight_t.contiguous()
    gate_w = module.gate_proj.weight.contiguous()

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
