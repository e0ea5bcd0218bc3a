"""The allocation-free after-gate entry point, moc_global_after_gate_noalloc_bf16.

It runs the kernels of moc_global_after_gate_bf16 / _residual_bf16 on the
library's own fixed device scratch array instead of a caller workspace, so
its outputs must equal that entry point's bit for bit (same kernels, same
fixed-order reductions).  Checked through the C ABI on two calls in a row,
the second with a smaller input (the scratch keeps the first call's
contents), with and without the residual, and the selection it reports.
"""
from __future__ import annotations

import pytest
import torch

from moc_amd import _native as N

DEV = "cuda"


def test_noalloc_rejects_oversized_shapes_before_device_work():
    lib = N.load()
    # 16 tokens of hidden 8192 and k 16384 need ~32 MB of partial sums
    rc = lib.moc_global_after_gate_noalloc_bf16(None, None, 16, 16384, 8192, None, None, 8192, 16384,
                                                None, None, None, None)
    assert rc == N.MOC_ERR_INVALID and "scratch" in N.last_error()
    assert lib.moc_global_after_gate_noalloc_bf16(None, None, 0, 5461, 2048, None, None, 2048, 1024, None,
                                                  None, None, None) == N.MOC_OK


def _inputs(nb, d, inter, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(nb, d, generator=g).to(torch.bfloat16)
    gate = (torch.randn(nb, inter, generator=g) * 0.9).to(torch.bfloat16)
    wu = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16)
    wdt = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16)
    res = torch.randn(nb, d, generator=g).to(torch.bfloat16)
    return [t.to(DEV) for t in (x, gate, wu, wdt, res)]


def _with_workspace(x, gate, wu, wdt, k, res):
    nb, d = x.shape
    inter = gate.shape[1]
    nbytes = N.query("moc_global_after_gate_workspace_size", nb, inter, k, d)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=DEV)
    y = torch.empty(nb, d, dtype=torch.bfloat16, device=DEV)
    io = torch.full((nb, k), -1, dtype=torch.int32, device=DEV)
    if res is None:
        N.call("moc_global_after_gate_bf16", x.data_ptr(), gate.data_ptr(), nb, inter, d, wu.data_ptr(),
               wdt.data_ptr(), wdt.stride(0), k, y.data_ptr(), io.data_ptr(), ws.data_ptr(), nbytes, N.stream_of(x))
    else:
        N.call("moc_global_after_gate_residual_bf16", x.data_ptr(), gate.data_ptr(), nb, inter, d,
               wu.data_ptr(), wdt.data_ptr(), wdt.stride(0), k, res.data_ptr(), y.data_ptr(), io.data_ptr(),
               ws.data_ptr(), nbytes, N.stream_of(x))
    return y, io


def _no_alloc(x, gate, wu, wdt, k, res):
    nb, d = x.shape
    inter = gate.shape[1]
    y = torch.empty(nb, d, dtype=torch.bfloat16, device=DEV)
    io = torch.full((nb, k), -1, dtype=torch.int32, device=DEV)
    N.call("moc_global_after_gate_noalloc_bf16", x.data_ptr(), gate.data_ptr(), nb, inter, d,
           wu.data_ptr(), wdt.data_ptr(), wdt.stride(0), k, None if res is None else res.data_ptr(), y.data_ptr(),
           io.data_ptr(), N.stream_of(x))
    return y, io


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry_point():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    N.load()
    d, inter, k = 2048, 5461, 1024
    # 16 tokens (dense-U form, the largest scratch use at this shape), then 1
    # token and 4 tokens on the scratch the previous call left behind
    for step, nb in enumerate((16, 1, 4)):
        x, gate, wu, wdt, res = _inputs(nb, d, inter, 900 + step)
        for r in (None, res):
            print(f"[no-alloc] call nb={nb} residual={r is not None}", flush=True)
            y_ref, io_ref = _with_workspace(x, gate, wu, wdt, k, r)
            y, io = _no_alloc(x, gate, wu, wdt, k, r)
            torch.cuda.synchronize()
            assert torch.equal(io, io_ref), f"selection differs at nb={nb}"
            assert torch.equal(y, y_ref), f"y differs at nb={nb}"
            assert int(io.min()) >= 0


@pytest.mark.gpu
def test_noalloc_captured_in_graph_matches_workspace_entry_point():
    """The entry point captured in a HIP graph (after an eager first call,
    which clears the scratch counters), replayed three times with new inputs
    copied into the captured buffers and eager calls of the workspace entry
    point between the replays: every replay equals that entry point on the
    same input bit for bit (output and selection)."""
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    N.load()
    d, inter, k, nb = 2048, 5461, 1024, 4
    x, gate, wu, wdt, res = _inputs(nb, d, inter, 950)
    _no_alloc(x, gate, wu, wdt, k, res)  # the first call on the device is eager
    torch.cuda.synchronize()
    xs, gs, rs = x.clone(), gate.clone(), res.clone()
    y = torch.empty(nb, d, dtype=torch.bfloat16, device=DEV)
    io = torch.full((nb, k), -1, dtype=torch.int32, device=DEV)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):  # captures on torch's own capture stream
        N.call("moc_global_after_gate_noalloc_bf16", xs.data_ptr(), gs.data_ptr(), nb, inter, d,
               wu.data_ptr(), wdt.data_ptr(), wdt.stride(0), k, rs.data_ptr(), y.data_ptr(), io.data_ptr(),
               N.stream_of(xs))
    for rep in range(3):
        xn, gn, _, _, rn = _inputs(nb, d, inter, 960 + rep)
        xs.copy_(xn)
        gs.copy_(gn)
        rs.copy_(rn)
        print(f"[no-alloc] graph replay {rep}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        y_ref, io_ref = _with_workspace(xn, gn, wu, wdt, k, rn)
        torch.cuda.synchronize()
        assert torch.equal(io, io_ref), f"selection differs on replay {rep}"
        assert torch.equal(y, y_ref), f"y differs on replay {rep}"
