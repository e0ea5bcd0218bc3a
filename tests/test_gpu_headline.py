"""GPU parity of the headline workload at its full size: the 1b MoC FFN layer
(X [64, 256, 2048] bf16, d_ffn 5461, K 1024; benchmark_training_latency.py:
20-31), forward and backward, on the inputs bench.py times (the same seeded
draw), against the CPU oracle.

At 16384 tokens the [rows, I] GEMMs take several rounds of 256x256 tiles, so
the layer runs its two-stream schedule (the W_down row copy beside the
Top-K, dWd beside gZ and the backward aux kernel, the joins) and the weight
gradients take the two-part K fix-up over 176 tiles.  Smaller layer tests
never reach those branches.

The oracle is handed the device's own bf16 G and U (from the G,U pair launch
the layer makes) and gZ (the layer's gZ launch), as in the other layer
tests, so the selection is compared on identical inputs: the indices the
layer saves for its backward must equal the oracle's bit for bit, and out,
dX, dWg, dWu and dWd must agree within rtol/atol 2e-2 (moc/ffn.py:124-259,
372-497).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moc_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
T, D, INTER, K = 64 * 256, 2048, 5461, 1024


@pytest.fixture(scope="module", autouse=True)
def _lib():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    from moc_amd import _native
    _native.load()


def bench_inputs():
    """bench.py's seeded_inputs(16384, 2048, 5461): X ~ N(0,1), W_gate, W_up
    [I, d] and W_down [d, I] ~ N(0, 0.02), dD ~ N(0,1), drawn on the CPU in
    that order from one generator seeded 1234."""
    g = torch.Generator().manual_seed(1234)
    x = torch.randn(T, D, generator=g).to(torch.bfloat16)
    wg = (torch.randn(INTER, D, generator=g) * 0.02).to(torch.bfloat16)
    wu = (torch.randn(INTER, D, generator=g) * 0.02).to(torch.bfloat16)
    wd = (torch.randn(D, INTER, generator=g) * 0.02).to(torch.bfloat16)
    go = torch.randn(T, D, generator=g).to(torch.bfloat16)
    return x, wg, wu, wd, go


@pytest.fixture(scope="module")
def oracle_1b():
    """Inputs, the oracle's forward/backward on the device's own G, U, gZ."""
    from moc_amd import kernels as KR
    x, wg, wu, wd, go = bench_inputs()
    xd = x.to(DEV)
    g, u = KR.linear_pair(xd, wg.to(DEV), wu.to(DEV))
    gz = KR.gemm(KR.aligned_rows(go.to(DEV)), KR.aligned_rows(wd.to(DEV)))
    g, u, gz = g.cpu(), u.cpu(), gz.cpu()
    torch.set_num_threads(min(16, max(1, torch.get_num_threads())))
    fwd = O.ffn_forward(x, wg, wu, wd, K, "moc_gcp", g_override=g, u_override=u)
    ref = (fwd["out"],) + O.ffn_backward(x, wg, wu, wd, fwd, go, gcp=True, gz_override=gz)
    return (x, wg, wu, wd, go), fwd["idx"], ref


def close(a, b, rtol, atol, what):
    a = a.detach().float().cpu().reshape(-1)
    b = b.detach().float().cpu().reshape(-1)
    err = (a - b).abs()
    bad = err > atol + rtol * b.abs()
    assert not bool(bad.any()), f"{what}: max err {err.max().item():.4g} ({int(bad.sum())} elems)"


@pytest.mark.timeout(600)
@pytest.mark.parametrize("ffn_type", ["moc_gcp", "moc"])
def test_layer_1b_full_size_matches_oracle(oracle_1b, ffn_type):
    from moc_amd import build_ffn
    from moc_amd import ffn as F
    (x, wg, wu, wd, go), idx_ref, ref = oracle_1b
    dev = torch.device(DEV)
    # the shape takes the two-stream schedule bench.py times
    assert F._side_for(dev, T, INTER) is not None
    m = build_ffn(D, INTER, ffn_type, k=K).to(DEV, torch.bfloat16).train()
    with torch.no_grad():
        for p, w in zip((m.gate_proj.weight, m.up_proj.weight, m.down_proj.weight), (wg, wu, wd)):
            p.copy_(w)
    xd = x.reshape(64, 256, D).to(DEV)
    god = go.reshape(64, 256, D).to(DEV)
    runs = []
    for _ in range(2):  # two steps back to back, as the bench's steps run
        m.zero_grad(set_to_none=True)
        xr = xd.detach().clone().requires_grad_(True)
        saved = []

        def pack(t):
            saved.append(t)
            return t

        with torch.autograd.graph.saved_tensors_hooks(pack, lambda t: t):
            out = m(xr)
        out.backward(god)
        torch.cuda.synchronize()
        sel = [s for s in saved if s.dtype == torch.int16 and s.shape[-1] == K]
        assert len(sel) == 1, [(tuple(s.shape), s.dtype) for s in saved]
        runs.append((sel[0].reshape(T, K).cpu(), out.detach().cpu(), xr.grad.cpu(),
                     m.gate_proj.weight.grad.cpu(), m.up_proj.weight.grad.cpu(),
                     m.down_proj.weight.grad.cpu()))
    # the saved selection, in ascending channel order, is the oracle's
    assert np.array_equal(runs[0][0].numpy().astype(np.int64), idx_ref)
    # the two steps are bit-identical (deterministic kernels, no stale state)
    for a, b in zip(runs[0], runs[1]):
        assert torch.equal(a, b)
    for name, a, b in zip(("out", "dx", "dWg", "dWu", "dWd"), runs[0][1:], ref):
        close(a, b, 2e-2, 2e-2, f"{ffn_type} {name}")
