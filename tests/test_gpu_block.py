"""GPU parity of the FFN's neighbours fused around the MoC FFN in training and
prefill: the pre-norm (RMSNorm, moc/model.py:20-28) as a row kernel and the
residual add (moc/model.py:85) in the Down GEMM's epilogue.

- moc_rmsnorm_rows_bf16 against the model's stock RMSNorm (torch ops) and
  against the formula in float64;
- moc_rmsnorm_backward_bf16 against float64 autograd of the formula;
- moc_gemm_residual_bf16 against the plain GEMM plus a bf16 add, bit for bit,
  on shapes that take each of the GEMM's output paths (whole tiles, the
  two-part fix-up, split-K, 128-row tiles);
- the fused block h + FFN(RMSNorm(h)), forward and backward, against stock
  RMSNorm + the CPU oracle's FFN (on the device's own G, U, gZ) + add, in
  the one-call native form (config 5's layer shape) and the per-kernel,
  two-stream form (a 1b-shape layer at 4096 tokens), within 2e-2;
- a 2-layer 350m-shape model: one training step with the fused blocks
  against the same model with them switched off.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moc_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _lib():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    from moc_amd import _native
    _native.load()


def _stock_rmsnorm(h, w, eps):
    """RMSNorm.forward of the model host (moc/model.py:26-28), torch ops."""
    hf = h.float()
    return (hf * torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + eps)).to(h.dtype) * w


def _ulps(a, b):
    """Distance in bf16 ulps (units of the order-preserving integer code)."""
    def code(t):
        i = t.contiguous().view(torch.int16).to(torch.int32)
        return torch.where(i < 0, -(i & 0x7FFF), i)
    return (code(a) - code(b)).abs()


def _close(a, b, rtol, atol, what):
    a = a.detach().float().cpu().reshape(-1)
    b = b.detach().float().cpu().reshape(-1)
    if isinstance(atol, torch.Tensor):
        atol = atol.reshape(-1)
    err = (a - b).abs()
    bad = err > atol + rtol * b.abs()
    assert not bool(bad.any()), f"{what}: max err {err.max().item():.4g} ({int(bad.sum())} elems)"


@pytest.mark.parametrize("rows,d", [(1, 8), (3, 768), (4096, 1024), (257, 2048), (64, 4096), (5, 8192)])
def test_rmsnorm_rows_matches_stock_norm(rows, d):
    from moc_amd import kernels as K
    g = torch.Generator(device=DEV).manual_seed(rows + d)
    h = (torch.randn(rows, d, device=DEV, generator=g) * 3).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(d, device=DEV, generator=g)).to(torch.bfloat16)
    y, rstd = K.rmsnorm_rows(h, w, 1e-6)
    ref = _stock_rmsnorm(h, w, 1e-6)
    # the row's mean square is summed in another order and 1/sqrt rounds
    # differently from torch's rsqrt: bf16(x r) may move by one ulp, and
    # the product with w by one more
    assert bool((_ulps(y, ref) <= 2).all()), int(_ulps(y, ref).max())
    assert (y != ref).float().mean().item() < 1e-2
    r64 = 1.0 / torch.sqrt(h.double().pow(2).mean(-1) + 1e-6)
    assert torch.allclose(rstd.double(), r64, rtol=2e-6, atol=0)


@pytest.mark.parametrize("rows,d", [(2, 8), (1000, 1024), (333, 2048), (17, 4096)])
def test_rmsnorm_backward_matches_autograd(rows, d):
    from moc_amd import kernels as K
    g = torch.Generator(device=DEV).manual_seed(7 * rows + d)
    h = (torch.randn(rows, d, device=DEV, generator=g) * 2).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(d, device=DEV, generator=g)).to(torch.bfloat16)
    dy = torch.randn(rows, d, device=DEV, generator=g).to(torch.bfloat16)
    dres = torch.randn(rows, d, device=DEV, generator=g).to(torch.bfloat16)
    _, rstd = K.rmsnorm_rows(h, w, 1e-6)
    dx, dw = K.rmsnorm_backward(h, w, rstd, dy, dres=dres)
    hd = h.double().cpu().requires_grad_(True)
    wd = w.double().cpu().requires_grad_(True)
    y = hd * torch.rsqrt(hd.pow(2).mean(-1, keepdim=True) + 1e-6) * wd
    y.backward(dy.double().cpu())
    _close(dx, hd.grad + dres.double().cpu(), 2e-2, 2e-2, "dx")
    _close(dw, wd.grad, 2e-2, 2e-2 * max(1.0, rows ** 0.5), "dw")
    dx2, dw2 = K.rmsnorm_backward(h, w, rstd, dy)
    _close(dx2, hd.grad, 2e-2, 2e-2, "dx without dres")
    assert torch.equal(dw, dw2)  # dw does not depend on dres and is summed in a fixed order


@pytest.mark.parametrize("m,n,k", [(4096, 1024, 2736),   # 350m D: 128-row tiles, two-part fix-up
                                   (8192, 768, 2048),    # 130m D: 128-row whole tiles
                                   (16384, 2048, 5461),  # 1b D: whole 256x256 tiles, 4 rounds
                                   (300, 1000, 4000),    # few tiles: split-K and its reduction
                                   (1, 72, 64)])
def test_gemm_residual_equals_gemm_plus_add(m, n, k):
    from moc_amd import kernels as K
    g = torch.Generator(device=DEV).manual_seed(m + n + k)
    a = torch.randn(m, k, device=DEV, generator=g).to(torch.bfloat16)
    b = (torch.randn(n, k, device=DEV, generator=g) * 0.05).to(torch.bfloat16)
    r = torch.randn(m, n, device=DEV, generator=g).to(torch.bfloat16)
    plain = K.gemm(K.aligned_rows(a), K.aligned_rows(b).t())
    fused = K.gemm(K.aligned_rows(a), K.aligned_rows(b).t(), residual=r)
    want = (plain.float() + r.float()).to(torch.bfloat16)
    assert torch.equal(fused, want)


def _block_inputs(t, d, inter, seed):
    g = torch.Generator().manual_seed(seed)
    h = (torch.randn(t, d, generator=g) * 2).to(torch.bfloat16)
    wn = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16)
    wg = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16)
    wu = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16)
    wd = (torch.randn(d, inter, generator=g) * 0.02).to(torch.bfloat16)
    dout = torch.randn(t, d, generator=g).to(torch.bfloat16)
    return h, wn, wg, wu, wd, dout


def _block_reference(h, wn, wg, wu, wd, dout, k, omode, gcp):
    """The norm's output, then the oracle FFN on the device's own G, U and gZ
    + the residual add; the norm's backward by float64 autograd of its
    formula.  The norm output handed to the oracle is the row kernel's (the
    block's own bits, so that the selection is compared on identical
    inputs); its distance to the stock RMSNorm is bounded at two bf16 ulps
    here and in test_rmsnorm_rows_matches_stock_norm."""
    from moc_amd import kernels as K
    eps = 1e-6
    hd, wnd = h.to(DEV), wn.to(DEV)
    xn, _ = K.rmsnorm_rows(hd, wnd, eps)
    assert bool((_ulps(xn, _stock_rmsnorm(hd, wnd, eps)) <= 2).all())
    gdev, udev = K.linear_pair(xn, wg.to(DEV), wu.to(DEV))
    gz = K.gemm(K.aligned_rows(dout.to(DEV)), K.aligned_rows(wd.to(DEV)))
    xn_c = xn.cpu()
    fwd = O.ffn_forward(xn_c, wg, wu, wd, k, omode, g_override=gdev.cpu(), u_override=udev.cpu())
    dxn, dwg, dwu, dwd = O.ffn_backward(xn_c, wg, wu, wd, fwd, dout, gcp=gcp, gz_override=gz.cpu())
    out = (h.float() + fwd["out"].float()).to(torch.bfloat16)
    h64 = h.double().requires_grad_(True)
    w64 = wn.double().requires_grad_(True)
    y = h64 * torch.rsqrt(h64.pow(2).mean(-1, keepdim=True) + eps) * w64
    y.backward(dxn.double())
    dh = h64.grad + dout.double()
    # the norm weight's gradient sums rows x dxn over all tokens; dxn carries
    # the bf16 rounding of the FFN's dX (one ulp where the device's
    # accumulation order rounds the other way), so its noise grows as the
    # square root of the token count: 4 sigma of one-ulp errors of each term
    terms = (dxn.double() * (h.double() * torch.rsqrt(h.double().pow(2).mean(-1, keepdim=True) + eps)))
    dw_noise = 4 * 2.0 ** -8 * terms.pow(2).sum(0).sqrt()
    return out, dh, w64.grad, dwg, dwu, dwd, fwd["idx"], dw_noise


def _run_block(mode, h, wn, wg, wu, wd, dout, k):
    from moc_amd import ffn as F
    from moc_amd.ffn import MoCSwiGLUFFN
    t, d = h.shape
    inter = wg.shape[0]
    m = MoCSwiGLUFFN(d, inter, k, mode=mode, index_save_dtype=torch.int16).to(DEV, torch.bfloat16)
    with torch.no_grad():
        m.gate_proj.weight.copy_(wg)
        m.up_proj.weight.copy_(wu)
        m.down_proj.weight.copy_(wd)
    w = torch.nn.Parameter(wn.to(DEV))
    hd = h.to(DEV).requires_grad_(True)
    assert F.block_ffn_ok(hd, w, m)
    saved = []

    def pack(x):
        saved.append(x)
        return x

    with torch.autograd.graph.saved_tensors_hooks(pack, lambda x: x):
        out = F.block_ffn(hd, w, 1e-6, m)
    out.backward(dout.to(DEV))
    idx = [s for s in saved if s.dtype == torch.int16]
    return (out, hd.grad, w.grad, m.gate_proj.weight.grad, m.up_proj.weight.grad,
            m.down_proj.weight.grad), idx[0].reshape(t, -1)


@pytest.mark.parametrize("mode,omode,gcp", [("moc_gcp", "moc_gcp", True), ("moc", "moc", False),
                                            ("moc_2_8", "moc_2_8", False)])
@pytest.mark.parametrize("t,d,inter,k,native", [(4096, 1024, 2736, 512, True),
                                                (4096, 2048, 5461, 1024, False)])
def test_block_ffn_matches_stock_norm_oracle_ffn_and_add(mode, omode, gcp, t, d, inter, k, native):
    from moc_amd import ffn as F
    h, wn, wg, wu, wd, dout = _block_inputs(t, d, inter, seed=t + inter)
    h2 = h.to(DEV)
    assert F._block_native(h2, wg.to(DEV), wu.to(DEV), wd.to(DEV)) == native
    if not native:  # the per-kernel form runs its two-stream schedule here
        assert F._side_for(torch.device(DEV), t, inter) is not None
    got, idx = _run_block(mode, h, wn, wg, wu, wd, dout, k)
    ref = _block_reference(h, wn, wg, wu, wd, dout, k, omode, gcp)
    # the indices the block saves for its backward are the oracle's
    assert np.array_equal(idx.cpu().numpy().astype(np.int64), ref[6])
    for name, a, b in zip(("out", "dh", "dnorm_w", "dWg", "dWu", "dWd"), got, ref[:6]):
        atol = 2e-2 + (ref[7].float() if name == "dnorm_w" else 0.0)
        _close(a, b, 2e-2, atol, f"{mode} {name}")


def test_model_two_layers_fused_block_matches_unfused():
    """A 2-layer decoder of the 350m preset's shape with moc_gcp FFNs: one
    training step with the fused blocks against the same model with the
    fusion switched off (stock RMSNorm module + FFN module + add)."""
    from moc_amd import MoCConfig, build_model
    from moc_amd import ffn as F
    cfg = MoCConfig(hidden_size=1024, intermediate_size=2736, num_hidden_layers=2,
                    num_attention_heads=16, vocab_size=32100, max_seq_len=256, k=512)
    torch.manual_seed(11)
    model = build_model(cfg, ffn_type="moc_gcp").to(DEV, torch.bfloat16)
    for b in model.blocks:  # norm weights away from one
        torch.nn.init.normal_(b.ffn_norm.weight, mean=1.0, std=0.1)
    tok = torch.randint(0, cfg.vocab_size, (16, 256), device=DEV,
                        generator=torch.Generator(device=DEV).manual_seed(3))
    res = {}
    for fuse in (True, False):
        F.FUSE_BLOCK_FFN = fuse
        try:
            model.zero_grad(set_to_none=True)
            _, loss = model(tok, labels=tok)
            loss.backward()
        finally:
            F.FUSE_BLOCK_FFN = True
        res[fuse] = (loss.detach().float().item(),
                     {n: p.grad.detach().float().clone() for n, p in model.named_parameters()})
    assert abs(res[True][0] - res[False][0]) < 2e-2 * abs(res[False][0])
    for name, g_fused in res[True][1].items():
        g_plain = res[False][1][name]
        rel = ((g_fused - g_plain).norm() / g_plain.norm().clamp_min(1e-30)).item()
        assert rel < 3e-2, f"{name}: relative gradient difference {rel:.3g}"
