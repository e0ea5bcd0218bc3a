"""GPU parity of the gfx950 kernels against the CPU oracle (marked gpu).

Integer/index outputs (Top-K indices, masks, 2:8 indices) must match the
oracle bit-exactly on identical inputs.  Floating outputs are bf16 and are
compared within rtol/atol 2e-2, or in bf16 ulps
where the arithmetic is the same sequence of rounded operations.  Inputs are
seeded on the CPU and copied to the device, so both sides see identical bits.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import moc_oracle as O

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _lib():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    from moc_amd import _native
    _native.load()  # raises if the library is missing: no silent fallback


def K():
    from moc_amd import kernels
    return kernels


def N():
    from moc_amd import _native
    return _native


def gen(seed):
    return torch.Generator().manual_seed(seed)


def bf16_ulp_diff(a: torch.Tensor, b: torch.Tensor) -> np.ndarray:
    """|difference| in bf16 units of last place (order-key distance)."""
    ka = O.order_keys(a.detach().cpu().to(torch.bfloat16)).astype(np.int64)
    kb = O.order_keys(b.detach().cpu().to(torch.bfloat16)).astype(np.int64)
    return np.abs(ka - kb)


def bf16_close(a, b, ulps: int = 1, atol: float = 1e-3) -> None:
    """Each element within `ulps` bf16 ulps of b, or within atol (near zero
    the ulp distance of two roundings of a cancelling sum is meaningless)."""
    a = a.detach().float().cpu()
    b = b.detach().float().cpu()
    assert a.shape == b.shape, (a.shape, b.shape)
    ulp = torch.from_numpy(bf16_ulp_diff(a, b))
    bad = (ulp > ulps) & ((a - b).abs() > atol)
    assert not bool(bad.any()), f"{int(bad.sum())} elements off, e.g. {a[bad][:4].tolist()} vs {b[bad][:4].tolist()}"


def close(a, b, rtol=2e-2, atol=2e-2):
    a = a.detach().float().cpu()
    b = b.detach().float().cpu()
    assert a.shape == b.shape, (a.shape, b.shape)
    err = (a - b).abs()
    bad = err > atol + rtol * b.abs()
    assert not bool(bad.any()), f"max err {err.max().item():.4g} at {torch.nonzero(bad)[:4].tolist()}"


@pytest.mark.parametrize("rows,cols,off", [(2048, 5461, 0), (3, 13, 1), (17, 1000, 3), (1, 7, 5)])
def test_aligned_rows_copy(rows, cols, off):
    """aligned_rows() of a matrix whose rows are not 16-byte aligned (a view
    starting `off` elements into its storage): the padded copy holds the
    values and zero pad columns."""
    g = gen(rows + cols)
    base = torch.randn(rows * cols + off, generator=g).to(torch.bfloat16).to(DEV)
    t = base[off:].view(rows, cols)
    a = K().aligned_rows(t)
    assert a.stride(0) % 8 == 0 and a.data_ptr() % 16 == 0
    assert torch.equal(a, t)
    full = a.as_strided((rows, a.stride(0)), (a.stride(0), 1))
    assert not bool(full[:, cols:].any())


# ----------------------------------------------------------------------- GEMM
@pytest.mark.parametrize("a_kc", [True, False])
@pytest.mark.parametrize("b_kc", [True, False])
@pytest.mark.parametrize("mnk", [(128, 128, 64), (136, 72, 93), (130, 67, 93), (1, 300, 40),
                                 (264, 5464, 200), (257, 5461, 200), (520, 600, 5461),
                                 (300, 264, 1000)])
def test_gemm_bf16_layouts(a_kc, b_kc, mnk):
    M, Nn, Kk = mnk
    g = gen(1)
    a = torch.randn(M, Kk, generator=g).to(torch.bfloat16)
    b = torch.randn(Kk, Nn, generator=g).to(torch.bfloat16)
    ref = a.float() @ b.float()
    ad = a.to(DEV) if a_kc else a.t().contiguous().to(DEV).t()
    bd = b.t().contiguous().to(DEV).t() if b_kc else b.to(DEV)
    if a_kc and Kk % 8:  # K-contiguous rows need a pitch that is a multiple of 8
        ad = K().aligned_rows(ad)
    out = K().gemm(ad, bd, out_dtype=torch.float32)
    close(out, ref, rtol=1e-4, atol=1e-3)
    out16 = K().gemm(ad, bd)
    bf16_close(out16, ref, ulps=1, atol=1e-3)


@pytest.mark.parametrize("a_kc,b_kc", [(True, True), (False, False), (True, False), (False, True)])
def test_gemm_weight_gradient_shape(a_kc, b_kc):
    """176 output tiles of 256x256 (the weight-gradient shape class) against
    a torch fp32 reference on the device; repeated calls are bit-identical."""
    M, Nn, Kk = 2048, 5461, 1000
    g = torch.Generator(device=DEV).manual_seed(7)
    a = torch.randn(M, Kk, device=DEV, generator=g).to(torch.bfloat16)
    b = torch.randn(Kk, Nn, device=DEV, generator=g).to(torch.bfloat16)
    ref = a.float() @ b.float()
    ad = K().aligned_rows(a) if a_kc else a.t().contiguous().t()
    bd = K().aligned_rows(b.t().contiguous()).t() if b_kc else K().aligned_rows(b)
    first = K().gemm(ad, bd, out_dtype=torch.float32)
    close(first, ref, rtol=1e-4, atol=2e-3)
    again = K().gemm(ad, bd, out_dtype=torch.float32)
    assert torch.equal(first, again)
    out16 = K().gemm(ad, bd)
    bf16_close(out16, ref, ulps=1, atol=2e-3)


@pytest.mark.parametrize("layout", ["mnmn", "kcmn", "kckc"])
@pytest.mark.parametrize("mnk", [(768, 2048, 8192), (520, 300, 5000), (72, 1000, 2048)])
def test_gemm_split_k(layout, mnk):
    """Products with few output tiles split K over f32 partials in a
    workspace: results match the fp32 reference, do not depend on timing
    (repeat equality) and agree with the unsplit kernel to f32 rounding."""
    M, Nn, Kk = mnk
    g = torch.Generator(device=DEV).manual_seed(11)
    a = torch.randn(M, Kk, device=DEV, generator=g).to(torch.bfloat16)
    b = torch.randn(Kk, Nn, device=DEV, generator=g).to(torch.bfloat16)
    ref = a.float() @ b.float()
    ad = K().aligned_rows(a) if layout in ("kcmn", "kckc") else a.t().contiguous().t()
    bd = K().aligned_rows(b.t().contiguous()).t() if layout == "kckc" else K().aligned_rows(b)
    ws = N().query("moc_gemm_workspace_size", N().MOC_BF16, M, Nn, Kk, 0)
    assert ws > 0, "shape expected to split"
    first = K().gemm(ad, bd, out_dtype=torch.float32)
    close(first, ref, rtol=1e-4, atol=3e-3)
    assert torch.equal(first, K().gemm(ad, bd, out_dtype=torch.float32))
    out16 = K().gemm(ad, bd)
    bf16_close(out16, ref, ulps=1, atol=3e-3)
    # the unsplit kernel (moc_gemm, no workspace) on the same operands
    flat = torch.empty(M, Nn, device=DEV, dtype=torch.float32)
    a_, as0, as1 = K()._operand(ad, True)
    b_, bs0, bs1 = K()._operand(bd, True)
    N().call("moc_gemm", N().MOC_BF16, M, Nn, Kk, a_.data_ptr(), as0, as1, b_.data_ptr(), bs0, bs1,
             0, None, 0, 0, None, 0, 0, flat.data_ptr(), Nn, N().MOC_F32, N().stream_of(ad))
    close(first, flat, rtol=1e-5, atol=3e-3)  # f32 sums of K products in another order


def test_gemm_split_k_dual():
    """dX-shaped dual product at a small width: the split runs across both
    products' K tiles."""
    g = torch.Generator(device=DEV).manual_seed(12)
    T, I, d = 4096, 2048, 768
    gg = torch.randn(T, I, device=DEV, generator=g).to(torch.bfloat16)
    gu = torch.randn(T, I, device=DEV, generator=g).to(torch.bfloat16)
    wg = (torch.randn(I, d, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    wu = (torch.randn(I, d, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    assert N().query("moc_gemm_workspace_size", N().MOC_BF16, T, d, I, I) > 0
    out = K().gemm(gg, wg, a2=gu, b2=wu, out_dtype=torch.float32)
    ref = gg.float() @ wg.float() + gu.float() @ wu.float()
    close(out, ref, rtol=1e-4, atol=1e-3)


@pytest.mark.parametrize("mkn", [
    (16384, 2048, 5461, 5461),   # 1b gate/up: 1408 + 1408 tiles, one launch
    (8192, 768, 2048, 2048),     # 130m: 256 + 256 tiles, one launch
    (1000, 200, 1300, 700),      # ragged: 4 x (6 + 3) tiles -> two moc_gemm_ws calls
    (300, 64, 50, 90),           # one tile each, split-K plans
])
def test_gemm_pair_equals_two_launches(mkn):
    """moc_gemm_pair (G = x Wg^T and U = x Wu^T with the two tile grids side
    by side in one launch) equals the two single-product launches bit for bit,
    leaves the pad columns of padded outputs alone, and matches fp32."""
    M, Kd, n1, n2 = mkn
    g = torch.Generator(device=DEV).manual_seed(21)
    x = torch.randn(M, Kd, device=DEV, generator=g).to(torch.bfloat16)
    w1 = (torch.randn(n1, Kd, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(n2, Kd, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    o1 = K().padded_empty(M, n1, torch.bfloat16, DEV)
    o2 = K().padded_empty(M, n2, torch.bfloat16, DEV)
    for o in (o1, o2):
        o.as_strided((M, o.stride(0)), (o.stride(0), 1)).fill_(7.0)
    K().linear_pair(x, w1, w2, out1=o1, out2=o2)
    torch.cuda.synchronize()
    assert torch.equal(o1, K().linear(x, w1)) and torch.equal(o2, K().linear(x, w2))
    for o, n in ((o1, n1), (o2, n2)):
        pad = o.as_strided((M, o.stride(0)), (o.stride(0), 1))[:, n:]
        assert pad.numel() == 0 or bool((pad == 7.0).all())
    sub = slice(0, min(M, 512))
    bf16_close(o1[sub], x[sub].float() @ w1.float().t(), ulps=1, atol=1e-3)
    bf16_close(o2[sub], x[sub].float() @ w2.float().t(), ulps=1, atol=1e-3)


def _unsplit(ad, bd, M, Nn, Kk, a2=None, b2=None, K2=0):
    """The GEMM without a workspace (moc_gemm: whole tiles only), f32 out."""
    flat = torch.empty(M, Nn, device=DEV, dtype=torch.float32)
    a_, as0, as1 = K()._operand(ad, True)
    b_, bs0, bs1 = K()._operand(bd, True)
    p2 = [None, 0, 0, None, 0, 0]
    if a2 is not None:
        a2_, a2s0, a2s1 = K()._operand(a2, True)
        b2_, b2s0, b2s1 = K()._operand(b2, True)
        p2 = [a2_.data_ptr(), a2s0, a2s1, b2_.data_ptr(), b2s0, b2s1]
    N().call("moc_gemm", N().MOC_BF16, M, Nn, Kk, a_.data_ptr(), as0, as1, b_.data_ptr(), bs0, bs1,
             K2, *p2, flat.data_ptr(), Nn, N().MOC_F32, N().stream_of(ad))
    return flat


@pytest.mark.parametrize("layout,mnk", [
    ("mnmn", (5461, 2048, 16384)),   # 1b dW_gate / dW_up: 176 tiles, each in two K ranges
    ("mnmn", (2048, 5461, 16384)),   # 1b dW_down
    ("kckc", (5461, 2000, 16001)),   # ragged M, N and K (K % 64 != 0)
    ("kcmn", (1000, 3000, 9000)),    # 48 tiles: split-K plan, not the fix-up
])
def test_gemm_tail_fixup(layout, mnk):
    """Products with more tiles than half the CUs but fewer than all of them
    run each tile as two K ranges on two workgroups; the one that finishes
    second adds the other's f32 partial.  Results match the fp32 reference,
    repeat bit for bit (the arrival counters are left zero for the next
    call), and agree with the whole-tile kernel to f32 rounding."""
    M, Nn, Kk = mnk
    g = torch.Generator(device=DEV).manual_seed(13)
    a = torch.randn(M, Kk, device=DEV, generator=g).to(torch.bfloat16)
    b = torch.randn(Kk, Nn, device=DEV, generator=g).to(torch.bfloat16)
    ad = K().aligned_rows(a) if layout in ("kcmn", "kckc") else K().aligned_rows(a.t().contiguous()).t()
    bd = K().aligned_rows(b.t().contiguous()).t() if layout == "kckc" else K().aligned_rows(b)
    assert N().query("moc_gemm_workspace_size", N().MOC_BF16, M, Nn, Kk, 0) > 0
    first = K().gemm(ad, bd, out_dtype=torch.float32)
    ref = a.float() @ b.float()
    close(first, ref, rtol=1e-4, atol=2e-2)
    assert torch.equal(first, K().gemm(ad, bd, out_dtype=torch.float32))
    bf16_close(K().gemm(ad, bd), ref, ulps=1, atol=2e-2)
    close(first, _unsplit(ad, bd, M, Nn, Kk), rtol=1e-5, atol=1e-2)


def test_gemm_tail_fixup_dual():
    """A dual product (dX form) with 160 tiles, each in two K ranges that
    split the second product."""
    g = torch.Generator(device=DEV).manual_seed(14)
    T, I, d = 5000, 1000, 2048
    gg = torch.randn(T, I, device=DEV, generator=g).to(torch.bfloat16)
    gu = torch.randn(T, I, device=DEV, generator=g).to(torch.bfloat16)
    wg = (torch.randn(I, d, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    wu = (torch.randn(I, d, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    gg, gu = K().aligned_rows(gg), K().aligned_rows(gu)
    assert N().query("moc_gemm_workspace_size", N().MOC_BF16, T, d, I, I) > 0
    out = K().gemm(gg, wg, a2=gu, b2=wu, out_dtype=torch.float32)
    ref = gg.float() @ wg.float() + gu.float() @ wu.float()
    close(out, ref, rtol=1e-4, atol=1e-3)
    assert torch.equal(out, K().gemm(gg, wg, a2=gu, b2=wu, out_dtype=torch.float32))
    close(out, _unsplit(gg, wg, T, d, I, gu, wu, I), rtol=1e-5, atol=1e-3)


@pytest.mark.parametrize("layout,mnk", [
    ("kckc", (8192, 768, 2048)),   # 130m D = Z W_down^T: 96 tiles of 256x256 -> 192 of 128x256
    ("kcmn", (8192, 768, 2048)),
    ("kckc", (8100, 700, 1000)),   # ragged M (not a multiple of 128) and N
    ("kckc", (8192, 768, 1001)),   # K % 8 != 0: the straddling chunk of A and B zeroed
])
def test_gemm_short_tiles(layout, mnk):
    """Products whose 256x256 tiles would fill more than a quarter but at
    most half of the CUs run 128x256 tiles whole: results match the fp32
    reference, repeat bit for bit, and the workspace-free entry gives the
    same bits (no split either way)."""
    M, Nn, Kk = mnk
    tiles = ((M + 255) // 256) * ((Nn + 255) // 256)
    cus = K().cu_count(torch.cuda.current_device())
    assert 4 * tiles > cus and 2 * tiles <= cus
    g = torch.Generator(device=DEV).manual_seed(16)
    a = torch.randn(M, Kk, device=DEV, generator=g).to(torch.bfloat16)
    b = (torch.randn(Kk, Nn, device=DEV, generator=g) * 0.05).to(torch.bfloat16)
    ad = K().aligned_rows(a)
    bd = K().aligned_rows(b.t().contiguous()).t() if layout == "kckc" else K().aligned_rows(b)
    first = K().gemm(ad, bd, out_dtype=torch.float32)
    ref = a.float() @ b.float()
    close(first, ref, rtol=1e-4, atol=2e-3)
    assert torch.equal(first, K().gemm(ad, bd, out_dtype=torch.float32))
    assert torch.equal(first, _unsplit(ad, bd, M, Nn, Kk))
    bf16_close(K().gemm(ad, bd), ref, ulps=1, atol=2e-3)


def test_gemm_short_tiles_dual():
    """A dX-shaped dual product with short K (M 8192, N 768, K 1024 + 1024)
    on 128x256 tiles against the fp32 reference."""
    g = torch.Generator(device=DEV).manual_seed(17)
    T, I, d = 8192, 1024, 768
    gg = torch.randn(T, I, device=DEV, generator=g).to(torch.bfloat16)
    gu = torch.randn(T, I, device=DEV, generator=g).to(torch.bfloat16)
    wg = (torch.randn(I, d, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    wu = (torch.randn(I, d, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    out = K().gemm(gg, wg, a2=gu, b2=wu, out_dtype=torch.float32)
    ref = gg.float() @ wg.float() + gu.float() @ wu.float()
    close(out, ref, rtol=1e-4, atol=1e-3)
    assert torch.equal(out, K().gemm(gg, wg, a2=gu, b2=wu, out_dtype=torch.float32))
    assert torch.equal(out, _unsplit(gg, wg, T, d, I, gu, wu, I))
    bf16_close(K().gemm(gg, wg, a2=gu, b2=wu), ref, ulps=1, atol=1e-3)


@pytest.mark.parametrize("mnk", [(4096, 1024, 2736), (4000, 1000, 2736), (4096, 1024, 1001)])
def test_gemm_short_tiles_fixup(mnk):
    """Products whose 256x256 tiles fill at most a third of the CUs but whose
    128x256 tiles fill more (the 350m layer's D: 4096 x 1024 x 2736) run the
    128-row tiles in two K parts with the fix-up instead of a K split:
    against the fp32 reference, bit for bit on repeats (the fix-up's sum of
    two partials does not depend on which part finishes first)."""
    M, Nn, Kk = mnk
    tiles = ((M + 255) // 256) * ((Nn + 255) // 256)
    cus = K().cu_count(torch.cuda.current_device())
    assert 3 * tiles <= cus < 6 * tiles
    g = torch.Generator(device=DEV).manual_seed(18)
    a = K().aligned_rows(torch.randn(M, Kk, device=DEV, generator=g).to(torch.bfloat16))
    w = K().aligned_rows((torch.randn(Nn, Kk, device=DEV, generator=g) * 0.05).to(torch.bfloat16))
    first = K().gemm(a, w.t(), out_dtype=torch.float32)
    ref = a.float() @ w.float().t()
    close(first, ref, rtol=1e-4, atol=2e-3)
    for _ in range(3):
        assert torch.equal(first, K().gemm(a, w.t(), out_dtype=torch.float32))
    bf16_close(K().gemm(a, w.t()), ref, ulps=1, atol=2e-3)


def test_gemm_short_tiles_fixup_dual():
    """A dX-shaped dual product (4096 x 1024 x (1024 + 1024)) on 128-row
    tiles in two K parts, against the fp32 reference and bit for bit on
    repeats."""
    g = torch.Generator(device=DEV).manual_seed(19)
    T, I, d = 4096, 1024, 1024
    gg = K().aligned_rows(torch.randn(T, I, device=DEV, generator=g).to(torch.bfloat16))
    gu = K().aligned_rows(torch.randn(T, I, device=DEV, generator=g).to(torch.bfloat16))
    wg = (torch.randn(I, d, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    wu = (torch.randn(I, d, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    out = K().gemm(gg, wg, a2=gu, b2=wu, out_dtype=torch.float32)
    ref = gg.float() @ wg.float() + gu.float() @ wu.float()
    close(out, ref, rtol=1e-4, atol=1e-3)
    for _ in range(3):
        assert torch.equal(out, K().gemm(gg, wg, a2=gu, b2=wu, out_dtype=torch.float32))


def test_gemm_workspace_shared_by_split_and_fixup():
    """Split-K and fix-up launches take turns on the stream's one workspace:
    the split-K partials leave the fix-up's arrival counters untouched."""
    g = torch.Generator(device=DEV).manual_seed(15)
    a = K().aligned_rows(torch.randn(5461, 4096, device=DEV, generator=g).to(torch.bfloat16))
    b = K().aligned_rows(torch.randn(4096, 2048, device=DEV, generator=g).to(torch.bfloat16))
    c = K().aligned_rows(torch.randn(1000, 4096, device=DEV, generator=g).to(torch.bfloat16))
    fix0 = K().gemm(a, b, out_dtype=torch.float32)
    split0 = K().gemm(c, b, out_dtype=torch.float32)
    for _ in range(2):
        assert torch.equal(K().gemm(a, b, out_dtype=torch.float32), fix0)
        assert torch.equal(K().gemm(c, b, out_dtype=torch.float32), split0)
    close(fix0, a.float() @ b.float(), rtol=1e-4, atol=1e-2)
    close(split0, c.float() @ b.float(), rtol=1e-4, atol=1e-2)


def test_gemm_dual_product_and_f32():
    g = gen(2)
    a, a2 = torch.randn(200, 72, generator=g), torch.randn(200, 40, generator=g)
    b, b2 = torch.randn(72, 96, generator=g), torch.randn(40, 96, generator=g)
    ref = a @ b + a2 @ b2
    dual = K().gemm(a.bfloat16().to(DEV), b.bfloat16().to(DEV), a2=a2.bfloat16().to(DEV),
                    b2=b2.bfloat16().to(DEV), out_dtype=torch.float32)
    close(dual, a.bfloat16().float() @ b.bfloat16().float() + a2.bfloat16().float() @ b2.bfloat16().float(),
          rtol=1e-4, atol=1e-3)
    f32 = K().gemm(a.to(DEV), b.to(DEV), a2=a2.to(DEV), b2=b2.to(DEV))
    close(f32, ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("layout", ["kckc", "kcmn", "mnkc", "mnmn"])
@pytest.mark.parametrize("mnk", [(512, 1376, 512), (512, 512, 1376), (67, 45, 130), (1, 5, 7),
                                 (300, 260, 64), (68, 44, 132), (64, 128, 4096), (2048, 512, 512)])
def test_gemm_f32_tiled(layout, mnk):
    """The f32 GEMM (fp32 MFMA, 64x64 tiles, K split over f32 partials summed
    in a fixed order when that shortens the busiest CU's work) in all four
    operand layouts, against float64; repeat calls are identical.  Extents
    not a multiple of 4 along an operand's contiguous dimension take the
    generic kernel (67, 45, 130 and 1, 5, 7 in the MN layouts)."""
    M, Nn, Kk = mnk
    g = gen(M * 7 + Nn + Kk)
    a, b = torch.randn(M, Kk, generator=g), torch.randn(Kk, Nn, generator=g)
    ref = (a.double() @ b.double()).float()
    ad = a.to(DEV) if layout[:2] == "kc" else a.t().contiguous().t().to(DEV)
    bd = b.t().contiguous().t().to(DEV) if layout[2:] == "kc" else b.to(DEV)
    if layout[2:] == "kc":
        bd = b.t().contiguous().to(DEV).t()
    got = K().gemm(ad, bd)
    close(got, ref, rtol=1e-5, atol=1e-5 * (Kk ** 0.5) * 4)
    assert torch.equal(K().gemm(ad, bd), got)


def test_gemm_f32_dual_product_tiled():
    """dX-shaped f32 sum of two products (first K a multiple of the K step)."""
    g = gen(5)
    a, a2 = torch.randn(200, 64, generator=g), torch.randn(200, 40, generator=g)
    b, b2 = torch.randn(64, 96, generator=g), torch.randn(40, 96, generator=g)
    ref = (a.double() @ b.double() + a2.double() @ b2.double()).float()
    got = K().gemm(a.to(DEV), b.to(DEV), a2=a2.to(DEV), b2=b2.to(DEV))
    close(got, ref, rtol=1e-5, atol=1e-4)


# ---------------------------------------------------------------------- Top-K
@pytest.mark.parametrize("name", ["topk_bf16_ties", "topk_bf16_rand"])
def test_topk_golden_bitexact(name):
    d = dict(np.load(GOLD / f"{name}.npz"))
    s = O.torch_from_bf16_bits(d["scores_bits"]).to(DEV)
    _, idx, _ = K().topk_rows(s, int(d["k"]))
    assert np.array_equal(idx.cpu().numpy(), d["idx"])


def test_topk_golden_f32_bitexact():
    d = dict(np.load(GOLD / "topk_f32_ties.npz"))
    _, idx, _ = K().topk_rows(torch.from_numpy(d["scores"]).to(DEV), int(d["k"]))
    assert np.array_equal(idx.cpu().numpy(), d["idx"])


@pytest.mark.parametrize("dtype,rows,inter,k", [
    (torch.bfloat16, 64, 5461, 1024),   # 1b decode/training shape
    (torch.bfloat16, 300, 2048, 384),   # 130m
    (torch.float32, 96, 1376, 256),     # 60m (f32, config 1)
    (torch.bfloat16, 7, 37, 37),        # k == inter
    (torch.bfloat16, 5, 16384, 1),      # widest supported row, k == 1
    (torch.float32, 3, 9000, 4500),
])
def test_topk_bitexact_vs_oracle(dtype, rows, inter, k):
    s = (torch.randn(rows, inter, generator=gen(rows + inter)) * 0.9).to(dtype)
    vals, idx, mask = K().topk_rows(s.to(DEV), k, want_mask=True)
    want = O.topk_indices(s, k)
    assert np.array_equal(idx.cpu().numpy(), want)
    assert torch.equal(vals.cpu(), O.gather_rows(s, want))
    bits = mask.cpu().numpy().view(np.uint32)
    m = np.zeros((rows, inter), dtype=bool)
    for c in range(inter):
        m[:, c] = (bits[:, c // 32] >> (c % 32)) & 1
    assert np.array_equal(m, O.topk_mask(want, inter))


@pytest.mark.parametrize("k", [1, 100, 1024, 2600, 4000, 5461])
def test_topk_wide_range_rows_vs_oracle(k):
    """bf16 rows whose values span ~140 binades (some rows all negative, some
    holding NaN or inf), so the k-th largest key falls inside, at the edge of
    and below the 4096-key window under each row's largest key."""
    g = gen(k)
    rows, inter = 48, 5461
    mag = torch.exp2(torch.rand(rows, inter, generator=g) * 140 - 70)
    sign = torch.where(torch.rand(rows, inter, generator=g) < 0.3, -1.0, 1.0)
    s = (sign * mag).to(torch.bfloat16)
    s[::4] = -s[::4].abs()                               # all-negative rows
    s[1::6, 17] = float("nan")
    s[2::6, 33] = float("inf")
    s[3::6, 40:60] = 2.0 ** 60                           # a block of equal top keys
    _, idx, _ = K().topk_rows(s.to(DEV), k)
    assert np.array_equal(idx.cpu().numpy(), O.topk_indices(s, k))


@pytest.mark.parametrize("inter,k", [(961, 1), (961, 480), (2048, 384), (2736, 512), (2736, 2736),
                                     (4096, 100), (4096, 4000), (5461, 1024), (8192, 3000)])
def test_topk_two_wave_bf16_rows_vs_oracle(inter, k):
    """bf16 rows of 961-4032 channels take two waves per row, of 4033-8192
    four: the same
    selection as the oracle on rows spanning ~140 binades (all-negative rows,
    NaN, inf, a block of equal top keys, signed zeros) and on rows of heavy
    ties, indices and bit mask."""
    g = gen(inter + k)
    rows = 40
    mag = torch.exp2(torch.rand(rows, inter, generator=g) * 140 - 70)
    sign = torch.where(torch.rand(rows, inter, generator=g) < 0.3, -1.0, 1.0)
    s = (sign * mag).to(torch.bfloat16)
    s[::4] = -s[::4].abs()
    s[1::6, 17] = float("nan")
    s[2::6, 33] = float("inf")
    s[3::6, 40:60] = 2.0 ** 60
    ties = torch.tensor(np.random.default_rng(inter).choice([0.0, -0.0, 1.0, -2.0, 0.5], size=(8, inter)),
                        dtype=torch.bfloat16)
    s = torch.cat([s, ties])
    vals, idx, mask = K().topk_rows(s.to(DEV), k, want_mask=True)
    want = O.topk_indices(s, k)
    assert np.array_equal(idx.cpu().numpy(), want)
    # the selected entries' raw bits (NaN payloads included)
    assert np.array_equal(vals.cpu().view(torch.int16).numpy(),
                          np.take_along_axis(s.view(torch.int16).numpy(), want.astype(np.int64), 1))
    bits = mask.cpu().numpy().view(np.uint32)
    m = (bits[:, np.arange(inter) // 32] >> (np.arange(inter) % 32)) & 1
    assert np.array_equal(m.astype(bool), O.topk_mask(want, inter))


def test_topk_heavy_ties_and_index_dtypes():
    vals = torch.tensor(np.random.default_rng(3).choice([0.0, -0.0, 1.0, -2.0, 0.5, float("inf")],
                                                        size=(33, 700)), dtype=torch.float32)
    for dt in (torch.bfloat16, torch.float32):
        s = vals.to(dt)
        want = O.topk_indices(s, 111)
        for idt in (torch.int16, torch.int32, torch.int64):
            _, idx, _ = K().topk_rows(s.to(DEV), 111, idx_dtype=idt)
            assert idx.dtype == idt and np.array_equal(idx.cpu().numpy().astype(np.int64), want)


def test_topk_strided_rows_and_post_silu_transform():
    s = (torch.randn(20, 600, generator=gen(5)) * 2).to(torch.bfloat16)
    sd = s.to(DEV)
    _, idx, _ = K().topk_rows(sd[:, :555], 100)  # leading dimension 600, width 555
    assert np.array_equal(idx.cpu().numpy(), O.topk_indices(s[:, :555].contiguous(), 100))
    vals, idx, _ = K().topk_rows(sd, 64, score_transform=1)
    want = O.topk_indices(O.silu_abs_scores(s), 64)
    # the transformed score is computed on the device; its bf16 rounding can
    # differ from the CPU's in rare near-ties, so compare tie-aware
    score = O.silu_abs_scores(s).float()
    got = idx.cpu().numpy()
    for r in range(s.shape[0]):
        thr = torch.sort(score[r], descending=True).values[63].item()
        gs = {i for i in got[r] if score[r, i] > thr * (1 + 2 ** -7)}
        ws = {i for i in want[r] if score[r, i] > thr * (1 + 2 ** -7)}
        assert gs == ws
    assert torch.equal(vals.cpu(), O.gather_rows(s, got))  # raw pre-SiLU gates


def test_select_2of8_bitexact():
    d = dict(np.load(GOLD / "sel28_bf16_tail.npz"))
    s = O.torch_from_bf16_bits(d["scores_bits"])
    vals, idx = K().select_2of8(s.to(DEV))
    assert np.array_equal(idx.cpu().numpy(), d["idx"])
    for dt, inter in ((torch.bfloat16, 5461), (torch.float32, 2736), (torch.bfloat16, 5464)):
        s = torch.randn(50, inter, generator=gen(inter)).to(dt)
        vals, idx = K().select_2of8(s.to(DEV), idx_dtype=torch.int16)
        want = O.select_2of8_indices(s)
        assert np.array_equal(idx.cpu().numpy().astype(np.int64), want)
        assert torch.equal(vals.cpu(), O.gather_rows(s, want))


# ------------------------------------------------------------- training aux
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(300, 2048, 384), (64, 5461, 1024)])
def test_sparse_aux_forward_backward(dtype, shape):
    """Row kernels (bf16 pitches up to 8192, f32 up to 4096) and, for f32
    rows past that, the element kernels with a zero-fill, against the oracle."""
    rows, inter, k = shape
    g = gen(6)
    G = torch.randn(rows, inter, generator=g).to(dtype)
    U = torch.randn(rows, inter, generator=g).to(dtype)
    GZ = torch.randn(rows, inter, generator=g).to(dtype)
    idx = O.topk_indices(G, k)
    vals = O.gather_rows(G, idx)
    u_s, s_s, z_s, z_full = O.sparse_forward_aux(vals, idx, U, inter)
    ti = torch.from_numpy(idx).to(torch.int16).to(DEV)
    du, ds, dz, dzf = K().sparse_forward_aux(vals.to(DEV), ti, U.to(DEV), inter)
    assert torch.equal(du.cpu(), u_s)
    if dtype == torch.bfloat16:
        bf16_close(ds, s_s, ulps=1, atol=0)
        bf16_close(dz, z_s, ulps=2, atol=0)
        bf16_close(dzf, z_full, ulps=2, atol=0)
    else:
        close(ds, s_s, rtol=1e-5, atol=1e-6)
        close(dz, z_s, rtol=1e-5, atol=1e-6)
        close(dzf, z_full, rtol=1e-5, atol=1e-6)
    # scatter / gather round trip
    dense = K().scatter_sparse_to_dense(z_s.to(DEV), ti, inter)
    want = torch.zeros(rows, inter, dtype=dtype).scatter_(1, torch.from_numpy(idx), z_s)
    assert torch.equal(dense.cpu(), want)
    assert torch.equal(K().gather_dense_to_sparse(dense, ti).cpu(), z_s)
    # GCP recompute + backward aux
    rs, rz = O.gcp_recompute(vals, u_s)
    ks, kz = K().gcp_recompute(vals.to(DEV), u_s.to(DEV))
    tol = dict(rtol=1e-5, atol=1e-6) if dtype == torch.float32 else dict(rtol=2e-2, atol=2e-2)
    close(ks, rs, **tol)
    close(kz, rz, **tol)
    gg, gu = O.sparse_backward_aux(idx, vals, u_s, rs, GZ, inter)
    kg, ku = K().sparse_backward_aux(ti, vals.to(DEV), u_s.to(DEV), rs.to(DEV), GZ.to(DEV), inter)
    close(kg, gg, **tol)
    close(ku, gu, **tol)
    kg2, ku2 = K().sparse_backward_aux(ti, vals.to(DEV), u_s.to(DEV), None, GZ.to(DEV), inter)
    close(kg2, gg, **tol)
    if dtype == torch.bfloat16:
        # the fused GCP recompute + scatter equals the two-step form bit for bit
        fs, fz = K().gcp_recompute_scatter(vals.to(DEV), u_s.to(DEV), ti, inter)
        assert torch.equal(fs.cpu(), ks.cpu())
        assert torch.equal(fz.cpu(), K().scatter_sparse_to_dense(kz, ti, inter).cpu())


@pytest.mark.parametrize("idx_dtype", [torch.int16, torch.int32, torch.int64])
@pytest.mark.parametrize("k", [1024, 383])
def test_sparse_aux_row_kernels_vector_and_element_entry_loads(idx_dtype, k):
    """The row kernels (forward aux, GCP recompute + scatter, backward aux)
    read a row's sparse entries four at a time (8-byte loads and stores)
    when k is a multiple of 4 and the rows are aligned, else one by one:
    both forms give the same bits.  Misaligned copies of the sparse
    inputs (views one element into a buffer) force the element form."""
    rows, inter = 256, 5461
    g = gen(7)
    G = torch.randn(rows, inter, generator=g).to(torch.bfloat16)
    GZ = torch.randn(rows, inter, generator=g).to(torch.bfloat16).to(DEV)
    U = torch.randn(rows, k, generator=g).to(torch.bfloat16)
    idx = O.topk_indices(G, k)
    vals = O.gather_rows(G, idx).to(DEV)
    u_s = U.to(DEV)
    ti = torch.from_numpy(idx).to(idx_dtype).to(DEV)

    def shifted(t):  # same values, base one element past an aligned buffer
        buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=DEV)
        v = buf[1:].view(t.shape)
        v.copy_(t)
        return v

    Gd = K().aligned_rows(G.to(DEV))  # 16-byte aligned rows: the row kernel
    f1 = K().sparse_forward_aux(vals, ti, Gd, inter)
    f2 = K().sparse_forward_aux(shifted(vals), shifted(ti), Gd, inter)
    for a, b in zip(f1, f2):
        assert torch.equal(a, b)
    s1, z1 = K().gcp_recompute_scatter(vals, u_s, ti, inter)
    s2, z2 = K().gcp_recompute_scatter(shifted(vals), shifted(u_s), shifted(ti), inter)
    assert torch.equal(s1, s2) and torch.equal(z1, z2)
    gg1, gu1 = K().sparse_backward_aux(ti, vals, u_s, s1, GZ, inter)
    gg2, gu2 = K().sparse_backward_aux(shifted(ti), shifted(vals), shifted(u_s), shifted(s1), GZ, inter)
    assert torch.equal(gg1, gg2) and torch.equal(gu1, gu2)
    # and against the oracle
    rs, rz = O.gcp_recompute(vals.cpu(), U)
    close(s1, rs, rtol=2e-2, atol=2e-2)
    gg, gu = O.sparse_backward_aux(idx, vals.cpu(), U, rs, GZ.cpu(), inter)
    close(gg1, gg, rtol=2e-2, atol=2e-2)
    close(gu1, gu, rtol=2e-2, atol=2e-2)


# ------------------------------------------------------------------- decode
@pytest.mark.parametrize("nb", [1, 4, 16])
def test_global_decode_path_1b(nb):
    d, inter, k = 2048, 5461, 1024
    g = gen(100 + nb)
    x = torch.randn(nb, d, generator=g).to(torch.bfloat16)
    wg = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16)
    wu = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16)
    wd = (torch.randn(d, inter, generator=g) * 0.02).to(torch.bfloat16)
    xd, wgd, wud = x.to(DEV), wg.to(DEV), wu.to(DEV)
    wdt = wd.t().contiguous().to(DEV)
    G = K().gemv(xd, wgd)
    Gc = G.cpu()
    bf16_close(Gc, x.float() @ wg.float().t(), ulps=1, atol=1e-3)
    y_ref, idx_ref, z_ref = O.masked_reference(x, wg, wu, wd, k, g_override=Gc)
    vals, idx, _ = K().topk_rows(G, k)
    assert np.array_equal(idx.cpu().numpy(), idx_ref)
    z = K().selected_up_silu(xd, vals, idx, wud)
    bf16_close(z, z_ref, ulps=2, atol=1e-4)
    y = K().selected_down(z, idx, wdt)
    close(y, O.selected_down(z.cpu(), idx_ref, wd.t().contiguous()), rtol=1e-2, atol=1e-3)
    y2 = K().global_after_gate(xd, G, wud, wdt, k)
    close(y2, y_ref)
    # the fused path sums the same f32 products in another order
    close(y2, y, rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("nb,inter,d", [(1, 5461, 2048), (3, 5461, 2048), (4, 5461, 2048),
                                         (5, 5461, 2048), (16, 5461, 2048), (4, 1000, 256),
                                         (8, 777, 4096), (7, 50, 1024), (12, 3001, 384)])
def test_global_decode_layer_entry(nb, inter, d):
    """moc_global_decode_bf16 against gemv + global_after_gate on the same
    G: the same selected channels bit for bit, y within one bf16 ulp (where
    hidden % 256 == 0 the layer entry's after-gate kernel sums each output
    column in another f32 order) and within 2e-2 of the oracle on that
    selection; two calls in a row give the same bits, and a call of the
    selected-row path in between (same workspace, its counters) changes
    nothing.  (8, 777, 4096) takes the GEMV fallback that launches twice;
    (4, 1000, 256) and (12, 3001, 384) the selected-row after-gate kernel;
    every G row is also checked against the f32 product."""
    k = max(1, inter // 5)
    g = gen(360 + nb + inter)
    x = torch.randn(nb, d, generator=g).to(torch.bfloat16).to(DEV)
    wg = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    wu = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    wdt = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    G = K().gemv(x, wg)
    Gc = G.cpu()
    bf16_close(Gc, x.float().cpu() @ wg.float().cpu().t(), ulps=1, atol=1e-3)
    i_two = torch.empty(nb, k, dtype=torch.int32, device=DEV)
    y_two = K().global_after_gate(x, G, wu, wdt, k, idx_out=i_two)
    i_one = torch.empty(nb, k, dtype=torch.int32, device=DEV)
    ws = K().global_decode_workspace(nb, inter, k, d, DEV)
    y_first = None
    for _ in range(2):  # the counters are left zero for the next call
        y_one = K().global_decode(x, wg, wu, wdt, k, workspace=ws, idx_out=i_one)
        assert torch.equal(i_one, i_two)
        if y_first is None:
            y_first = y_one.clone()
            # the selected-row kernel on the same workspace in between
            K().global_after_gate(x, G, wu, wdt, k, workspace=ws[:K().global_after_gate_workspace_bytes(
                nb, inter, k, d)])
        assert torch.equal(y_one, y_first)
    bf16_close(y_one, y_two, ulps=1, atol=1e-4)
    y_ref, idx_ref, _ = O.masked_reference(x.cpu(), wg.cpu(), wu.cpu(), wdt.cpu().t().contiguous(), k,
                                           g_override=Gc)
    assert np.array_equal(i_one.cpu().numpy(), idx_ref)
    close(y_one, y_ref)


@pytest.mark.parametrize("nb", [1, 4, 16])
def test_down_t_padded_pitch_same_bits(nb):
    """W_down^T at the module's decode layout (rows padded by 128 bytes,
    down_weight_t_for_decode) gives the same bits as the contiguous matrix
    on every decode entry that reads it: the layer entries, the after-gate
    kernel (plain and residual), the selected Down, the 2:8 selected Down."""
    d, inter, k = 2048, 5461, 1024
    g = gen(390 + nb)
    x = torch.randn(nb, d, generator=g).to(torch.bfloat16).to(DEV)
    res = torch.randn(nb, d, generator=g).to(torch.bfloat16).to(DEV)
    nw = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16).to(DEV)
    wg = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    wu = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    wd = (torch.randn(d, inter, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    wdt = wd.t().contiguous()
    wdp = K().down_weight_t_for_decode(wd)
    assert wdp.shape == wdt.shape and wdp.stride(0) == d + 64 and torch.equal(wdp, wdt)
    ws = K().global_decode_workspace(nb, inter, k, d, DEV)
    assert torch.equal(K().global_decode(x, wg, wu, wdp, k, workspace=ws),
                       K().global_decode(x, wg, wu, wdt, k, workspace=ws))
    if nb <= 4:
        assert torch.equal(K().global_decode_rmsnorm_residual(x, nw, 1e-6, wg, wu, wdp, k, workspace=ws),
                           K().global_decode_rmsnorm_residual(x, nw, 1e-6, wg, wu, wdt, k, workspace=ws))
    G = K().gemv(x, wg)
    for r in (None, res):
        assert torch.equal(K().global_after_gate(x, G, wu, wdp, k, residual=r),
                           K().global_after_gate(x, G, wu, wdt, k, residual=r))
    vals, idx, _ = K().topk_rows(G, k)
    z = K().selected_up_silu(x, vals, idx, wu)
    assert torch.equal(K().selected_down(z, idx, wdp), K().selected_down(z, idx, wdt))
    wd8 = (torch.randn(d, 5464, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    wg8 = (torch.randn(5464, d, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    wu8 = (torch.randn(5464, d, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    idx8, sz8 = K().grouped_top2_up_silu(x, wg8, wu8)
    wd8p, wd8t = K().down_weight_t_for_decode(wd8), wd8.t().contiguous()
    assert torch.equal(K().selected_grouped_down(sz8, idx8, wd8p), K().selected_grouped_down(sz8, idx8, wd8t))
    assert torch.equal(K().selected_grouped_down(sz8, idx8, wd8p, residual=res),
                       K().selected_grouped_down(sz8, idx8, wd8t, residual=res))


@pytest.mark.parametrize("nb", [1, 2, 3, 4])
def test_global_decode_rmsnorm_residual(nb):
    """moc_global_decode_rmsnorm_residual_bf16: the decoder layer's FFN half
    x + FFN(RMSNorm(x)) in two launches.  Its norm and gate rows are the
    gemv_rmsnorm kernel's (same bits), so the selection equals the oracle's
    Top-K of gemv_rmsnorm's G bit for bit, and y is within 2e-2 of bf16(x +
    bf16(oracle FFN of gemv_rmsnorm's xn)); a second call gives the same
    bits."""
    d, inter, k, eps = 2048, 5461, 1024, 1e-6
    g = gen(380 + nb)
    x = (torch.randn(nb, d, generator=g) * 2).to(torch.bfloat16).to(DEV)
    nw = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16).to(DEV)
    wg = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    wu = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    wdt = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    G, xn = K().gemv_rmsnorm(x, nw, eps, wg)
    io = torch.full((nb, k), -1, dtype=torch.int32, device=DEV)
    ws = K().global_decode_workspace(nb, inter, k, d, DEV)
    y = K().global_decode_rmsnorm_residual(x, nw, eps, wg, wu, wdt, k, workspace=ws, idx_out=io)
    y2 = K().global_decode_rmsnorm_residual(x, nw, eps, wg, wu, wdt, k, workspace=ws)
    assert torch.equal(y, y2)
    ffn_ref, idx_ref, _ = O.masked_reference(xn.cpu(), wg.cpu(), wu.cpu(), wdt.cpu().t().contiguous(), k,
                                             g_override=G.cpu())
    assert np.array_equal(io.cpu().numpy(), idx_ref)
    close(y, (x.cpu().float() + ffn_ref.float()).to(torch.bfloat16))


@pytest.mark.parametrize("nb", [1, 2, 3, 4])
def test_gemv_rmsnorm_fused_prologue(nb):
    """The gate GEMV with the FFN's RMSNorm in front: xn matches the
    reference formula (x.float() * rsqrt(mean(x^2) + eps)).to(bf16) * w to
    one bf16 ulp (the f32 mean is summed in another order), and y equals the
    plain GEMV of that xn bit for bit (same dot products)."""
    d, inter, eps = 2048, 5461, 1e-6
    g = gen(300 + nb)
    x = (torch.randn(nb, d, generator=g) * 3).to(torch.bfloat16).to(DEV)
    nw = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16).to(DEV)
    wg = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    y, xn = K().gemv_rmsnorm(x, nw, eps, wg)
    xf = x.float()
    want = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(torch.bfloat16) * nw
    bf16_close(xn, want.float().cpu(), ulps=1, atol=0)
    assert torch.equal(y, K().gemv(xn, wg))


@pytest.mark.parametrize("nb", [1, 4])
def test_global_after_gate_residual(nb):
    """The residual add in the after-gate kernel's last step equals the
    bf16 add of the residual and the plain result, bit for bit."""
    d, inter, k = 2048, 5461, 1024
    g = gen(320 + nb)
    x = torch.randn(nb, d, generator=g).to(torch.bfloat16).to(DEV)
    res = torch.randn(nb, d, generator=g).to(torch.bfloat16).to(DEV)
    wg = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    wu = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    wdt = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    G = K().gemv(x, wg)
    y = K().global_after_gate(x, G, wu, wdt, k)
    yr = K().global_after_gate(x, G, wu, wdt, k, residual=res)
    assert torch.equal(yr, res + y)


@pytest.mark.parametrize("nb", [1, 3, 4])
def test_grouped_2of8_rmsnorm_and_residual(nb):
    """The 2:8 decode kernels with the FFN's neighbours inside: gate/up of
    RMSNorm(x) equals gate/up of the kernel-side norm (gemv_rmsnorm's xn,
    same rounding) bit for bit, and the residual form of the selected Down
    equals residual + Down."""
    d, inter, eps = 2048, 5464, 1e-6
    g = gen(340 + nb)
    x = (torch.randn(nb, d, generator=g) * 2).to(torch.bfloat16).to(DEV)
    nw = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16).to(DEV)
    wg = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    wu = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    wdt = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    _, xn = K().gemv_rmsnorm(x, nw, eps, wg)
    idx_f, sz_f = K().grouped_top2_up_silu(x, wg, wu, norm_weight=nw, eps=eps)
    idx, sz = K().grouped_top2_up_silu(xn, wg, wu)
    assert torch.equal(idx_f, idx) and torch.equal(sz_f, sz)
    y = K().selected_grouped_down(sz, idx, wdt)
    yr = K().selected_grouped_down(sz, idx, wdt, residual=x)
    assert torch.equal(yr, x + y)


def test_grouped_2of8_integer_inputs_bitexact():
    """Integer-valued bf16 inputs make G and U exact, so the fused kernel's
    selection can be compared bit-exactly with the oracle."""
    rng = np.random.default_rng(9)
    for nb, d, inter in ((3, 64, 96), (40, 64, 96), (600, 256, 400)):
        x = torch.tensor(rng.integers(-3, 4, (nb, d)), dtype=torch.bfloat16)
        wg = torch.tensor(rng.integers(-2, 3, (inter, d)), dtype=torch.bfloat16)
        wu = torch.tensor(rng.integers(-2, 3, (inter, d)), dtype=torch.bfloat16)
        wd = torch.tensor(rng.integers(-2, 3, (d, inter)), dtype=torch.bfloat16) * 0.125
        idx_ref, sz_ref, _ = O.grouped_top2_up_silu(x, wg, wu)
        idx, sz = K().grouped_top2_up_silu(x.to(DEV), wg.to(DEV), wu.to(DEV))
        assert np.array_equal(idx.cpu().numpy(), idx_ref)
        bf16_close(sz, sz_ref, ulps=1, atol=0)
        y = K().selected_grouped_down(sz, idx, wd.t().contiguous().to(DEV))
        close(y, O.selected_down(sz.cpu(), idx_ref, wd.t().contiguous()), rtol=1e-2, atol=1e-2)


def exact_projection_inputs(nb, d, inter, seed):
    """x, W_gate, W_up whose products are exact in f32 in any summation
    order: integer x in [-1, 1], weights (integers in [-2, 2]) * 2^-7, so
    every partial sum is a multiple of 2^-7 below 2^5 in magnitude (G has the
    1b shape's spread, std ~0.4).  G and U are then the same bits on the
    device and in the oracle whatever the kernel's accumulation order, and
    the many equal values exercise the tie rule."""
    rng = np.random.default_rng(seed)
    x = torch.tensor(rng.integers(-1, 2, (nb, d)), dtype=torch.bfloat16)
    wg = (torch.tensor(rng.integers(-2, 3, (inter, d)), dtype=torch.float32) / 128).to(torch.bfloat16)
    wu = (torch.tensor(rng.integers(-2, 3, (inter, d)), dtype=torch.float32) / 128).to(torch.bfloat16)
    wd = (torch.randn(d, inter, generator=gen(seed)) * 0.02).to(torch.bfloat16)
    return x, wg, wu, wd


@pytest.mark.parametrize("nb", [1, 3, 4, 9, 16])
def test_global_decode_exact_inputs_bitexact(nb):
    """The layer entry (gate + dense-U GEMV, then the column-owning
    after-gate kernel) on exact projections: G and U are the same bits on
    the device and in the oracle whatever the accumulation order, and G holds
    few distinct values (ties at the threshold in every row), so the
    kernel's own selection (idx_out) is compared with the oracle's Top-K of
    the exact G bit for bit without handing it the device's G; y within 2e-2
    of the oracle (W_down^T at the module's padded row pitch)."""
    d, inter, k = 2048, 5461, 1024
    x, wg, wu, wd = exact_projection_inputs(nb, d, inter, 600 + nb)
    xd, wgd, wud = x.to(DEV), wg.to(DEV), wu.to(DEV)
    wdp = K().down_weight_t_for_decode(wd.to(DEV))
    io = torch.full((nb, k), -1, dtype=torch.int32, device=DEV)
    y = K().global_decode(xd, wgd, wud, wdp, k, idx_out=io)
    y_ref, idx_ref, _ = O.masked_reference(x, wg, wu, wd, k)
    assert np.array_equal(io.cpu().numpy(), idx_ref)
    close(y, y_ref)


@pytest.mark.parametrize("hidden,inter,k", [(1024, 2736, 512), (2048, 5461, 1), (2048, 5461, 5461),
                                            (2048, 5461, 4000), (256, 100, 7), (768, 8192, 2048)])
def test_global_decode_layer_entry_shapes(hidden, inter, k):
    """The column-owning layer at other shapes, on exact projections so
    the selection is compared with the oracle's directly: k of 1 and of
    every channel, k = 4000 of 5461 (the k-th largest gate value is
    negative, below the selection's 32-binade window under the row maximum:
    the byte-digit passes run), a 100-channel row, I = 8192 (16 channels per
    thread); idx_out bit-exact, y within 2e-2 of the oracle, at 1 and 2
    tokens."""
    for nb in (1, 2):
        x, wg, wu, wd = exact_projection_inputs(nb, hidden, inter, hidden + inter + k + nb)
        io = torch.full((nb, k), -1, dtype=torch.int32, device=DEV)
        y = K().global_decode(x.to(DEV), wg.to(DEV), wu.to(DEV), K().down_weight_t_for_decode(wd.to(DEV)), k,
                              idx_out=io)
        y_ref, idx_ref, _ = O.masked_reference(x, wg, wu, wd, k)
        assert np.array_equal(io.cpu().numpy(), idx_ref), (nb, hidden, inter, k)
        close(y, y_ref)


@pytest.mark.parametrize("nb", [1, 4, 16, 64, 300, 4096])
def test_grouped_2of8_1b_exact_inputs(nb):
    """MoC 2:8 at the 1b shape (config 4 at nb = 4096): with exact
    projections the fused gate/up kernel's selection equals the oracle's bit
    for bit on every row (decode kernel up to 16 tokens, the MFMA GEMM with
    the selecting epilogue above), sz within one bf16 ulp and y within
    2e-2 on every element."""
    d, inter = 2048, 5464
    x, wg, wu, wd = exact_projection_inputs(nb, d, inter, 200 + nb)
    idx_ref, sz_ref, _ = O.grouped_top2_up_silu(x, wg, wu)
    idx, sz = K().grouped_top2_up_silu(x.to(DEV), wg.to(DEV), wu.to(DEV))
    assert np.array_equal(idx.cpu().numpy(), idx_ref)
    bf16_close(sz, sz_ref, ulps=1, atol=0)
    wdt = wd.t().contiguous()
    y = K().selected_grouped_down(sz, idx, wdt.to(DEV))
    close(y, O.selected_down(sz_ref, idx_ref, wdt))


@pytest.mark.parametrize("nb", [1, 3, 4, 9, 16])
def test_moc28_decode_exact_inputs(nb):
    """The 2:8 decode layer entry (gate/up GEMV pair, then one launch that
    picks the top 2 of every 8 channels and sums the selected Down rows per
    column block) on exact projections: its selection (idx_out) equals the
    oracle's bit for bit on every group, ties included, without handing it
    the device's G; y within 2e-2 of the oracle's Down of the oracle's sz;
    the residual form equals residual + y bit for bit (one rounding of the
    FFN, then of the sum); W_down^T at the module's padded pitch."""
    d, inter = 2048, 5464
    x, wg, wu, wd = exact_projection_inputs(nb, d, inter, 640 + nb)
    idx_ref, sz_ref, _ = O.grouped_top2_up_silu(x, wg, wu)
    xd, wgd, wud = x.to(DEV), wg.to(DEV), wu.to(DEV)
    wdp = K().down_weight_t_for_decode(wd.to(DEV))
    io = torch.full((nb, inter // 4), -1, dtype=torch.int64, device=DEV)
    y = K().moc28_decode(xd, wgd, wud, wdp, idx_out=io)
    assert np.array_equal(io.cpu().numpy(), idx_ref)
    wdt = wd.t().contiguous()
    close(y, O.selected_down(sz_ref, idx_ref, wdt))
    y_two = K().selected_grouped_down(*reversed(K().grouped_top2_up_silu(xd, wgd, wud)), wdp)
    close(y, y_two)
    res = torch.randn(nb, d, generator=gen(650 + nb)).to(torch.bfloat16).to(DEV)
    assert torch.equal(K().moc28_decode(xd, wgd, wud, wdp, residual=res), res + y)


@pytest.mark.parametrize("nb", [1, 2, 3, 4])
def test_moc28_decode_rmsnorm_residual(nb):
    """The 2:8 decode layer as the decoder's FFN half x + FFN(RMSNorm(x)):
    its norm and gate rows are the gemv_rmsnorm kernel's (same bits), so the
    selection equals the oracle's top-2-of-8 of gemv_rmsnorm's G bit for bit;
    y within 2e-2 of bf16(x + bf16(oracle FFN of gemv_rmsnorm's xn)); the
    same as the two-kernel 2:8 path (norm inside the gate/up kernel, the
    residual inside the selected Down) within 2e-2; a second call on the
    same workspace gives the same bits."""
    d, inter, eps = 2048, 5464, 1e-6
    g = gen(660 + nb)
    x = (torch.randn(nb, d, generator=g) * 2).to(torch.bfloat16).to(DEV)
    nw = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16).to(DEV)
    wg = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    wu = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    wdt = K().down_weight_t_for_decode((torch.randn(d, inter, generator=g) * 0.02).to(torch.bfloat16).to(DEV))
    G, xn = K().gemv_rmsnorm(x, nw, eps, wg)
    U = K().gemv(xn, wu)
    io = torch.full((nb, inter // 4), -1, dtype=torch.int64, device=DEV)
    ws = torch.zeros(N().query("moc_moc28_decode_workspace_size", nb, inter, d), dtype=torch.uint8, device=DEV)
    y = K().moc28_decode(x, wg, wu, wdt, norm_weight=nw, eps=eps, residual=x, workspace=ws, idx_out=io)
    assert torch.equal(y, K().moc28_decode(x, wg, wu, wdt, norm_weight=nw, eps=eps, residual=x, workspace=ws))
    wd_cpu = wdt[:, :d].cpu().t().contiguous()
    ffn_ref, idx_ref, _ = O.masked_reference(xn.cpu(), wg.cpu(), wu.cpu(), wd_cpu, inter // 4, grouped=True,
                                             g_override=G.cpu(), u_override=U.cpu())
    assert np.array_equal(io.cpu().numpy(), idx_ref)
    close(y, (x.cpu().float() + ffn_ref.float()).to(torch.bfloat16))
    idx2, sz2 = K().grouped_top2_up_silu(x, wg, wu, norm_weight=nw, eps=eps)
    assert torch.equal(idx2, io)
    close(y, K().selected_grouped_down(sz2, idx2, wdt, residual=x))


@pytest.mark.parametrize("nb,hidden,inter", [(1, 256, 8), (16, 256, 8), (2, 768, 8192), (12, 768, 8192),
                                             (5, 1024, 2736), (1, 2048, 4096), (16, 2048, 4104),
                                             (8, 4096, 1024), (2, 8192, 1024), (12, 6144, 2048)])
def test_moc28_decode_shapes(nb, hidden, inter):
    """The 2:8 decode layer at other shapes on exact projections: one group
    (inter 8, k 2), the largest inter (8192, two groups per thread), inter
    either side of the one-group-per-thread limit (4096 / 4104), 64- and
    128-column workgroups (up to 8 tokens / beyond), column-block counts
    that are and are not a multiple of the 8 XCDs, hidden sizes past the
    row-per-wave GEMV's 4096 (the streaming and pipelined GEMV forms);
    selection bit-exact against the oracle, y within 2e-2."""
    x, wg, wu, wd = exact_projection_inputs(nb, hidden, inter, 670 + nb + inter)
    idx_ref, sz_ref, _ = O.grouped_top2_up_silu(x, wg, wu)
    io = torch.full((nb, inter // 4), -1, dtype=torch.int64, device=DEV)
    y = K().moc28_decode(x.to(DEV), wg.to(DEV), wu.to(DEV), K().down_weight_t_for_decode(wd.to(DEV)),
                         idx_out=io)
    assert np.array_equal(io.cpu().numpy(), idx_ref), (nb, hidden, inter)
    close(y, O.selected_down(sz_ref, idx_ref, wd.t().contiguous()))


def plain_linear(x, w):
    """x @ w.T on the MFMA GEMM without a K split (moc_gemm with no
    workspace): the accumulation order of the 2:8 selecting GEMM."""
    M, Kd = x.shape
    out = torch.empty(M, w.shape[0], dtype=torch.bfloat16, device=DEV)
    N().call("moc_gemm", N().MOC_BF16, M, w.shape[0], Kd, x.data_ptr(), x.stride(0), 1, w.data_ptr(),
             1, w.stride(0), 0, None, 0, 0, None, 0, 0, out.data_ptr(), out.stride(0), N().MOC_BF16,
             N().stream_of(x))
    return out


@pytest.mark.parametrize("nb", [300, 4096])
def test_grouped_2of8_1b_device_projections(nb):
    """Random N(0,1) tokens and N(0,0.02) weights at the 1b shape: the oracle
    gets the device's own bf16 G and U (the same MFMA GEMM the fused kernel
    runs, without a K split); the selection must match bit for bit on every
    row, sz and y within 2e-2 (no row may differ)."""
    d, inter = 2048, 5464
    g = gen(260 + nb)
    x = torch.randn(nb, d, generator=g).to(torch.bfloat16)
    wg = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16)
    wu = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16)
    wd = (torch.randn(d, inter, generator=g) * 0.02).to(torch.bfloat16)
    xd = x.to(DEV)
    G = plain_linear(xd, wg.to(DEV)).cpu()
    U = plain_linear(xd, wu.to(DEV)).cpu()
    idx_ref, sz_ref, _ = O.grouped_top2_up_silu(x, wg, wu, g_override=G, u_override=U)
    idx, sz = K().grouped_top2_up_silu(xd, wg.to(DEV), wu.to(DEV))
    assert np.array_equal(idx.cpu().numpy(), idx_ref)
    close(sz, sz_ref)
    bf16_close(sz, sz_ref, ulps=1, atol=0)
    wdt = wd.t().contiguous()
    y = K().selected_grouped_down(sz, idx, wdt.to(DEV))
    close(y, O.selected_down(sz_ref, idx_ref, wdt))
    y_ref, idx_m, _ = O.masked_reference(x, wg, wu, wd, inter // 4, grouped=True, g_override=G,
                                         u_override=U)
    assert np.array_equal(idx_m, idx_ref)
    close(y, y_ref)


def random_2of8(nb, inter, seed):
    """A random 2:8 selection in moc_grouped_top2_up_silu_bf16's layout:
    per 8-group two distinct channels in either order, N(0,1) bf16 values."""
    g = gen(seed)
    groups = inter // 8
    pos = torch.argsort(torch.rand(nb, groups, 8, generator=g), dim=-1)[..., :2]
    idx = (pos + 8 * torch.arange(groups)[None, :, None]).reshape(nb, groups * 2)
    sz = torch.randn(nb, groups * 2, generator=g).to(torch.bfloat16)
    return idx.to(torch.int64), sz


def packed28(sz, idx, inter):
    """moc_pack28_bf16 into fresh buffers -> (ap, ld_ap, meta, meta_rows)."""
    nb = sz.shape[0]
    nt = (inter + 63) // 64
    ld_ap = 32 * nt
    meta_rows = (nb + 255) // 256 * 256
    ap = torch.full((nb, ld_ap), 7.0, dtype=torch.bfloat16, device=DEV)  # pad columns must be zeroed
    meta = torch.full((nt, meta_rows, 2), -1, dtype=torch.int32, device=DEV)
    N().call("moc_pack28_bf16", sz.data_ptr(), idx.data_ptr(), nb, inter, ap.data_ptr(), ld_ap,
             meta.data_ptr(), meta_rows, None, N().stream_of(sz))
    return ap, ld_ap, meta, meta_rows


def sparse28_down(ap, ld_ap, meta, meta_rows, inter, w, w_kc):
    nb = ap.shape[0]
    hidden = w.shape[0] if w_kc else w.shape[1]
    y = torch.empty(nb, hidden, dtype=torch.bfloat16, device=DEV)
    ws_bytes = N().query("moc_sparse28_down_workspace_size", nb, inter, hidden)
    ws = torch.zeros(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
    N().call("moc_sparse28_down_bf16", ap.data_ptr(), ld_ap, meta.data_ptr(), meta_rows, nb, inter,
             w.data_ptr(), w.stride(0), int(w_kc), hidden, y.data_ptr(), y.stride(0), ws.data_ptr(),
             ws_bytes, N().stream_of(ap))
    return y, ws


@pytest.mark.parametrize("nb,hidden,inter", [(65, 64, 200), (300, 2048, 5464), (1000, 768, 2048),
                                             (700, 72, 96), (4096, 2048, 5464)])
@pytest.mark.parametrize("w_kc", [0, 1])
def test_sparse28_down_vs_oracle(nb, hidden, inter, w_kc):
    """The 2:4-packed 2:8 Down on the structured-sparse MFMA against the
    oracle's gathered Down (f32 sums of the selected rows): whole tiles,
    partial channel tiles (inter % 64 != 0), split-K (65 tokens: one tile
    row), the two-part K split (4096 tokens: 128 tiles) and both W layouts;
    every element within 2e-2.  The workspace's counters are zero again
    after the call."""
    idx, sz = random_2of8(nb, inter, 300 + nb + inter)
    wd = (torch.randn(hidden, inter, generator=gen(301 + nb)) * 0.02).to(torch.bfloat16)
    wdt = wd.t().contiguous()
    ap, ld_ap, meta, meta_rows = packed28(sz.to(DEV), idx.to(DEV), inter)
    w = (wd if w_kc else wdt).to(DEV)
    y, ws = sparse28_down(ap, ld_ap, meta, meta_rows, inter, w, w_kc)
    close(y, O.selected_down(sz, idx.numpy(), wdt))
    assert int(ws[:4096].count_nonzero()) == 0
    # the op path (pack + sparse GEMM over W_down^T inside one entry point)
    y2 = K().selected_grouped_down(sz.to(DEV), idx.to(DEV), wdt.to(DEV))
    if nb > 64:
        assert torch.equal(y2, sparse28_down(ap, ld_ap, meta, meta_rows, inter, wdt.to(DEV), 0)[0])


@pytest.mark.parametrize("nb,hidden,inter", [(300, 2048, 5464), (4096, 2048, 5464), (130, 64, 200)])
def test_grouped_2of8_packed_epilogue(nb, hidden, inter):
    """The gate/up kernel's packed epilogue writes exactly what
    moc_pack28_bf16 makes of the (idx, sz) the same kernel writes unpacked
    (every stored value and position bit of every token), and the module's
    prefill path (packed gate/up, then the sparse Down) matches the oracle."""
    g = gen(40 + nb)
    x = torch.randn(nb, hidden, generator=g).to(torch.bfloat16).to(DEV)
    wg = (torch.randn(inter, hidden, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    wu = (torch.randn(inter, hidden, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    idx, sz = K().grouped_top2_up_silu(x, wg, wu)
    ap_ref, _, meta_ref, _ = packed28(sz, idx, inter)
    ap, meta = K().packed28_buffers(nb, inter, DEV)
    K().grouped_top2_up_silu_packed(x, wg, wu, ap, meta)
    assert torch.equal(ap, ap_ref)
    assert torch.equal(meta[:, :nb], meta_ref[:, :nb])
    from moc_amd.inference.inference_ffn import InferenceMoCSwiGLUFFN
    m = InferenceMoCSwiGLUFFN(hidden, inter, inter // 4, grouped_a=2, grouped_b=8).to(DEV, torch.bfloat16)
    with torch.no_grad():
        m.gate_proj.weight.copy_(wg)
        m.up_proj.weight.copy_(wu)
        m.down_proj.weight.copy_((torch.randn(hidden, inter, generator=g) * 0.02).to(torch.bfloat16))
    y = m(x, mode="moc_inference_grouped_top2of8")
    wdt = m.down_proj.weight.t().contiguous().cpu()
    close(y, O.selected_down(sz.cpu(), idx.cpu().numpy(), wdt))
    y2 = m(x, mode="moc_inference_grouped_top2of8")  # workspace reused: same result
    assert torch.equal(y, y2)


def test_pack28_layout_and_bad_indices():
    """moc_pack28_bf16 against a CPU packing of the documented layout (values
    in channel order per 4-group, zeros elsewhere, 2-bit positions), and an
    index outside its 8-group turns that token's output into NaN."""
    nb, inter = 70, 136  # 3 channel tiles, the last one partial
    idx, sz = random_2of8(nb, inter, 17)
    ap, ld_ap, meta, meta_rows = packed28(sz.to(DEV), idx.to(DEV), inter)
    nt = (inter + 63) // 64
    want_ap = torch.zeros(nb, ld_ap, dtype=torch.bfloat16)
    want_meta = torch.zeros(nt, meta_rows, 2, dtype=torch.int64)
    dense = torch.zeros(nb, nt * 64, dtype=torch.bfloat16)
    for r in range(nb):
        dense[r, idx[r]] = sz[r]
    sel = torch.zeros(nb, nt * 64, dtype=torch.bool)
    sel.scatter_(1, idx, True)
    for r in range(meta_rows):
        for q in range(nt * 16):  # 4-groups
            chans = [c for c in range(4 * q, 4 * q + 4) if r < nb and sel[r, c]]
            if len(chans) == 2:
                p = [chans[0] - 4 * q, chans[1] - 4 * q]
            elif len(chans) == 1:
                p = [0, 1] if chans[0] == 4 * q else [0, chans[0] - 4 * q]
            else:
                p = [0, 1]
            if r < nb:
                for slot in range(2):
                    c = 4 * q + p[slot]
                    want_ap[r, 2 * q + slot] = dense[r, c] if sel[r, c] else 0.0
            t, rem = divmod(q, 16)
            s, rem = divmod(rem, 8)
            h, j = divmod(rem, 4)
            for slot in range(2):
                want_meta[t, r, h] |= p[slot] << (16 * s + 2 * (2 * j + slot))
    assert torch.equal(ap.cpu(), want_ap)
    assert torch.equal(meta.cpu().to(torch.int64) & 0xFFFFFFFF, want_meta)
    bad = idx.clone()
    bad[5, 6] = bad[5, 6] + 8  # channel of the next group
    ap, ld_ap, meta, meta_rows = packed28(sz.to(DEV), bad.to(DEV), inter)
    wd = (torch.randn(64, inter, generator=gen(5)) * 0.02).to(torch.bfloat16).to(DEV)
    y, _ = sparse28_down(ap, ld_ap, meta, meta_rows, inter, wd, 1)
    assert bool(torch.isnan(y[5]).all()) and not bool(torch.isnan(y[4]).any())


def tie_heavy_rows(nb, inter, kind, seed):
    g = gen(seed)
    if kind == "levels":  # seven values: ~780 channels share each one
        v = torch.randint(-3, 4, (nb, inter), generator=g).float() * 0.25
    elif kind == "zeros":  # +-0 and a few levels; -0.0 ranks equal to +0.0
        v = torch.randint(-1, 2, (nb, inter), generator=g).float()
        v = torch.where(v == 0, torch.where(torch.rand(nb, inter, generator=g) < 0.5,
                                            torch.tensor(-0.0), torch.tensor(0.0)), v)
    else:  # the 1b decode distribution: ~6 values in the threshold's bf16 bucket
        v = torch.randn(nb, inter, generator=g) * 0.9
    return v.to(torch.bfloat16)


@pytest.mark.parametrize("nb", [1, 4, 16])
@pytest.mark.parametrize("kind", ["levels", "zeros", "gauss"])
def test_after_gate_selection_bitexact(nb, kind):
    """The fused after-gate kernel ranks every gate row itself (each
    workgroup of a token repeats the radix select); its selection, read back
    through idx_out, equals the oracle's Top-K bit for bit on tie-heavy 1b
    rows, for the plain and the residual form, and y agrees with the oracle
    computed on that selection."""
    d, inter, k = 2048, 5461, 1024
    G = tie_heavy_rows(nb, inter, kind, 500 + nb)
    g = gen(510 + nb)
    x = torch.randn(nb, d, generator=g).to(torch.bfloat16)
    wu = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16)
    wdt = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16)
    res = torch.randn(nb, d, generator=g).to(torch.bfloat16)
    idx_ref = O.topk_indices(G, k)
    xd, Gd, wud, wdtd = x.to(DEV), G.to(DEV), wu.to(DEV), wdt.to(DEV)
    io = torch.full((nb, k), -1, dtype=torch.int32, device=DEV)
    y = K().global_after_gate(xd, Gd, wud, wdtd, k, idx_out=io)
    assert np.array_equal(io.cpu().numpy(), idx_ref)
    io2 = torch.full((nb, k), -1, dtype=torch.int32, device=DEV)
    yr = K().global_after_gate(xd, Gd, wud, wdtd, k, idx_out=io2, residual=res.to(DEV))
    assert torch.equal(io2, io)
    assert torch.equal(yr, res.to(DEV) + y)
    vals = O.gather_rows(G, idx_ref)
    z_ref = O.selected_up_silu(x, vals, idx_ref, wu)
    close(y, O.selected_down(z_ref, idx_ref, wdt))


@pytest.mark.parametrize("hidden,inter,k", [(512, 100, 7), (1024, 2736, 512), (4096, 16384, 4000),
                                            (2048, 5461, 1), (2048, 5461, 5461), (1536, 777, 300),
                                            (768, 777, 300)])
def test_after_gate_one_token_shapes(hidden, inter, k):
    """One token at shapes other than the 1b one (small and wide rows, k of
    1 and of every channel, hidden not a multiple of the 256-column block):
    selection bit-exact, y within 2e-2 of the oracle on that selection,
    residual form equal to the bf16 add."""
    g = gen(inter + k)
    G = tie_heavy_rows(1, inter, "gauss", inter)
    x = torch.randn(1, hidden, generator=g).to(torch.bfloat16)
    wu = (torch.randn(inter, hidden, generator=g) * 0.02).to(torch.bfloat16)
    wdt = (torch.randn(inter, hidden, generator=g) * 0.02).to(torch.bfloat16)
    res = torch.randn(1, hidden, generator=g).to(torch.bfloat16).to(DEV)
    idx_ref = O.topk_indices(G, k)
    io = torch.full((1, k), -1, dtype=torch.int32, device=DEV)
    xd, Gd, wud, wdtd = x.to(DEV), G.to(DEV), wu.to(DEV), wdt.to(DEV)
    y = K().global_after_gate(xd, Gd, wud, wdtd, k, idx_out=io)
    assert np.array_equal(io.cpu().numpy(), idx_ref)
    z_ref = O.selected_up_silu(x, O.gather_rows(G, idx_ref), idx_ref, wu)
    close(y, O.selected_down(z_ref, idx_ref, wdt))
    yr = K().global_after_gate(xd, Gd, wud, wdtd, k, residual=res)
    assert torch.equal(yr, res + y)


@pytest.mark.parametrize("rows,inter,k,gcp", [(1024, 2048, 384, True), (300, 132, 100, False)])
def test_backward_aux_in_place_matches(rows, inter, k, gcp):
    """gZ in dL/dU's own rows (the layer backward's grouped weight-gradient
    order, [gG | gU] stacked at one pitch): the aux kernel reads each row
    whole before writing it, so dL/dG and dL/dU equal, bit for bit, the
    ones computed from a separate gZ buffer."""
    from moc_amd import _native as N
    g = gen(960 + rows)
    scores = torch.randn(rows, inter, generator=g).to(torch.bfloat16).to(DEV)
    _, idx, _ = K().topk_rows(scores, k, idx_dtype=torch.int16, want_vals=False)
    gs = (torch.randn(rows, k, generator=g) * 4).to(torch.bfloat16).to(DEV)
    us = torch.randn(rows, k, generator=g).to(torch.bfloat16).to(DEV)
    ss = None if gcp else torch.randn(rows, k, generator=g).to(torch.bfloat16).to(DEV)
    gz = K().padded_empty(rows, inter, torch.bfloat16, DEV)
    gz.copy_(torch.randn(rows, inter, generator=g).to(torch.bfloat16))
    ref_g, ref_u, _ = K().sparse_backward_aux(idx, gs, us, ss, gz, inter, stacked=True)
    pitch = K().row_pitch(inter, torch.bfloat16)
    buf = torch.full((rows, 2 * pitch), float("nan"), dtype=torch.bfloat16, device=DEV)
    buf[:, pitch:pitch + inter].copy_(gz)
    gg, gu = buf[:, :inter], buf[:, pitch:pitch + inter]
    N.call("moc_sparse_backward_aux", N.dtype_code(torch.bfloat16), idx.data_ptr(), N.idx_code(idx.dtype),
           gs.data_ptr(), us.data_ptr(), N.ptr(ss), gu.data_ptr(), 2 * pitch, rows, k, inter,
           gg.data_ptr(), gu.data_ptr(), 2 * pitch, N.stream_of(gs))
    torch.cuda.synchronize()
    assert torch.equal(gg.view(torch.int16), ref_g.view(torch.int16))
    assert torch.equal(gu.view(torch.int16), ref_u.view(torch.int16))
    # another pitch for gZ than for the outputs is refused
    with pytest.raises(ValueError, match="gz_full may only be grad_u"):
        N.call("moc_sparse_backward_aux", N.dtype_code(torch.bfloat16), idx.data_ptr(), N.idx_code(idx.dtype),
               gs.data_ptr(), us.data_ptr(), N.ptr(ss), gu.data_ptr(), pitch, rows, k, inter,
               gg.data_ptr(), gu.data_ptr(), 2 * pitch, N.stream_of(gs))


@pytest.mark.parametrize("rows,inter,k", [(4096, 5461, 1024), (300, 132, 100)])
def test_backward_aux_recomputed_s_matches_gcp_recompute(rows, inter, k):
    """The GCP backward keeps no S: the aux kernel recomputes it from g_s.
    Its dL/dG and dL/dU equal, bit for bit, the ones computed from the GCP
    recompute's own S (moc_gcp_recompute_scatter), on gate values spanning
    zeros, negatives and large magnitudes."""
    g = gen(950 + rows)
    scores = torch.randn(rows, inter, generator=g).to(torch.bfloat16).to(DEV)
    _, idx, _ = K().topk_rows(scores, k, idx_dtype=torch.int16, want_vals=False)
    gs = (torch.randn(rows, k, generator=g) * 4).to(torch.bfloat16)
    gs[:, :3] = torch.tensor([0.0, -0.0, 30.0])
    gs, us = gs.to(DEV), torch.randn(rows, k, generator=g).to(torch.bfloat16).to(DEV)
    gz = K().padded_empty(rows, inter, torch.bfloat16, DEV)
    gz.copy_(torch.randn(rows, inter, generator=g).to(torch.bfloat16))
    s_rec, _ = K().gcp_recompute_scatter(gs, us, idx, inter)
    a = K().sparse_backward_aux(idx, gs, us, s_rec, gz, inter)
    b = K().sparse_backward_aux(idx, gs, us, None, gz, inter)
    w = (inter + 7) // 8 * 8
    for p, q in zip(a, b):
        pv = p.as_strided((rows, w), p.stride()).view(torch.int16)
        qv = q.as_strided((rows, w), q.stride()).view(torch.int16)
        assert torch.equal(pv, qv)
