"""Pins oracle/moc_oracle.py (CPU only).

Each check is independent of the oracle's own formulas: brute force, torch
library routines (bf16 casts, topk, sigmoid/silu, autograd in float64),
closed forms, and the fixtures under tests/golden/ (written by
tests/golden/make_golden.py from brute force and float64 autograd).  Each is
chosen so that a plausible slip (wrong tie direction, transposed operand,
dropped term of SiLU', wrong rounding point) fails.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import moc_oracle as O

GOLD = Path(__file__).resolve().parent / "golden"


def load(name):
    return dict(np.load(GOLD / f"{name}.npz", allow_pickle=False))


# ------------------------------------------------------------------ bf16 bits
def test_bf16_rounding_matches_torch_cast():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 20000),
        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -9,
                  3.3895314e38, -3.3895314e38, 1e-45, 65504.0], dtype=np.float32)])
    ours = O.bf16_bits(x)
    ref = O.torch_bf16_bits(torch.from_numpy(x).to(torch.bfloat16))
    nan = np.isnan(x)
    assert np.array_equal(ours[~nan], ref[~nan])
    assert np.all((ours[nan] & 0x7FFF) > 0x7F80)


def test_order_keys_follow_numeric_order():
    rng = np.random.default_rng(1)
    v = torch.from_numpy(rng.standard_normal(4000).astype(np.float32) * 5)
    for t in (v, v.to(torch.bfloat16)):
        keys = O.order_keys(t).astype(np.int64)
        vals = t.float().numpy()
        i, j = rng.integers(0, len(vals), (2, 20000))
        assert np.array_equal(np.sign(keys[i] - keys[j]), np.sign(vals[i] - vals[j]))
    z = O.order_keys(torch.tensor([0.0, -0.0, float("nan"), float("inf")]))
    assert z[0] == z[1] and z[2] > z[3]


# ------------------------------------------------------------------ selection
@pytest.mark.parametrize("name", ["topk_bf16_ties", "topk_bf16_rand"])
def test_topk_golden_bf16(name):
    g = load(name)
    scores = O.torch_from_bf16_bits(g["scores_bits"])
    assert np.array_equal(O.topk_indices(scores, int(g["k"])), g["idx"])


def test_topk_golden_f32():
    g = load("topk_f32_ties")
    assert np.array_equal(O.topk_indices(torch.from_numpy(g["scores"]), int(g["k"])), g["idx"])


def test_topk_brute_force_random_ties():
    rng = np.random.default_rng(2)
    for _ in range(30):
        inter = int(rng.integers(1, 70))
        k = int(rng.integers(1, inter + 1))
        vals = rng.choice([-2.0, -1.0, 0.0, 0.5, 1.0, 3.0], size=(3, inter)).astype(np.float32)
        got = O.topk_indices(torch.from_numpy(vals).to(torch.bfloat16), k)
        for r in range(3):
            want = sorted(sorted(range(inter), key=lambda i: (-vals[r, i], i))[:k])
            assert got[r].tolist() == want


def test_topk_matches_torch_topk_up_to_ties():
    gen = torch.Generator().manual_seed(3)
    g = (torch.randn(64, 5461, generator=gen) * 0.9).to(torch.bfloat16)
    k = 1024
    ours = O.topk_indices(g, k)
    tv, ti = torch.topk(g.float(), k, dim=-1)
    for r in range(g.shape[0]):
        thr = tv[r, -1].item()
        row = g[r].float()
        strict_ours = {i for i in ours[r].tolist() if row[i] > thr}
        strict_torch = {i for i in ti[r].tolist() if row[i] > thr}
        assert strict_ours == strict_torch
        assert sum(row[i] == thr for i in ours[r].tolist()) == sum(row[i] == thr for i in ti[r].tolist())


def test_topk_invariants_and_special_cases():
    gen = torch.Generator().manual_seed(4)
    g = torch.randn(8, 300, generator=gen).to(torch.bfloat16)
    idx = O.topk_indices(g, 50)
    for r in range(8):
        sel = set(idx[r].tolist())
        assert len(sel) == 50 and list(idx[r]) == sorted(idx[r])
        rest = [g[r, i].item() for i in range(300) if i not in sel]
        assert min(g[r, i].item() for i in sel) >= max(rest)
    same = torch.ones(2, 17)
    assert O.topk_indices(same, 5).tolist() == [[0, 1, 2, 3, 4]] * 2
    assert O.topk_indices(g, 300).tolist() == [list(range(300))] * 8
    am = O.topk_indices(g, 1)[:, 0]
    assert np.array_equal(am, torch.argmax(g.float(), dim=1).numpy())  # torch argmax: first max


def test_2of8_golden_and_brute_force():
    g = load("sel28_bf16_tail")
    s = O.torch_from_bf16_bits(g["scores_bits"])
    assert np.array_equal(O.select_2of8_indices(s), g["idx"])
    for inter, kp in [(8, 2), (5461, 1366), (5464, 1366), (2736, 684), (9, 3), (1, 1)]:
        assert O.moc28_effective_k(inter) == kp
    rng = np.random.default_rng(5)
    v = torch.from_numpy(rng.standard_normal((4, 5461)).astype(np.float32))
    idx = O.select_2of8_indices(v)
    assert idx.shape == (4, 1366)
    grp = v[:, :5456].reshape(4, 682, 8)
    top2 = torch.topk(grp, 2, dim=-1).indices + torch.arange(682).view(1, 682, 1) * 8
    assert np.array_equal(idx[:, :1364].reshape(4, 682, 2), top2.numpy())


# -------------------------------------------------------- elementwise helpers
def test_sparse_forward_aux_closed_form():
    gen = torch.Generator().manual_seed(6)
    rows, inter, k = 5, 50, 12
    g = torch.randn(rows, inter, generator=gen).to(torch.bfloat16)
    u = torch.randn(rows, inter, generator=gen).to(torch.bfloat16)
    idx = O.topk_indices(g, k)
    vals = O.gather_rows(g, idx)
    u_s, s_s, z_s, z_full = O.sparse_forward_aux(vals, idx, u, inter)
    gd = vals.double()
    s_exact = gd * torch.sigmoid(gd)
    assert torch.allclose(s_s.double(), s_exact, rtol=2 ** -8, atol=0)
    assert torch.equal(z_s, (s_s.float() * u_s.float()).to(torch.bfloat16))
    assert torch.equal(u_s, O.gather_rows(u, idx))
    m = torch.from_numpy(O.topk_mask(idx, inter))
    assert torch.all(z_full[~m] == 0)
    assert torch.equal(O.gather_rows(z_full, idx), z_s)


def test_backward_aux_matches_autograd_f32():
    gen = torch.Generator().manual_seed(7)
    rows, inter, k = 6, 30, 7
    g = torch.randn(rows, inter, generator=gen)
    idx = O.topk_indices(g, k)
    gs = O.gather_rows(g, idx).double().requires_grad_(True)
    us = torch.randn(rows, k, generator=gen).double().requires_grad_(True)
    gz = torch.randn(rows, inter, generator=gen)
    gzs = O.gather_rows(gz, idx).double()
    (F.silu(gs) * us * gzs).sum().backward()
    s_s = F.silu(gs.detach()).float()
    gg, gu = O.sparse_backward_aux(idx, gs.detach().float(), us.detach().float(), s_s, gz, inter)
    assert torch.allclose(O.gather_rows(gg, idx).double(), gs.grad, rtol=1e-5, atol=1e-6)
    assert torch.allclose(O.gather_rows(gu, idx).double(), us.grad, rtol=1e-5, atol=1e-6)
    m = torch.from_numpy(O.topk_mask(idx, inter))
    assert torch.all(gg[~m] == 0) and torch.all(gu[~m] == 0)


def test_backward_aux_bf16_chain_close_to_exact():
    gen = torch.Generator().manual_seed(8)
    rows, inter, k = 16, 64, 16
    g = torch.randn(rows, inter, generator=gen).to(torch.bfloat16)
    idx = O.topk_indices(g, k)
    gs = O.gather_rows(g, idx)
    us = torch.randn(rows, k, generator=gen).to(torch.bfloat16)
    gz = torch.randn(rows, inter, generator=gen).to(torch.bfloat16)
    s_s, _ = O.gcp_recompute(gs, us)
    gg, gu = O.sparse_backward_aux(idx, gs, us, s_s, gz, inter)
    gd, ud, zd = gs.double(), us.double(), O.gather_rows(gz, idx).double()
    sig = torch.sigmoid(gd)
    exact_gg = ud * zd * sig * (1 + gd * (1 - sig))
    assert torch.allclose(O.gather_rows(gg, idx).double(), exact_gg, rtol=2e-2, atol=2e-2)
    assert torch.allclose(O.gather_rows(gu, idx).double(), F.silu(gd) * zd, rtol=2e-2, atol=2e-2)


def test_gcp_recompute_matches_torch_silu():
    gen = torch.Generator().manual_seed(9)
    g = torch.randn(1000, generator=gen).to(torch.bfloat16)
    u = torch.randn(1000, generator=gen).to(torch.bfloat16)
    s, z = O.gcp_recompute(g, u)
    assert torch.equal(s, F.silu(g.float()).to(torch.bfloat16))
    assert torch.equal(z, (s.float() * u.float()).to(torch.bfloat16))


# ------------------------------------------------------------------- the FFN
@pytest.mark.parametrize("name", ["ffn_small_f64", "ffn_odd_f64"])
@pytest.mark.parametrize("gcp", [True, False])
def test_ffn_oracle_matches_golden_autograd(name, gcp):
    g = load(name)
    t = lambda a: torch.from_numpy(a).float()  # noqa: E731
    x, wg, wu, wd, go = t(g["x"]), t(g["wg"]), t(g["wu"]), t(g["wd"]), t(g["go"])
    k = int(g["k"])
    fwd = O.ffn_forward(x, wg, wu, wd, k, "moc_gcp" if gcp else "moc")
    assert np.array_equal(fwd["idx"], g["idx"])
    assert np.allclose(fwd["out"].numpy(), g["out"], rtol=1e-5, atol=1e-5)
    dx, dwg, dwu, dwd = O.ffn_backward(x, wg, wu, wd, fwd, go, gcp=gcp)
    for got, want in ((dx, g["dx"]), (dwg, g["dwg"]), (dwu, g["dwu"]), (dwd, g["dwd"])):
        assert np.allclose(got.numpy(), want, rtol=1e-5, atol=1e-5)


def test_ffn_oracle_bf16_close_to_f64_autograd():
    gen = torch.Generator().manual_seed(10)
    x = torch.randn(2, 64, 96, generator=gen).to(torch.bfloat16)
    wg = (torch.randn(200, 96, generator=gen) * 0.05).to(torch.bfloat16)
    wu = (torch.randn(200, 96, generator=gen) * 0.05).to(torch.bfloat16)
    wd = (torch.randn(96, 200, generator=gen) * 0.05).to(torch.bfloat16)
    go = torch.randn(2, 64, 96, generator=gen).to(torch.bfloat16)
    fwd = O.ffn_forward(x, wg, wu, wd, 40, "moc_gcp")
    out, dx, dwg, dwu, dwd = O.dense_masked_autograd(x, wg, wu, wd, fwd["idx"], go)
    assert torch.allclose(fwd["out"].double(), out.reshape(fwd["out"].shape), rtol=2e-2, atol=2e-2)
    got = O.ffn_backward(x, wg, wu, wd, fwd, go, gcp=True)
    # bf16 materialises every intermediate, so compare against the exact
    # float64 gradients relative to each tensor's scale
    for a, b in zip(got, (dx, dwg, dwu, dwd)):
        b = b.reshape(a.shape)
        assert (a.double() - b).abs().max() <= 2e-2 * b.abs().max()


def test_mode_selection_variants():
    gen = torch.Generator().manual_seed(11)
    x = torch.randn(10, 32, generator=gen)
    wg = torch.randn(48, 32, generator=gen) * 0.2
    wu = torch.randn(48, 32, generator=gen) * 0.2
    wd = torch.randn(32, 48, generator=gen) * 0.2
    f28 = O.ffn_forward(x, wg, wu, wd, None, "moc_2_8")
    assert f28["idx"].shape == (10, 12)
    f_ps = O.ffn_forward(x, wg, wu, wd, 9, "moc_post_silu_abs")
    g = x @ wg.t()
    score = F.silu(g).abs()
    for r in range(10):
        thr = torch.topk(score[r], 9).values[-1]
        assert set(np.nonzero((score[r] > thr).numpy())[0]) <= set(f_ps["idx"][r].tolist())
    # vals handed to the sparse machinery are the pre-SiLU gates (moc/ffn.py:338)
    assert torch.equal(f_ps["vals"], O.gather_rows(g, f_ps["idx"]))


def test_masked_reference_consistent_with_training_forward():
    gen = torch.Generator().manual_seed(12)
    x = torch.randn(4, 64, generator=gen).to(torch.bfloat16)
    wg = (torch.randn(120, 64, generator=gen) * 0.1).to(torch.bfloat16)
    wu = (torch.randn(120, 64, generator=gen) * 0.1).to(torch.bfloat16)
    wd = (torch.randn(64, 120, generator=gen) * 0.1).to(torch.bfloat16)
    y, idx, z = O.masked_reference(x, wg, wu, wd, 30)
    fwd = O.ffn_forward(x, wg, wu, wd, 30, "moc")
    assert np.array_equal(idx, fwd["idx"])
    assert torch.allclose(y.float(), fwd["out"].float(), rtol=2e-2, atol=2e-2)
    yd, *_ = O.dense_masked_autograd(x, wg, wu, wd, idx, torch.zeros(4, 64))
    assert torch.allclose(y.double(), yd, rtol=2e-2, atol=2e-2)
    # selected up / down restatements agree with the masked reference
    vals = O.gather_rows(x.float() @ wg.float().t(), idx).to(torch.bfloat16)
    vals = O.gather_rows((x.float() @ wg.float().t()).to(torch.bfloat16), idx)
    z2 = O.selected_up_silu(x, vals, idx, wu)
    assert torch.equal(z2, z)
    y2 = O.selected_down(z, idx, wd.t().contiguous())
    assert torch.allclose(y2.float(), y.float(), rtol=1e-2, atol=1e-3)


def test_grouped_kernel_a_oracle():
    gen = torch.Generator().manual_seed(13)
    x = torch.randn(5, 64, generator=gen).to(torch.bfloat16)
    wg = (torch.randn(48, 64, generator=gen) * 0.1).to(torch.bfloat16)
    wu = (torch.randn(48, 64, generator=gen) * 0.1).to(torch.bfloat16)
    idx, sz, g = O.grouped_top2_up_silu(x, wg, wu)
    assert idx.shape == (5, 12)
    gv = g.float()
    for b in range(5):
        for grp in range(6):
            vals = gv[b, grp * 8:(grp + 1) * 8].tolist()
            want = sorted(range(8), key=lambda i: (-vals[i], i))[:2]
            assert idx[b, 2 * grp:2 * grp + 2].tolist() == [grp * 8 + w for w in want]
    u = (x.float() @ wu.float().t()).to(torch.bfloat16).float()
    gs = O.gather_rows(gv, idx).double()
    exact = F.silu(gs) * O.gather_rows(u, idx).double()
    assert torch.allclose(sz.double(), exact, rtol=1e-2, atol=1e-3)
