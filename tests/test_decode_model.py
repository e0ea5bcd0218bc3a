"""End-to-end decode model (moc_amd/inference/decode_model.py; the model of
the reference's benchmarks/inference/benchmark_decode.py:101-363).

CPU: RoPE against its closed form (a rotation of each pair by p * theta_i),
RMSNorm against its formula, and the static KV cache: logits of tokens fed
one at a time after a prompt equal the logits of one forward over the whole
sequence.  GPU: for each row (dense, global MoC, MoC 2:8) the whole-step
graph replays give the eager step's logits and tokens, and the prompt goes
through the >16-token forms of the FFN ops.
"""
from __future__ import annotations

import math

import pytest
import torch

from moc_amd.inference.decode_model import (DecodeConfig, DecoderModel, apply_rope, make_step,
                                             rope_tables, run_decode, RMSNorm)

DEV = "cuda"


def test_rope_is_the_pairwise_rotation():
    d, n = 16, 11
    cos, sin = rope_tables(d, n)
    x = torch.randn(3, n, d, generator=torch.Generator().manual_seed(1), dtype=torch.float64)
    y = apply_rope(x, cos.double(), sin.double())
    theta = 10000.0 ** (-torch.arange(0, d, 2, dtype=torch.float64) / d)
    ang = torch.arange(n, dtype=torch.float64)[:, None] * theta[None, :]
    zc = torch.complex(x[..., 0::2], x[..., 1::2]) * torch.exp(1j * ang)
    want = torch.stack((zc.real, zc.imag), dim=-1).flatten(-2)
    assert torch.allclose(y, want, atol=1e-6)
    assert torch.equal(y[:, 0], x[:, 0])  # position 0: identity


def test_rmsnorm_formula():
    m = RMSNorm(8)
    with torch.no_grad():
        m.weight.copy_(torch.arange(1, 9, dtype=torch.float32))
    x = torch.tensor([[3.0, -4.0, 0, 0, 0, 0, 0, 0]])
    rms = math.sqrt(25.0 / 8 + 1e-6)
    assert torch.allclose(m(x), x / rms * m.weight, atol=1e-6)


def test_incremental_decode_matches_full_forward_cpu():
    cfg = DecodeConfig(hidden=64, intermediate=176, heads=4, layers=2, vocab=97, k=32, max_seq=16)
    m = DecoderModel("dense", cfg).init_weights(3, std=0.1)
    m.allocate_cache()
    tok = torch.randint(0, cfg.vocab, (1, 12), generator=torch.Generator().manual_seed(4))
    full = m.forward_prompt(tok)
    m.reset_cache()
    m.forward_prompt(tok[:, :7])
    pos = torch.zeros((), dtype=torch.int64)
    steps = []
    for i in range(7, 12):
        pos.fill_(i)
        steps.append(m.forward_step(tok[:, i:i + 1], pos))
    assert torch.allclose(torch.cat(steps, 1), full[:, 7:12], atol=1e-5, rtol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("row", ["dense", "global_moc", "moc_2_8"])
def test_decode_graph_matches_eager(row):
    cfg = DecodeConfig(layers=2, max_seq=40)
    m = DecoderModel(row, cfg).to(DEV, torch.bfloat16).init_weights(7)
    m.allocate_cache()
    prompt = torch.randint(0, cfg.vocab, (1, 24), generator=torch.Generator().manual_seed(8)).to(DEV)
    eager = make_step(m, "eager")
    graph = make_step(m, "whole_graph")
    layer_graph = make_step(m, "layer_graph")
    _, toks_e = run_decode(m, prompt, 8, eager)
    _, toks_g = run_decode(m, prompt, 8, graph)
    _, toks_l = run_decode(m, prompt, 8, layer_graph)
    assert torch.equal(toks_e, toks_g)
    assert torch.equal(toks_e, toks_l)
    # one step from the same cache state: identical logits
    m.reset_cache()
    m.forward_prompt(prompt)
    cur = toks_e[:, :1]
    le = eager(cur, 24).clone()
    m.reset_cache()
    m.forward_prompt(prompt)
    lg = graph(cur, 24).clone()
    m.reset_cache()
    m.forward_prompt(prompt)
    ll = layer_graph(cur, 24).clone()
    torch.cuda.synchronize()
    assert torch.allclose(le.float(), ll.float(), atol=2e-2, rtol=2e-2)
    assert bool(torch.isfinite(le.float()).all())
    # the same kernels on the same inputs; allow library GEMMs that split K
    # with atomics their last-bit differences
    assert torch.allclose(le.float(), lg.float(), atol=2e-2, rtol=2e-2)


@pytest.mark.gpu
@pytest.mark.parametrize("row", ["global_moc", "moc_2_8"])
def test_decode_fused_ffn_neighbours_match_unfused(row):
    """MoC decode with ffn_norm fused into the gate (or gate/up) kernel and
    the residual add into the down kernel gives the unfused layer's logits
    (the RMSNorm statistics are summed in another order: bf16 tolerance)
    and the same greedy tokens."""
    cfg = DecodeConfig(layers=2, max_seq=40)
    fused = DecoderModel(row, cfg, fuse=True).to(DEV, torch.bfloat16).init_weights(9)
    plain = DecoderModel(row, cfg, fuse=False).to(DEV, torch.bfloat16)
    plain.load_state_dict(fused.state_dict())
    for m in (fused, plain):
        m.allocate_cache()
    prompt = torch.randint(0, cfg.vocab, (1, 24), generator=torch.Generator().manual_seed(10)).to(DEV)
    _, tf = run_decode(fused, prompt, 6, make_step(fused, "whole_graph"))
    _, tp = run_decode(plain, prompt, 6, make_step(plain, "eager"))
    assert torch.equal(tf, tp)
    for m in (fused, plain):
        m.reset_cache()
        m.forward_prompt(prompt)
    pos = torch.full((), 24, dtype=torch.int64, device=DEV)
    lf = fused.forward_step(tf[:, :1], pos).float()
    lp = plain.forward_step(tf[:, :1], pos).float()
    assert torch.allclose(lf, lp, atol=5e-2, rtol=5e-2)


class _FFNRecorder:
    """Records every FFN call of a decode model: ("ffn", x, y) for the
    module's forward (x is the FFN input after ffn_norm) and ("fused", x, y,
    norm weight, eps) for fused_decode_residual (x before the norm, y = x +
    FFN(norm(x))).  With graph_only, only calls made while a HIP graph is
    being captured are kept: their clones are written again by every replay,
    so after a replay they hold that replay's FFN inputs and outputs."""

    def __init__(self, model, graph_only: bool):
        self.calls = []
        self.graph_only = graph_only
        for i, layer in enumerate(model.layers):
            layer.ffn.register_forward_hook(
                lambda mod, args, out, _i=i: self._add(_i, "ffn", args[0], out))
            orig = layer.ffn.fused_decode_residual

            def fused(x, w, eps, _orig=orig, _i=i):
                y = _orig(x, w, eps)
                self._add(_i, "fused", x, y, w, eps)
                return y

            layer.ffn.fused_decode_residual = fused

    def _add(self, i, kind, x, y, w=None, eps=None):
        if self.graph_only and not torch.cuda.is_current_stream_capturing():
            return
        self.calls.append((i, kind, x.detach().clone(), y.detach().clone(), w, eps))


def _ffn_oracle(ffn, row, x):
    """The FFN of one decode layer on the CPU oracle, for FFN input x [n, h]
    (bf16 on the device): global MoC is masked_reference with the device's
    own gate scores (the same GEMV/GEMM the layer runs, so the selection is
    compared on identical inputs); MoC 2:8 is kernel A (grouped top-2 + up
    SiLU) then kernel B (selected Down) of the reference's Triton path."""
    from moc_amd import kernels as K
    from oracle import moc_oracle as O
    wg, wu, wd = (w.detach() for w in (ffn.gate_proj.weight, ffn.up_proj.weight, ffn.down_proj.weight))
    if row == "global_moc":
        g = (K.gemv(x, wg) if x.shape[0] <= 16 else K.linear(x, wg)).cpu()
        y, _, _ = O.masked_reference(x.cpu(), wg.cpu(), wu.cpu(), wd.cpu(), ffn.config.k, g_override=g)
        return y
    idx, sz, _ = O.grouped_top2_up_silu(x.cpu(), wg.cpu(), wu.cpu())
    return O.selected_down(sz, idx, wd.t().contiguous().cpu())


def _check_calls(calls, model, row):
    from oracle import moc_oracle as O
    assert calls, "no FFN call was recorded"
    for i, kind, x, y, w, eps in calls:
        ffn = model.layers[i].ffn
        if kind == "ffn":
            ref = _ffn_oracle(ffn, row, x)
        else:
            xf = x.float()
            xn = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype) * w
            if row == "global_moc":
                from moc_amd import kernels as K
                _, xn = K.gemv_rmsnorm(x, w, eps, ffn.gate_proj.weight)  # the device's own x_norm
            ref = (x.cpu().float() + _ffn_oracle(ffn, row, xn).float()).to(x.dtype)
        a, b = y.float().cpu().reshape(ref.shape), ref.float()
        err = (a - b).abs()
        bad = err > 2e-2 + 2e-2 * b.abs()
        assert not bool(bad.any()), (i, kind, tuple(x.shape), err.max().item())
        assert O is not None


@pytest.mark.gpu
@pytest.mark.parametrize("fuse", [True, False])
@pytest.mark.parametrize("row", ["global_moc", "moc_2_8"])
def test_decode_ffn_calls_match_oracle_eager(row, fuse):
    """Every FFN call of a 2-layer decode (the 24-token prompt through the
    >16-token op forms, then 4 greedy single-token steps) against the
    oracle on that call's own input: out within 2e-2."""
    cfg = DecodeConfig(layers=2, max_seq=40)
    m = DecoderModel(row, cfg, fuse=fuse).to(DEV, torch.bfloat16).init_weights(11)
    m.allocate_cache()
    rec = _FFNRecorder(m, graph_only=False)
    prompt = torch.randint(0, cfg.vocab, (1, 24), generator=torch.Generator().manual_seed(12)).to(DEV)
    run_decode(m, prompt, 4, make_step(m, "eager"))
    torch.cuda.synchronize()
    kinds = {k for _, k, *_ in rec.calls}
    assert kinds == ({"ffn", "fused"} if fuse else {"ffn"}), kinds
    _check_calls(rec.calls, m, row)


@pytest.mark.gpu
@pytest.mark.parametrize("fuse", [True, False])
@pytest.mark.parametrize("row", ["global_moc", "moc_2_8"])
def test_decode_ffn_calls_match_oracle_whole_graph(row, fuse):
    """The whole-step HIP graph (the scope of the decode benchmark's rows):
    after each of three replays, every layer's FFN input and output as that
    replay computed them, against the oracle."""
    cfg = DecodeConfig(layers=2, max_seq=40)
    m = DecoderModel(row, cfg, fuse=fuse).to(DEV, torch.bfloat16).init_weights(13)
    m.allocate_cache()
    rec = _FFNRecorder(m, graph_only=True)
    prompt = torch.randint(0, cfg.vocab, (1, 24), generator=torch.Generator().manual_seed(14)).to(DEV)
    step = make_step(m, "whole_graph")
    assert len(rec.calls) == cfg.layers
    m.reset_cache()
    cur = m.forward_prompt(prompt)[:, -1:, :].argmax(dim=-1)
    for i in range(3):
        cur = step(cur, 24 + i).argmax(dim=-1)
        torch.cuda.synchronize()
        _check_calls(rec.calls, m, row)
