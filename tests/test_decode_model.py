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
