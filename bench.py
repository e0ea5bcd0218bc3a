"""Benchmark of the MoC sparse SwiGLU FFN hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Prints ONE JSON line.  The headline (`value`) is the MoC+GCP FFN layer
forward+backward latency at the 1b preset shape (X [64, 256, 2048] bf16,
d_ffn 5461, K 1024), the shape of the reference's training-latency harness
(benchmarks/training/benchmark_training_latency.py:20-31).  A step is one
forward and one backward of that layer over one batch of synthetic inputs
already resident in HBM; weight gradients are cleared (set to None) before
each step as the reference harness does (:55-57).

The same line carries:
  roofline      the MFMA GEMM engine (the dominant kernel of the step):
                algorithmic FLOP of the nine FFN GEMMs (7 launches: G and U
                share one, dX sums two products) / the time the GPU spends in
                those launches inside the timed steps (union of their
                event-bracketed intervals), against the 2.5 PFLOP/s dense bf16
                peak; `isolated`: the same launches timed back to back;
  roofline_decode  global-MoC decode (config 3, B=1): union-of-selected-rows
                bytes / layer time against 8 TB/s, cold weights (rotation
                over 8 weight sets > 2x the 256 MB MALL), HIP-graph replays;
  cpu_baseline  the repo's CPU restatement (oracle/) of the reference path,
                timed on this host on a bounded token sample and scaled to
                the full layer;
  configs       each of the five configs: latency, throughput, roofline
                fraction and its own CPU baseline (config 1: 60m fp32 MoC
                forward; 2: 130m MoC+GCP fwd+bwd; 3: decode B=1/4/16; 4: MoC
                2:8 prefill of 4096 tokens; 5: 350m model training step,
                moc_gcp and dense, tokens/s and peak memory).

Only one GPU is used; --gpus N with N > 1 exits with a message.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "MoC FFN layer µs (fwd+bwd; decode) at 1b shape + % HBM/MFMA roofline"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0

D1B, I1B, K1B = 2048, 5461, 1024
PROBE_STEPS = 5
BATCH1B, SEQ1B = 64, 256


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=int(os.environ.get("WORLD_SIZE", "1")))
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="approximate CPU time budget of the cpu_baseline sample")
    p.add_argument("--decode-groups", type=int, default=80)
    p.add_argument("--decode-iters", type=int, default=100)
    p.add_argument("--skip-extra", action="store_true", help="headline + rooflines only")
    p.add_argument("--cfg5", action="store_true",
                   help="only the 350m-model training step (config 5): tokens/s and peak "
                        "memory, moc_gcp vs dense, one JSON line")
    p.add_argument("--cfg5-steps", type=int, default=10)
    p.add_argument("--gemm-k-sweep", action="store_true",
                   help="only time C[16384, N] = A B for N 5461 and 2048 over K 256 ... 8192 "
                        "(padded outputs) and fit the per-round fixed cost and per-K-tile cost")
    p.add_argument("--trace-summary", metavar="DIR", default=None,
                   help="no GPU work: summarise a rocprofv3 --kernel-trace --stats --output-format csv "
                        "output directory (per-kernel totals; with --trace-headline, the GEMM "
                        "launches of the headline's timed steps) as markdown")
    p.add_argument("--trace-steps", type=float, default=1.0,
                   help="with --trace-summary: steps the traced run made (per-step columns)")
    p.add_argument("--trace-by-grid", action="store_true",
                   help="with --trace-summary: also split every kernel's dispatches by grid size "
                        "(mean and median duration per kernel and grid, from *kernel_trace.csv)")
    p.add_argument("--trace-headline", action="store_true",
                   help="with --trace-summary: the trace is of `bench.py --skip-extra`; report the "
                        "seven GEMM launches of its timed fwd+bwd steps")
    p.add_argument("--cfg5-row", choices=["moc_gcp", "dense", "moc_gcp_unfused"], default=None,
                   help="with --cfg5: only this row, and no FFN-layer timing (for kernel traces)")
    p.add_argument("--only", choices=["cfg1", "cfg2", "cfg4"], default=None,
                   help="run one config's GPU leg alone (for kernel traces) and print its JSON")
    p.add_argument("--decode-e2e", action="store_true",
                   help="only end-to-end greedy decode of a 24-layer 1b-shape decoder (dense, "
                        "global MoC, MoC 2:8; eager and whole-step graph): ms/token, one JSON line")
    p.add_argument("--roofline-only", action="store_true",
                   help="only the seven GEMM launches of the roofline (for rocprofv3 kernel "
                        "traces whose per-kernel averages match roofline.per_launch)")
    p.add_argument("--pmc-target", choices=["gemm", "dx", "copy", "decode", "down28", "down28_dense",
                                            "topk"],
                   default=None,
                   help="only launch one workload a few times (for rocprofv3 --pmc runs): the G,U "
                        "pair GEMM of the 1b layer, its dX GEMM (two products), a plain 256 MiB "
                        "copy kernel (counter scale), the B=1 decode layer over 8 weight sets, or "
                        "config 4's 2:8 Down (down28: structured-sparse MFMA over the packed "
                        "selection; down28_dense: the same selection scattered dense), or the "
                        "row Top-K of the 1b training rows (topk: G of the bench input, "
                        "16384 x 5461 bf16, K 1024, three calls)")
    return p.parse_args()


def cfg5_model_flop(cfg, batch: int, seq: int) -> float:
    """Algorithmic FLOP of one training step of the decoder (forward +
    backward = 3 x forward): 2 FLOP per token per parameter of every matmul
    (q/k/v and output projections, gate/up/down, LM head; not the embedding
    lookup) plus the attention products QK^T and PV (2 x 2 x S^2 x d per
    sequence and layer, over the full square).  The MoC FFN's nine GEMMs are
    dense products in the reference (moc/ffn.py:389-494), so the count is
    the same for both FFN types."""
    L, d, inter, v = cfg.num_hidden_layers, cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size
    tokens = batch * seq
    fwd = 2 * tokens * (L * (4 * d * d + 3 * d * inter) + v * d) + L * 2 * 2 * batch * seq * seq * d
    return 3.0 * fwd


def cfg5_bench(steps: int, only: str | None = None) -> dict:
    """Config 5: a 350m LLaMA training step (24 layers, d=1024, I=2736,
    K=512), bf16 parameters, AdamW (0.9/0.999, wd 0, fused=False, lr 1e-3),
    tokens [16, 256] uniform over the 32100-token vocabulary with labels =
    tokens; 5 warmup steps (the reference harness's default,
    benchmark_training_throughput.py:135), then `steps` timed steps; peak
    memory over the timed steps (the method of
    benchmark_training_throughput.py:51-114 and benchmark_memory.py:51-107).
    Attention, norms and embeddings are stock PyTorch; the FFN is this
    build's.  Beside the wall-clock step: the model's algorithmic FLOP over
    it, and one FFN layer of the step's shape timed on its own (GPU-bound,
    so the two FFNs compare without the host's launch time, which at this
    size is close to the GPU's work).  Rows: moc_gcp (the FFN's pre-norm and
    residual add fused around it), dense, and moc_gcp with that fusion
    switched off."""
    import torch
    from moc_amd import PRESETS, build_model
    from dataclasses import replace
    out = {}
    cfg = replace(PRESETS["350m"], vocab_size=32100, max_seq_len=256)
    flop = cfg5_model_flop(cfg, 16, 256)
    from moc_amd import ffn as F
    for row in ("moc_gcp", "dense", "moc_gcp_unfused") if only is None else (only,):
        # moc_gcp_unfused: the same model with the FFN's pre-norm and residual
        # add as stock PyTorch ops around the FFN (the fusion switched off)
        ffn_type = "moc_gcp" if row == "moc_gcp_unfused" else row
        F.FUSE_BLOCK_FFN = row != "moc_gcp_unfused"
        torch.manual_seed(1234)
        model = build_model(cfg, ffn_type=ffn_type).to("cuda", torch.bfloat16)
        opt = torch.optim.AdamW(model.parameters(), lr=1e-3, betas=(0.9, 0.999), weight_decay=0.0,
                                fused=False)
        gen = torch.Generator().manual_seed(1234)
        tok = torch.randint(0, 32100, (16, 256), generator=gen).cuda()

        def step():
            _, loss = model(tok, labels=tok)
            loss.backward()
            opt.step()
            opt.zero_grad(set_to_none=True)
            return loss

        loss0 = step().detach()
        for _ in range(4):
            step()
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        t0 = time.perf_counter()
        for _ in range(steps):
            loss = step().detach()
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / steps
        peak = torch.cuda.max_memory_allocated()
        tf = flop / dt / 1e12
        res = {"ms_per_step": round(dt * 1e3, 2), "tokens_per_s": round(16 * 256 / dt, 1),
               "peak_mem_gib": round(peak / 2**30, 3),
               "loss_first": round(float(loss0), 4), "loss_last": round(float(loss), 4),
               "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": BF16_PEAK_TFLOPS,
                            "unit": "TFLOP/s", "frac": round(tf / BF16_PEAK_TFLOPS, 4),
                            "algorithmic_tflop_per_step": round(flop / 1e12, 3)}}
        out[row] = res
        log(f"cfg5 {row}: {out[row]}")
        del model, opt
        torch.cuda.empty_cache()
    F.FUSE_BLOCK_FFN = True
    if only is not None:
        return out
    out["ffn_layer"] = cfg5_ffn_layer()
    log(f"cfg5 ffn layer: {out['ffn_layer']}")
    return out


def cfg5_ffn_layer(steps: int = 20, warmup: int = 5) -> dict:
    """One FFN layer of config 5's shape (16 x 256 tokens, d 1024, I 2736,
    K 512), fwd+bwd on its own: moc_gcp (this build) against the dense
    SwiGLU FFN (stock PyTorch, hipBLASLt), same seeded inputs; the nine
    dense-equivalent GEMMs' FLOP over the step."""
    import torch
    from moc_amd import build_ffn
    t, d, inter, k = 16 * 256, 1024, 2736, 512
    x, wg, wu, wd, go = seeded_inputs(t, d, inter)
    xd = x.reshape(16, 256, d).cuda().requires_grad_(True)
    god = go.reshape(16, 256, d).cuda()
    flop = 9 * 2.0 * t * d * inter
    res = {}
    for ffn_type in ("moc_gcp", "dense"):
        m = build_ffn(d, inter, ffn_type, k=k).to("cuda", torch.bfloat16).train()
        with torch.no_grad():
            for p_, w in zip((m.gate_proj.weight, m.up_proj.weight, m.down_proj.weight), (wg, wu, wd)):
                p_.copy_(w)
        ms, f, b = time_train_layer(m, xd, god, steps, warmup)
        tf = flop / (ms * 1e-3) / 1e12
        res[ffn_type] = {"us": round(ms * 1e3, 1), "fwd_us": round(f["median"] * 1e3, 1),
                         "bwd_us": round(b["median"] * 1e3, 1), "achieved": round(tf, 1),
                         "frac": round(tf / BF16_PEAK_TFLOPS, 4)}
        del m
    res["algorithmic_gflop"] = round(flop / 1e9, 1)
    return res


def pmc_target(which: str) -> None:
    """Minimal launches for the counter runs behind roofline.traffic."""
    import torch
    from moc_amd import _native as N
    from moc_amd import kernels as K
    N.load()
    if which == "gemm":
        x, wg, _, _, _ = seeded_inputs(BATCH1B * SEQ1B, D1B, I1B)
        x, wg = x.cuda(), wg.cuda()
        wu = (torch.randn(I1B, D1B, generator=torch.Generator().manual_seed(5)) * 0.02)
        wu = wu.to(torch.bfloat16).cuda()
        g = K.padded_empty(x.shape[0], I1B, torch.bfloat16, x.device)
        u = K.padded_empty(x.shape[0], I1B, torch.bfloat16, x.device)
        for _ in range(5):
            K.linear_pair(x, wg, wu, out1=g, out2=u)
    elif which == "dx":
        t, d, inter, k = BATCH1B * SEQ1B, D1B, I1B, K1B
        x, wg, wu, _, _ = seeded_inputs(t, d, inter)
        gen = torch.Generator(device="cuda").manual_seed(7)
        zs = torch.randn(t, k, device="cuda", generator=gen).to(torch.bfloat16)
        idx = torch.argsort(torch.rand(t, inter, device="cuda", generator=gen), dim=1)[:, :k]
        idx = idx.sort(dim=1).values.to(torch.int16)
        gg = K.scatter_sparse_to_dense(zs, idx, inter)
        gu = K.scatter_sparse_to_dense(zs, idx, inter)
        wg_a, wu_a = K.aligned_rows(wg.cuda()), K.aligned_rows(wu.cuda())
        for _ in range(5):
            K.gemm(gg, wg_a, a2=gu, b2=wu_a)
    elif which == "decode":
        gen = torch.Generator(device="cuda").manual_seed(1234)
        layers = []
        for _ in range(8):
            wg = (torch.randn(I1B, D1B, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
            wu = (torch.randn(I1B, D1B, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
            wdt = K.down_weight_t_for_decode(
                (torch.randn(D1B, I1B, device="cuda", generator=gen) * 0.02).to(torch.bfloat16))
            layers.append((wg, wu, wdt))
        x = torch.randn(1, D1B, device="cuda", generator=gen).to(torch.bfloat16)
        y = torch.empty(1, D1B, device="cuda", dtype=torch.bfloat16)
        ws = K.global_decode_workspace(1, I1B, K1B, D1B, "cuda")
        for _ in range(3):
            for wg, wu, wdt in layers:
                K.global_decode(x, wg, wu, wdt, K1B, workspace=ws, out=y)
    elif which == "topk":
        # the 1b layer's selection: G = X Wg^T of the bench input (one GEMM
        # launch first), then the row Top-K three times, as the layer calls it
        x, wg, _, _, _ = seeded_inputs(BATCH1B * SEQ1B, D1B, I1B)
        g = K.padded_empty(x.shape[0], I1B, torch.bfloat16, "cuda")
        K.linear(x.cuda(), wg.cuda(), out=g)
        for _ in range(3):
            K.topk_rows(g, K1B, idx_dtype=torch.int16)
        torch.cuda.synchronize()
        log("pmc target topk: 3 Top-K launches done")
        return
    elif which in ("down28", "down28_dense"):
        # config 4's Down: 4096 tokens, the 1b shape padded to 5464 channels;
        # the 2:4-packed selection on the structured-sparse MFMA, or the same
        # selection scattered dense on the dense MFMA
        t, d, inter = 4096, D1B, 5464
        gen = torch.Generator(device="cuda").manual_seed(11)
        groups = inter // 8
        pos = torch.argsort(torch.rand(t, groups, 8, device="cuda", generator=gen), dim=-1)[..., :2]
        idx = (pos + 8 * torch.arange(groups, device="cuda")[None, :, None]).reshape(t, groups * 2)
        sz = torch.randn(t, groups * 2, device="cuda", generator=gen).to(torch.bfloat16)
        wdt = (torch.randn(inter, d, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
        if which == "down28":
            ap, meta = K.packed28_buffers(t, inter, "cuda")
            nt, ld_ap, meta_rows = K.packed28_layout(t, inter)
            N.call("moc_pack28_bf16", sz.data_ptr(), idx.data_ptr(), t, inter, ap.data_ptr(), ld_ap,
                   meta.data_ptr(), meta_rows, None, N.stream_of(sz))
            ws = K.sparse28_down_workspace(t, inter, d, "cuda")
            for _ in range(5):
                K.sparse28_down(ap, meta, inter, wdt, workspace=ws)
        else:
            z = K.scatter_sparse_to_dense(sz, idx, inter)
            for _ in range(5):
                K.gemm(z, wdt)
    else:
        rows, cols = 16384, 8192  # 256 MiB of bf16 read and written
        src = torch.ones(rows, cols, device="cuda", dtype=torch.bfloat16)
        dst = torch.empty_like(src)
        for _ in range(5):
            N.call("moc_copy_pad_2d", N.MOC_BF16, src.data_ptr(), rows, cols, cols, dst.data_ptr(),
                   cols, cols, N.stream_of(src))
    torch.cuda.synchronize()
    log(f"pmc target {which}: 5 launches done")


# ----------------------------------------------------------------- helpers
def seeded_inputs(t, d, inter, seed=1234, dtype=None):
    """X ~ N(0,1), W_gate/W_up [I,d], W_down [d,I] ~ N(0,0.02), dD ~ N(0,1),
    drawn on the CPU in that order from one seeded generator."""
    import torch
    dtype = dtype or torch.bfloat16
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(t, d, generator=g).to(dtype)
    wg = (torch.randn(inter, d, generator=g) * 0.02).to(dtype)
    wu = (torch.randn(inter, d, generator=g) * 0.02).to(dtype)
    wd = (torch.randn(d, inter, generator=g) * 0.02).to(dtype)
    go = torch.randn(t, d, generator=g).to(dtype)
    return x, wg, wu, wd, go


def summarize(samples):
    s = sorted(samples)
    n = len(s)
    return {"mean": statistics.mean(s), "median": statistics.median(s),
            "p10": s[int(0.10 * (n - 1))], "p90": s[int(0.90 * (n - 1))], "n": n}


def build_layer(d, inter, k, ws, mode="moc_gcp"):
    import torch
    from moc_amd import build_ffn
    m = build_ffn(d, inter, mode, k=k).to("cuda", torch.bfloat16).train()
    with torch.no_grad():
        for p, w in zip((m.gate_proj.weight, m.up_proj.weight, m.down_proj.weight), ws):
            p.copy_(w)
    return m


def time_train_layer(m, x, go, steps, warmup, probe: list | None = None,
                     step_starts: list | None = None):
    """Reference method: untimed warmup, then K timed fwd+bwd steps bracketed
    by a device synchronisation; per-step events split fwd and bwd.  With
    `probe` (a list), every GEMM launch of the timed steps is also bracketed
    by timing events on its own stream and recorded there."""
    import torch
    from moc_amd import kernels as K
    for _ in range(warmup):
        m.zero_grad(set_to_none=True)
        x.grad = None
        m(x).backward(go)
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
           torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    K.set_gemm_probe(probe)
    try:
        t0 = time.perf_counter()
        for e0, e1, e2 in ev:
            m.zero_grad(set_to_none=True)
            x.grad = None
            e0.record()
            y = m(x)
            e1.record()
            y.backward(go)
            e2.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    finally:
        K.set_gemm_probe(None)
    if step_starts is not None:
        step_starts.extend(e0 for e0, _, _ in ev)
    fwd = [a.elapsed_time(b) for a, b, _ in ev]
    bwd = [b.elapsed_time(c) for _, b, c in ev]
    return wall * 1e3 / steps, summarize(fwd), summarize(bwd)


# L2-miss (MALL/HBM side) bytes of one G,U pair launch at the 1b shape, from the
# FETCH_SIZE / WRITE_SIZE counter runs in profiles/gemm_GU_pair_traffic.md, each
# scaled by what the counter reads for a copy kernel of known size
# (FETCH_SIZE x 2.000, WRITE_SIZE x 1.000).
GEMM_GU_TRAFFIC_BYTES = 1120.2e6 + 358.6e6
# the same for the B=1 decode layer (the gate + dense-U GEMV pair, then the
# column-owning select/down kernel), profiles/decode_B1_traffic.md
DECODE_B1_TRAFFIC_BYTES = 44.80e6 + 0.09e6 + 4.59e6


def gemm_roofline(t, d, inter, k, ws, x, go, reps=10):
    """HIP-event time of the seven GEMM launches of one MoC FFN fwd+bwd step at
    the layer's real shapes (the kernels and operand layouts the layer uses)."""
    import torch
    from moc_amd import kernels as K
    wg, wu, wd = [w.cuda() for w in ws]
    x2 = K.aligned_rows(x.reshape(-1, d))
    go2 = K.aligned_rows(go.reshape(-1, d))
    wd_a = K.aligned_rows(wd)
    g = K.padded_empty(t, inter, torch.bfloat16, x.device)
    u = K.padded_empty(t, inter, torch.bfloat16, x.device)
    # a realistic sparse z_full / grad tensors: K of I channels per row
    gen = torch.Generator(device="cuda").manual_seed(7)
    zs = torch.randn(t, k, device="cuda", generator=gen).to(torch.bfloat16)
    idx = torch.argsort(torch.rand(t, inter, device="cuda", generator=gen), dim=1)[:, :k]
    idx = idx.sort(dim=1).values.to(torch.int16)
    z_full = K.scatter_sparse_to_dense(zs, idx, inter)
    gz = K.padded_empty(t, inter, torch.bfloat16, x.device)
    gg = K.scatter_sparse_to_dense(zs, idx, inter)
    gu = K.scatter_sparse_to_dense(zs, idx, inter)
    wg_a, wu_a = K.aligned_rows(wg), K.aligned_rows(wu)
    unit = 2.0 * t * d * inter
    launches = [
        ("G, U = X Wg^T, X Wu^T (one launch)", lambda: K.linear_pair(x2, wg, wu, out1=g, out2=u), 2),
        ("D = Z Wd^T", lambda: K.gemm(z_full, wd_a.t()), 1),
        ("dWd = dD^T Z", lambda: K.gemm(go2.t(), z_full), 1),
        ("gZ = dD Wd", lambda: K.gemm(go2, wd_a, out=gz), 1),
        ("dWg = gG^T X", lambda: K.gemm(gg.t(), x2), 1),
        ("dWu = gU^T X", lambda: K.gemm(gu.t(), x2), 1),
        ("dX = gG Wg + gU Wu", lambda: K.gemm(gg, wg_a, a2=gu, b2=wu_a), 2),
    ]
    for _ in range(3):  # warm every launch (clocks, caches) before timing any
        for _, fn, _ in launches:
            fn()
    torch.cuda.synchronize()
    per = []
    tot_ms, tot_flop = 0.0, 0.0
    for name, fn, mult in launches:
        # two untimed launches first: the first launch after a switch of
        # workload runs several % slower than the steady state
        fn()
        fn()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(reps)]
        for a, b in ev:
            a.record()
            fn()
            b.record()
        torch.cuda.synchronize()
        ms = statistics.median(a.elapsed_time(b) for a, b in ev)
        flop = unit * mult
        tot_ms += ms
        tot_flop += flop
        per.append({"gemm": name, "us": round(ms * 1e3, 2),
                    "tflops": round(flop / (ms * 1e-3) / 1e12, 1)})
    achieved = tot_flop / (tot_ms * 1e-3) / 1e12
    return {
        "bound": "mfma", "achieved": round(achieved, 1), "peak": BF16_PEAK_TFLOPS,
        "unit": "TFLOP/s", "frac": round(achieved / BF16_PEAK_TFLOPS, 4),
        "traffic": GEMM_GU_TRAFFIC_BYTES if (t, d, inter) == (BATCH1B * SEQ1B, D1B, I1B) else None,
        "traffic_note": "bytes per G,U pair launch (L2 misses to MALL/HBM; counter runs scaled by a "
                        "copy kernel, profiles/gemm_GU_pair_traffic.md)",
        "kernel": "gemm_pp_kernel (v_mfma_f32_32x32x16_bf16), 7 launches/step",
        "algorithmic_flop_per_step": tot_flop, "gemm_ms_per_step": round(tot_ms, 4),
        "per_launch": per,
    }


def decode_bench(nb, sets=8, groups=40, iters=50, moc28=False):
    """Global-MoC decode layer (config 3): gate GEMV + Top-K + selected Up*SiLU
    + selected Down, captured in one HIP graph that walks `sets` distinct
    weight sets (cold MALL), replayed groups x iters times.  moc28: the MoC
    2:8 decode layer instead (d_ffn 5464, top 2 of every 8 channels; the
    reference's single-layer B=1 row, results/inference_ffn.md:19)."""
    import torch
    from moc_amd import kernels as K
    d, inter, k = (D1B, 5464, 5464 // 4) if moc28 else (D1B, I1B, K1B)
    gen = torch.Generator(device="cuda").manual_seed(1234)
    layers = []
    for _ in range(sets):
        wg = (torch.randn(inter, d, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
        wu = (torch.randn(inter, d, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
        wd = (torch.randn(d, inter, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
        wdt = K.down_weight_t_for_decode(wd)  # the module's layout (padded row pitch)
        del wd
        layers.append((wg, wu, wdt))
    x = torch.randn(nb, d, device="cuda", generator=gen).to(torch.bfloat16)
    gate = [torch.empty(nb, inter, device="cuda", dtype=torch.bfloat16) for _ in range(sets)]
    ys = [torch.empty(nb, d, device="cuda", dtype=torch.bfloat16) for _ in range(sets)]
    if moc28:
        ws = torch.empty(K.moc28_decode_workspace_bytes(nb, inter, d), dtype=torch.uint8, device="cuda")
    else:
        ws = K.global_decode_workspace(nb, inter, k, d, "cuda")

    def run_all():
        for (wg, wu, wdt), y in zip(layers, ys):
            if moc28:
                K.moc28_decode(x, wg, wu, wdt, workspace=ws, out=y)
            else:
                K.global_decode(x, wg, wu, wdt, k, workspace=ws, out=y)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            run_all()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run_all()
    for _ in range(30):
        graph.replay()
    torch.cuda.synchronize()
    samples = []
    for _ in range(groups):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(iters):
            graph.replay()
        b.record()
        torch.cuda.synchronize()
        samples.append(a.elapsed_time(b) * 1e3 / (iters * sets))
    # algorithmic bytes: all of W_gate + the union of selected rows of W_up and
    # W_down^T + activations (x in, G out+in, y out), counted from the masks
    union = []
    for (wg, wu, wdt), g in zip(layers, gate):
        if moc28:
            idx = torch.empty(nb, k, dtype=torch.int64, device="cuda")
            K.moc28_decode(x, wg, wu, wdt, workspace=ws, idx_out=idx)
        else:
            K.gemv(x, wg, out=g)
            _, idx, _ = K.topk_rows(g, k, want_vals=False)
        union.append(int(torch.unique(idx).numel()))
    u_avg = sum(union) / len(union)
    act = 2 * nb * d * 2 + 2 * nb * inter * 2
    bytes_layer = 2 * d * inter + 2 * 2 * d * u_avg + act
    st = summarize(samples)
    achieved = bytes_layer / (st["median"] * 1e-6) / 1e9
    if moc28:
        del layers, graph
        torch.cuda.empty_cache()
        return {"nb": nb, "us_median": round(st["median"], 3), "us_mean": round(st["mean"], 3),
                "us_p10": round(st["p10"], 3), "us_p90": round(st["p90"], 3),
                "union_rows": round(u_avg, 1), "bytes": int(bytes_layer),
                "achieved_GBs": round(achieved, 1), "frac_hbm": round(achieved / HBM_PEAK_GBS, 4)}
    # the gate GEMV alone, to report the dominant decode kernel separately
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2):
        for (wg, _, _), g in zip(layers, gate):
            K.gemv(x, wg, out=g)
    for _ in range(10):
        g2.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(iters * 4):
        g2.replay()
    b.record()
    torch.cuda.synchronize()
    gemv_us = a.elapsed_time(b) * 1e3 / (iters * 4 * sets)
    gemv_gbs = (2 * d * inter) / (gemv_us * 1e-6) / 1e9
    del layers, graph, g2
    torch.cuda.empty_cache()
    return {
        "nb": nb, "us_median": round(st["median"], 3), "us_mean": round(st["mean"], 3),
        "us_p10": round(st["p10"], 3), "us_p90": round(st["p90"], 3),
        "union_rows": round(u_avg, 1), "bytes": int(bytes_layer),
        "achieved_GBs": round(achieved, 1), "frac_hbm": round(achieved / HBM_PEAK_GBS, 4),
        "gate_gemv_us": round(gemv_us, 3), "gate_gemv_GBs": round(gemv_gbs, 1),
    }


def moc28_prefill_bench(t=4096, reps=20):
    """MoC 2:8 prefill (config 4): fused gate/up + top-2-of-8 + compacted down."""
    import torch
    from moc_amd.inference.inference_ffn import InferenceMoCSwiGLUFFN
    d, inter = D1B, 5464
    m = InferenceMoCSwiGLUFFN(d, inter, inter // 4, grouped_a=2, grouped_b=8)
    m = m.to("cuda", torch.bfloat16).eval()
    gen = torch.Generator(device="cuda").manual_seed(1234)
    with torch.no_grad():
        for p in m.parameters():
            p.copy_(torch.randn(p.shape, device="cuda", generator=gen) * 0.02)
            p.requires_grad_(False)
        m.gate_proj.weight[5461:].zero_()
        m.up_proj.weight[5461:].zero_()
        m.down_proj.weight[:, 5461:].zero_()
    x = torch.randn(t, d, device="cuda", generator=gen).to(torch.bfloat16)
    runner = m.make_moc2_8_graph_runner(batch_size=t)
    for _ in range(5):
        runner(x)
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(reps)]
    for a, b in evs:
        a.record()
        runner.graph.replay()
        b.record()
    torch.cuda.synchronize()
    us = statistics.median(a.elapsed_time(b) for a, b in evs) * 1e3
    kp = inter // 4
    flop = 2 * 2 * t * d * inter + 2 * t * kp * d
    tf = flop / (us * 1e-6) / 1e12
    del m, runner
    torch.cuda.empty_cache()
    # the Down runs on the structured-sparse MFMA over the 2:4-packed
    # selection: half the dense product's MFMA work, twice the compacted
    # product's own FLOP (each 2:8 group keeps 2 of 8 channels, stored as 2
    # of every 4)
    down_alg = 2 * t * kp * d
    return {"tokens": t, "us": round(us, 2), "algorithmic_gflop": round(flop / 1e9, 1),
            "tflops": round(tf, 1), "frac_mfma": round(tf / BF16_PEAK_TFLOPS, 4),
            "down": {"kernel": "gemm_pp_kernel<..., SP> (v_smfmac_f32_32x32x32_bf16, 2:4-packed A)",
                     "algorithmic_gflop": round(down_alg / 1e9, 1),
                     "executed_gflop": round(2 * down_alg / 1e9, 1),
                     "dense_equivalent_gflop": round(2 * t * inter * d / 1e9, 1)}}


def cpu_baseline(seconds: float):
    """The oracle's CPU restatement of the reference path (moc_gcp forward +
    backward), on a bounded token sample of the 1b workload, scaled to the
    full 16384-token layer."""
    import torch
    from oracle import moc_oracle as O
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    ts = 4096
    x, wg, wu, wd, go = seeded_inputs(ts, D1B, I1B, seed=4321)
    times = []
    t_start = time.perf_counter()
    for i in range(6):
        t0 = time.perf_counter()
        f = O.ffn_forward(x, wg, wu, wd, K1B, "moc_gcp")
        O.ffn_backward(x, wg, wu, wd, f, go, gcp=True)
        dt = time.perf_counter() - t0
        if i > 0:
            times.append(dt)
        if len(times) >= 3 and time.perf_counter() - t_start > seconds:
            break
    med = statistics.median(times)
    total_tokens = BATCH1B * SEQ1B
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(med * total_tokens / ts * 1e6, 1), "unit": "us",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"oracle moc_gcp fwd+bwd on {ts} of {total_tokens} tokens at the 1b shape "
                      f"(bf16 storage, f32 matmul), median of {len(times)} reps after 1 warmup, "
                      f"scaled x{total_tokens // ts}",
            "cpu_model": cpu_model or platform.processor()}


FP32_PEAK_TFLOPS = 157.3


def in_step_gemm(records, step_starts):
    """GEMM time inside the timed fwd+bwd steps, from the probe's records
    (every GEMM launch bracketed by timing events on the stream it ran on).
    Launches on the two streams can overlap, so the GEMM time of a step is
    the length of the union of its launch intervals (relative to the step's
    start event); per launch position, the mean bracketed duration."""
    steps = len(step_starts)
    per_step = len(records) // steps
    busy, flops = [], []
    for i, ref in enumerate(step_starts):
        rs = records[i * per_step:(i + 1) * per_step]
        iv = sorted((ref.elapsed_time(a), ref.elapsed_time(b)) for _, a, b, _ in rs)
        tot, cur_s, cur_e = 0.0, None, None
        for s0, e0 in iv:
            if cur_e is None or s0 > cur_e:
                if cur_e is not None:
                    tot += cur_e - cur_s
                cur_s, cur_e = s0, e0
            else:
                cur_e = max(cur_e, e0)
        tot += cur_e - cur_s
        busy.append(tot)
        flops.append(sum(f for _, _, _, f in rs))
    ms = statistics.median(busy)
    flop = flops[0]
    launches = []
    for j in range(per_step):
        rs = records[j::per_step]
        us = statistics.mean(a.elapsed_time(b) for _, a, b, _ in rs) * 1e3
        launches.append({"gemm": rs[0][0], "us": round(us, 1),
                         "tflops": round(rs[0][3] / (us * 1e-6) / 1e12, 1)})
    achieved = flop / (ms * 1e-3) / 1e12
    return {"gemm_ms_per_step": round(ms, 4), "algorithmic_flop_per_step": flop,
            "achieved": round(achieved, 1), "frac": round(achieved / BF16_PEAK_TFLOPS, 4),
            "per_launch": launches}


def gather_report(x, wg, k, tiles=(256, 64, 16)):
    """Executed vs algorithmic FLOP of the training step's GEMMs over the
    channel dimension, from the real selection of the bench input.  The
    layer runs every product densely over all I channels on MFMA tiles; the
    algorithmic count takes only each token's K selected channels; a
    gathered-row GEMM over an M-tile of tokens would have to run over the
    union of the tile's selections, whose share of I is measured here for
    several tile heights (1 - (1 - K/I)^m for independent tokens)."""
    import torch
    from moc_amd import kernels as K
    t, d = x.shape[0] * x.shape[1], x.shape[-1]
    inter = wg.shape[0]
    g = K.linear(x.reshape(-1, d).to(torch.bfloat16), wg)
    _, _, mask = K.topk_rows(g, k, want_vals=False, want_mask=True)
    bits = torch.zeros(t, (inter + 31) // 32 * 32, dtype=torch.bool, device=x.device)
    words = mask.view(torch.int32)
    for b in range(32):
        bits[:, b::32] = ((words >> b) & 1).bool()
    bits = bits[:, :inter]
    union = {}
    for m in tiles:
        tb = bits[: (t // m) * m].view(t // m, m, inter).any(dim=1)
        union[f"tile_{m}_tokens"] = round(tb.float().mean().item(), 4)
    dense = 2.0 * t * d * inter
    sparse = 2.0 * t * d * k
    # D, dWd, gZ (needed only at selected positions), dWg, dWu, dX (2 products)
    prods = 7
    return {"products_over_channels": prods,
            "executed_gflop_dense": round(prods * dense / 1e9, 1),
            "algorithmic_gflop_selected": round(prods * sparse / 1e9, 1),
            "gathered_gflop_at_tile_256": round(prods * dense * union["tile_256_tokens"] / 1e9, 1),
            "union_share_of_channels": union,
            "note": "G and U (2 products) are dense in the reference too; the other 7 products "
                    "touch only selected channels per token, but a 256-token MFMA tile's union "
                    "of selections covers about all channels, so gathering rows would not cut "
                    "the executed FLOP"}


def cfg2_bench(steps=20, warmup=5, probe_steps=3):
    """Config 2: the 130m layer (8 x 1024 tokens, d 768, I 2048, k 384,
    moc_gcp) fwd+bwd; then probe_steps more steps with the GEMM launches
    bracketed by timing events (the probe costs host time at this size, so
    the headline latency comes from the unprobed steps)."""
    x2, wg2, wu2, wd2, go2 = seeded_inputs(8 * 1024, 768, 2048)
    m2 = build_layer(768, 2048, 384, [w.cuda() for w in (wg2, wu2, wd2)])
    x2d = x2.reshape(8, 1024, 768).cuda().requires_grad_(True)
    go2d = go2.reshape(8, 1024, 768).cuda()
    ms2, f2, b2 = time_train_layer(m2, x2d, go2d, steps, warmup)
    rec2, starts2 = [], []
    if probe_steps:
        time_train_layer(m2, x2d, go2d, probe_steps, 1, probe=rec2, step_starts=starts2)
    flop2 = 9 * 2 * 8192 * 768 * 2048
    tf2 = flop2 / (ms2 * 1e-3) / 1e12
    return {
        "us": round(ms2 * 1e3, 1), "fwd_us": round(f2["median"] * 1e3, 1),
        "bwd_us": round(b2["median"] * 1e3, 1), "tokens_per_s": round(8192 / (ms2 * 1e-3), 1),
        "roofline": {"bound": "mfma", "achieved": round(tf2, 1), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tf2 / BF16_PEAK_TFLOPS, 4),
                     "algorithmic_gflop": round(flop2 / 1e9, 1),
                     "gemm_in_step": in_step_gemm(rec2, starts2) if probe_steps else None}}


def cfg1_bench(reps=50):
    """Config 1: one MoC FFN layer forward at the 60m preset shape in fp32
    (X [2, 256, 512], I 1376, K 256; `moc` mode), eager launches."""
    import torch
    from moc_amd.ffn import MoCSwiGLUFFN
    d, inter, k = 512, 1376, 256
    x, wg, wu, wd, _ = seeded_inputs(512, d, inter, dtype=torch.float32)
    m = MoCSwiGLUFFN(d, inter, k, mode="moc").to("cuda")
    with torch.no_grad():
        for p_, w in zip((m.gate_proj.weight, m.up_proj.weight, m.down_proj.weight), (wg, wu, wd)):
            p_.copy_(w)
    xd = x.reshape(2, 256, d).cuda()
    with torch.no_grad():
        for _ in range(10):
            m(xd)
        torch.cuda.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(reps)]
        for a, b in ev:
            a.record()
            m(xd)
            b.record()
        torch.cuda.synchronize()
    st = summarize([a.elapsed_time(b) * 1e3 for a, b in ev])
    # algorithmic: gate + up GEMMs + the down projection of the K selected channels
    flop = 2 * 2 * 512 * d * inter + 2 * 512 * k * d
    tf = flop / (st["median"] * 1e-6) / 1e12
    return {"us": round(st["median"], 2), "us_p10": round(st["p10"], 2), "us_p90": round(st["p90"], 2),
            "tokens_per_s": round(512 / (st["median"] * 1e-6), 1), "dtype": "f32",
            "roofline": {"bound": "fp32 (latency-bound at this size)", "achieved": round(tf, 2),
                         "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tf / FP32_PEAK_TFLOPS, 4),
                         "algorithmic_gflop": round(flop / 1e9, 3)}}


def _cpu_setup():
    import torch
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    return threads


def _cpu_time(fn, reps=3, budget_s=8.0):
    """Median wall time of fn() after one untimed call, at least `reps`
    timed calls unless the budget runs out after the first."""
    fn()
    times = []
    t_start = time.perf_counter()
    while len(times) < reps:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s:
            break
    return statistics.median(times), len(times)


def cpu_cfg1():
    import torch
    from oracle import moc_oracle as O
    th = _cpu_setup()
    d, inter, k = 512, 1376, 256
    x, wg, wu, wd, _ = seeded_inputs(512, d, inter, dtype=torch.float32)
    med, n = _cpu_time(lambda: O.ffn_forward(x, wg, wu, wd, k, "moc"), reps=10)
    return {"value": round(med * 1e6, 1), "unit": "us", "cores": th, "kind": "port",
            "sample": f"oracle `moc` forward, the whole workload (512 tokens, f32), median of {n}"}


def cpu_cfg2():
    from oracle import moc_oracle as O
    th = _cpu_setup()
    t, d, inter, k = 8192, 768, 2048, 384
    x, wg, wu, wd, go = seeded_inputs(t, d, inter)

    def run():
        f = O.ffn_forward(x, wg, wu, wd, k, "moc_gcp")
        O.ffn_backward(x, wg, wu, wd, f, go, gcp=True)

    med, n = _cpu_time(run, reps=2)
    return {"value": round(med * 1e6, 1), "unit": "us", "cores": th, "kind": "port",
            "sample": f"oracle moc_gcp fwd+bwd, the whole workload (8192 tokens; bf16 storage, "
                      f"f32 matmul), median of {n}"}


def cpu_decode(nb):
    import torch
    from oracle import moc_oracle as O
    th = _cpu_setup()
    d, inter, k = D1B, I1B, K1B
    g = torch.Generator().manual_seed(1234)
    wg = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16)
    wu = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16)
    wd = (torch.randn(d, inter, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(nb, d, generator=g).to(torch.bfloat16)
    med, n = _cpu_time(lambda: O.masked_reference(x, wg, wu, wd, k), reps=10, budget_s=3.0)
    return {"value": round(med * 1e6, 1), "unit": "us", "cores": th, "kind": "port",
            "sample": f"oracle masked_reference, the whole workload ({nb} token(s), bf16 storage, "
                      f"f32 matmul), median of {n}"}


def cpu_cfg4():
    import torch
    from oracle import moc_oracle as O
    th = _cpu_setup()
    t, d, inter = 4096, D1B, 5464
    g = torch.Generator().manual_seed(1234)
    x = torch.randn(t, d, generator=g).to(torch.bfloat16)
    wg = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16)
    wu = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16)
    wdt = (torch.randn(inter, d, generator=g) * 0.02).to(torch.bfloat16)

    def run():
        idx, sz, _ = O.grouped_top2_up_silu(x, wg, wu)
        O.selected_down(sz, idx, wdt)

    med, n = _cpu_time(run, reps=1, budget_s=10.0)
    return {"value": round(med * 1e6, 1), "unit": "us", "cores": th, "kind": "port",
            "sample": f"oracle 2:8 gate/up + top-2-of-8 + compacted down, the whole workload (4096 "
                      f"tokens; bf16 storage, f32 matmul), median of {n}"}


def cpu_cfg5():
    """Config 5 on the CPU: the 350m decoder's training step with the
    oracle's moc_gcp FFN (forward and backward as an autograd Function),
    stock PyTorch attention/norms/embeddings and AdamW, batch 16 x 256, f32.
    A bounded sample: one transformer block's fwd+bwd and AdamW update, and
    the rest of the step (embedding, final norm, LM head, loss, their AdamW)
    are timed separately; the 24-layer step is rest + 24 x block."""
    import torch
    from dataclasses import replace
    from oracle import moc_oracle as O
    from moc_amd import PRESETS, build_model
    from moc_amd.model import TransformerBlock
    th = _cpu_setup()

    class OracleGCP(torch.autograd.Function):
        @staticmethod
        def forward(ctx, x, wg, wu, wd, k):
            x2 = x.reshape(-1, x.shape[-1])
            f = O.ffn_forward(x2, wg, wu, wd, k, "moc_gcp")
            ctx.f, ctx.shape = f, x.shape
            ctx.save_for_backward(x2, wg, wu, wd)
            return f["out"].reshape(x.shape).to(x.dtype)

        @staticmethod
        def backward(ctx, go):
            x2, wg, wu, wd = ctx.saved_tensors
            dx, dwg, dwu, dwd = O.ffn_backward(x2, wg, wu, wd, ctx.f, go.reshape(x2.shape), gcp=True)
            return (dx.reshape(ctx.shape).to(x2.dtype), dwg.to(wg.dtype), dwu.to(wu.dtype),
                    dwd.to(wd.dtype), None)

    class OracleFFN(torch.nn.Module):
        def __init__(self, ffn, k):
            super().__init__()
            self.gate_proj, self.up_proj, self.down_proj = ffn.gate_proj, ffn.up_proj, ffn.down_proj
            self.k = k

        def forward(self, x):
            return OracleGCP.apply(x, self.gate_proj.weight, self.up_proj.weight,
                                   self.down_proj.weight, self.k)

    def adamw(params):
        return torch.optim.AdamW(params, lr=1e-3, betas=(0.9, 0.999), weight_decay=0.0, fused=False)

    torch.manual_seed(1234)
    cfg = replace(PRESETS["350m"], vocab_size=32100, max_seq_len=256)
    # one block: fwd + bwd on a [16, 256, d] activation, then its AdamW update
    blk = TransformerBlock(cfg, ffn_type="dense")
    blk.ffn = OracleFFN(blk.ffn, cfg.k)
    opt_b = adamw(blk.parameters())
    h = torch.randn(16, 256, cfg.hidden_size, generator=torch.Generator().manual_seed(1))
    h.requires_grad_(True)

    def block_step():
        blk(h).sum().backward()
        opt_b.step()
        opt_b.zero_grad(set_to_none=True)

    t_block, _ = _cpu_time(block_step, reps=2, budget_s=4.0)
    # the rest: a model with no blocks (embedding, norm, LM head, loss, AdamW)
    rest = build_model(replace(cfg, num_hidden_layers=0), ffn_type="dense")
    opt_r = adamw(rest.parameters())
    tok = torch.randint(0, 32100, (16, 256), generator=torch.Generator().manual_seed(1234))

    def rest_step():
        _, loss = rest(tok, labels=tok)
        loss.backward()
        opt_r.step()
        opt_r.zero_grad(set_to_none=True)

    t_rest, _ = _cpu_time(rest_step, reps=2, budget_s=4.0)
    step = t_rest + cfg.num_hidden_layers * t_block
    return {"value": round(16 * 256 / step, 1), "unit": "tokens/s", "cores": th, "kind": "port",
            "ms_per_step": round(step * 1e3, 1),
            "sample": f"350m decoder step, f32, 16x256 tokens: one block (attention + oracle moc_gcp "
                      f"FFN) fwd+bwd+AdamW {t_block * 1e3:.0f} ms and the rest (embedding, LM head, "
                      f"loss, AdamW) {t_rest * 1e3:.0f} ms timed; step = rest + "
                      f"{cfg.num_hidden_layers} x block"}


def gemm_k_sweep() -> dict:
    """Time C[16384, N] = A[16384, K] B[K, N] (bf16, padded 16-byte aligned
    outputs) for N in (5461, 2048) and K from 256 to 8192; per N, fit the
    time per round of 256 tiles as t0 + nK tk (nK = K / 64 K tiles)."""
    import torch
    from moc_amd import kernels as K
    g = torch.Generator(device="cuda").manual_seed(1)
    m, res = 16384, {}
    for n in (5461, 2048):
        out = K.padded_empty(m, n, torch.bfloat16, "cuda")
        a_all = torch.randn(m, 8192, device="cuda", generator=g).to(torch.bfloat16)
        w_all = (torch.randn(n, 8192, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
        tiles = ((m + 255) // 256) * ((n + 255) // 256)
        rounds = -(-tiles // K.cu_count(torch.cuda.current_device()))
        pts = []
        for kk in (256, 512, 1024, 2048, 4096, 8192):
            a, w = a_all[:, :kk], w_all[:, :kk]
            fn = lambda: K.gemm(a, w.t(), out=out)  # noqa: E731
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                  for _ in range(15)]
            for e0, e1 in ev:
                e0.record()
                fn()
                e1.record()
            torch.cuda.synchronize()
            us = statistics.median(e0.elapsed_time(e1) for e0, e1 in ev) * 1e3
            pts.append((kk, us))
        xs = [kk / 64 for kk, _ in pts]
        ys = [us / rounds for _, us in pts]
        mx, my = statistics.mean(xs), statistics.mean(ys)
        tk = sum((x - mx) * (y - my) for x, y in zip(xs, ys)) / sum((x - mx) ** 2 for x in xs)
        res[f"N{n}"] = {"tiles": tiles, "rounds": rounds,
                        "us_by_K": {str(kk): round(us, 1) for kk, us in pts},
                        "fit_t0_us_per_round": round(my - tk * mx, 2), "fit_us_per_K_tile": round(tk, 3)}
        log(f"gemm K sweep N={n}: {res[f'N{n}']}")
    return res


def trace_by_grid(d: str) -> None:
    """Per (kernel, grid size) of a rocprofv3 kernel trace: dispatches, mean
    and median duration (one kernel template serving launches of several
    shapes, told apart by their grids)."""
    import csv
    import glob
    trace = glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True)
    runs = {}
    for r in csv.DictReader(open(trace[0])):
        grid = int(r.get("Grid_Size_X") or r.get("Grid_Size") or 0)
        runs.setdefault((r["Kernel_Name"], grid), []).append(
            (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    print("\n| kernel | grid (threads) | dispatches | mean us | median us |\n|---|---:|---:|---:|---:|")
    for (name, grid), v in sorted(runs.items(), key=lambda kv: -sum(kv[1])):
        name = name if len(name) < 100 else name[:97] + "..."
        print(f"| `{name}` | {grid} | {len(v)} | {statistics.mean(v):.2f} | {statistics.median(v):.2f} |")


def trace_summary(d: str, steps: float, headline: bool) -> None:
    """Markdown summary of a rocprofv3 CSV output directory: the kernels by
    total time (from *kernel_stats.csv), and with `headline` the GEMM
    launches of the timed steps of `bench.py --skip-extra` (from
    *kernel_trace.csv): per launch the mean and median duration over the
    timed steps, and the union of a step's GEMM intervals."""
    import csv
    import glob
    stats = glob.glob(os.path.join(d, "**", "*kernel_stats.csv"), recursive=True)
    if stats:
        rows = list(csv.DictReader(open(stats[0])))
        tot = sum(float(r["TotalDurationNs"]) for r in rows)
        print(f"Kernels: {len(rows)}; total kernel time {tot / 1e6:.3f} ms; per step ({steps:g} steps) "
              f"{tot / 1e6 / steps:.3f} ms\n")
        print("| kernel | calls | total ms | ms per step | mean us |\n|---|---:|---:|---:|---:|")
        for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"]))[:30]:
            name = r["Name"] if len(r["Name"]) < 100 else r["Name"][:97] + "..."
            print(f"| `{name}` | {r['Calls']} | {float(r['TotalDurationNs']) / 1e6:.3f} | "
                  f"{float(r['TotalDurationNs']) / 1e6 / steps:.3f} | {float(r['AverageNs']) / 1e3:.2f} |")
    if not headline:
        return
    trace = glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True)
    ev = []
    for r in csv.DictReader(open(trace[0])):
        if "gemm_pp_kernel" in r["Kernel_Name"]:
            # grid sizes are in work-items: workgroups = grid / workgroup size
            grid = int(r.get("Grid_Size_X") or r.get("Grid_Size") or 0)
            wg = int(r.get("Workgroup_Size_X") or r.get("Workgroup_Size") or 1)
            ev.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), grid // wg, r["Kernel_Name"]))
    ev.sort()
    per_step = 7
    warm, timed = 5, 20  # bench.py's headline: 5 warmup steps, then the timed ones
    names = ["G, U pair", "D = Z Wd^T", "dWd = dD^T Z", "gZ = dD Wd", "dWg = gG^T X", "dWu = gU^T X",
             "dX = gG Wg + gU Wu"]
    by_launch = {n: [] for n in names}
    unions = []
    for st in range(warm, warm + timed):
        step = ev[st * per_step:(st + 1) * per_step]
        # forward: pair then D; backward: dWd (side stream) and gZ overlap, then dWg, dWu, dX
        fwd = step[:2]
        bwd = sorted(step[2:], key=lambda e: (e[2] != 352, e[0]))  # the 352-workgroup launches first
        w352 = [e for e in bwd if e[2] == 352]
        other = [e for e in bwd if e[2] != 352]
        gz = [e for e in other if e[2] != 512][0]
        dx = [e for e in other if e[2] == 512][0]
        for n, e in zip(names, [fwd[0], fwd[1], w352[0], gz, w352[1], w352[2], dx]):
            by_launch[n].append((e[1] - e[0]) / 1e3)
        iv = sorted((e[0], e[1]) for e in step)
        tot, cs, ce = 0, iv[0][0], iv[0][1]
        for a, b in iv[1:]:
            if a > ce:
                tot += ce - cs
                cs, ce = a, b
            else:
                ce = max(ce, b)
        unions.append((tot + ce - cs) / 1e3)
    print("\n| GEMM launch | trace mean us | trace median us |\n|---|---:|---:|")
    for n in names:
        v = by_launch[n]
        print(f"| {n} | {statistics.mean(v):.1f} | {statistics.median(v):.1f} |")
    u = statistics.median(unions)
    flop = 9 * 2.0 * BATCH1B * SEQ1B * D1B * I1B
    print(f"\nUnion of a timed step's GEMM intervals (median of {timed} steps): {u:.1f} us -> "
          f"{flop / 1e12:.3f} TFLOP / {u:.1f} us = {flop / (u * 1e-6) / 1e12:.0f} TFLOP/s = "
          f"{flop / (u * 1e-6) / 1e12 / BF16_PEAK_TFLOPS:.3f} of 2.5 PFLOP/s")


def main():
    args = parse_args()
    if args.trace_summary:
        trace_summary(args.trace_summary, args.trace_steps, args.trace_headline)
        if args.trace_by_grid:
            trace_by_grid(args.trace_summary)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; the MoC FFN path has no "
                                   "multi-GPU mode (bench.py --gpus 1)", "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no ROCm device visible"}))
        sys.exit(1)
    if args.pmc_target:
        pmc_target(args.pmc_target)
        return
    if args.decode_e2e:
        from moc_amd import _native
        from moc_amd.inference.decode_model import measure_decode
        _native.load()
        rows = []
        for row, scope, fuse in (("dense", "whole_graph", False), ("global_moc", "whole_graph", True),
                                 ("global_moc", "whole_graph", False), ("moc_2_8", "whole_graph", True),
                                 ("moc_2_8", "whole_graph", False), ("dense", "layer_graph", False),
                                 ("global_moc", "layer_graph", True), ("moc_2_8", "layer_graph", True),
                                 ("dense", "eager", False), ("global_moc", "eager", True),
                                 ("moc_2_8", "eager", True)):
            log(f"decode e2e {row} {scope} fuse={fuse}")
            rows.append(measure_decode(row, scope=scope, fuse=fuse))
            torch.cuda.empty_cache()
        print(json.dumps({"workload": "greedy decode, 24 layers, d=2048, I=5464, 16 heads, prompt "
                                      "128 + 128 generated tokens, batch 1, bf16, random weights "
                                      "and prompt (seed 1234)",
                          "reference_a800_ms_per_token": {"dense": 4.310, "global_moc": 4.003,
                                                          "moc_2_8": 3.586},
                          "rows": rows}), flush=True)
        return
    if args.gemm_k_sweep:
        from moc_amd import _native
        _native.load()
        print(json.dumps({"gemm_k_sweep": gemm_k_sweep()}), flush=True)
        return
    if args.roofline_only:
        from moc_amd import _native
        _native.load()
        t = BATCH1B * SEQ1B
        x, wg, wu, wd, go = seeded_inputs(t, D1B, I1B)
        xd = x.reshape(BATCH1B, SEQ1B, D1B).cuda()
        god = go.reshape(BATCH1B, SEQ1B, D1B).cuda()
        print(json.dumps({"roofline": gemm_roofline(t, D1B, I1B, K1B, (wg, wu, wd), xd, god)}), flush=True)
        return
    if args.only:
        fn = {"cfg1": cfg1_bench, "cfg2": cfg2_bench, "cfg4": moc28_prefill_bench}[args.only]
        print(json.dumps({"config": args.only, "result": fn()}), flush=True)
        return
    if args.cfg5:
        print(json.dumps({"config": "350m LLaMA training step (config 5), 16x256 tokens, bf16",
                          "steps": args.cfg5_steps,
                          "result": cfg5_bench(args.cfg5_steps, args.cfg5_row)}))
        return
    from moc_amd import _native
    _native.load()  # the HIP library must be there: no fallback

    t = BATCH1B * SEQ1B
    log("1b MoC+GCP FFN fwd+bwd: building inputs")
    x, wg, wu, wd, go = seeded_inputs(t, D1B, I1B)
    ws = (wg, wu, wd)
    m = build_layer(D1B, I1B, K1B, [w.cuda() for w in ws])
    xd = x.reshape(BATCH1B, SEQ1B, D1B).cuda().requires_grad_(True)
    god = go.reshape(BATCH1B, SEQ1B, D1B).cuda()
    ms_step, fwd, bwd = time_train_layer(m, xd, god, args.steps, args.warmup)
    log(f"fwd+bwd {ms_step:.3f} ms/step (fwd {fwd['median']:.3f}, bwd {bwd['median']:.3f})")
    # the GEMM launches' in-step time comes from separate probed steps (the
    # probe adds two timing events per launch, so it stays out of `value`)
    rec, starts = [], []
    time_train_layer(m, xd, god, PROBE_STEPS, 1, probe=rec, step_starts=starts)
    inst = in_step_gemm(rec, starts)
    iso = gemm_roofline(t, D1B, I1B, K1B, ws, xd.detach(), god)
    log(f"GEMMs in the timed steps {inst['gemm_ms_per_step']:.3f} ms ({inst['achieved']} TFLOP/s), "
        f"isolated {iso['gemm_ms_per_step']:.3f} ms ({iso['achieved']} TFLOP/s)")
    roof = {"bound": "mfma", "achieved": inst["achieved"], "peak": BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": inst["frac"], "traffic": iso.pop("traffic"),
            "traffic_note": iso.pop("traffic_note"), "kernel": iso.pop("kernel"),
            "method": f"algorithmic FLOP of the step's nine GEMMs (7 launches) / the time the GPU "
                      f"spent in them inside {PROBE_STEPS} fwd+bwd steps run after the timed ones with "
                      "every GEMM launch bracketed by timing events on its own stream (union of the "
                      "launch intervals; per_launch: mean bracketed duration, which includes the "
                      "slowdown of launches that overlap another stream's); `isolated`: the same "
                      "launches timed back to back; `layer_step`: the same FLOP over the whole "
                      "timed fwd+bwd step (`value`)",
            "algorithmic_flop_per_step": inst["algorithmic_flop_per_step"],
            "gemm_ms_per_step": inst["gemm_ms_per_step"], "per_launch": inst["per_launch"],
            "isolated": {k: iso[k] for k in ("achieved", "frac", "gemm_ms_per_step", "per_launch")},
            "layer_step": layer_step_roofline(inst["algorithmic_flop_per_step"], ms_step)}
    gath = gather_report(xd.detach(), m.gate_proj.weight.detach(), K1B)
    log(f"gather report: union share {gath['union_share_of_channels']}")
    del m, xd, god
    torch.cuda.empty_cache()

    configs = {}
    log("decode B=1")
    dec = {1: decode_bench(1, groups=args.decode_groups, iters=args.decode_iters)}
    d1 = dec[1]
    roof_dec = {"bound": "hbm", "achieved": d1["achieved_GBs"], "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": d1["frac_hbm"], "traffic": DECODE_B1_TRAFFIC_BYTES,
                "kernel": "decode layer (gate + dense-U GEMV pair, then Top-K + z + selected Down "
                          "in one launch), B=1",
                "us": d1["us_median"], "bytes": d1["bytes"]}
    cpu_on = not args.no_cpu_baseline
    if not args.skip_extra:
        log("config 1: 60m fp32 MoC forward")
        configs["1_60m_moc_fwd_f32"] = cfg1_bench()
        log("config 2: 130m MoC+GCP fwd+bwd")
        configs["2_130m_moc_gcp_fwd_bwd"] = cfg2_bench()
        for nb in (4, 16):
            log(f"decode B={nb}")
            dec[nb] = decode_bench(nb, groups=args.decode_groups, iters=args.decode_iters)
        configs["3_decode_1b"] = {f"B{nb}": {**r, "tokens_per_s": round(nb / (r["us_median"] * 1e-6), 1)}
                                  for nb, r in dec.items()}
        log("MoC 2:8 decode B=1/4/16")
        configs["3b_moc28_decode_1b"] = {
            "workload": "MoC 2:8 decode layer, d=2048, d_ffn=5464, top 2 of every 8 channels, bf16 "
                        "(the reference's single-layer row: 56.011 us at B=1 on A800, "
                        "results/inference_ffn.md:19)",
            **{f"B{nb}": decode_bench(nb, groups=args.decode_groups, iters=args.decode_iters, moc28=True)
               for nb in (1, 4, 16)}}
        log("config 4: 2:8 prefill")
        configs["4_moc28_prefill_4096"] = moc28_prefill_bench()
        log("config 5: 350m training step")
        configs["5_350m_step"] = cfg5_bench(args.cfg5_steps)
        if cpu_on:
            log("cpu baselines of configs 1-5")
            configs["1_60m_moc_fwd_f32"]["cpu_baseline"] = cpu_cfg1()
            configs["2_130m_moc_gcp_fwd_bwd"]["cpu_baseline"] = cpu_cfg2()
            configs["3_decode_1b"]["cpu_baseline"] = {f"B{nb}": cpu_decode(nb) for nb in (1, 4, 16)}
            configs["4_moc28_prefill_4096"]["cpu_baseline"] = cpu_cfg4()
            configs["5_350m_step"]["cpu_baseline"] = cpu_cfg5()

    cpu = None
    if cpu_on:
        log("cpu baseline (headline)")
        cpu = cpu_baseline(args.cpu_seconds)

    out = {
        "metric": METRIC, "value": round(ms_step * 1e3, 1), "unit": "us",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: X~N(0,1), W~N(0,0.02), dD~N(0,1), seed 1234 (no checkpoints)",
        "config": {"workload": "moc_gcp FFN layer fwd+bwd, 1b preset shape", "tokens": t,
                   "batch": BATCH1B, "seq_len": SEQ1B, "hidden": D1B, "intermediate": I1B,
                   "k": K1B, "parallelism": "none (one GPU)"},
        "tokens_per_s": round(t / (ms_step * 1e-3), 1),
        "fwd_ms": summarize_round(fwd), "bwd_ms": summarize_round(bwd),
        "roofline": roof, "roofline_decode": roof_dec, "cpu_baseline": cpu, "configs": configs,
        "gemm_flop_executed_vs_algorithmic": gath,
        "device": torch.cuda.get_device_name(0),
    }
    print(json.dumps(out), flush=True)


def layer_step_roofline(flop: float, ms_step: float) -> dict:
    """The step's GEMM FLOP over the whole fwd+bwd step time (Top-K, sparse
    aux kernels and stream joins included)."""
    tf = flop / (ms_step * 1e-3) / 1e12
    return {"achieved": round(tf, 1), "frac": round(tf / BF16_PEAK_TFLOPS, 4), "ms": round(ms_step, 4)}


def summarize_round(s):
    return {k: (round(v, 4) if isinstance(v, float) else v) for k, v in s.items()}


if __name__ == "__main__":
    main()
