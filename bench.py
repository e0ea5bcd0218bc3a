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
                share one, dX sums two products) / their summed HIP-event time,
                against the 2.5 PFLOP/s dense bf16 peak;
  roofline_decode  global-MoC decode (config 3, B=1): union-of-selected-rows
                bytes / layer time against 8 TB/s, cold weights (rotation
                over 8 weight sets > 2x the 256 MB MALL), HIP-graph replays;
  cpu_baseline  the repo's CPU restatement (oracle/) of the reference path,
                timed on this host on a bounded token sample and scaled to
                the full layer;
  extra         the other configs: decode B=1/4/16, 2:8 prefill (config 4),
                130m MoC+GCP fwd+bwd (config 2), fwd/bwd split.

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
    p.add_argument("--decode-groups", type=int, default=40)
    p.add_argument("--decode-iters", type=int, default=50)
    p.add_argument("--skip-extra", action="store_true", help="headline + rooflines only")
    p.add_argument("--cfg5", action="store_true",
                   help="only the 350m-model training step (config 5): tokens/s and peak "
                        "memory, moc_gcp vs dense, one JSON line")
    p.add_argument("--cfg5-steps", type=int, default=10)
    p.add_argument("--decode-e2e", action="store_true",
                   help="only end-to-end greedy decode of a 24-layer 1b-shape decoder (dense, "
                        "global MoC, MoC 2:8; eager and whole-step graph): ms/token, one JSON line")
    p.add_argument("--roofline-only", action="store_true",
                   help="only the seven GEMM launches of the roofline (for rocprofv3 kernel "
                        "traces whose per-kernel averages match roofline.per_launch)")
    p.add_argument("--pmc-target", choices=["gemm", "copy", "decode"], default=None,
                   help="only launch one workload a few times (for rocprofv3 --pmc runs): the G "
                        "GEMM of the 1b layer, a plain 256 MiB copy kernel (counter scale), or "
                        "the B=1 decode layer over 8 weight sets")
    return p.parse_args()


def cfg5_bench(steps: int) -> dict:
    """Config 5: a 350m LLaMA training step (24 layers, d=1024, I=2736,
    K=512), bf16 parameters, AdamW (0.9/0.999, wd 0, fused=False, lr 1e-3),
    tokens [16, 256] uniform over the 32100-token vocabulary with labels =
    tokens; 1 warmup step, then `steps` timed steps; peak memory after the
    warmup (the method of benchmark_training_throughput.py:51-114 and
    benchmark_memory.py:51-107).  Attention, norms and embeddings are stock
    PyTorch; the FFN is this build's."""
    import torch
    from moc_amd import PRESETS, build_model
    from dataclasses import replace
    out = {}
    for ffn_type in ("moc_gcp", "dense"):
        torch.manual_seed(1234)
        cfg = replace(PRESETS["350m"], vocab_size=32100, max_seq_len=256)
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
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        t0 = time.perf_counter()
        for _ in range(steps):
            loss = step().detach()
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / steps
        out[ffn_type] = {"ms_per_step": round(dt * 1e3, 2), "tokens_per_s": round(16 * 256 / dt, 1),
                         "peak_mem_gib": round(torch.cuda.max_memory_allocated() / 2**30, 3),
                         "loss_first": round(float(loss0), 4), "loss_last": round(float(loss), 4)}
        log(f"cfg5 {ffn_type}: {out[ffn_type]}")
        del model, opt
        torch.cuda.empty_cache()
    return out


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
    elif which == "decode":
        gen = torch.Generator(device="cuda").manual_seed(1234)
        layers = []
        for _ in range(8):
            wg = (torch.randn(I1B, D1B, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
            wu = (torch.randn(I1B, D1B, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
            wdt = (torch.randn(I1B, D1B, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
            layers.append((wg, wu, wdt))
        x = torch.randn(1, D1B, device="cuda", generator=gen).to(torch.bfloat16)
        gate = torch.empty(1, I1B, device="cuda", dtype=torch.bfloat16)
        y = torch.empty(1, D1B, device="cuda", dtype=torch.bfloat16)
        ws = K.global_after_gate_workspace(1, I1B, K1B, D1B, "cuda")
        for _ in range(3):
            for wg, wu, wdt in layers:
                K.gemv(x, wg, out=gate)
                K.global_after_gate(x, gate, wu, wdt, K1B, workspace=ws, out=y)
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


def time_train_layer(m, x, go, steps, warmup):
    """Reference method: untimed warmup, then K timed fwd+bwd steps bracketed
    by a device synchronisation; per-step events split fwd and bwd."""
    import torch
    for _ in range(warmup):
        m.zero_grad(set_to_none=True)
        x.grad = None
        m(x).backward(go)
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
           torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
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
    fwd = [a.elapsed_time(b) for a, b, _ in ev]
    bwd = [b.elapsed_time(c) for _, b, c in ev]
    return wall * 1e3 / steps, summarize(fwd), summarize(bwd)


# L2-miss (MALL/HBM side) bytes of one G,U pair launch at the 1b shape, from the
# FETCH_SIZE / WRITE_SIZE counter runs in profiles/gemm_GU_pair_traffic.md, each
# scaled by what the counter reads for a copy kernel of known size
# (FETCH_SIZE x 2.000, WRITE_SIZE x 1.000).
GEMM_GU_TRAFFIC_BYTES = 1133.3e6 + 358.6e6
# the same for the B=1 decode layer (gate GEMV + fused select/up/down),
# profiles/decode_B1_traffic.md
DECODE_B1_TRAFFIC_BYTES = 22.48e6 + 9.33e6


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


def decode_bench(nb, sets=8, groups=40, iters=50):
    """Global-MoC decode layer (config 3): gate GEMV + Top-K + selected Up*SiLU
    + selected Down, captured in one HIP graph that walks `sets` distinct
    weight sets (cold MALL), replayed groups x iters times."""
    import torch
    from moc_amd import kernels as K
    d, inter, k = D1B, I1B, K1B
    gen = torch.Generator(device="cuda").manual_seed(1234)
    layers = []
    for _ in range(sets):
        wg = (torch.randn(inter, d, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
        wu = (torch.randn(inter, d, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
        wd = (torch.randn(d, inter, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
        wdt = wd.t().contiguous()
        del wd
        layers.append((wg, wu, wdt))
    x = torch.randn(nb, d, device="cuda", generator=gen).to(torch.bfloat16)
    gate = [torch.empty(nb, inter, device="cuda", dtype=torch.bfloat16) for _ in range(sets)]
    ys = [torch.empty(nb, d, device="cuda", dtype=torch.bfloat16) for _ in range(sets)]
    ws = K.global_after_gate_workspace(nb, inter, k, d, "cuda")

    def run_all():
        for (wg, wu, wdt), g, y in zip(layers, gate, ys):
            K.gemv(x, wg, out=g)
            K.global_after_gate(x, g, wu, wdt, k, workspace=ws, out=y)

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
    for g in gate:
        _, idx, _ = K.topk_rows(g, k, want_vals=False)
        union.append(int(torch.unique(idx).numel()))
    u_avg = sum(union) / len(union)
    act = 2 * nb * d * 2 + 2 * nb * inter * 2
    bytes_layer = 2 * d * inter + 2 * 2 * d * u_avg + act
    st = summarize(samples)
    achieved = bytes_layer / (st["median"] * 1e-6) / 1e9
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
    return {"tokens": t, "us": round(us, 2), "algorithmic_gflop": round(flop / 1e9, 1),
            "tflops": round(tf, 1), "frac_mfma": round(tf / BF16_PEAK_TFLOPS, 4)}


def cpu_baseline(seconds: float):
    """The oracle's CPU restatement of the reference path (moc_gcp forward +
    backward), on a bounded token sample of the 1b workload, scaled to the
    full 16384-token layer."""
    import torch
    from oracle import moc_oracle as O
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    ts = 1024
    x, wg, wu, wd, go = seeded_inputs(ts, D1B, I1B, seed=4321)
    times = []
    t_start = time.perf_counter()
    for i in range(12):
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


def main():
    args = parse_args()
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
                                 ("moc_2_8", "whole_graph", False), ("dense", "eager", False),
                                 ("global_moc", "eager", True), ("moc_2_8", "eager", True)):
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
    if args.roofline_only:
        from moc_amd import _native
        _native.load()
        t = BATCH1B * SEQ1B
        x, wg, wu, wd, go = seeded_inputs(t, D1B, I1B)
        xd = x.reshape(BATCH1B, SEQ1B, D1B).cuda()
        god = go.reshape(BATCH1B, SEQ1B, D1B).cuda()
        print(json.dumps({"roofline": gemm_roofline(t, D1B, I1B, K1B, (wg, wu, wd), xd, god)}), flush=True)
        return
    if args.cfg5:
        print(json.dumps({"config": "350m LLaMA training step (config 5), 16x256 tokens, bf16",
                          "steps": args.cfg5_steps, "result": cfg5_bench(args.cfg5_steps)}))
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
    roof = gemm_roofline(t, D1B, I1B, K1B, ws, xd.detach(), god)
    log(f"GEMMs {roof['gemm_ms_per_step']:.3f} ms, {roof['achieved']} TFLOP/s")
    del m, xd, god
    torch.cuda.empty_cache()

    extra = {"fwd_ms": summarize_round(fwd), "bwd_ms": summarize_round(bwd)}
    log("decode B=1")
    dec = [decode_bench(1, groups=args.decode_groups, iters=args.decode_iters)]
    d1 = dec[0]
    roof_dec = {"bound": "hbm", "achieved": d1["achieved_GBs"], "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": d1["frac_hbm"], "traffic": DECODE_B1_TRAFFIC_BYTES,
                "kernel": "decode layer (gate GEMV + Top-K + selected Up + selected Down), B=1",
                "us": d1["us_median"], "bytes": d1["bytes"]}
    if not args.skip_extra:
        for nb in (4, 16):
            log(f"decode B={nb}")
            dec.append(decode_bench(nb, groups=args.decode_groups, iters=args.decode_iters))
        log("2:8 prefill")
        extra["moc28_prefill_4096"] = moc28_prefill_bench()
        log("130m MoC+GCP fwd+bwd")
        x2, wg2, wu2, wd2, go2 = seeded_inputs(8 * 1024, 768, 2048)
        m2 = build_layer(768, 2048, 384, [w.cuda() for w in (wg2, wu2, wd2)])
        x2d = x2.reshape(8, 1024, 768).cuda().requires_grad_(True)
        ms2, f2, b2 = time_train_layer(m2, x2d, go2.reshape(8, 1024, 768).cuda(), 20, 5)
        flop2 = 9 * 2 * 8192 * 768 * 2048
        extra["cfg2_130m_fwd_bwd"] = {"us": round(ms2 * 1e3, 1),
                                      "tflops_gemm_equiv": round(flop2 / (ms2 * 1e-3) / 1e12, 1)}
        del m2, x2d
    extra["decode"] = dec

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline")
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
        "roofline": roof, "roofline_decode": roof_dec, "cpu_baseline": cpu, "extra": extra,
        "device": torch.cuda.get_device_name(0),
    }
    print(json.dumps(out), flush=True)


def summarize_round(s):
    return {k: (round(v, 4) if isinstance(v, float) else v) for k, v in s.items()}


if __name__ == "__main__":
    main()
