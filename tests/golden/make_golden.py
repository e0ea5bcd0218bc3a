"""Writes the small golden fixtures under tests/golden/ (run from the repo root).

    python tests/golden/make_golden.py

The reference (xiaohuangji/MoC) ships no tests, fixtures or golden vectors,
so these vectors are computed here from first principles, independently of
oracle/moc_oracle.py:

* selection: brute force in pure Python, sorted(range(I), key=(-value, index))
  on the exact input values, i.e. the stable-descending rule of the
  reference's CUB Top-K (optimized_global_moc_ext.cu:59-82) and the
  lowest-index-among-maxima rule of its 2:8 kernel
  (triton_fused_ffn_kernels.py:103-114);
* FFN forward/backward: torch autograd in float64 of the dense masked formula
  D = (SiLU(X W_g^T) * (X W_u^T) * M) W_d^T with M from the brute-force
  selection (moc/ffn.py:141-163, 423-497 compute exactly this map).

Inputs are seeded; the FFN inputs are re-drawn until every row has a clear
margin between its K-th and (K+1)-th gate value, so float32 rounding cannot
flip the selection.
"""
from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent


def brute_topk(row: list[float], k: int) -> list[int]:
    def key(i):
        v = row[i]
        if math.isnan(v):
            return (0, -math.inf, i)  # NaN ranks first
        return (1, -v, i)
    return sorted(sorted(range(len(row)), key=key)[:k])


def brute_2of8(row: list[float]) -> list[int]:
    out = []
    for c0 in range(0, len(row), 8):
        grp = list(range(c0, min(c0 + 8, len(row))))
        order = sorted(grp, key=lambda i: (-row[i], i))
        out.extend(order[:min(2, len(grp))])
    return out


def bf16_values(gen: torch.Generator, shape, choices) -> torch.Tensor:
    pick = torch.randint(0, len(choices), shape, generator=gen)
    return torch.tensor(choices, dtype=torch.float32)[pick].to(torch.bfloat16)


def topk_cases():
    gen = torch.Generator().manual_seed(20241)
    cases = {}
    # heavy ties in bf16, including signed zeros and infinities
    choices = [0.0, -0.0, 1.0, -1.0, 0.5, 2.0, 2.0, -3.0, float("inf"), float("-inf"), 0.75]
    s = bf16_values(gen, (6, 40), choices)
    k = 13
    vals = s.float().tolist()
    idx = [brute_topk(r, k) for r in vals]
    cases["topk_bf16_ties"] = dict(scores_bits=s.view(torch.int16).numpy().view(np.uint16),
                                   k=np.int64(k), idx=np.array(idx, dtype=np.int64))
    # random bf16 at a realistic scale, odd width
    s = (torch.randn(5, 300, generator=gen) * 0.9).to(torch.bfloat16)
    k = 61
    idx = [brute_topk(r, k) for r in s.float().tolist()]
    cases["topk_bf16_rand"] = dict(scores_bits=s.view(torch.int16).numpy().view(np.uint16),
                                   k=np.int64(k), idx=np.array(idx, dtype=np.int64))
    # float32 with ties and signed zeros
    f = torch.tensor(np.random.default_rng(7).choice(
        [0.0, -0.0, 1.5, -1.5, 3.25, 1e-30, -1e-30, 7.0], size=(4, 33)), dtype=torch.float32)
    k = 9
    idx = [brute_topk(r, k) for r in f.tolist()]
    cases["topk_f32_ties"] = dict(scores=f.numpy(), k=np.int64(k), idx=np.array(idx, dtype=np.int64))
    # 2:8 with a tail group of 5 channels (I = 21)
    s = bf16_values(gen, (7, 21), [0.0, 1.0, -1.0, 2.0, 0.25, -0.5])
    idx = [brute_2of8(r) for r in s.float().tolist()]
    cases["sel28_bf16_tail"] = dict(scores_bits=s.view(torch.int16).numpy().view(np.uint16),
                                    idx=np.array(idx, dtype=np.int64))
    return cases


def ffn_case(seed: int, t: int, d: int, inter: int, k: int):
    gen = torch.Generator().manual_seed(seed)
    for _ in range(1000):
        x = torch.randn(t, d, generator=gen)
        wg = torch.randn(inter, d, generator=gen) * 0.3
        wu = torch.randn(inter, d, generator=gen) * 0.3
        wd = torch.randn(d, inter, generator=gen) * 0.3
        g = (x.double() @ wg.double().t())
        srt = torch.sort(g, dim=1, descending=True).values
        margin = (srt[:, k - 1] - srt[:, k]).min().item()
        if margin > 1e-3:
            break
    else:
        raise RuntimeError("could not draw a well-separated FFN case")
    go = torch.randn(t, d, generator=gen)
    idx = np.array([brute_topk(r, k) for r in g.tolist()], dtype=np.int64)
    xs = x.double().requires_grad_(True)
    ws = [w.double().requires_grad_(True) for w in (wg, wu, wd)]
    m = torch.zeros(t, inter, dtype=torch.float64)
    m.scatter_(1, torch.from_numpy(idx), 1.0)
    z = torch.nn.functional.silu(xs @ ws[0].t()) * (xs @ ws[1].t()) * m
    out = z @ ws[2].t()
    out.backward(go.double())
    return dict(x=x.numpy(), wg=wg.numpy(), wu=wu.numpy(), wd=wd.numpy(), go=go.numpy(),
                k=np.int64(k), idx=idx, out=out.detach().numpy(), dx=xs.grad.numpy(),
                dwg=ws[0].grad.numpy(), dwu=ws[1].grad.numpy(), dwd=ws[2].grad.numpy())


def main():
    for name, arrays in topk_cases().items():
        np.savez(OUT / f"{name}.npz", **arrays)
    np.savez(OUT / "ffn_small_f64.npz", **ffn_case(seed=11, t=12, d=16, inter=40, k=9))
    np.savez(OUT / "ffn_odd_f64.npz", **ffn_case(seed=12, t=7, d=24, inter=37, k=8))
    print("wrote", sorted(p.name for p in OUT.glob("*.npz")))


if __name__ == "__main__":
    main()
