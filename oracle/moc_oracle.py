"""CPU oracle for the MoC sparse SwiGLU FFN hot path.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import this module, and only as the checker
(or the timed CPU baseline).  The product path (moc_amd/) never imports it.

It restates the reference's algorithm on the CPU: selection and bf16
bit-level work in numpy, FFN arithmetic in torch-CPU float32/float64.  Every
function cites the reference lines (xiaohuangji/MoC) it follows.

Selection rule (the reference leaves ties to torch.topk, which guarantees
nothing; its CUB decode kernel is a stable descending sort, i.e. lower index
first, optimized_global_moc_ext.cu:39-83, and its 2:8 Triton kernel takes the
lowest index among maxima, triton_fused_ffn_kernels.py:103-114): values
descending, ties to the lower channel index, -0.0 == +0.0, NaN above +inf.
Top-K indices are returned in ascending channel order.

Parity pins: every function here is checked in tests/test_oracle.py against
brute force on small inputs, torch library routines (bf16 casts, autograd of
the dense masked formula in float64, torch.topk up to ties) and closed forms,
and against the fixtures under tests/golden/.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

# --------------------------------------------------------------------- bf16
def bf16_bits(x) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even, NaN -> 0x7FC0.

    Same rounding as float_to_bf16_bits (optimized_global_moc_ext.cu:19-24)
    plus the canonical NaN torch produces."""
    u = np.ascontiguousarray(np.asarray(x, dtype=np.float32)).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, 0x7FC0, r)
    return r.astype(np.uint16)


def bf16_to_f32(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x) -> np.ndarray:
    return bf16_to_f32(bf16_bits(x))


def torch_bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def torch_from_bf16_bits(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


# --------------------------------------------------------------- order keys
def _keys_from_bits(bits: np.ndarray, nbits: int) -> np.ndarray:
    """Order keys of raw IEEE bit patterns of width nbits (16: bf16, 32: f32)."""
    sign = np.uint32(1 << (nbits - 1))
    full = np.uint32((1 << nbits) - 1)
    expmask = np.uint32(((1 << (nbits - 1)) - 1))
    inf = np.uint32(0x7F80 if nbits == 16 else 0x7F800000)
    bits = np.where(bits == sign, np.uint32(0), bits)
    keys = np.where(bits & sign, (~bits) & full, bits | sign).astype(np.uint32)
    keys = np.where((bits & expmask) > inf, full, keys)
    return keys.astype(np.uint32)


# the key of every bf16 bit pattern: a bf16 tensor's keys are one table lookup
_BF16_KEYS = _keys_from_bits(np.arange(1 << 16, dtype=np.uint32), 16)


def order_keys(scores) -> np.ndarray:
    """Unsigned keys whose order is the numeric order of the scores.

    bf16 tensors give 16-bit keys, float32 tensors 32-bit keys, following the
    sign-flip encoding of bf16_order_key (optimized_global_moc_ext.cu:26-29)
    with -0 folded onto +0 and NaN mapped to the largest key."""
    if isinstance(scores, torch.Tensor):
        if scores.dtype == torch.bfloat16:
            return _BF16_KEYS[torch_bf16_bits(scores)]
        if scores.dtype == torch.float32:
            bits = scores.detach().cpu().contiguous().numpy().view(np.uint32).astype(np.uint32)
            return _keys_from_bits(bits, 32)
        raise ValueError(f"unsupported dtype {scores.dtype}")
    arr = np.asarray(scores)
    if arr.dtype == np.uint16:
        return _BF16_KEYS[arr]
    if arr.dtype == np.float32:
        return _keys_from_bits(arr.view(np.uint32).astype(np.uint32), 32)
    raise ValueError(f"unsupported array dtype {arr.dtype}")


def silu_abs_scores(g: torch.Tensor) -> torch.Tensor:
    """|SiLU(g)| in g's dtype (moc/ffn.py:335)."""
    gf = g.float()
    return (gf / (1.0 + torch.exp(-gf))).abs().to(g.dtype)


# ---------------------------------------------------------------- selection
def topk_indices(scores: torch.Tensor, k: int) -> np.ndarray:
    """Row-wise Top-K channel indices [rows, k], ascending channel order.

    Follows torch.topk(g, k, dim=-1, largest=True, sorted=False)
    (moc/ffn.py:144,392; inference_ffn.py:147-153) with the stable-descending
    tie rule of the CUB kernel (optimized_global_moc_ext.cu:59-82): the first
    k of a stable sort by descending key.  That set is every key above the
    row's k-th largest key plus, of the keys equal to it, the ones of lowest
    channel index; it is formed that way here (a partition finds the k-th
    key), in blocks of rows, so that rows of a full training batch take
    seconds instead of a full sort each."""
    keys = order_keys(scores.reshape(-1, scores.shape[-1]))
    rows, inter = keys.shape
    if not 1 <= k <= inter:
        raise ValueError(f"k={k} must be in [1, {inter}]")
    out = np.empty((rows, k), dtype=np.int64)
    for r0 in range(0, rows, 1024):
        kb = keys[r0:r0 + 1024]
        kth = np.partition(kb, inter - k, axis=1)[:, inter - k][:, None]
        above = kb > kth
        tied = kb == kth
        need = (k - above.sum(axis=1, dtype=np.int64))[:, None]
        take = above | (tied & (np.cumsum(tied, axis=1, dtype=np.int32) <= need))
        out[r0:r0 + 1024] = np.nonzero(take)[1].reshape(-1, k)
    return out


def topk_mask(idx: np.ndarray, inter: int) -> np.ndarray:
    rows = idx.shape[0]
    m = np.zeros((rows, inter), dtype=bool)
    np.put_along_axis(m, idx, True, axis=1)
    return m


def moc28_effective_k(inter: int) -> int:
    """K' = 2*floor(I/8) + min(2, I mod 8) (moc/ffn.py:62-65)."""
    full, tail = divmod(int(inter), 8)
    return full * 2 + min(2, tail)


def select_2of8_indices(scores: torch.Tensor) -> np.ndarray:
    """[rows, K'] indices, (top-1, top-2) per aligned 8-group; a trailing group
    of t < 8 channels gives top-min(2, t) (moc/ffn.py:68-108).  Ties: lowest
    index among maxima (triton_fused_ffn_kernels.py:103-114)."""
    keys = order_keys(scores.reshape(-1, scores.shape[-1])).astype(np.int64)
    rows, inter = keys.shape
    out = np.zeros((rows, moc28_effective_k(inter)), dtype=np.int64)
    col = 0
    for c0 in range(0, inter, 8):
        grp = keys[:, c0:c0 + 8]
        take = min(2, grp.shape[1])
        order = np.argsort(-grp, axis=1, kind="stable")[:, :take]
        out[:, col:col + take] = order + c0
        col += take
    return out


def gather_rows(t: torch.Tensor, idx: np.ndarray) -> torch.Tensor:
    t2 = t.reshape(-1, t.shape[-1])
    return torch.gather(t2, 1, torch.from_numpy(idx).to(torch.int64))


# ------------------------------------------------------------- sparse aux ops
def sparse_forward_aux(vals: torch.Tensor, idx: np.ndarray, u_full: torch.Tensor, inter: int):
    """u_s, s_s, z_s, z_full as _forward_sparse_aux_kernel
    (moc/training/triton_sparse_aux.py:17-49): s = g*sigmoid(g); bf16 rounds
    s, then z = s_bf16 * u."""
    dt = vals.dtype
    g = vals.reshape(-1, vals.shape[-1]).float()
    u_s = gather_rows(u_full, idx)
    s = g * torch.sigmoid(g)
    s_s = s.to(dt)
    z_s = (s_s.float() * u_s.float()).to(dt)
    rows = g.shape[0]
    z_full = torch.zeros(rows, inter, dtype=dt)
    z_full.scatter_(1, torch.from_numpy(idx), z_s)
    return u_s.to(dt), s_s, z_s, z_full


def gcp_recompute(g_s: torch.Tensor, u_s: torch.Tensor):
    """s = F.silu(g), z = s*u, each materialised in the tensor dtype
    (moc/ffn.py:435-436)."""
    dt = g_s.dtype
    gf = g_s.float()
    s = (gf / (1.0 + torch.exp(-gf))).to(dt)
    z = (s.float() * u_s.float()).to(dt)
    return s, z


def sparse_backward_aux(idx: np.ndarray, g_s, u_s, s_s, gz_full, inter: int):
    """Dense grad_g, grad_u (moc/training/triton_sparse_aux.py:363-423).
    bf16: every elementwise op materialises a bf16 tensor (:376-400);
    float32: the fused kernel (:139-182)."""
    dt = g_s.dtype
    rows = g_s.reshape(-1, g_s.shape[-1]).shape[0]
    g = g_s.reshape(rows, -1).float()
    u = u_s.reshape(rows, -1).float()
    s = s_s.reshape(rows, -1).float()
    gz = gather_rows(gz_full.reshape(rows, -1), idx).float()
    if dt == torch.bfloat16:
        r = lambda t: t.to(torch.bfloat16).float()  # noqa: E731
        gs = r(u * gz)
        gu = r(s * gz)
        sig = r(torch.sigmoid(g))
        t1 = r(1.0 - sig)
        t2 = r(g * t1)
        t3 = r(1.0 + t2)
        d = r(sig * t3)
        gg = r(gs * d)
    else:
        sig = torch.sigmoid(g)
        d = sig * (1.0 + g * (1.0 - sig))
        gg = u * gz * d
        gu = s * gz
    ti = torch.from_numpy(idx)
    grad_g = torch.zeros(rows, inter, dtype=dt).scatter_(1, ti, gg.to(dt))
    grad_u = torch.zeros(rows, inter, dtype=dt).scatter_(1, ti, gu.to(dt))
    return grad_g, grad_u


# ----------------------------------------------------------------- the FFN
def mm(a: torch.Tensor, b: torch.Tensor, out_dtype) -> torch.Tensor:
    """GEMM with f32 accumulation (f64 for f64 inputs), result in out_dtype."""
    acc = torch.float64 if a.dtype == torch.float64 else torch.float32
    return (a.to(acc) @ b.to(acc)).to(out_dtype)


def select(g: torch.Tensor, k: int, mode: str) -> np.ndarray:
    if mode in ("moc", "moc_gcp"):
        return topk_indices(g, k)
    if mode == "moc_2_8":
        return select_2of8_indices(g)
    if mode == "moc_post_silu_abs":
        return topk_indices(silu_abs_scores(g), k)
    raise ValueError(f"unknown mode {mode}")


def ffn_forward(x, gate_w, up_w, down_w, k: int, mode: str = "moc_gcp", g_override=None,
                idx_override=None, u_override=None):
    """Forward of _MoCFunction / _MoCGCPFunction / _MoC28Function /
    _MoCPostSiluFunction (moc/ffn.py:130-173, 266-308, 322-367, 378-421).

    g_override lets a parity test hand in the device's own G so that the
    selection is compared on identical inputs; idx_override replaces the
    selection itself (for scores the device derives from G, such as
    |SiLU(G)|); u_override hands in the device's bf16 U, whose last-bit
    rounding depends on the GEMM's accumulation order.  Returns a dict of
    the saved/intermediate tensors plus D."""
    dt = x.dtype
    d = x.shape[-1]
    inter = gate_w.shape[0]
    x2 = x.reshape(-1, d)
    g = mm(x2, gate_w.t(), dt) if g_override is None else g_override.reshape(-1, inter).to(dt)
    idx = select(g, k, mode) if idx_override is None else np.asarray(idx_override, dtype=np.int64)
    vals = gather_rows(g, idx)
    u = mm(x2, up_w.t(), dt) if u_override is None else u_override.reshape(-1, inter).to(dt)
    u_s, s_s, z_s, z_full = sparse_forward_aux(vals, idx, u, inter)
    out = mm(z_full, down_w.t(), dt)
    return {"g": g, "idx": idx, "vals": vals, "u_s": u_s, "s_s": s_s, "z_s": z_s,
            "z_full": z_full, "out": out.reshape(*x.shape[:-1], down_w.shape[0])}


def ffn_backward(x, gate_w, up_w, down_w, fwd: dict, grad_out, gcp: bool = True,
                 gz_override=None):
    """_MoCGCPFunction.backward (moc/ffn.py:423-497) or, with gcp=False,
    _MoCFunction.backward (moc/ffn.py:175-259).  Returns (dx, dWg, dWu, dWd).

    gz_override hands in the device's bf16 grad_z_full = grad_out @ W_down
    (moc/ffn.py:450), so that a one-ulp rounding difference of that GEMM is
    not amplified by the weight-gradient reductions that follow it."""
    dt = x.dtype
    d = x.shape[-1]
    inter = gate_w.shape[0]
    x2 = x.reshape(-1, d)
    go = grad_out.reshape(-1, grad_out.shape[-1]).to(dt)
    idx = fwd["idx"]
    g_s, u_s = fwd["vals"], fwd["u_s"]
    if gcp:
        s_s, z_s = gcp_recompute(g_s, u_s)
    else:
        s_s, z_s = fwd["s_s"], fwd["z_s"]
    z_full = torch.zeros(x2.shape[0], inter, dtype=dt).scatter_(1, torch.from_numpy(idx), z_s)
    grad_down_w = mm(go.t(), z_full, down_w.dtype)
    gz = mm(go, down_w, dt) if gz_override is None else gz_override.reshape(-1, inter).to(dt)
    grad_g, grad_u = sparse_backward_aux(idx, g_s, u_s, s_s, gz, inter)
    grad_gate_w = mm(grad_g.t(), x2, gate_w.dtype)
    grad_up_w = mm(grad_u.t(), x2, up_w.dtype)
    acc = torch.float64 if dt == torch.float64 else torch.float32
    dx = (grad_g.to(acc) @ gate_w.to(acc) + grad_u.to(acc) @ up_w.to(acc)).to(dt)
    return dx.reshape(x.shape), grad_gate_w, grad_up_w, grad_down_w


def dense_masked_autograd(x, gate_w, up_w, down_w, idx: np.ndarray, grad_out, dtype=torch.float64):
    """Independent check: D = (SiLU(G) * U * M) W_down^T with the mask M held
    constant, differentiated by torch autograd in `dtype`."""
    xs = x.detach().to(dtype).requires_grad_(True)
    wg = gate_w.detach().to(dtype).requires_grad_(True)
    wu = up_w.detach().to(dtype).requires_grad_(True)
    wd = down_w.detach().to(dtype).requires_grad_(True)
    inter = gate_w.shape[0]
    x2 = xs.reshape(-1, xs.shape[-1])
    m = torch.from_numpy(topk_mask(idx, inter)).to(dtype)
    z = F.silu(x2 @ wg.t()) * (x2 @ wu.t()) * m
    out = z @ wd.t()
    out.backward(grad_out.reshape(out.shape).to(dtype))
    return out.detach(), xs.grad.detach(), wg.grad.detach(), wu.grad.detach(), wd.grad.detach()


# ---------------------------------------------------------------- inference
def masked_reference(x, gate_w, up_w, down_w, k: int, grouped: bool = False, g_override=None,
                     u_override=None):
    """InferenceMoCSwiGLUFFN.masked_reference (moc/inference/inference_ffn.py:
    169-180): G, U in bf16, z = bf16(bf16(SiLU(g)) * u), y = z_full W_down^T."""
    dt = x.dtype
    x2 = x.reshape(-1, x.shape[-1])
    g = mm(x2, gate_w.t(), dt) if g_override is None else g_override.reshape(x2.shape[0], -1).to(dt)
    u = mm(x2, up_w.t(), dt) if u_override is None else u_override.reshape(x2.shape[0], -1).to(dt)
    idx = select_2of8_indices(g) if grouped else topk_indices(g, k)
    vals = gather_rows(g, idx).float()
    s = (vals / (1.0 + torch.exp(-vals))).to(dt)
    z = (s.float() * gather_rows(u, idx).float()).to(dt)
    z_full = torch.zeros_like(g).scatter_(1, torch.from_numpy(idx), z)
    y = mm(z_full, down_w.t(), dt)
    return y, idx, z


def selected_up_silu(x, vals, idx: np.ndarray, w_up):
    """z[b,k] = bf16(bf16(SiLU(vals)) * bf16(x_b . W_up[idx]))
    (optimized_global_moc_ext.cu:127-162 with masked_reference rounding)."""
    dt = x.dtype
    u = torch.stack([w_up[torch.from_numpy(idx[b])].float() @ x[b].float() for b in range(x.shape[0])])
    u = u.to(dt).float()
    v = vals.float()
    s = (v / (1.0 + torch.exp(-v))).to(dt).float()
    return (s * u).to(dt)


def selected_down(z, idx: np.ndarray, w_down_t):
    """y[b,h] = bf16(sum_k z[b,k] W_down_t[idx[b,k], h]), f32 accumulation
    (optimized_global_moc_ext.cu:247-285)."""
    rows = [z[b].float() @ w_down_t[torch.from_numpy(idx[b])].float() for b in range(z.shape[0])]
    return torch.stack(rows).to(z.dtype)


def grouped_top2_up_silu(x, gate_w, up_w, g_override=None, u_override=None):
    """Kernel A of the 2:8 path (triton_fused_ffn_kernels.py:29-156): G, U
    rounded to bf16 before selection; sz = (g*sigmoid(g))*u in f32, stored
    in x's dtype; idx int64 (top-1, top-2) per group.  g_override/u_override
    replace the two projections (e.g. by the device's own bf16 results)."""
    dt = x.dtype
    g = mm(x, gate_w.t(), dt) if g_override is None else g_override.to(dt)
    u = mm(x, up_w.t(), dt) if u_override is None else u_override.to(dt)
    idx = select_2of8_indices(g)
    gs = gather_rows(g, idx).float()
    us = gather_rows(u, idx).float()
    sz = ((gs * torch.sigmoid(gs)) * us).to(dt)
    return idx, sz, g
