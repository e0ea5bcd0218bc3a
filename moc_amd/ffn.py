"""Mixture-of-Channels SwiGLU FFN on MI355X (module API of moc/ffn.py).

Public names, constructor arguments, attributes and state_dict keys follow
moc/ffn.py:111-121,500-609 so that models, checkpoints and harnesses written
against the reference load unchanged:

  dense     - StandardSwiGLUFFN, the dense baseline (stock torch modules).
  moc       - MoC, selected activations saved for backward.
  moc_gcp   - MoC with gate checkpointing: saves x, idx, G*M, U*M and
              recomputes S*M, Z*M in backward (moc/ffn.py:372-497).
  moc_2_8   - top-2 of every aligned 8-channel group (moc/ffn.py:262-310).
  moc_post_silu_abs - Top-K of |SiLU(G)| (moc/ffn.py:313-369).

Every MoC mode runs on the gfx950 kernels of libmoc_amd.so: MFMA GEMMs for
the nine projections, the LDS radix-select Top-K, and the sparse aux
kernels.  The `*_triton_aux` mode names are accepted for compatibility and
behave like their plain counterparts (with the reference's requirement of
int16 saved indices).  There is no CPU path: MoC modes raise on non-device
tensors.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _native as N
from . import kernels as K

_MODES = (
    "moc",
    "moc_gcp",
    "moc_triton_aux",
    "moc_gcp_triton_aux",
    "moc_2_8",
    "moc_2_8_triton_aux",
    "moc_post_silu_abs",
    "moc_post_silu_abs_triton_aux",
)


# index_save_dtype that saves the selection as a bit mask (ceil(I / 32)
# int32 words per token instead of K indices: the compact saved-mask format,
# an extension of moc/ffn.py:147,395,417); the backward expands it back to
# indices (moc_mask_to_idx).  Top-K selections only.
INDEX_SAVE_BITMASK = "bitmask"


def _pack_topk_idx_dtype(dtype, inter: int):
    """Index dtype check of _pack_topk_idx (moc/ffn.py:27-41) with the static
    bound max_allowed_idx = inter - 1 the reference always passes."""
    if dtype is None:
        return torch.int64
    if isinstance(dtype, str) and dtype == INDEX_SAVE_BITMASK:
        return torch.int16 if inter - 1 <= torch.iinfo(torch.int16).max else torch.int32
    info = torch.iinfo(dtype)
    if inter - 1 > info.max:
        raise ValueError(f"topk_idx range [0, {inter - 1}] cannot be stored as {dtype}")
    return dtype


def _moc_2_8_effective_k(intermediate_size: int) -> int:
    """Structure-determined K' for MoC 2:8 selection (moc/ffn.py:62-65)."""
    full_groups, tail = divmod(intermediate_size, 8)
    return full_groups * 2 + min(2, tail)


class StandardSwiGLUFFN(nn.Module):
    """Standard LLaMA-style SwiGLU FFN (moc/ffn.py:111-121)."""

    def __init__(self, hidden_size: int, intermediate_size: int):
        super().__init__()
        self.gate_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.up_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.down_proj = nn.Linear(intermediate_size, hidden_size, bias=False)

    def forward(self, x):
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


def _check_inputs(x, gate_w, up_w, down_w, strict_aux: bool, index_save_dtype):
    if strict_aux and not (index_save_dtype == torch.int16 or index_save_dtype == INDEX_SAVE_BITMASK):
        raise ValueError("MoC fused helper kernels require compact saved indices.")
    for t in (x, gate_w, up_w, down_w):
        if not t.is_cuda:
            raise ValueError("MoC HIP kernels require ROCm device tensors.")
    if not (x.dtype == gate_w.dtype == up_w.dtype == down_w.dtype):
        raise ValueError(
            f"MoC HIP kernels need one compute dtype, got x={x.dtype}, weights="
            f"{gate_w.dtype}/{up_w.dtype}/{down_w.dtype}")


_SIDE_STREAMS: dict = {}


def _side_stream(device) -> torch.cuda.Stream:
    """A second stream per device (default priority) for independent work: a
    256x256-tile GEMM whose tile count leaves CUs idle in its last round (or
    a short selection/elementwise kernel) overlaps another one instead."""
    key = device.index if device.index is not None else torch.cuda.current_device()
    s = _SIDE_STREAMS.get(key)
    if s is None:
        s = torch.cuda.Stream(device=device)
        _SIDE_STREAMS[key] = s
    return s


def _on_side(side, tensors, fn):
    """Run fn() on `side` after the current stream's queued work; tensors
    made on the current stream and used there are kept alive for it.  With
    side None, fn() runs on the current stream."""
    if side is None:
        fn()
        return
    side.wait_stream(torch.cuda.current_stream(side.device))
    with torch.cuda.stream(side):
        fn()
    for t in tensors:
        t.record_stream(side)


def _side_for(device, rows: int, inter: int):
    """The side stream when the [rows, inter] GEMMs take several rounds of
    256x256 tiles (their half-empty last rounds are worth filling), else None:
    for one round or less the stream handoffs cost more host time (~40 us
    per layer) than the overlap gains."""
    if K.gemm_tiles(rows, inter) > K.cu_count(device.index if device.index is not None
                                               else torch.cuda.current_device()):
        return _side_stream(device)
    return None


_SELECTION_CODE = {"topk": 0, "post_silu_abs": 1, "2of8": 2}
_LAYER_WS: dict = {}
# The one-call native layer for single-stream shapes; False runs the same
# launches one host call per kernel (the tests compare the two).
USE_NATIVE_LAYER = True


def _layer_ok(x2, *weights, dtypes=(torch.bfloat16,)) -> bool:
    """True if the one-call native layer (moc_ffn_forward_bf16 / _f32,
    moc_ffn_backward_bf16) takes these operands: one of `dtypes`, all alike,
    several rows, every row 16-byte aligned without a copy (hidden and
    intermediate sizes multiples of 16 bytes, contiguous weights)."""
    # the GEMM timing probe brackets every GEMM launch from Python
    if not USE_NATIVE_LAYER or K._GEMM_PROBE is not None or x2.dtype not in dtypes:
        return False
    per16 = 16 // x2.element_size()
    if x2.shape[0] < 2 or x2.shape[1] % per16 or x2.stride(1) != 1 or x2.stride(0) % per16 or x2.data_ptr() % 16:
        return False
    for w in weights:
        if w.dtype != x2.dtype or not w.is_contiguous() or w.data_ptr() % 16 or w.shape[1] % per16:
            return False
    return True


def _layer_ws_bytes(key, query, *args) -> int:
    n = _LAYER_WS.get(key)
    if n is None:
        n = _LAYER_WS[key] = N.query(query, *args)
    return n


def _layer_forward(x, x2, gate_w, up_w, down_w, k, selection: str, idx_dtype, save_s: bool):
    """_forward_common's launches as one native call (same results)."""
    rows, d = x2.shape
    inter = gate_w.shape[0]
    dev = x2.device
    dt = x2.dtype
    f32 = dt == torch.float32
    pitch = K.row_pitch(inter, dt)
    kk = _moc_2_8_effective_k(inter) if selection == "2of8" else k
    g = torch.empty((rows, pitch), dtype=dt, device=dev)
    u = torch.empty((rows, pitch), dtype=dt, device=dev)
    vals = torch.empty((rows, kk), dtype=dt, device=dev)
    idx = torch.empty((rows, kk), dtype=idx_dtype, device=dev)
    u_s = torch.empty((rows, kk), dtype=dt, device=dev)
    s_s = torch.empty((rows, kk), dtype=dt, device=dev) if save_s else None
    z_s = torch.empty((rows, kk), dtype=dt, device=dev) if save_s else None
    d_out = down_w.shape[0]
    out = torch.empty((rows, d_out), dtype=dt, device=dev)
    query = "moc_ffn_forward_f32_workspace_size" if f32 else "moc_ffn_forward_workspace_size"
    nbytes = _layer_ws_bytes(("f", f32, dev.index, rows, d, inter), query, rows, d, inter)
    ws = K._gemm_workspace(dev, nbytes) if nbytes > 0 else None
    N.call("moc_ffn_forward_f32" if f32 else "moc_ffn_forward_bf16", rows, d, inter, kk,
             _SELECTION_CODE[selection], x2.data_ptr(),
             x2.stride(0), gate_w.data_ptr(), d, up_w.data_ptr(), d, down_w.data_ptr(), inter,
             g.data_ptr(), u.data_ptr(), pitch, vals.data_ptr(), idx.data_ptr(), N.idx_code(idx_dtype),
             u_s.data_ptr(), N.ptr(s_s), N.ptr(z_s), out.data_ptr(), d_out, N.ptr(ws), nbytes,
             N.stream_of(x2))
    shp = (*x.shape[:-1], kk)
    return (out.reshape(*x.shape[:-1], d_out), idx.reshape(shp), vals.reshape(shp), u_s.reshape(shp),
            None if s_s is None else s_s.reshape(shp), None if z_s is None else z_s.reshape(shp))


def _forward_common(x, gate_w, up_w, down_w, k, selection: str, idx_dtype, save_s: bool,
                    want_mask: bool = False, residual=None):
    """Shared MoC forward: G -> select -> U -> sparse aux -> D.

    Follows _MoCFunction.forward (moc/ffn.py:130-173) and the variants at
    :266-308 (2:8), :322-367 (post-SiLU) and :378-421 (GCP).  With
    `residual` ([rows, d] bf16), returns residual + D from D's epilogue."""
    d = x.shape[-1]
    inter = gate_w.shape[0]
    x2 = K.aligned_rows(x.reshape(-1, d))
    rows = x2.shape[0]
    # bf16: G = x Wg^T and U = x Wu^T as one MFMA launch (their tile grids
    # side by side: two products that each end in a half-empty round of the
    # CUs share it); the 16-byte-row copy of W_down (when its rows need one),
    # which the backward reuses, then runs on the side stream beside the
    # selection.  f32: U on the side stream beside G and the selection.
    side = _side_for(x.device, rows, inter)
    if side is None and not want_mask and residual is None and down_w.shape[0] == d and \
            _layer_ok(x2, gate_w, up_w, down_w, dtypes=(torch.bfloat16, torch.float32)):
        # one native call for the whole single-stream forward (host-bound shapes)
        return _layer_forward(x, x2, gate_w, up_w, down_w, k, selection, idx_dtype, save_s)
    g = K.padded_empty(rows, inter, x.dtype, x.device)
    u = K.padded_empty(rows, inter, x.dtype, x.device)
    wd = (K.padded_empty(down_w.shape[0], down_w.shape[1], down_w.dtype, x.device)
          if K.needs_alignment(down_w) else down_w)
    if x.dtype == torch.bfloat16:
        K.linear_pair(x2, gate_w, up_w, out1=g, out2=u)
        if wd is not down_w:
            _on_side(side, (down_w, wd), lambda: K.aligned_rows(down_w, out=wd))
    else:
        def side_work():
            K.linear(x2, up_w, out=u)
            K.aligned_rows(down_w, out=wd)

        _on_side(side, (x2, up_w, u, down_w, wd), side_work)
        K.linear(x2, gate_w, out=g)
    mask = None
    if selection == "topk":
        vals, idx, mask = K.topk_rows(g, k, idx_dtype=idx_dtype, want_mask=want_mask)
    elif selection == "post_silu_abs":
        vals, idx, mask = K.topk_rows(g, k, idx_dtype=idx_dtype, score_transform=1, want_mask=want_mask)
    elif selection == "2of8":
        if want_mask:
            raise ValueError("the bit-mask index format is for Top-K selections, not MoC 2:8")
        vals, idx = K.select_2of8(g, idx_dtype=idx_dtype)
    else:
        raise ValueError(selection)
    del g
    if side is not None:
        torch.cuda.current_stream(x.device).wait_stream(side)
    u_s, s_s, z_s, z_full = K.sparse_forward_aux(vals, idx, u, inter, want_s=save_s, want_z=save_s)
    del u
    out = K.gemm(z_full, wd.t(), residual=residual)
    del z_full
    kk = idx.shape[-1]
    shp = (*x.shape[:-1], kk)
    res = (out.reshape(*x.shape[:-1], down_w.shape[0]), idx.reshape(shp), vals.reshape(shp),
           u_s.reshape(shp), None if s_s is None else s_s.reshape(shp),
           None if z_s is None else z_s.reshape(shp))
    if not want_mask:
        return res
    return res + (mask.reshape(*x.shape[:-1], mask.shape[-1]),)


def _saved_index(idx, mask, bitmask: bool):
    """What the forward saves for the selection: the indices, or the mask."""
    return mask if bitmask else idx


def _restore_index(ctx, saved):
    """The backward's indices: the saved ones, or the saved mask expanded."""
    if not ctx.bitmask:
        return saved
    rows_shape = saved.shape[:-1]
    idx = K.mask_to_idx(saved.reshape(-1, saved.shape[-1]), ctx.inter, ctx.k,
                        idx_dtype=_pack_topk_idx_dtype(INDEX_SAVE_BITMASK, ctx.inter))
    return idx.reshape(*rows_shape, ctx.k)


def _backward_common(grad_out, x, idx, g_s, u_s, s_s, z_s, gate_w, up_w, down_w, gcp: bool,
                     grad_dtype=None):
    """Shared MoC backward (moc/ffn.py:175-259 and the GCP form :423-497).
    x and the weights are in the compute dtype; the weight gradients come out
    in grad_dtype (the parameters' dtype, default the weights' dtype), dX in
    x's dtype.

    dWd = go^T Z, gZ = go Wd, (gG, gU) = sparse_backward_aux, dWg = gG^T x,
    dWu = gU^T x, dX = gG Wg + gU Wu (one MFMA pass over both products).

    When gZ takes several rounds of tiles, dWd (176 tiles of 256x256 at the
    1b shape: two thirds of the CUs) runs on the side stream beside gZ and
    the aux kernel.  dWg, dWu and dX run in order (overlapping them measured
    slower at the 1b shape: the concurrent GEMMs split each XCD's L2 between
    their tile groups; small ones split K instead)."""
    d = x.shape[-1]
    inter = gate_w.shape[0]
    dev = x.device
    main = torch.cuda.current_stream(dev)
    x2 = K.aligned_rows(x.reshape(-1, d))
    side = _side_for(dev, x2.shape[0], inter)
    go = K.aligned_rows(grad_out.reshape(-1, grad_out.shape[-1]).to(x.dtype))
    if side is None and _layer_ok(x2, gate_w, up_w, down_w) and _layer_ok(go) \
            and (not gcp or K.row_pitch(inter, x.dtype) <= 8192):
        # one native call for the whole single-stream backward
        return _layer_backward(x, x2, go, idx, g_s, u_s, s_s, z_s, gate_w, up_w, down_w, gcp,
                               grad_dtype or down_w.dtype)
    if gcp and x.dtype == torch.bfloat16 and K.row_pitch(inter, torch.bfloat16) <= 8192:
        # S is not kept: the aux kernel recomputes it from g_s (the same bits)
        s_s, z_full = K.gcp_recompute_scatter(g_s, u_s, idx, inter, want_s=False)
    else:
        if gcp:
            s_s, z_s = K.gcp_recompute(g_s, u_s)
        z_full = K.scatter_sparse_to_dense(z_s, idx, inter)
    grad_dtype = grad_dtype or down_w.dtype
    grad_down_w = torch.empty(go.shape[1], inter, dtype=grad_dtype, device=dev)
    _on_side(side, (go, z_full, grad_down_w), lambda: K.gemm(go.t(), z_full, out=grad_down_w,
                                                             out_dtype=grad_down_w.dtype))
    del z_full
    wd = K.aligned_rows(down_w)
    gz = K.padded_empty(go.shape[0], inter, x.dtype, dev)
    K.gemm(go, wd, out=gz)
    pitch = K.row_pitch(inter, x.dtype)
    if _stack_weight_grads(dev, inter, d, pitch, x.dtype):
        # dWg and dWu as one GEMM over the stacked [gG | gU]: twice the tiles
        # of each, so a K split half as deep and half the partial tiles
        grad_g, grad_u, ggu = K.sparse_backward_aux(idx, g_s, u_s, s_s, gz, inter, stacked=True)
        del gz
        dw = K.gemm(ggu.t(), x2, out_dtype=grad_dtype)
        grad_gate_w, grad_up_w = dw[:inter], dw[pitch:pitch + inter]
    else:
        grad_g, grad_u = K.sparse_backward_aux(idx, g_s, u_s, s_s, gz, inter)
        del gz
        grad_gate_w = K.gemm(grad_g.t(), x2, out_dtype=grad_dtype)
        grad_up_w = K.gemm(grad_u.t(), x2, out_dtype=grad_dtype)
    grad_x = K.gemm(grad_g, K.aligned_rows(gate_w), a2=grad_u, b2=K.aligned_rows(up_w))
    if side is not None:
        main.wait_stream(side)
    return grad_x.reshape(x.shape).to(x.dtype), grad_gate_w, grad_up_w, grad_down_w


def _layer_backward(x, x2, go, idx, g_s, u_s, s_s, z_s, gate_w, up_w, down_w, gcp: bool, grad_dtype):
    """_backward_common's launches as one native call (same results)."""
    rows, d = x2.shape
    inter = gate_w.shape[0]
    dev = x2.device
    bf16 = torch.bfloat16
    pitch = K.row_pitch(inter, bf16)
    idx2 = idx.reshape(rows, -1)
    kk = idx2.shape[1]
    g2, u2 = g_s.reshape(rows, kk), u_s.reshape(rows, kk)
    s2 = None if gcp else s_s.reshape(rows, kk)
    z2 = None if gcp else z_s.reshape(rows, kk)
    for t in (idx2, g2, u2, s2, z2):
        if t is not None and not t.is_contiguous():
            raise ValueError("saved selection tensors must be contiguous")
    stacked = _stack_weight_grads(dev, inter, d, pitch, bf16)
    zbuf = torch.empty((rows, pitch), dtype=bf16, device=dev)
    ggu = torch.empty((rows, 2 * pitch), dtype=bf16, device=dev)
    s_tmp = None  # GCP: the aux kernel recomputes S from g_s
    dx = torch.empty((rows, d), dtype=bf16, device=dev)
    if stacked:
        dw = torch.empty((2 * pitch, d), dtype=grad_dtype, device=dev)
        dwg, dwu = dw[:inter], dw[pitch:pitch + inter]
    else:
        dwg = torch.empty((inter, d), dtype=grad_dtype, device=dev)
        dwu = torch.empty((inter, d), dtype=grad_dtype, device=dev)
    d_out = go.shape[1]
    dwd = torch.empty((d_out, inter), dtype=grad_dtype, device=dev)
    nbytes = _layer_ws_bytes(("b", dev.index, rows, d, inter, stacked), "moc_ffn_backward_workspace_size",
                             rows, d, inter, 2 * pitch, int(stacked))
    ws = K._gemm_workspace(dev, nbytes) if nbytes > 0 else None
    gg = ggu.data_ptr()
    N.call("moc_ffn_backward_bf16", rows, d, inter, kk, go.data_ptr(), go.stride(0), x2.data_ptr(),
             x2.stride(0), idx2.data_ptr(), N.idx_code(idx2.dtype), g2.data_ptr(), u2.data_ptr(),
             N.ptr(s2), N.ptr(z2), gate_w.data_ptr(), d, up_w.data_ptr(), d, down_w.data_ptr(), inter,
             zbuf.data_ptr(), pitch, gg, gg + 2 * pitch, 2 * pitch, int(stacked), N.ptr(s_tmp),
             dx.data_ptr(), d, dwg.data_ptr(), dwu.data_ptr(), d, dwd.data_ptr(), inter,
             N.dtype_code(grad_dtype), N.ptr(ws), nbytes, N.stream_of(x2))
    return dx.reshape(x.shape).to(x.dtype), dwg, dwu, dwd


def _stack_weight_grads(dev, inter: int, d: int, pitch: int, dtype) -> bool:
    """dWg and dWu as one stacked GEMM when each alone leaves most CUs idle
    (split-K territory: the 130m and 350m shapes).  At the 1b shape (176
    tiles each) two launches with their own two-part K splits measured
    faster than one stacked launch (632-649 us against 660 us)."""
    if dtype != torch.bfloat16 or 2 * pitch > 8192:  # the backward row kernel's limit
        return False
    return 2 * K.gemm_tiles(inter, d) <= K.cu_count(dev.index) // 2


def _autocast_dtype(x):
    """The autocast dtype the reference's matmuls would run in for x
    (moc/ffn.py:50-59), or None outside torch.autocast."""
    if x.is_cuda and torch.is_autocast_enabled("cuda"):
        return torch.get_autocast_dtype("cuda")
    return None


def _in_compute_dtype(cdt, *ts):
    """ts cast to the compute dtype (temporaries; None: unchanged)."""
    if cdt is None:
        return ts
    return tuple(t if t.dtype == cdt else t.to(cdt) for t in ts)


def _moc_forward(ctx, selection, x, gate_w, up_w, down_w, k, index_save_dtype, use_triton_aux,
                 gcp: bool):
    """Forward of every MoC Function.  Under torch.autocast x and the weights
    are cast to the autocast dtype here, inside the Function: the casts are
    temporaries, and what is saved for backward is the cast x plus the
    parameters themselves (as the reference saves them, moc/ffn.py:166-169,
    417), not copies of the weights."""
    cdt = _autocast_dtype(x)
    xc, wg, wu, wd = _in_compute_dtype(cdt, x, gate_w, up_w, down_w)
    _check_inputs(xc, wg, wu, wd, use_triton_aux, index_save_dtype)
    inter = gate_w.shape[0]
    idx_dtype = _pack_topk_idx_dtype(index_save_dtype, inter)
    bitmask = index_save_dtype == INDEX_SAVE_BITMASK
    out, idx, vals, u_s, s_s, z_s, *mask = _forward_common(
        xc, wg, wu, wd, k, selection, idx_dtype, save_s=not gcp, want_mask=bitmask)
    sel = _saved_index(idx, mask[0] if mask else None, bitmask)
    if gcp:
        ctx.save_for_backward(xc, sel, vals, u_s, gate_w, up_w, down_w)
    else:
        ctx.save_for_backward(xc, sel, vals, u_s, s_s, z_s, gate_w, up_w, down_w)
    ctx.k = idx.shape[-1]
    ctx.inter = inter
    ctx.bitmask = bitmask
    ctx.compute_dtype = cdt
    ctx.x_dtype = x.dtype
    ctx.gcp = gcp
    return out


def _moc_backward(ctx, grad_out):
    if ctx.gcp:
        x, saved, g_s, u_s, gate_w, up_w, down_w = ctx.saved_tensors
        s_s = z_s = None
    else:
        x, saved, g_s, u_s, s_s, z_s, gate_w, up_w, down_w = ctx.saved_tensors
    idx = _restore_index(ctx, saved)
    wg, wu, wd = _in_compute_dtype(ctx.compute_dtype, gate_w, up_w, down_w)
    dx, dwg, dwu, dwd = _backward_common(grad_out, x, idx, g_s, u_s, s_s, z_s, wg, wu, wd,
                                         gcp=ctx.gcp, grad_dtype=gate_w.dtype)
    return dx.to(ctx.x_dtype), dwg, dwu, dwd, None, None, None


class _MoCFunction(torch.autograd.Function):
    """MoC autograd path that keeps selected activations for backward
    (moc/ffn.py:124-259)."""

    @staticmethod
    def forward(ctx, x, gate_w, up_w, down_w, k, index_save_dtype=None, use_triton_aux=False):
        return _moc_forward(ctx, "topk", x, gate_w, up_w, down_w, k, index_save_dtype,
                            use_triton_aux, gcp=False)

    backward = staticmethod(_moc_backward)


class _MoC28Function(torch.autograd.Function):
    """MoC with structured 2:8 selection; reuses the MoC backward
    (moc/ffn.py:262-310)."""

    @staticmethod
    def forward(ctx, x, gate_w, up_w, down_w, k, index_save_dtype=None, use_triton_aux=False):
        return _moc_forward(ctx, "2of8", x, gate_w, up_w, down_w, k, index_save_dtype,
                            use_triton_aux, gcp=False)

    backward = staticmethod(_moc_backward)


class _MoCPostSiluFunction(torch.autograd.Function):
    """MoC with Top-K on |SiLU(G)|; the pre-SiLU gates at those channels feed
    the shared sparse machinery (moc/ffn.py:313-369)."""

    @staticmethod
    def forward(ctx, x, gate_w, up_w, down_w, k, index_save_dtype=None, use_triton_aux=False):
        return _moc_forward(ctx, "post_silu_abs", x, gate_w, up_w, down_w, k, index_save_dtype,
                            use_triton_aux, gcp=False)

    backward = staticmethod(_moc_backward)


class _MoCGCPFunction(torch.autograd.Function):
    """MoC with selected-activation checkpointing (moc/ffn.py:372-497): saves
    x, idx, G*M, U*M; S*M and Z*M are recomputed in backward."""

    @staticmethod
    def forward(ctx, x, gate_w, up_w, down_w, k, index_save_dtype=None, use_triton_aux=False):
        return _moc_forward(ctx, "topk", x, gate_w, up_w, down_w, k, index_save_dtype,
                            use_triton_aux, gcp=True)

    backward = staticmethod(_moc_backward)


class MoCSwiGLUFFN(nn.Module):
    """MoC SwiGLU FFN with selectable backward strategy (moc/ffn.py:500-581).

    mode='moc'     : save sparse selected activations.
    mode='moc_gcp' : recompute selected activations in backward.
    """

    def __init__(self, hidden_size: int, intermediate_size: int, k: int | None = None,
                 mode: str = "moc", index_save_dtype=None):
        super().__init__()
        if mode not in _MODES:
            raise ValueError(
                f"Unknown mode '{mode}'. Use 'moc', 'moc_gcp', "
                "'moc_triton_aux', 'moc_gcp_triton_aux', "
                "'moc_2_8', 'moc_2_8_triton_aux', "
                "'moc_post_silu_abs', or 'moc_post_silu_abs_triton_aux'."
            )
        self.mode = mode
        self.requested_k = k
        if mode.startswith("moc_2_8"):
            self.k_effective = _moc_2_8_effective_k(intermediate_size)
        else:
            if k is None:
                raise ValueError("MoC FFN requires `k` outside moc_2_8 modes.")
            self.k_effective = k
        self.k = self.k_effective
        self.index_save_dtype = index_save_dtype
        self.gate_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.up_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.down_proj = nn.Linear(intermediate_size, hidden_size, bias=False)

    def forward(self, x):
        wg, wu, wd = self.gate_proj.weight, self.up_proj.weight, self.down_proj.weight
        aux = self.mode.endswith("_triton_aux")
        if self.mode in ("moc_gcp", "moc_gcp_triton_aux"):
            fn = _MoCGCPFunction
        elif self.mode in ("moc_2_8", "moc_2_8_triton_aux"):
            fn = _MoC28Function
        elif self.mode in ("moc_post_silu_abs", "moc_post_silu_abs_triton_aux"):
            fn = _MoCPostSiluFunction
        else:
            fn = _MoCFunction
        return fn.apply(x, wg, wu, wd, self.k, self.index_save_dtype, aux)


# ------------------------------------------------------------ decoder block
# The FFN half of a pre-norm block, h + FFN(RMSNorm(h)) (TransformerBlock.
# forward, moc/model.py:83-86; RMSNorm :20-28), with the norm as one row
# kernel in front of the FFN and the residual add in the Down GEMM's
# epilogue; the backward runs the FFN backward on the recomputed norm output
# and then the norm's backward with the residual gradient added.  The
# library's own fusion of the FFN's neighbours (no reference counterpart:
# the reference runs stock PyTorch ops around its FFN).
FUSE_BLOCK_FFN = True

_SELECTION_OF_MODE = {"moc": ("topk", False), "moc_triton_aux": ("topk", False),
                      "moc_gcp": ("topk", True), "moc_gcp_triton_aux": ("topk", True),
                      "moc_2_8": ("2of8", False), "moc_2_8_triton_aux": ("2of8", False),
                      "moc_post_silu_abs": ("post_silu_abs", False),
                      "moc_post_silu_abs_triton_aux": ("post_silu_abs", False)}


def block_ffn_ok(h, norm_weight, ffn) -> bool:
    """True if block_ffn takes this block: a MoC FFN, bf16 activations,
    norm weight and FFN weights on the device, no autocast, hidden a
    multiple of 8 up to 4096."""
    if not FUSE_BLOCK_FFN or not isinstance(ffn, MoCSwiGLUFFN) or ffn.mode not in _SELECTION_OF_MODE:
        return False
    if not h.is_cuda or h.dtype != torch.bfloat16 or norm_weight.dtype != torch.bfloat16:
        return False
    if _autocast_dtype(h) is not None:
        return False
    d = h.shape[-1]
    if d % 8 or d > 4096:
        return False
    return all(w.dtype == torch.bfloat16 and w.is_cuda for w in
               (ffn.gate_proj.weight, ffn.up_proj.weight, ffn.down_proj.weight))


def block_ffn(h, norm_weight, eps: float, ffn) -> torch.Tensor:
    """h + ffn(RMSNorm(h)) with the norm (weight norm_weight, eps) and the
    residual fused around the MoC FFN `ffn` (block_ffn_ok must hold)."""
    selection, gcp = _SELECTION_OF_MODE[ffn.mode]
    return _MoCBlockFunction.apply(h, norm_weight, ffn.gate_proj.weight, ffn.up_proj.weight,
                                   ffn.down_proj.weight, float(eps), ffn.k, ffn.index_save_dtype,
                                   ffn.mode.endswith("_triton_aux"), selection, gcp)


def _block_native(h2, wg, wu, wd) -> bool:
    """The one-call block entry points take this shape (single-stream)."""
    return _side_for(h2.device, h2.shape[0], wg.shape[0]) is None and h2.shape[1] == wd.shape[0] and \
        _layer_ok(h2, wg, wu, wd)


class _MoCBlockFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, h, norm_w, gate_w, up_w, down_w, eps, k, index_save_dtype, use_triton_aux, selection,
                gcp):
        _check_inputs(h, gate_w, up_w, down_w, use_triton_aux, index_save_dtype)
        d = h.shape[-1]
        inter = gate_w.shape[0]
        h2 = K.aligned_rows(h.reshape(-1, d))
        rows = h2.shape[0]
        idx_dtype = _pack_topk_idx_dtype(index_save_dtype, inter)
        bitmask = index_save_dtype == INDEX_SAVE_BITMASK
        mask = None
        if not bitmask and _block_native(h2, gate_w, up_w, down_w):
            out, idx, vals, u_s, s_s, z_s, rstd = _block_forward_native(
                h2, norm_w, eps, gate_w, up_w, down_w, k, selection, idx_dtype, save_s=not gcp)
        else:
            xn, rstd = K.rmsnorm_rows(h2, norm_w, eps)
            out, idx, vals, u_s, s_s, z_s, *mk = _forward_common(
                xn, gate_w, up_w, down_w, k, selection, idx_dtype, save_s=not gcp, want_mask=bitmask,
                residual=h2)
            mask = mk[0] if mk else None
            del xn
        sel = _saved_index(idx, mask, bitmask)
        if gcp:
            ctx.save_for_backward(h2, rstd, norm_w, sel, vals, u_s, gate_w, up_w, down_w)
        else:
            ctx.save_for_backward(h2, rstd, norm_w, sel, vals, u_s, s_s, z_s, gate_w, up_w, down_w)
        ctx.k = idx.shape[-1]
        ctx.inter = inter
        ctx.bitmask = bitmask
        ctx.gcp = gcp
        ctx.eps = eps
        ctx.h_shape = h.shape
        return out.reshape(h.shape)

    @staticmethod
    def backward(ctx, dout):
        if ctx.gcp:
            h2, rstd, norm_w, saved, g_s, u_s, wg, wu, wd = ctx.saved_tensors
            s_s = z_s = None
        else:
            h2, rstd, norm_w, saved, g_s, u_s, s_s, z_s, wg, wu, wd = ctx.saved_tensors
        idx = _restore_index(ctx, saved)
        d = h2.shape[1]
        go = K.aligned_rows(dout.reshape(-1, d).to(h2.dtype))
        if _block_native(h2, wg, wu, wd) and _layer_ok(go) and \
                (not ctx.gcp or K.row_pitch(ctx.inter, h2.dtype) <= 8192):
            dh, dnw, dwg, dwu, dwd = _block_backward_native(ctx, go, h2, rstd, norm_w, idx, g_s, u_s, s_s,
                                                            z_s, wg, wu, wd)
        else:
            xn, _ = K.rmsnorm_rows(h2, norm_w, ctx.eps, want_rstd=False)
            dxn, dwg, dwu, dwd = _backward_common(go, xn, idx, g_s, u_s, s_s, z_s, wg, wu, wd, gcp=ctx.gcp)
            del xn
            dh, dnw = K.rmsnorm_backward(h2, norm_w, rstd, dxn.reshape(-1, d), dres=go)
        return (dh.reshape(ctx.h_shape), dnw, dwg, dwu, dwd, None, None, None, None, None, None)


def _block_forward_native(h2, norm_w, eps, gate_w, up_w, down_w, k, selection, idx_dtype, save_s):
    """moc_ffn_block_forward_bf16: the norm, the FFN and the residual add in
    one call (the launches of the unfused path in the same order)."""
    rows, d = h2.shape
    inter = gate_w.shape[0]
    dev = h2.device
    dt = h2.dtype
    pitch = K.row_pitch(inter, dt)
    kk = _moc_2_8_effective_k(inter) if selection == "2of8" else k
    xn = torch.empty((rows, d), dtype=dt, device=dev)
    rstd = torch.empty(rows, dtype=torch.float32, device=dev)
    g = torch.empty((rows, pitch), dtype=dt, device=dev)
    u = torch.empty((rows, pitch), dtype=dt, device=dev)
    vals = torch.empty((rows, kk), dtype=dt, device=dev)
    idx = torch.empty((rows, kk), dtype=idx_dtype, device=dev)
    u_s = torch.empty((rows, kk), dtype=dt, device=dev)
    s_s = torch.empty((rows, kk), dtype=dt, device=dev) if save_s else None
    z_s = torch.empty((rows, kk), dtype=dt, device=dev) if save_s else None
    out = torch.empty((rows, d), dtype=dt, device=dev)
    nbytes = _layer_ws_bytes(("f", False, dev.index, rows, d, inter), "moc_ffn_forward_workspace_size",
                             rows, d, inter)
    ws = K._gemm_workspace(dev, nbytes) if nbytes > 0 else None
    N.call("moc_ffn_block_forward_bf16", rows, d, inter, kk, _SELECTION_CODE[selection], h2.data_ptr(),
           h2.stride(0), norm_w.contiguous().data_ptr(), float(eps), xn.data_ptr(), d, rstd.data_ptr(),
           gate_w.data_ptr(), d, up_w.data_ptr(), d, down_w.data_ptr(), inter, g.data_ptr(), u.data_ptr(),
           pitch, vals.data_ptr(), idx.data_ptr(), N.idx_code(idx_dtype), u_s.data_ptr(), N.ptr(s_s),
           N.ptr(z_s), out.data_ptr(), d, N.ptr(ws), nbytes, N.stream_of(h2))
    return out, idx, vals, u_s, s_s, z_s, rstd


def _block_backward_native(ctx, go, h2, rstd, norm_w, idx, g_s, u_s, s_s, z_s, gate_w, up_w, down_w):
    """moc_ffn_block_backward_bf16: norm recompute, FFN backward and the
    norm's backward with the residual gradient in one call."""
    rows, d = h2.shape
    inter = gate_w.shape[0]
    dev = h2.device
    bf16 = torch.bfloat16
    pitch = K.row_pitch(inter, bf16)
    idx2 = idx.reshape(rows, -1)
    kk = idx2.shape[1]
    g2, u2 = g_s.reshape(rows, kk), u_s.reshape(rows, kk)
    s2 = None if ctx.gcp else s_s.reshape(rows, kk)
    z2 = None if ctx.gcp else z_s.reshape(rows, kk)
    for t in (idx2, g2, u2, s2, z2):
        if t is not None and not t.is_contiguous():
            raise ValueError("saved selection tensors must be contiguous")
    grad_dtype = down_w.dtype
    stacked = _stack_weight_grads(dev, inter, d, pitch, bf16)
    xn = torch.empty((rows, d), dtype=bf16, device=dev)
    zbuf = torch.empty((rows, pitch), dtype=bf16, device=dev)
    ggu = torch.empty((rows, 2 * pitch), dtype=bf16, device=dev)
    s_tmp = None  # GCP: the aux kernel recomputes S from g_s
    dh = torch.empty((rows, d), dtype=bf16, device=dev)
    if stacked:
        dw = torch.empty((2 * pitch, d), dtype=grad_dtype, device=dev)
        dwg, dwu = dw[:inter], dw[pitch:pitch + inter]
    else:
        dwg = torch.empty((inter, d), dtype=grad_dtype, device=dev)
        dwu = torch.empty((inter, d), dtype=grad_dtype, device=dev)
    dwd = torch.empty((d, inter), dtype=grad_dtype, device=dev)
    dnw = torch.empty(d, dtype=norm_w.dtype, device=dev)
    nbytes = _layer_ws_bytes(("bb", dev.index, rows, d, inter, stacked), "moc_ffn_block_backward_workspace_size",
                             rows, d, inter, 2 * pitch, int(stacked))
    ws = K._gemm_workspace(dev, nbytes)
    gg = ggu.data_ptr()
    N.call("moc_ffn_block_backward_bf16", rows, d, inter, kk, go.data_ptr(), go.stride(0), h2.data_ptr(),
           h2.stride(0), norm_w.contiguous().data_ptr(), float(ctx.eps), rstd.data_ptr(), xn.data_ptr(), d,
           idx2.data_ptr(), N.idx_code(idx2.dtype), g2.data_ptr(), u2.data_ptr(), N.ptr(s2), N.ptr(z2),
           gate_w.data_ptr(), d, up_w.data_ptr(), d, down_w.data_ptr(), inter, zbuf.data_ptr(), pitch, gg,
           gg + 2 * pitch, 2 * pitch, int(stacked), N.ptr(s_tmp), dh.data_ptr(), d, dwg.data_ptr(),
           dwu.data_ptr(), d, dwd.data_ptr(), inter, N.dtype_code(grad_dtype), dnw.data_ptr(),
           N.dtype_code(norm_w.dtype), ws.data_ptr(), nbytes, N.stream_of(h2))
    return dh, dnw, dwg, dwu, dwd


def build_ffn(hidden_size: int, intermediate_size: int, ffn_type: str = "dense", k=None):
    """Factory for Dense FFN, MoC, MoC+GCP, MoC 2:8 and post-SiLU variants
    (moc/ffn.py:584-609)."""
    if ffn_type == "dense":
        return StandardSwiGLUFFN(hidden_size, intermediate_size)
    if ffn_type in ("moc", "moc_gcp", "moc_2_8", "moc_post_silu_abs"):
        if k is None and ffn_type != "moc_2_8":
            raise ValueError("MoC FFN requires `k`")
        mode = {
            "moc": "moc_triton_aux",
            "moc_gcp": "moc_gcp_triton_aux",
            "moc_2_8": "moc_2_8_triton_aux",
            "moc_post_silu_abs": "moc_post_silu_abs_triton_aux",
        }[ffn_type]
        return MoCSwiGLUFFN(hidden_size, intermediate_size, k, mode=mode,
                            index_save_dtype=torch.int16)
    raise ValueError(f"Unknown ffn_type '{ffn_type}'")
