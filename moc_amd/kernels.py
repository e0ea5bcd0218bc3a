"""Python entry points over the gfx950 kernels of libmoc_amd.so.

Each function validates shapes, strides and dtypes, allocates its outputs
with torch (device memory only), and launches on torch's current stream.
There is no CPU or eager fallback: non-device tensors raise ValueError and a
missing library raises NativeLibraryMissing.

Internal [rows, intermediate] activations are allocated with a leading
dimension padded to a multiple of 8 elements so that every MFMA operand row
is 16-byte aligned; functions return the logical [:, :intermediate] view.
"""
from __future__ import annotations

import torch

from . import _native as N


def round_up(x: int, m: int) -> int:
    return (x + m - 1) // m * m


def _empty(shape, dtype, device):
    return torch.empty(shape, dtype=dtype, device=device)


def _rows_view(t: torch.Tensor) -> tuple[torch.Tensor, int]:
    """2-D [rows, cols] view with unit column stride; returns (view, ld)."""
    if t.dim() != 2:
        raise ValueError(f"expected a 2-D tensor, got shape {tuple(t.shape)}")
    if t.stride(1) != 1 and t.shape[1] > 1:
        t = t.contiguous()
    ld = t.stride(0) if t.shape[0] > 1 else max(t.shape[1], 1)
    return t, ld


def row_pitch(cols: int, dtype) -> int:
    """Row pitch (elements) of a padded [rows, cols] allocation: a multiple of
    8 elements (16 bytes, the MFMA load unit), and of 128 bytes once a row
    spans 1 KB, so that the GEMM's 128-byte row segments are whole L2 lines
    (one request each instead of two)."""
    esz = dtype.itemsize
    cols = max(cols, 1)
    if cols * esz >= 1024:
        return round_up(cols * esz, 128) // esz
    return round_up(cols, 8)


def padded_empty(rows: int, cols: int, dtype, device) -> torch.Tensor:
    """[rows, cols] view of a [rows, row_pitch(cols)] allocation."""
    return _empty((rows, row_pitch(cols, dtype)), dtype, device).narrow(1, 0, cols)


_CUS: dict = {}


def cu_count(device_index: int) -> int:
    """Compute units of a device (cached)."""
    n = _CUS.get(device_index)
    if n is None:
        n = _CUS[device_index] = torch.cuda.get_device_properties(device_index).multi_processor_count
    return n


def gemm_tiles(m: int, n: int) -> int:
    """Workgroups (256x256 output tiles) of a bf16 GEMM with an [m, n] output."""
    return ((m + 255) // 256) * ((n + 255) // 256)


def needs_alignment(t: torch.Tensor) -> bool:
    """True if aligned_rows(t) would copy: a bf16 matrix whose rows are not
    16-byte aligned."""
    t, ld = _rows_view(t)
    return t.dtype == torch.bfloat16 and not (ld % 8 == 0 and t.data_ptr() % 16 == 0)


def aligned_rows(t: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Row-major copy (if needed) whose rows are 16-byte aligned for MFMA loads.
    `out`, if given, is the destination of the copy (a padded_empty of t's
    shape); it is ignored when t needs no copy."""
    t, ld = _rows_view(t)
    if not needs_alignment(t):
        return t
    if out is None:
        out = padded_empty(t.shape[0], t.shape[1], t.dtype, t.device)
    elif out.shape != t.shape or out.dtype != t.dtype or out.stride(1) != 1 or out.stride(0) % 8:
        raise ValueError("aligned_rows: out must be a padded [rows, cols] bf16 view")
    N.call("moc_copy_pad_2d", N.MOC_BF16, t.data_ptr(), t.shape[0], t.shape[1], ld,
           out.data_ptr(), out.stride(0), out.stride(0), N.stream_of(t))
    return out


# ----------------------------------------------------------------- selection
def topk_rows(scores: torch.Tensor, k: int, *, idx_dtype=torch.int64, want_vals: bool = True,
              want_mask: bool = False, score_transform: int = 0):
    """Row-wise Top-K of a [rows, I] tensor -> (vals | None, idx, mask | None).

    idx is in ascending channel order; ties go to the lower channel index.
    """
    N.require_device(scores)
    s, ld = _rows_view(scores)
    rows, inter = s.shape
    dev = s.device
    idx = _empty((rows, k), idx_dtype, dev)
    vals = _empty((rows, k), s.dtype, dev) if want_vals else None
    words = (inter + 31) // 32
    mask = _empty((rows, words), torch.int32, dev) if want_mask else None
    N.call("moc_topk_rows", N.dtype_code(s.dtype), s.data_ptr(), rows, inter, ld, int(k),
           int(score_transform), N.ptr(vals), idx.data_ptr(), N.idx_code(idx_dtype),
           N.ptr(mask), words, N.stream_of(s))
    return vals, idx, mask


def mask_to_idx(mask: torch.Tensor, inter: int, k: int, *, idx_dtype=torch.int16) -> torch.Tensor:
    """[rows, ceil(inter/32)] int32 selection mask -> [rows, k] channel
    indices in ascending order (the first k set bits of each row)."""
    N.require_device(mask)
    m, ld = _rows_view(mask)
    if m.dtype != torch.int32:
        raise ValueError("mask must be int32 words")
    rows = m.shape[0]
    idx = _empty((rows, k), idx_dtype, m.device)
    N.call("moc_mask_to_idx", m.data_ptr(), rows, int(inter), ld, int(k), idx.data_ptr(),
           N.idx_code(idx_dtype), N.stream_of(m))
    return idx


def moc28_effective_k(inter: int) -> int:
    full, tail = divmod(int(inter), 8)
    return full * 2 + min(2, tail)


def select_2of8(scores: torch.Tensor, *, idx_dtype=torch.int64):
    """Top-2 of every aligned 8-channel group -> (vals, idx), (top-1, top-2) per group."""
    N.require_device(scores)
    s, ld = _rows_view(scores)
    rows, inter = s.shape
    kout = moc28_effective_k(inter)
    idx = _empty((rows, kout), idx_dtype, s.device)
    vals = _empty((rows, kout), s.dtype, s.device)
    N.call("moc_select_2of8", N.dtype_code(s.dtype), s.data_ptr(), rows, inter, ld,
           vals.data_ptr(), idx.data_ptr(), N.idx_code(idx_dtype), N.stream_of(s))
    return vals, idx


# ----------------------------------------------------------- training helpers
def _sparse_2d(t: torch.Tensor) -> torch.Tensor:
    return t.reshape(-1, t.shape[-1]).contiguous()


def sparse_forward_aux(topk_vals: torch.Tensor, topk_idx: torch.Tensor, u_full: torch.Tensor,
                       inter: int, *, want_s: bool = True, want_z: bool = True,
                       want_full: bool = True):
    """-> (u_sparse, s_sparse | None, z_sparse | None, z_full | None); z_full is a
    [rows, inter] view of a padded, zero-filled buffer."""
    N.require_device(topk_vals, topk_idx, u_full)
    vals = _sparse_2d(topk_vals)
    idx = _sparse_2d(topk_idx)
    rows, k = vals.shape
    u, u_ld = _rows_view(u_full.reshape(rows, -1) if u_full.dim() != 2 else u_full)
    if u.shape[1] < inter:
        raise ValueError(f"u_full has {u.shape[1]} columns, expected >= {inter}")
    dt, dev = vals.dtype, vals.device
    if u.dtype != dt:
        raise ValueError(f"dtype mismatch: topk_vals {dt}, u_full {u.dtype}")
    u_s = _empty((rows, k), dt, dev)
    s_s = _empty((rows, k), dt, dev) if want_s else None
    z_s = _empty((rows, k), dt, dev) if want_z else None
    z_full = padded_empty(rows, inter, dt, dev) if want_full else None
    N.call("moc_sparse_forward_aux", N.dtype_code(dt), vals.data_ptr(), idx.data_ptr(),
           N.idx_code(idx.dtype), u.data_ptr(), u_ld, rows, k, inter, u_s.data_ptr(),
           N.ptr(s_s), N.ptr(z_s), N.ptr(z_full),
           z_full.stride(0) if z_full is not None else inter, N.stream_of(vals))
    return u_s, s_s, z_s, z_full


def scatter_sparse_to_dense(sparse: torch.Tensor, topk_idx: torch.Tensor, inter: int) -> torch.Tensor:
    """[rows, k] -> zero-filled [rows, inter] (view of a padded buffer)."""
    N.require_device(sparse, topk_idx)
    sp = _sparse_2d(sparse)
    idx = _sparse_2d(topk_idx)
    rows, k = sp.shape
    dense = padded_empty(rows, inter, sp.dtype, sp.device)
    N.call("moc_scatter_sparse_to_dense", N.dtype_code(sp.dtype), sp.data_ptr(), idx.data_ptr(),
           N.idx_code(idx.dtype), rows, k, inter, dense.data_ptr(), dense.stride(0),
           N.stream_of(sp))
    return dense


def gather_dense_to_sparse(dense: torch.Tensor, topk_idx: torch.Tensor) -> torch.Tensor:
    N.require_device(dense, topk_idx)
    idx = _sparse_2d(topk_idx)
    rows, k = idx.shape
    d, ld = _rows_view(dense.reshape(rows, -1) if dense.dim() != 2 else dense)
    out = _empty((rows, k), d.dtype, d.device)
    N.call("moc_gather_dense_to_sparse", N.dtype_code(d.dtype), d.data_ptr(), ld, idx.data_ptr(),
           N.idx_code(idx.dtype), rows, k, out.data_ptr(), N.stream_of(d))
    return out


def gcp_recompute(g_sparse: torch.Tensor, u_sparse: torch.Tensor):
    """GCP recompute -> (s = SiLU(g), z = s * u)."""
    N.require_device(g_sparse, u_sparse)
    g = g_sparse.contiguous()
    u = u_sparse.contiguous()
    s = torch.empty_like(g)
    z = torch.empty_like(g)
    N.call("moc_gcp_recompute", N.dtype_code(g.dtype), g.data_ptr(), u.data_ptr(), g.numel(),
           s.data_ptr(), z.data_ptr(), N.stream_of(g))
    return s, z


def gcp_recompute_scatter(g_sparse: torch.Tensor, u_sparse: torch.Tensor, topk_idx: torch.Tensor,
                          inter: int, want_s: bool = True):
    """GCP recompute fused with the scatter of z -> (s_sparse | None, z_full);
    z_full is a zero-filled [rows, inter] view of a padded buffer.  bf16."""
    N.require_device(g_sparse, u_sparse, topk_idx)
    g = _sparse_2d(g_sparse)
    u = _sparse_2d(u_sparse)
    idx = _sparse_2d(topk_idx)
    rows, k = g.shape
    s = torch.empty_like(g) if want_s else None
    z_full = padded_empty(rows, inter, g.dtype, g.device)
    N.call("moc_gcp_recompute_scatter", N.dtype_code(g.dtype), g.data_ptr(), u.data_ptr(),
           idx.data_ptr(), N.idx_code(idx.dtype), rows, k, inter, N.ptr(s), z_full.data_ptr(),
           z_full.stride(0), N.stream_of(g))
    return (s.reshape(g_sparse.shape) if want_s else None), z_full


def sparse_backward_aux(topk_idx: torch.Tensor, g_sparse: torch.Tensor, u_sparse: torch.Tensor,
                        s_sparse: torch.Tensor | None, grad_z_full: torch.Tensor, inter: int,
                        stacked: bool = False):
    """-> (grad_g, grad_u) as zero-filled [rows, inter] views of padded buffers.
    stacked: both are views of one [rows, 2 pitch] buffer (grad_g in columns
    [0, inter), grad_u from column pitch), returned third, so that
    [grad_g | grad_u]^T x is one GEMM."""
    N.require_device(topk_idx, g_sparse, u_sparse, s_sparse, grad_z_full)
    idx = _sparse_2d(topk_idx)
    g = _sparse_2d(g_sparse)
    u = _sparse_2d(u_sparse)
    s = _sparse_2d(s_sparse) if s_sparse is not None else None
    rows, k = g.shape
    gz, gz_ld = _rows_view(grad_z_full.reshape(rows, -1) if grad_z_full.dim() != 2 else grad_z_full)
    if gz.dtype != g.dtype:
        raise ValueError(f"dtype mismatch: g_sparse {g.dtype}, grad_z_full {gz.dtype}")
    if stacked:
        pitch = row_pitch(inter, g.dtype)
        buf = _empty((rows, 2 * pitch), g.dtype, g.device)
        gg, gu = buf[:, :inter], buf[:, pitch:pitch + inter]
    else:
        gg = padded_empty(rows, inter, g.dtype, g.device)
        gu = padded_empty(rows, inter, g.dtype, g.device)
    N.call("moc_sparse_backward_aux", N.dtype_code(g.dtype), idx.data_ptr(), N.idx_code(idx.dtype),
           g.data_ptr(), u.data_ptr(), N.ptr(s), gz.data_ptr(), gz_ld, rows, k, inter,
           gg.data_ptr(), gu.data_ptr(), gg.stride(0), N.stream_of(g))
    return (gg, gu, buf) if stacked else (gg, gu)


# ---------------------------------------------------------------------- GEMM
def _operand(t: torch.Tensor, bf16: bool) -> tuple[torch.Tensor, int, int]:
    """Return (tensor, stride0, stride1) of a 2-D operand usable by moc_gemm.

    bf16 operands need a unit stride along one dimension, the other stride a
    multiple of 8 elements and a 16-byte aligned base; anything else is copied
    into an aligned row-major buffer.  Strides of size-1 dimensions carry no
    information and are normalised.
    """
    if t.dim() != 2:
        raise ValueError(f"GEMM operands must be 2-D, got {tuple(t.shape)}")
    r, c = t.shape
    s0, s1 = t.stride()
    if not bf16:
        return t, s0, s1
    if r == 1:
        s0 = round_up(max(c, 1), 8)
    if c == 1:
        s1 = round_up(max(r, 1), 8) if s0 == 1 else 1
    aligned = t.data_ptr() % 16 == 0
    if aligned and s1 == 1 and s0 % 8 == 0:
        return t, s0, s1
    if aligned and s0 == 1 and s1 % 8 == 0:
        return t, s0, s1
    tt = aligned_rows(t)
    return tt, (tt.stride(0) if r > 1 else round_up(max(c, 1), 8)), 1


# Per-stream workspaces (GEMM fix-up/split-K partials, decode partial sums).
# Both start with arrival counters that must be zero when a kernel starts and
# that every kernel leaves zero, so a buffer is created zeroed and reused
# without clearing; one buffer per (device, stream) keeps kernels that run
# concurrently on different streams apart.
_STREAM_WS_LIMIT = 8        # cached streams per device and cache; the oldest goes first
_GEMM_WS: dict = {}
_WS_CACHE: dict = {}
# buffers a captured HIP graph still uses: kept alive until the process ends
# (one per captured buffer that was later outgrown or evicted)
_WS_CAPTURED: list = []


def _stream_workspace(cache: dict, device, nbytes: int, minimum: int = 1) -> torch.Tensor:
    """The zeroed workspace of the current stream on `device` from `cache`,
    grown on demand.  A buffer handed out during a HIP graph capture is
    marked: when it is outgrown or evicted it is kept alive (the graph keeps
    writing to it on every replay); any other outgrown buffer is freed (the
    caching allocator orders its reuse after the work queued on its
    stream).  At most _STREAM_WS_LIMIT streams per device keep a buffer."""
    stream = torch.cuda.current_stream(device)
    key = (device.index, stream.cuda_stream)
    ent = cache.pop(key, None)  # re-inserted below: the dict's order is least-recent first
    if ent is None or ent[0].numel() < nbytes:
        if ent is not None and ent[1]:
            _WS_CAPTURED.append(ent[0])
        ent = [torch.zeros((max(nbytes, minimum),), dtype=torch.uint8, device=device), False]
    if torch.cuda.is_current_stream_capturing():
        ent[1] = True
    cache[key] = ent
    same_dev = [k for k in cache if k[0] == device.index]
    for old in same_dev[:max(0, len(same_dev) - _STREAM_WS_LIMIT)]:
        gone = cache.pop(old)
        if gone[1]:
            _WS_CAPTURED.append(gone[0])
    return ent[0]


# Optional timing probe: when a list is installed with set_gemm_probe(), every
# GEMM launch made through gemm() / linear_pair() is bracketed by two timing
# events on the stream it runs on and recorded as (events, FLOP), so a
# harness can sum the GEMM time inside a real training step.
_GEMM_PROBE: list | None = None


def set_gemm_probe(records: list | None) -> None:
    """Install (a list) or remove (None) the GEMM timing probe."""
    global _GEMM_PROBE
    _GEMM_PROBE = records


def _probe_begin():
    if _GEMM_PROBE is None:
        return None
    ev = torch.cuda.Event(enable_timing=True)
    ev.record()
    return ev


def _probe_end(ev, name: str, flop: float) -> None:
    if ev is None:
        return
    end = torch.cuda.Event(enable_timing=True)
    end.record()
    _GEMM_PROBE.append((name, ev, end, flop))


def _gemm_workspace(device, nbytes: int) -> torch.Tensor:
    """The GEMM workspace of the current stream on `device` (its first 4 KB
    hold the fix-up's arrival counters), grown on demand."""
    return _stream_workspace(_GEMM_WS, device, nbytes)


def gemm(a: torch.Tensor, b: torch.Tensor, *, a2: torch.Tensor | None = None,
         b2: torch.Tensor | None = None, out: torch.Tensor | None = None,
         out_dtype: torch.dtype | None = None, residual: torch.Tensor | None = None) -> torch.Tensor:
    """C = a @ b (+ a2 @ b2) on the MFMA engine; a: [M, K], b: [K, N].  With
    `residual` (bf16 [M, N], bf16 operands, one product): C = residual +
    a @ b, added in the GEMM's epilogue (bf16(bf16(a @ b) + residual))."""
    if residual is not None:
        return _gemm_residual(a, b, residual, out)
    N.require_device(a, b, a2, b2, out)
    if a.dtype != b.dtype or (a2 is not None and (a2.dtype != a.dtype or b2.dtype != a.dtype)):
        raise ValueError("moc gemm operands must share one dtype")
    M, K = a.shape
    K_, Nn = b.shape
    if K != K_:
        raise ValueError(f"gemm shape mismatch {tuple(a.shape)} @ {tuple(b.shape)}")
    bf16 = a.dtype == torch.bfloat16
    out_dtype = out_dtype or a.dtype
    if not bf16 and out_dtype != torch.float32:
        raise ValueError("f32 GEMM produces f32")
    if out is None:
        out = _empty((M, Nn), out_dtype, a.device)
    if out.shape != (M, Nn) or (out.stride(1) != 1 and Nn > 1):
        raise ValueError("gemm out must be [M, N] with unit column stride")
    aa, as0, as1 = _operand(a, bf16)
    bb, bs0, bs1 = _operand(b, bf16)
    K2 = 0
    a2p = b2p = None
    a2s0 = a2s1 = b2s0 = b2s1 = 0
    if a2 is not None:
        K2 = a2.shape[1]
        if a2.shape[0] != M or b2.shape != (K2, Nn):
            raise ValueError("second GEMM pair has mismatched shapes")
        a2p, a2s0, a2s1 = _operand(a2, bf16)
        b2p, b2s0, b2s1 = _operand(b2, bf16)
    ldc = out.stride(0) if M > 1 else max(Nn, 1)
    code = N.dtype_code(a.dtype)
    # products with fewer tiles than CUs split K over a workspace of f32
    # partial tiles (f32 GEMMs decide inside the library)
    ws_bytes = 0
    if not bf16 or gemm_tiles(M, Nn) < cu_count(a.get_device()):
        ws_bytes = N.query("moc_gemm_workspace_size", code, M, Nn, K, K2)
    ws = _gemm_workspace(a.device, ws_bytes) if ws_bytes > 0 else None
    probe = _probe_begin()
    N.call("moc_gemm_ws", code, M, Nn, K, aa.data_ptr(), as0, as1, bb.data_ptr(),
           bs0, bs1, K2, N.ptr(a2p), a2s0, a2s1, N.ptr(b2p), b2s0, b2s1, out.data_ptr(), ldc,
           N.dtype_code(out_dtype), N.ptr(ws), ws_bytes, N.stream_of(a))
    _probe_end(probe, f"gemm {M}x{Nn}x{K}" + (f"+{K2}" if K2 else ""), 2.0 * M * Nn * (K + K2))
    return out


def _gemm_residual(a, b, residual, out):
    N.require_device(a, b, residual, out)
    if not (a.dtype == b.dtype == residual.dtype == torch.bfloat16):
        raise ValueError("gemm with a residual takes bf16 operands and a bf16 residual")
    M, Kd = a.shape
    K_, Nn = b.shape
    if Kd != K_ or residual.shape != (M, Nn):
        raise ValueError(f"gemm shape mismatch {tuple(a.shape)} @ {tuple(b.shape)} + {tuple(residual.shape)}")
    if out is None:
        out = _empty((M, Nn), torch.bfloat16, a.device)
    if out.shape != (M, Nn) or out.dtype != torch.bfloat16 or (out.stride(1) != 1 and Nn > 1):
        raise ValueError("gemm out must be bf16 [M, N] with unit column stride")
    r = aligned_rows(residual)
    aa, as0, as1 = _operand(a, True)
    bb, bs0, bs1 = _operand(b, True)
    ws_bytes = 0
    if gemm_tiles(M, Nn) < cu_count(a.get_device()):
        ws_bytes = N.query("moc_gemm_workspace_size", N.MOC_BF16, M, Nn, Kd, 0)
    ws = _gemm_workspace(a.device, ws_bytes) if ws_bytes > 0 else None
    probe = _probe_begin()
    N.call("moc_gemm_residual_bf16", M, Nn, Kd, aa.data_ptr(), as0, as1, bb.data_ptr(), bs0, bs1,
           out.data_ptr(), out.stride(0) if M > 1 else max(Nn, 1), r.data_ptr(),
           r.stride(0) if M > 1 else round_up(max(Nn, 1), 8), N.ptr(ws), ws_bytes, N.stream_of(a))
    _probe_end(probe, f"gemm {M}x{Nn}x{Kd} +res", 2.0 * M * Nn * Kd)
    return out


def rmsnorm_rows(x2d: torch.Tensor, weight: torch.Tensor, eps: float, *, out: torch.Tensor | None = None,
                 want_rstd: bool = True):
    """(y, rstd): the pre-norm y = bf16(bf16(x / rms(x)) * weight) of every
    row of a bf16 [rows, d] tensor (RMSNorm.forward of moc/model.py:26-28),
    rstd = 1 / rms(x) per row in f32 (None unless want_rstd)."""
    N.require_device(x2d, weight, out)
    if x2d.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise ValueError("rmsnorm_rows takes bf16 rows and a bf16 weight")
    xa = aligned_rows(x2d)
    rows, d = xa.shape
    w = weight.contiguous()
    if w.shape != (d,):
        raise ValueError(f"norm weight must be [{d}]")
    y = padded_empty(rows, d, torch.bfloat16, x2d.device) if out is None else out
    rstd = torch.empty(rows, dtype=torch.float32, device=x2d.device) if want_rstd else None
    N.call("moc_rmsnorm_rows_bf16", xa.data_ptr(), xa.stride(0) if rows > 1 else round_up(d, 8), rows, d,
           w.data_ptr(), float(eps), y.data_ptr(), y.stride(0) if rows > 1 else round_up(d, 8),
           N.ptr(rstd), N.stream_of(x2d))
    return y, rstd


def rmsnorm_backward(x2d: torch.Tensor, weight: torch.Tensor, rstd: torch.Tensor, dy: torch.Tensor,
                     dres: torch.Tensor | None = None, dw_dtype=None):
    """(dx, dw) of rmsnorm_rows given dy, plus dres (the gradient of a
    residual branch around the norm, added to dx)."""
    N.require_device(x2d, weight, rstd, dy, dres)
    xa, ga = aligned_rows(x2d), aligned_rows(dy)
    ra = None if dres is None else aligned_rows(dres)
    rows, d = xa.shape
    w = weight.contiguous()
    dw_dtype = dw_dtype or weight.dtype
    dx = padded_empty(rows, d, torch.bfloat16, x2d.device)
    dw = torch.empty(d, dtype=dw_dtype, device=x2d.device)
    nbytes = N.query("moc_rmsnorm_backward_workspace_size", rows, d)
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=x2d.device)
    ld = lambda t: t.stride(0) if rows > 1 else round_up(d, 8)  # noqa: E731
    N.call("moc_rmsnorm_backward_bf16", xa.data_ptr(), ld(xa), rows, d, w.data_ptr(),
           rstd.contiguous().data_ptr(), ga.data_ptr(), ld(ga), N.ptr(ra), 0 if ra is None else ld(ra),
           dx.data_ptr(), ld(dx), dw.data_ptr(), N.dtype_code(dw_dtype), ws.data_ptr(), ws.numel(),
           N.stream_of(x2d))
    return dx, dw


def linear(x2d: torch.Tensor, weight: torch.Tensor, *, out: torch.Tensor | None = None,
           out_dtype=None) -> torch.Tensor:
    """x2d @ weight.T for an nn.Linear weight [out_features, in_features]."""
    return gemm(x2d, weight.t(), out=out, out_dtype=out_dtype)


def linear_pair(x2d: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, *,
                out1: torch.Tensor | None = None,
                out2: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """(x2d @ w1.T, x2d @ w2.T) for two nn.Linear weights of one input, bf16,
    in one MFMA launch when the pair fills the CUs (moc_gemm_pair)."""
    N.require_device(x2d, w1, w2, out1, out2)
    if not (x2d.dtype == w1.dtype == w2.dtype == torch.bfloat16):
        raise ValueError("linear_pair takes bf16 operands")
    M, Kd = x2d.shape
    if w1.shape[1] != Kd or w2.shape[1] != Kd:
        raise ValueError(f"linear_pair shape mismatch {tuple(x2d.shape)} x {tuple(w1.shape)}, "
                         f"{tuple(w2.shape)}")
    n1, n2 = w1.shape[0], w2.shape[0]
    xa, wa, wb = aligned_rows(x2d), aligned_rows(w1), aligned_rows(w2)
    outs = []
    for o, n in ((out1, n1), (out2, n2)):
        if o is None:
            o = _empty((M, n), torch.bfloat16, x2d.device)
        if o.shape != (M, n) or (o.stride(1) != 1 and n > 1) or o.dtype != torch.bfloat16:
            raise ValueError("linear_pair outputs must be bf16 [M, N] with unit column stride")
        outs.append(o)
    lda = xa.stride(0) if M > 1 else round_up(max(Kd, 1), 8)
    ld1 = wa.stride(0) if n1 > 1 else round_up(max(Kd, 1), 8)
    ld2 = wb.stride(0) if n2 > 1 else round_up(max(Kd, 1), 8)
    ldc = [o.stride(0) if M > 1 else max(o.shape[1], 1) for o in outs]
    ws_bytes = 0
    for n in (n1, n2):
        if gemm_tiles(M, n) < cu_count(x2d.get_device()):
            ws_bytes = max(ws_bytes, N.query("moc_gemm_workspace_size", N.dtype_code(torch.bfloat16),
                                             M, n, Kd, 0))
    ws = _gemm_workspace(x2d.device, ws_bytes) if ws_bytes > 0 else None
    probe = _probe_begin()
    N.call("moc_gemm_pair", M, Kd, xa.data_ptr(), lda, wa.data_ptr(), ld1, n1, outs[0].data_ptr(),
           ldc[0], wb.data_ptr(), ld2, n2, outs[1].data_ptr(), ldc[1], N.ptr(ws), ws_bytes,
           N.stream_of(x2d))
    _probe_end(probe, f"gemm pair {M}x({n1}+{n2})x{Kd}", 2.0 * M * Kd * (n1 + n2))
    return outs[0], outs[1]


# -------------------------------------------------------------------- decode
def gemv(x: torch.Tensor, weight: torch.Tensor, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """[nb <= 16, hidden] @ weight[rows, hidden].T -> [nb, rows] (bf16)."""
    N.require_device(x, weight)
    xx = aligned_rows(x)
    w = aligned_rows(weight)
    nb, hidden = xx.shape
    rows = w.shape[0]
    if w.shape[1] != hidden:
        raise ValueError(f"gemv shape mismatch {tuple(x.shape)} x {tuple(weight.shape)}")
    y = _empty((nb, rows), torch.bfloat16, x.device) if out is None else out
    if y.shape != (nb, rows) or not y.is_contiguous():
        raise ValueError("gemv out must be a contiguous [nb, rows] tensor")
    N.call("moc_gemv_bf16", xx.data_ptr(), xx.stride(0) if nb > 1 else round_up(hidden, 8), nb,
           w.data_ptr(), w.stride(0), rows, hidden, y.data_ptr(), rows, N.stream_of(x))
    return y


def gemv_rmsnorm(x: torch.Tensor, norm_weight: torch.Tensor, eps: float, weight: torch.Tensor, *,
                 out: torch.Tensor | None = None, xn_out: torch.Tensor | None = None):
    """(y, xn): xn = RMSNorm(x) (f32 statistics, bf16 rounding as torch's
    (x.float() * r).to(bf16) * w), y = xn @ weight.T, for <= 4 tokens."""
    N.require_device(x, norm_weight, weight)
    xx = aligned_rows(x)
    w = aligned_rows(weight)
    nw = norm_weight.contiguous()
    nb, hidden = xx.shape
    rows = w.shape[0]
    if w.shape[1] != hidden or nw.shape != (hidden,):
        raise ValueError("gemv_rmsnorm shape mismatch")
    for t in (xx, w, nw):
        if t.dtype != torch.bfloat16:
            raise ValueError("gemv_rmsnorm is bf16 only")
    y = _empty((nb, rows), torch.bfloat16, x.device) if out is None else out
    xn = _empty((nb, hidden), torch.bfloat16, x.device) if xn_out is None else xn_out
    N.call("moc_gemv_rmsnorm_bf16", xx.data_ptr(), xx.stride(0) if nb > 1 else round_up(hidden, 8), nb,
           nw.data_ptr(), float(eps), xn.data_ptr(), xn.stride(0) if nb > 1 else round_up(hidden, 8),
           w.data_ptr(), w.stride(0), rows, hidden, y.data_ptr(), rows, N.stream_of(x))
    return y, xn


def _bf16_contig(*ts):
    for t in ts:
        if t.dtype != torch.bfloat16:
            raise ValueError(f"expected bfloat16, got {t.dtype}")
    return [t.contiguous() for t in ts]


# Extra elements per row of the decode kernels' W_down^T (MOC_DOWN_T_PITCH_PAD
# of include/moc_amd.h): 128 bytes, so that the rows' column blocks do not all
# fall on the same memory channels.
DOWN_T_PITCH_PAD = 64


def down_weight_t_for_decode(down_weight: torch.Tensor) -> torch.Tensor:
    """W_down [hidden, inter] -> W_down^T [inter, hidden] as the decode
    kernels read it best: a view of rows at a pitch of round8(hidden) +
    DOWN_T_PITCH_PAD elements (the pad is never read)."""
    hidden, inter = down_weight.shape
    pitch = round_up(hidden, 8) + DOWN_T_PITCH_PAD
    buf = torch.empty((inter, pitch), dtype=down_weight.dtype, device=down_weight.device)
    view = buf[:, :hidden]
    view.copy_(down_weight.detach().t())
    return view


def _down_t_rows(wdt: torch.Tensor):
    """(tensor, row pitch) of a bf16 W_down^T [inter, hidden]: a view with
    unit column stride, 16-byte aligned rows and a pitch of a multiple of 8
    is passed as it is; anything else is made contiguous."""
    if wdt.dtype != torch.bfloat16:
        raise ValueError(f"expected bfloat16, got {wdt.dtype}")
    if (wdt.dim() == 2 and wdt.stride(1) == 1 and wdt.stride(0) >= wdt.shape[1]
            and wdt.stride(0) % 8 == 0 and wdt.data_ptr() % 16 == 0):
        return wdt, wdt.stride(0)
    c = wdt.contiguous()
    return c, c.shape[1] if c.dim() == 2 else 0


def selected_up_silu(x, topk_vals, topk_idx, up_weight) -> torch.Tensor:
    N.require_device(x, topk_vals, topk_idx, up_weight)
    x, vals, w = _bf16_contig(x, topk_vals, up_weight)
    idx = topk_idx.contiguous()
    nb, hidden = x.shape
    k = idx.shape[1]
    z = _empty((nb, k), torch.bfloat16, x.device)
    N.call("moc_selected_up_silu_bf16", x.data_ptr(), nb, hidden, vals.data_ptr(), idx.data_ptr(),
           N.idx_code(idx.dtype), k, w.data_ptr(), w.shape[0], z.data_ptr(), N.stream_of(x))
    return z


def selected_down(sparse_z, topk_idx, down_weight_t) -> torch.Tensor:
    N.require_device(sparse_z, topk_idx, down_weight_t)
    (z,) = _bf16_contig(sparse_z)
    wdt, ldw = _down_t_rows(down_weight_t)
    idx = topk_idx.contiguous()
    nb, k = z.shape
    inter, hidden = wdt.shape
    y = _empty((nb, hidden), torch.bfloat16, z.device)
    ws_bytes = N.query("moc_selected_down_workspace_size", nb, k, hidden)
    ws = _empty((max(ws_bytes, 1),), torch.uint8, z.device)
    N.call("moc_selected_down_bf16", z.data_ptr(), idx.data_ptr(), N.idx_code(idx.dtype), nb, k,
           wdt.data_ptr(), ldw, inter, hidden, y.data_ptr(), ws.data_ptr(), ws_bytes, N.stream_of(z))
    return y


def global_after_gate_workspace_bytes(nb: int, inter: int, k: int, hidden: int) -> int:
    return N.query("moc_global_after_gate_workspace_size", nb, inter, int(k), hidden)


def _decode_workspace(device, nbytes: int) -> torch.Tensor:
    """The after-gate workspace of the current stream on `device`, grown on
    demand (callers without a workspace of their own: the moc_native op)."""
    return _stream_workspace(_WS_CACHE, device, nbytes, minimum=256)


def global_after_gate_workspace(nb: int, inter: int, k: int, hidden: int, device) -> torch.Tensor:
    """A fresh zero-initialised workspace for global_after_gate."""
    nbytes = global_after_gate_workspace_bytes(nb, inter, k, hidden)
    return torch.zeros((max(nbytes, 256),), dtype=torch.uint8, device=device)


def global_after_gate(x, gate_scores, up_weight, down_weight_t, k: int, *, workspace=None,
                      out=None, residual: torch.Tensor | None = None,
                      idx_out: torch.Tensor | None = None) -> torch.Tensor:
    """Top-K + selected Up * SiLU + selected Down after the gate; with
    `residual`, returns residual + that (bf16 add) from the same launch.
    `idx_out` (int32 [nb, k]) receives the selected channels in ascending
    order.  Without `workspace`, the stream's shared workspace is used."""
    N.require_device(x, gate_scores, up_weight, down_weight_t, idx_out)
    x, g, wu = _bf16_contig(x, gate_scores, up_weight)
    wdt, ldw = _down_t_rows(down_weight_t)
    nb, hidden = x.shape
    inter = g.shape[1]
    if wu.shape != (inter, hidden) or wdt.shape != (inter, hidden):
        raise ValueError("up_weight and down_weight_t must be [intermediate, hidden]")
    if idx_out is not None and (idx_out.dtype != torch.int32 or idx_out.shape != (nb, int(k))
                                or not idx_out.is_contiguous()):
        raise ValueError(f"idx_out must be a contiguous int32 [{nb}, {int(k)}] tensor")
    if nb > 16:
        # more tokens than the fused kernel takes: the same steps as separate
        # launches (row Top-K, selected Up * SiLU, selected Down), like the
        # reference's op, which accepts any batch (optimized_global_moc_ext.cu:457-540)
        vals, idx, _ = topk_rows(g, int(k), idx_dtype=torch.int32)
        z = selected_up_silu(x, vals, idx, wu)
        yy = selected_down(z, idx, wdt)
        if residual is not None:
            yy = residual.reshape(yy.shape) + yy
        if idx_out is not None:
            idx_out.copy_(idx)
        if out is None:
            return yy
        out.copy_(yy)
        return out
    y = _empty((nb, hidden), torch.bfloat16, x.device) if out is None else out
    ws_bytes = N.query("moc_global_after_gate_workspace_size", nb, inter, int(k), hidden)
    if workspace is None:
        workspace = _decode_workspace(x.device, ws_bytes)
    elif workspace.numel() < ws_bytes:
        raise ValueError(f"global_after_gate: workspace of {ws_bytes} bytes required")
    if residual is None:
        N.call("moc_global_after_gate_bf16", x.data_ptr(), g.data_ptr(), nb, inter, hidden,
               wu.data_ptr(), wdt.data_ptr(), ldw, int(k), y.data_ptr(), N.ptr(idx_out),
               workspace.data_ptr(), ws_bytes, N.stream_of(x))
        return y
    r = residual.reshape(nb, hidden)
    if r.dtype != torch.bfloat16 or not r.is_contiguous():
        raise ValueError("residual must be a contiguous bf16 [nb, hidden] tensor")
    N.call("moc_global_after_gate_residual_bf16", x.data_ptr(), g.data_ptr(), nb, inter, hidden,
           wu.data_ptr(), wdt.data_ptr(), ldw, int(k), r.data_ptr(), y.data_ptr(), N.ptr(idx_out),
           workspace.data_ptr(), ws_bytes, N.stream_of(x))
    return y


def global_decode_workspace(nb: int, inter: int, k: int, hidden: int, device) -> torch.Tensor:
    """A fresh zero-initialised workspace for global_decode."""
    nbytes = N.query("moc_global_decode_workspace_size", nb, inter, int(k), hidden)
    return torch.zeros((max(nbytes, 256),), dtype=torch.uint8, device=device)


def global_decode(x, gate_weight, up_weight, down_weight_t, k: int, *, workspace=None, out=None,
                  idx_out: torch.Tensor | None = None) -> torch.Tensor:
    """The global-MoC decode layer from x (<= 16 tokens): gate projection,
    then Top-K + selected Up * SiLU + selected Down; the result of
    global_after_gate(x, gemv(x, gate_weight), ...)."""
    N.require_device(x, gate_weight, up_weight, down_weight_t, idx_out)
    x, wg, wu = _bf16_contig(x, gate_weight, up_weight)
    wdt, ldw = _down_t_rows(down_weight_t)
    nb, hidden = x.shape
    inter = wg.shape[0]
    if nb > 16:
        raise ValueError(f"global_decode takes at most 16 tokens (got {nb})")
    if wg.shape != (inter, hidden) or wu.shape != (inter, hidden) or wdt.shape != (inter, hidden):
        raise ValueError("gate_weight, up_weight and down_weight_t must be [intermediate, hidden]")
    if idx_out is not None and (idx_out.dtype != torch.int32 or idx_out.shape != (nb, int(k))
                                or not idx_out.is_contiguous()):
        raise ValueError(f"idx_out must be a contiguous int32 [{nb}, {int(k)}] tensor")
    y = _empty((nb, hidden), torch.bfloat16, x.device) if out is None else out
    ws_bytes = N.query("moc_global_decode_workspace_size", nb, inter, int(k), hidden)
    if workspace is None:
        workspace = _decode_workspace(x.device, ws_bytes)
    elif workspace.numel() < ws_bytes:
        raise ValueError(f"global_decode: workspace of {ws_bytes} bytes required")
    N.call("moc_global_decode_bf16", x.data_ptr(), nb, hidden, wg.data_ptr(), wu.data_ptr(), inter,
           wdt.data_ptr(), ldw, int(k), y.data_ptr(), N.ptr(idx_out), workspace.data_ptr(), ws_bytes,
           N.stream_of(x))
    return y


def global_decode_rmsnorm_residual(x, norm_weight, eps: float, gate_weight, up_weight, down_weight_t,
                                   k: int, *, workspace=None, out=None,
                                   idx_out: torch.Tensor | None = None) -> torch.Tensor:
    """x + FFN(RMSNorm(x)) of a decoder layer, <= 4 tokens, global MoC: the
    norm inside the gate/up GEMV, the residual added by the after-gate
    kernel (moc_global_decode_rmsnorm_residual_bf16)."""
    N.require_device(x, norm_weight, gate_weight, up_weight, down_weight_t, idx_out)
    x, nw, wg, wu = _bf16_contig(x, norm_weight, gate_weight, up_weight)
    wdt, ldw = _down_t_rows(down_weight_t)
    nb, hidden = x.shape
    inter = wg.shape[0]
    if nb > 4:
        raise ValueError(f"global_decode_rmsnorm_residual takes at most 4 tokens (got {nb})")
    if wg.shape != (inter, hidden) or wu.shape != (inter, hidden) or wdt.shape != (inter, hidden) \
            or nw.shape != (hidden,):
        raise ValueError("norm_weight [hidden]; gate_weight, up_weight, down_weight_t [intermediate, hidden]")
    if idx_out is not None and (idx_out.dtype != torch.int32 or idx_out.shape != (nb, int(k))
                                or not idx_out.is_contiguous()):
        raise ValueError(f"idx_out must be a contiguous int32 [{nb}, {int(k)}] tensor")
    y = _empty((nb, hidden), torch.bfloat16, x.device) if out is None else out
    ws_bytes = N.query("moc_global_decode_workspace_size", nb, inter, int(k), hidden)
    if workspace is None:
        workspace = _decode_workspace(x.device, ws_bytes)
    elif workspace.numel() < ws_bytes:
        raise ValueError(f"global_decode_rmsnorm_residual: workspace of {ws_bytes} bytes required")
    N.call("moc_global_decode_rmsnorm_residual_bf16", x.data_ptr(), nb, hidden, nw.data_ptr(), float(eps),
           wg.data_ptr(), wu.data_ptr(), inter, wdt.data_ptr(), ldw, int(k), y.data_ptr(), N.ptr(idx_out),
           workspace.data_ptr(), ws_bytes, N.stream_of(x))
    return y


def global_decode_rmsnorm_residual_fits(nb: int, inter: int, k: int, hidden: int) -> bool:
    """Shapes moc_global_decode_rmsnorm_residual_bf16 takes."""
    return 1 <= nb <= 4 and hidden % 256 == 0 and hidden <= 4096 and inter <= 8192 and int(k) <= 4096


# ----------------------------------------------------------------------- 2:8
def grouped_top2_up_silu(x, gate_weight, up_weight, *, idx_out=None, sz_out=None,
                         norm_weight: torch.Tensor | None = None, eps: float = 1e-6):
    """-> (idx int64 [nb, inter/4], sparse_z bf16 [nb, inter/4]).  With
    norm_weight (<= 4 tokens): of RMSNorm(x) (the FFN's pre-norm) instead."""
    N.require_device(x, gate_weight, up_weight, norm_weight)
    x, wg, wu = _bf16_contig(x, gate_weight, up_weight)
    nb, hidden = x.shape
    inter = wg.shape[0]
    if inter % 8 != 0:
        raise ValueError(f"intermediate={inter} must be divisible by 8")
    if wg.shape != wu.shape or wg.shape[1] != hidden:
        raise ValueError(f"H mismatch: x={tuple(x.shape)}, gate={tuple(wg.shape)}, up={tuple(wu.shape)}")
    k = inter // 4
    idx = _empty((nb, k), torch.int64, x.device) if idx_out is None else idx_out
    sz = _empty((nb, k), torch.bfloat16, x.device) if sz_out is None else sz_out
    if idx.shape != (nb, k) or sz.shape != (nb, k) or not (idx.is_contiguous() and sz.is_contiguous()):
        raise ValueError(f"out shapes must be ({nb},{k})")
    if norm_weight is None:
        N.call("moc_grouped_top2_up_silu_bf16", x.data_ptr(), nb, hidden, wg.data_ptr(), wu.data_ptr(),
               inter, idx.data_ptr(), sz.data_ptr(), N.stream_of(x))
    else:
        nw = norm_weight.contiguous()
        if nw.dtype != torch.bfloat16 or nw.shape != (hidden,):
            raise ValueError("norm_weight must be a bf16 [hidden] tensor")
        N.call("moc_grouped_top2_up_silu_rmsnorm_bf16", x.data_ptr(), nb, hidden, nw.data_ptr(),
               float(eps), wg.data_ptr(), wu.data_ptr(), inter, idx.data_ptr(), sz.data_ptr(),
               N.stream_of(x))
    return idx, sz


def moc28_decode_fits(nb: int, inter: int, hidden: int, norm: bool = False) -> bool:
    """Shapes moc_moc28_decode_bf16 takes (norm: with the fused RMSNorm)."""
    return (1 <= nb <= (4 if norm else 16) and inter % 8 == 0 and 8 <= inter <= 8192
            and hidden % 256 == 0 and (not norm or hidden <= 4096))


def moc28_decode_workspace_bytes(nb: int, inter: int, hidden: int) -> int:
    """Workspace bytes of moc28_decode (no zeroing needed)."""
    return N.query("moc_moc28_decode_workspace_size", nb, inter, hidden)


def moc28_decode(x, gate_weight, up_weight, down_weight_t, *, norm_weight: torch.Tensor | None = None,
                 eps: float = 1e-6, residual: torch.Tensor | None = None, workspace=None, out=None,
                 idx_out: torch.Tensor | None = None) -> torch.Tensor:
    """The MoC 2:8 decode layer (<= 16 tokens) in two launches
    (moc_moc28_decode_bf16): the gate/up GEMV pair of x (of RMSNorm(x) with
    norm_weight, <= 4 tokens), then the top 2 of every 8 channels and the
    selected Down, + residual when given.  Same selection (idx_out int64
    [nb, inter/4]) and z as grouped_top2_up_silu, y as selected_grouped_down
    in another f32 order."""
    N.require_device(x, gate_weight, up_weight, down_weight_t, norm_weight, residual, idx_out)
    x, wg, wu = _bf16_contig(x, gate_weight, up_weight)
    wdt, ldw = _down_t_rows(down_weight_t)
    nb, hidden = x.shape
    inter = wg.shape[0]
    if not moc28_decode_fits(nb, inter, hidden, norm_weight is not None):
        raise ValueError(f"moc28_decode: unsupported shape nb={nb}, inter={inter}, hidden={hidden}")
    if wg.shape != (inter, hidden) or wu.shape != (inter, hidden) or wdt.shape != (inter, hidden):
        raise ValueError("gate_weight, up_weight and down_weight_t must be [intermediate, hidden]")
    nw = None
    if norm_weight is not None:
        nw = norm_weight.contiguous()
        if nw.dtype != torch.bfloat16 or nw.shape != (hidden,):
            raise ValueError("norm_weight must be a bf16 [hidden] tensor")
    r = None
    if residual is not None:
        r = residual.reshape(nb, hidden)
        if r.dtype != torch.bfloat16 or not r.is_contiguous():
            raise ValueError("residual must be a contiguous bf16 [nb, hidden] tensor")
    if idx_out is not None and (idx_out.dtype != torch.int64 or idx_out.shape != (nb, inter // 4)
                                or not idx_out.is_contiguous()):
        raise ValueError(f"idx_out must be a contiguous int64 [{nb}, {inter // 4}] tensor")
    y = _empty((nb, hidden), torch.bfloat16, x.device) if out is None else out
    ws_bytes = moc28_decode_workspace_bytes(nb, inter, hidden)
    if workspace is None:
        workspace = _decode_workspace(x.device, ws_bytes)
    elif workspace.numel() < ws_bytes:
        raise ValueError(f"moc28_decode: workspace of {ws_bytes} bytes required")
    N.call("moc_moc28_decode_bf16", x.data_ptr(), nb, hidden, N.ptr(nw), float(eps), wg.data_ptr(),
           wu.data_ptr(), inter, wdt.data_ptr(), ldw, N.ptr(r), y.data_ptr(), N.ptr(idx_out),
           workspace.data_ptr(), ws_bytes, N.stream_of(x))
    return y


def packed28_layout(nb: int, inter: int) -> tuple[int, int, int]:
    """(channel tiles, ld_ap, meta_rows) of the 2:4-packed 2:8 operand."""
    nt = (inter + 63) // 64
    return nt, 32 * nt, round_up(max(nb, 1), 256)


def packed28_buffers(nb: int, inter: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    """Empty (ap [nb, ld_ap] bf16, meta [nt, meta_rows, 2] int32) buffers."""
    nt, ld_ap, meta_rows = packed28_layout(nb, inter)
    return (_empty((nb, ld_ap), torch.bfloat16, device),
            _empty((nt, meta_rows, 2), torch.int32, device))


def grouped_top2_up_silu_packed(x, gate_weight, up_weight, ap, meta) -> None:
    """The 2:8 gate/up + top-2-of-8 with the selection written 2:4-packed
    (ap, meta from packed28_buffers) instead of as (idx, sz)."""
    N.require_device(x, gate_weight, up_weight, ap, meta)
    x, wg, wu = _bf16_contig(x, gate_weight, up_weight)
    nb, hidden = x.shape
    inter = wg.shape[0]
    if inter % 8 != 0:
        raise ValueError(f"intermediate={inter} must be divisible by 8")
    if wg.shape != wu.shape or wg.shape[1] != hidden:
        raise ValueError(f"H mismatch: x={tuple(x.shape)}, gate={tuple(wg.shape)}, up={tuple(wu.shape)}")
    nt, ld_ap, meta_rows = packed28_layout(nb, inter)
    _check_packed28(ap, meta, nb, nt, ld_ap, meta_rows)
    N.call("moc_grouped_top2_up_silu_packed_bf16", x.data_ptr(), nb, hidden, wg.data_ptr(),
           wu.data_ptr(), inter, ap.data_ptr(), ld_ap, meta.data_ptr(), meta.shape[1], N.stream_of(x))


def _check_packed28(ap, meta, nb: int, nt: int, ld_ap: int, meta_rows: int) -> None:
    """ap: [nb, ld_ap] rows (a row view of a larger buffer is fine); meta:
    [nt, R, 2] with R >= meta_rows (the tile stride may be a larger
    batch's)."""
    if (ap.shape != (nb, ld_ap) or ap.stride() != (ld_ap, 1) or meta.dim() != 3
            or meta.shape[0] != nt or meta.shape[2] != 2 or meta.shape[1] < meta_rows
            or meta.shape[1] % 256 or not meta.is_contiguous()):
        raise ValueError("packed buffers do not match packed28_layout")


def sparse28_down_workspace_bytes(nb: int, inter: int, hidden: int) -> int:
    return N.query("moc_sparse28_down_workspace_size", nb, inter, hidden)


def sparse28_down_workspace(nb: int, inter: int, hidden: int, device) -> torch.Tensor:
    """A zeroed workspace for sparse28_down (its counters start at zero and
    every call leaves them zero, so it is reused without clearing)."""
    b = sparse28_down_workspace_bytes(nb, inter, hidden)
    return torch.zeros((max(b, 1),), dtype=torch.uint8, device=device)


def sparse28_down(ap, meta, inter: int, down_weight_t, *, workspace, out=None) -> torch.Tensor:
    """y = A W_down (A 2:4-packed) on the structured-sparse MFMA; W_down
    given transposed [inter, hidden]."""
    N.require_device(ap, meta, down_weight_t, workspace, out)
    nb = ap.shape[0]
    if down_weight_t.dtype != torch.bfloat16:
        raise ValueError("down_weight_t must be a bf16 [inter, hidden] tensor")
    wdt, _ = _down_t_rows(down_weight_t)
    if wdt.shape[0] != inter:
        raise ValueError("down_weight_t must be a bf16 [inter, hidden] tensor")
    hidden = wdt.shape[1]
    nt, ld_ap, meta_rows = packed28_layout(nb, inter)
    _check_packed28(ap, meta, nb, nt, ld_ap, meta_rows)
    y = _empty((nb, hidden), torch.bfloat16, ap.device) if out is None else out
    if y.shape != (nb, hidden) or not y.is_contiguous():
        raise ValueError(f"out shape must be ({nb},{hidden})")
    ws_bytes = N.query("moc_sparse28_down_workspace_size", nb, inter, hidden)
    if workspace.numel() < ws_bytes:
        raise ValueError(f"sparse28_down needs a workspace of {ws_bytes} bytes")
    N.call("moc_sparse28_down_bf16", ap.data_ptr(), ld_ap, meta.data_ptr(), meta.shape[1], nb, inter,
           wdt.data_ptr(), wdt.stride(0), 0, hidden, y.data_ptr(), y.stride(0), workspace.data_ptr(),
           ws_bytes, N.stream_of(ap))
    return y


def selected_grouped_down_workspace_bytes(nb: int, k: int, inter: int, hidden: int) -> int:
    return N.query("moc_selected_grouped_down_workspace_size", nb, k, inter, hidden)


def selected_grouped_down(sparse_z, idx, down_weight_t, *, out=None, workspace=None,
                          residual: torch.Tensor | None = None) -> torch.Tensor:
    """y = sparse_z * W_down^T[idx]; with `residual` (<= 64 tokens),
    residual + y (bf16 add) from the same launches."""
    N.require_device(sparse_z, idx, down_weight_t, residual)
    (sz,) = _bf16_contig(sparse_z)
    wdt, ldw = _down_t_rows(down_weight_t)
    ii = idx.contiguous()
    if ii.dtype != torch.int64:
        raise ValueError("idx must be int64")
    nb, k = sz.shape
    inter, hidden = wdt.shape
    y = _empty((nb, hidden), torch.bfloat16, sz.device) if out is None else out
    if y.shape != (nb, hidden) or not y.is_contiguous():
        raise ValueError(f"out shape must be ({nb},{hidden})")
    ws_bytes = selected_grouped_down_workspace_bytes(nb, k, inter, hidden)
    ws = workspace if workspace is not None and workspace.numel() >= ws_bytes else \
        _empty((max(ws_bytes, 1),), torch.uint8, sz.device)
    if residual is None:
        N.call("moc_selected_grouped_down_bf16", sz.data_ptr(), ii.data_ptr(), nb, k, wdt.data_ptr(), ldw,
               inter, hidden, y.data_ptr(), ws.data_ptr(), ws_bytes, N.stream_of(sz))
        return y
    r = residual.reshape(nb, hidden)
    if r.dtype != torch.bfloat16 or not r.is_contiguous():
        raise ValueError("residual must be a contiguous bf16 [nb, hidden] tensor")
    if nb > 64:
        N.call("moc_selected_grouped_down_bf16", sz.data_ptr(), ii.data_ptr(), nb, k, wdt.data_ptr(), ldw,
               inter, hidden, y.data_ptr(), ws.data_ptr(), ws_bytes, N.stream_of(sz))
        y.copy_(r + y)
        return y
    N.call("moc_selected_grouped_down_residual_bf16", sz.data_ptr(), ii.data_ptr(), nb, k,
           wdt.data_ptr(), ldw, inter, hidden, r.data_ptr(), y.data_ptr(), ws.data_ptr(), ws_bytes,
           N.stream_of(sz))
    return y
