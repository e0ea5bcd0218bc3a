"""ctypes binding of libmoc_amd.so, the gfx950 HIP kernels behind the C ABI.

The library is loaded once, after torch, so that its HIP runtime dependency
resolves to the runtime torch already loaded (both carry the soname
libamdhip64.so.7).  Every call passes raw device pointers plus the HIP stream
torch is currently using, and a non-zero status becomes a Python exception:
MOC_ERR_INVALID -> ValueError, anything else -> RuntimeError, carrying the
library's own message (moc_last_error()).

There is no fallback: if the library is missing or the tensors are not on a
ROCm device, the call raises.
"""
from __future__ import annotations

import ctypes
import re
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libmoc_amd.so"
HEADER_PATH = Path(__file__).resolve().parent.parent / "include" / "moc_amd.h"

MOC_OK = 0
MOC_ERR_INVALID = -1
MOC_ERR_HIP = -2
MOC_BF16 = 0
MOC_F32 = 1
MOC_I16 = 0
MOC_I32 = 1
MOC_I64 = 2

_i64 = ctypes.c_int64
_int = ctypes.c_int
_vp = ctypes.c_void_p

# name -> (restype, argtypes); mirrors include/moc_amd.h
SIGNATURES: dict[str, tuple] = {
    "moc_last_error": (ctypes.c_char_p, []),
    "moc_abi_version": (_int, []),
    "moc_fill_zero": (_int, [_vp, _i64, _vp]),
    "moc_copy_pad_2d": (_int, [_int, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp]),
    "moc_topk_rows": (_int, [_int, _vp, _i64, _i64, _i64, _i64, _int, _vp, _vp, _int, _vp, _i64, _vp]),
    "moc_mask_to_idx": (_int, [_vp, _i64, _i64, _i64, _i64, _vp, _int, _vp]),
    "moc_moc28_effective_k": (_i64, [_i64]),
    "moc_select_2of8": (_int, [_int, _vp, _i64, _i64, _i64, _vp, _vp, _int, _vp]),
    "moc_sparse_forward_aux": (_int, [_int, _vp, _vp, _int, _vp, _i64, _i64, _i64, _i64,
                                      _vp, _vp, _vp, _vp, _i64, _vp]),
    "moc_scatter_sparse_to_dense": (_int, [_int, _vp, _vp, _int, _i64, _i64, _i64, _vp, _i64, _vp]),
    "moc_gather_dense_to_sparse": (_int, [_int, _vp, _i64, _vp, _int, _i64, _i64, _vp, _vp]),
    "moc_gcp_recompute": (_int, [_int, _vp, _vp, _i64, _vp, _vp, _vp]),
    "moc_gcp_recompute_scatter": (_int, [_int, _vp, _vp, _vp, _int, _i64, _i64, _i64, _vp, _vp,
                                         _i64, _vp]),
    "moc_sparse_backward_aux": (_int, [_int, _vp, _int, _vp, _vp, _vp, _vp, _i64, _i64, _i64,
                                       _i64, _vp, _vp, _i64, _vp]),
    "moc_gemm": (_int, [_int, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _i64, _vp,
                        _i64, _i64, _vp, _i64, _i64, _vp, _i64, _int, _vp]),
    "moc_gemm_ws": (_int, [_int, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _i64, _vp,
                           _i64, _i64, _vp, _i64, _i64, _vp, _i64, _int, _vp, _i64, _vp]),
    "moc_gemm_workspace_size": (_i64, [_int, _i64, _i64, _i64, _i64]),
    "moc_gemm_residual_bf16": (_int, [_i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64,
                                      _vp, _i64, _vp, _i64, _vp]),
    "moc_rmsnorm_rows_bf16": (_int, [_vp, _i64, _i64, _i64, _vp, ctypes.c_float, _vp, _i64, _vp, _vp]),
    "moc_rmsnorm_backward_workspace_size": (_i64, [_i64, _i64]),
    "moc_rmsnorm_backward_bf16": (_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _i64, _vp,
                                         _i64, _vp, _int, _vp, _i64, _vp]),
    "moc_ffn_block_forward_bf16": (_int, [_i64, _i64, _i64, _i64, _int, _vp, _i64, _vp, ctypes.c_float,
                                          _vp, _i64, _vp, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i64,
                                          _vp, _vp, _int, _vp, _vp, _vp, _vp, _i64, _vp, _i64, _vp]),
    "moc_ffn_block_backward_workspace_size": (_i64, [_i64, _i64, _i64, _i64, _int]),
    "moc_ffn_block_backward_bf16": (_int, [_i64, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp,
                                           ctypes.c_float, _vp, _vp, _i64, _vp, _int, _vp, _vp, _vp, _vp,
                                           _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i64,
                                           _int, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _i64, _int, _vp,
                                           _int, _vp, _i64, _vp]),
    "moc_ffn_forward_workspace_size": (_i64, [_i64, _i64, _i64]),
    "moc_ffn_forward_bf16": (_int, [_i64, _i64, _i64, _i64, _int, _vp, _i64, _vp, _i64, _vp, _i64, _vp,
                                    _i64, _vp, _vp, _i64, _vp, _vp, _int, _vp, _vp, _vp, _vp, _i64, _vp,
                                    _i64, _vp]),
    "moc_ffn_forward_f32_workspace_size": (_i64, [_i64, _i64, _i64]),
    "moc_ffn_forward_f32": (_int, [_i64, _i64, _i64, _i64, _int, _vp, _i64, _vp, _i64, _vp, _i64, _vp,
                                   _i64, _vp, _vp, _i64, _vp, _vp, _int, _vp, _vp, _vp, _vp, _i64, _vp,
                                   _i64, _vp]),
    "moc_ffn_backward_workspace_size": (_i64, [_i64, _i64, _i64, _i64, _int]),
    "moc_ffn_backward_bf16": (_int, [_i64, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp, _int, _vp, _vp,
                                     _vp, _vp, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp,
                                     _i64, _int, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _i64, _int, _vp,
                                     _i64, _vp]),
    "moc_gemm_pair": (_int, [_i64, _i64, _vp, _i64, _vp, _i64, _i64, _vp, _i64, _vp, _i64, _i64,
                             _vp, _i64, _vp, _i64, _vp]),
    "moc_gemv_bf16": (_int, [_vp, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _vp]),
    "moc_gemv_rmsnorm_bf16": (_int, [_vp, _i64, _i64, _vp, ctypes.c_float, _vp, _i64, _vp, _i64, _i64,
                                     _i64, _vp, _i64, _vp]),
    "moc_global_after_gate_residual_bf16": (_int, [_vp, _vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64,
                                                   _vp, _vp, _vp, _vp, _i64, _vp]),
    "moc_global_after_gate_noalloc_bf16": (_int, [_vp, _vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64,
                                                  _vp, _vp, _vp, _vp]),
    "moc_selected_up_silu_bf16": (_int, [_vp, _i64, _i64, _vp, _vp, _int, _i64, _vp, _i64, _vp, _vp]),
    "moc_selected_down_workspace_size": (_i64, [_i64, _i64, _i64]),
    "moc_selected_down_bf16": (_int, [_vp, _vp, _int, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _vp,
                                      _i64, _vp]),
    "moc_global_after_gate_workspace_size": (_i64, [_i64, _i64, _i64, _i64]),
    "moc_global_decode_workspace_size": (_i64, [_i64, _i64, _i64, _i64]),
    "moc_global_decode_bf16": (_int, [_vp, _i64, _i64, _vp, _vp, _i64, _vp, _i64, _i64, _vp, _vp, _vp,
                                      _i64, _vp]),
    "moc_global_decode_rmsnorm_residual_bf16": (_int, [_vp, _i64, _i64, _vp, ctypes.c_float, _vp, _vp,
                                                       _i64, _vp, _i64, _i64, _vp, _vp, _vp, _i64, _vp]),
    "moc_global_after_gate_bf16": (_int, [_vp, _vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _vp, _vp,
                                          _vp, _i64, _vp]),
    "moc_grouped_top2_up_silu_bf16": (_int, [_vp, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _vp]),
    "moc_moc28_decode_workspace_size": (_i64, [_i64, _i64, _i64]),
    "moc_moc28_decode_bf16": (_int, [_vp, _i64, _i64, _vp, ctypes.c_float, _vp, _vp, _i64, _vp, _i64, _vp,
                                     _vp, _vp, _vp, _i64, _vp]),
    "moc_grouped_top2_up_silu_rmsnorm_bf16": (_int, [_vp, _i64, _i64, _vp, ctypes.c_float, _vp, _vp,
                                                     _i64, _vp, _vp, _vp]),
    "moc_selected_grouped_down_residual_bf16": (_int, [_vp, _vp, _i64, _i64, _vp, _i64, _i64, _i64,
                                                       _vp, _vp, _vp, _i64, _vp]),
    "moc_selected_grouped_down_workspace_size": (_i64, [_i64, _i64, _i64, _i64]),
    "moc_selected_grouped_down_bf16": (_int, [_vp, _vp, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _vp,
                                              _i64, _vp]),
    "moc_pack28_bf16": (_int, [_vp, _vp, _i64, _i64, _vp, _i64, _vp, _i64, _vp, _vp]),
    "moc_grouped_top2_up_silu_packed_bf16": (_int, [_vp, _i64, _i64, _vp, _vp, _i64, _vp, _i64, _vp,
                                                    _i64, _vp]),
    "moc_sparse28_down_workspace_size": (_i64, [_i64, _i64, _i64]),
    "moc_sparse28_down_bf16": (_int, [_vp, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _int, _i64, _vp,
                                      _i64, _vp, _i64, _vp]),
}

_LIB = None
_LOCK = threading.Lock()


class NativeLibraryMissing(RuntimeError):
    pass


def header_function_names() -> list[str]:
    """Function names declared in include/moc_amd.h (the ABI contract)."""
    text = HEADER_PATH.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?[a-z0-9_]+\s*\*?\s*(moc_[a-z0-9_]+)\s*\(", text, flags=re.M)


def load():
    """Load libmoc_amd.so once and bind every signature; raises if absent."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is not None:
            return _LIB
        if not LIB_PATH.exists():
            raise NativeLibraryMissing(
                f"{LIB_PATH} is not built; run `python -m moc_amd.build` (hipcc, gfx950)")
        lib = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = lib
    return _LIB


def last_error() -> str:
    msg = load().moc_last_error()
    return msg.decode() if msg else ""


def check(status: int, what: str) -> None:
    if status == MOC_OK:
        return
    msg = last_error() or what
    if status == MOC_ERR_INVALID:
        raise ValueError(msg)
    raise RuntimeError(f"{what}: {msg}")


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args), name)


def query(name: str, *args) -> int:
    return int(getattr(load(), name)(*args))


def stream_of(t: torch.Tensor) -> int:
    """HIP stream torch currently uses on t's device (as an integer handle)."""
    return torch._C._cuda_getCurrentRawStream(t.get_device())


def require_device(*tensors: torch.Tensor) -> None:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("MoC HIP kernels require ROCm device tensors")
        d = t.get_device()
        if dev is None:
            dev = d
        elif d != dev:
            devs = sorted({str(x.device) for x in tensors if x is not None})
            raise ValueError(f"MoC HIP kernels need all tensors on one device, got {devs}")


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return MOC_BF16
    if dt == torch.float32:
        return MOC_F32
    raise ValueError(f"MoC HIP kernels support bfloat16 and float32, got {dt}")


def idx_code(dt: torch.dtype) -> int:
    if dt == torch.int16:
        return MOC_I16
    if dt == torch.int32:
        return MOC_I32
    if dt == torch.int64:
        return MOC_I64
    raise ValueError(f"index dtype must be int16/int32/int64, got {dt}")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
