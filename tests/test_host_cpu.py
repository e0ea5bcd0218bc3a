"""CPU-only checks of the boundary and host logic (no GPU compute).

* libmoc_amd.so loads and exports every function include/moc_amd.h declares;
* argument validation returns MOC_ERR_INVALID with the reference's messages
  before any device work (these calls never launch a kernel);
* the Python module API mirrors the reference (names, attributes, errors,
  state_dict keys) and the MoC path refuses CPU tensors instead of falling
  back to a CPU implementation;
* the product package never imports the oracle.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

import moc_amd
from moc_amd import _native as N
from moc_amd import build_ffn, build_model, PRESETS
from moc_amd.ffn import MoCSwiGLUFFN, _moc_2_8_effective_k
from moc_amd.inference.inference_ffn import InferenceMoCSwiGLUFFN

ROOT = Path(__file__).resolve().parent.parent


@pytest.fixture(scope="module")
def lib():
    if not N.LIB_PATH.exists():
        pytest.fail("libmoc_amd.so is not built (python -m moc_amd.build)")
    return N.load()


def test_library_exports_every_header_symbol(lib):
    names = N.header_function_names()
    assert len(names) >= 20
    assert set(names) == set(N.SIGNATURES), set(names) ^ set(N.SIGNATURES)
    for name in names:
        assert getattr(lib, name) is not None
    assert lib.moc_abi_version() == 3


def test_validation_errors_without_device_work(lib):
    # k > inter
    rc = lib.moc_topk_rows(N.MOC_BF16, None, 4, 100, 100, 101, 0, None, None, N.MOC_I64, None, 0, None)
    assert rc == N.MOC_ERR_INVALID
    assert "invalid k" in N.last_error()
    # int16 indices cannot address 40000 channels (moc/ffn.py:37-40)
    rc = lib.moc_topk_rows(N.MOC_BF16, None, 4, 16000, 16000, 10, 0, None, None, N.MOC_I16, None, 0, None)
    assert rc == N.MOC_OK or rc == N.MOC_ERR_INVALID  # null pointer or ok-range; no launch either way
    rc = lib.moc_select_2of8(N.MOC_BF16, None, 2, 40000, 40000, None, None, N.MOC_I16, None)
    assert rc == N.MOC_ERR_INVALID and "int16" in N.last_error()
    # 2:8 grouped kernel needs I % 8 == 0 (triton_grouped_moc_ops.py:46-47)
    rc = lib.moc_grouped_top2_up_silu_bf16(None, 1, 64, None, None, 5461, None, None, None)
    assert rc == N.MOC_ERR_INVALID and "divisible by 8" in N.last_error()
    # GEMM leading dimension must keep 16-byte rows
    rc = lib.moc_gemm(N.MOC_BF16, 4, 4, 4, ctypes.c_void_p(16), 5, 1, ctypes.c_void_p(16), 1, 8,
                      0, None, 0, 0, None, 0, 0, ctypes.c_void_p(16), 4, N.MOC_BF16, None)
    assert rc == N.MOC_ERR_INVALID and "multiples of 8" in N.last_error()
    # rows == 0 is a no-op
    assert lib.moc_topk_rows(N.MOC_F32, None, 0, 10, 10, 3, 0, None, None, N.MOC_I32, None, 0, None) == N.MOC_OK
    assert lib.moc_moc28_effective_k(5461) == 1366
    # the 2:8 decode layer: whole groups of 8, the fused norm up to 4 tokens
    rc = lib.moc_moc28_decode_bf16(None, 1, 2048, None, 1e-6, None, None, 5461, None, 2048, None, None, None,
                                   None, 0, None)
    assert rc == N.MOC_ERR_INVALID and "multiple of 8" in N.last_error()
    rc = lib.moc_moc28_decode_bf16(None, 5, 2048, ctypes.c_void_p(16), 1e-6, None, None, 5464, None, 2048, None,
                                   None, None, None, 0, None)
    assert rc == N.MOC_ERR_INVALID and "nb <= 4" in N.last_error()
    assert lib.moc_moc28_decode_bf16(None, 0, 2048, None, 1e-6, None, None, 5464, None, 2048, None, None, None,
                                     None, 0, None) == N.MOC_OK
    assert lib.moc_moc28_decode_workspace_size(16, 5464, 2048) > 0
    assert lib.moc_selected_down_workspace_size(1, 1024, 2048) > 0


def test_module_api_mirrors_reference():
    ffn = build_ffn(64, 176, "moc_gcp", k=32)
    assert isinstance(ffn, MoCSwiGLUFFN)
    assert ffn.mode == "moc_gcp_triton_aux" and ffn.index_save_dtype == torch.int16
    assert ffn.k == ffn.k_effective == ffn.requested_k == 32
    assert set(ffn.state_dict()) == {"gate_proj.weight", "up_proj.weight", "down_proj.weight"}
    assert ffn.gate_proj.weight.shape == (176, 64) and ffn.down_proj.weight.shape == (64, 176)
    f28 = build_ffn(2048, 5461, "moc_2_8", k=999)
    assert f28.k_effective == 1366 == _moc_2_8_effective_k(5461) and f28.requested_k == 999
    with pytest.raises(ValueError, match="requires `k`"):
        build_ffn(64, 176, "moc")
    with pytest.raises(ValueError, match="Unknown ffn_type"):
        build_ffn(64, 176, "nope")
    with pytest.raises(ValueError, match="Unknown mode"):
        MoCSwiGLUFFN(64, 176, 32, mode="bad")
    assert type(build_ffn(64, 176, "dense")).__name__ == "StandardSwiGLUFFN"


def test_moc_path_refuses_cpu_tensors():
    ffn = MoCSwiGLUFFN(64, 176, 32, mode="moc_gcp")
    with pytest.raises(ValueError, match="ROCm device"):
        ffn(torch.randn(3, 64))
    ffn = build_ffn(64, 176, "moc", k=32)
    with pytest.raises(ValueError):
        ffn(torch.randn(3, 64))


def test_inference_module_validation():
    with pytest.raises(ValueError, match=r"k=0 must be in"):
        InferenceMoCSwiGLUFFN(64, 128, 0)
    with pytest.raises(ValueError, match="set together"):
        InferenceMoCSwiGLUFFN(64, 128, 32, grouped_a=2)
    with pytest.raises(ValueError, match="grouped MoC requires"):
        InferenceMoCSwiGLUFFN(64, 128, 31, grouped_a=2, grouped_b=8)
    m = InferenceMoCSwiGLUFFN(64, 128, 32, grouped_a=2, grouped_b=8)
    assert m.config.grouped and m.config.k == 32
    x = torch.randn(2, 1, 64)
    x2, shp = m._flatten_decode_input(x)
    assert x2.shape == (2, 64) and m._restore_output_shape(x2, shp).shape == (2, 1, 64)
    with pytest.raises(ValueError, match="expected decode shape"):
        m._flatten_decode_input(torch.randn(2, 3, 64))


def test_build_model_and_presets():
    cfg = moc_amd.MoCConfig(hidden_size=64, intermediate_size=176, num_hidden_layers=2,
                            num_attention_heads=4, vocab_size=100, k=32)
    model = build_model(cfg, ffn_type="moc_gcp")
    assert model.blocks[0].ffn.mode == "moc_gcp_triton_aux"
    keys = set(model.state_dict())
    assert "blocks.1.ffn.down_proj.weight" in keys and "tok_emb.weight" in keys
    with pytest.raises(ValueError, match="ffn_type must be"):
        build_model(cfg, ffn_type="bad")
    assert PRESETS["1b"].intermediate_size == 5461 and PRESETS["350m"].k == 512
    assert moc_amd.count_parameters(PRESETS["60m"]) > 0


def test_custom_ops_registered_with_reference_names():
    from moc_amd import ops
    ops.register()
    for name in ("optimized_global_topk_bf16", "optimized_global_selected_up_silu_bf16",
                 "optimized_global_selected_down_bf16", "optimized_global_after_gate_bf16"):
        assert hasattr(torch.ops.moc_native, name)
    for name in ("optimized_global_topk_bf16", "fused_grouped_top2_up_silu", "selected_grouped_down"):
        assert hasattr(torch.ops.moc, name)
    with pytest.raises(Exception):
        torch.ops.moc_native.optimized_global_topk_bf16(torch.randn(2, 8).bfloat16(), 3)


def test_reference_import_path_resolves_to_this_package():
    """Callers written against the reference's `moc` package import unchanged
    (examples/quickstart.py:6, benchmark_training_latency.py:17,
    benchmark_ffn_latency.py) and get this package's objects."""
    import importlib

    import moc
    from moc import PRESETS as P2, build_model as bm2
    from moc.ffn import build_ffn as bf2, MoCSwiGLUFFN as M2
    from moc.inference.inference_ffn import InferenceMoCSwiGLUFFN as I2
    from moc.inference.optimized_global_moc_ops import load_optimized_global_moc_extension
    import moc.inference.triton_grouped_moc_ops as tg
    import moc.inference.triton_fused_ffn_kernels as tf
    import moc_amd.ffn
    assert P2 is PRESETS and bm2 is build_model and bf2 is build_ffn and M2 is MoCSwiGLUFFN
    assert I2 is InferenceMoCSwiGLUFFN
    assert moc.ffn is moc_amd.ffn and moc.ffn.__spec__.name == "moc_amd.ffn"
    assert tg.__name__ == "moc_amd.inference.grouped_moc_ops"
    assert hasattr(tf, "fused_gate_top2of8_selected_up_silu_into")
    assert callable(load_optimized_global_moc_extension)
    with pytest.raises(ModuleNotFoundError):
        importlib.import_module("moc.no_such_module")


def test_extension_object_checks_like_the_reference(lib):
    """load_optimized_global_moc_extension() returns an object with the
    reference pybind methods (optimized_global_moc_ext.cpp:78-86), whose
    argument checks raise the reference's messages before any device work."""
    from moc_amd.inference.optimized_global_moc_ops import load_optimized_global_moc_extension
    ext = load_optimized_global_moc_extension()
    assert ext is load_optimized_global_moc_extension()
    for name in ("cub_topk_bf16_512x11", "selected_up_silu_bf16", "selected_down_bf16_h32_k16",
                 "optimized_global_after_gate_bf16"):
        assert callable(getattr(ext, name))
    with pytest.raises(RuntimeError, match="scores must be CUDA"):
        ext.cub_topk_bf16_512x11(torch.randn(2, 64).bfloat16(), 3)
    with pytest.raises(RuntimeError, match="all tensors must be CUDA"):
        ext.selected_down_bf16_h32_k16(torch.zeros(1, 4).bfloat16(), torch.zeros(1, 4, dtype=torch.long),
                                       torch.zeros(8, 64).bfloat16())


def test_value_order_is_stable_descending():
    """The moc_native Top-K op's order: value descending, equal values by
    ascending channel (the reference's stable radix sort)."""
    from moc_amd.ops import value_order
    vals = torch.tensor([[1.0, 3.0, 3.0, -0.0, 0.0, 2.0]]).bfloat16()
    idx = torch.tensor([[0, 2, 5, 7, 8, 9]])
    v, i = value_order(vals, idx)
    assert i.tolist() == [[2, 5, 9, 0, 7, 8]]
    assert v.float().tolist() == [[3.0, 3.0, 2.0, 1.0, -0.0, 0.0]]
    # the two zeros rank equal in either order; NaN ranks above +inf
    z = torch.tensor([[0.0, -0.0, float("inf"), float("nan")], [-0.0, 0.0, 1.0, -1.0]]).bfloat16()
    _, i = value_order(z, torch.tensor([[3, 4, 5, 6], [3, 4, 5, 6]]))
    assert i.tolist() == [[6, 5, 3, 4], [5, 3, 4, 6]]


def test_product_never_imports_oracle():
    for path in (ROOT / "moc_amd").rglob("*.py"):
        text = path.read_text()
        assert not re.search(r"^\s*(from|import)\s+oracle", text, flags=re.M), path
