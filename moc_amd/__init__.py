"""MI355X-native Mixture-of-Channels sparse SwiGLU FFN (API of the `moc` package).

    from moc_amd import PRESETS, build_model, build_ffn

The MoC FFN modes run on hand-written gfx950 HIP kernels (libmoc_amd.so,
built by `python -m moc_amd.build`); importing this package loads no kernels.
"""
from .config import PRESETS, MoCConfig, count_parameters, get_config
from .ffn import MoCSwiGLUFFN, StandardSwiGLUFFN, build_ffn
from .model import LLaMAModel, build_model

__all__ = [
    "MoCConfig",
    "PRESETS",
    "count_parameters",
    "get_config",
    "MoCSwiGLUFFN",
    "StandardSwiGLUFFN",
    "build_ffn",
    "LLaMAModel",
    "build_model",
]
