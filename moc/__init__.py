"""The reference's import path (`moc`, xiaohuangji/MoC) served by moc_amd.

Code written against the reference imports unchanged:

    from moc import PRESETS, build_model                         # moc/__init__.py
    from moc.ffn import build_ffn                                # moc/ffn.py
    from moc.inference.inference_ffn import InferenceMoCSwiGLUFFN
    from moc.inference.optimized_global_moc_ops import load_optimized_global_moc_extension
    import moc.inference.triton_grouped_moc_ops                  # registers moc:: ops

Every `moc.<name>` module is the module object `moc_amd.<name>` itself (the
same classes, functions and module state), so isinstance checks, op
registration and caches are shared whichever path imported them.  The
reference's Triton-named inference modules resolve to the gfx950 modules that
replace them: `moc.inference.triton_grouped_moc_ops` ->
`moc_amd.inference.grouped_moc_ops`, `moc.inference.triton_fused_ffn_kernels`
-> `moc_amd.inference.fused_ffn_kernels`.
"""
from __future__ import annotations

import importlib
import importlib.abc
import importlib.util
import sys

from moc_amd import (  # noqa: F401  (the reference's top-level exports)
    PRESETS,
    LLaMAModel,
    MoCConfig,
    MoCSwiGLUFFN,
    StandardSwiGLUFFN,
    build_ffn,
    build_model,
    count_parameters,
    get_config,
)

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

_PREFIX = __name__ + "."
_TARGET = "moc_amd."
# reference module name (below `moc.`) -> moc_amd module name where they differ
_RENAMED = {
    "inference.triton_grouped_moc_ops": "inference.grouped_moc_ops",
    "inference.triton_fused_ffn_kernels": "inference.fused_ffn_kernels",
}


class _AliasImporter(importlib.abc.MetaPathFinder, importlib.abc.Loader):
    """Resolves `moc.<name>` to the already-importable `moc_amd.<name>`."""

    def __init__(self):
        self._own_spec: dict = {}

    @staticmethod
    def _target(fullname: str) -> str | None:
        if not fullname.startswith(_PREFIX):
            return None
        rel = fullname[len(_PREFIX):]
        return _TARGET + _RENAMED.get(rel, rel)

    def find_spec(self, fullname, path=None, target=None):
        name = self._target(fullname)
        if name is None or importlib.util.find_spec(name) is None:
            return None
        is_pkg = importlib.util.find_spec(name).submodule_search_locations is not None
        return importlib.util.spec_from_loader(fullname, self, is_package=is_pkg)

    def create_module(self, spec):
        module = importlib.import_module(self._target(spec.name))
        self._own_spec[id(module)] = module.__spec__
        return module

    def exec_module(self, module):
        # the import machinery re-labels the module's __spec__ with the alias;
        # give it back its own (it was executed already, under its own name)
        own = self._own_spec.pop(id(module), None)
        if own is not None:
            module.__spec__ = own


if not any(isinstance(f, _AliasImporter) for f in sys.meta_path):
    sys.meta_path.insert(0, _AliasImporter())
