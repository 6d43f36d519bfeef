"""Module aliases so that code importing SemBlend's kernel modules gets this package.

``install()`` registers ``semblend_core.{triton_kernels,rope_correction,partial_attention}``
and ``synapse_kv_connector.{triton_kernels,rope_correction,partial_attention}`` (the re-export
paths of synapse_kv_connector/{triton_kernels,rope_correction,partial_attention}.py) in
``sys.modules``. Parent packages that are not importable are created as empty namespace
modules; an importable parent is left as it is and only the three submodules are replaced.
"""

from __future__ import annotations

import importlib
import importlib.util
import sys
import types

from . import partial_attention, rope_correction, triton_kernels

_SUBMODULES = {
    "triton_kernels": triton_kernels,
    "rope_correction": rope_correction,
    "partial_attention": partial_attention,
}
_PARENTS = ("semblend_core", "synapse_kv_connector")


def install() -> list[str]:
    """Register the aliases; returns the module names that now point at this package."""
    names = []
    for parent in _PARENTS:
        if parent not in sys.modules:
            if importlib.util.find_spec(parent) is not None:
                importlib.import_module(parent)
            else:
                pkg = types.ModuleType(parent)
                pkg.__path__ = []  # namespace-like package with no files
                sys.modules[parent] = pkg
        pkg = sys.modules[parent]
        for sub, mod in _SUBMODULES.items():
            name = f"{parent}.{sub}"
            sys.modules[name] = mod
            setattr(pkg, sub, mod)
            names.append(name)
    return names
