"""Put the MI355X kernels behind QuantumDLBlocks' own import paths.

The reference's Born layers bind the kernel at import time,
``from ..kernels import flash_born_attention`` (Vengo/QuantumDLBlocks
src/qdlblocks/layers/attention.py:20; the call is at attention.py:704-713),
and the package re-exports it (src/qdlblocks/kernels/__init__.py:3-10,
src/qdlblocks/__init__.py:48).  ``install()`` rebinds those names to this
package's objects, and registers ``qdlblocks.kernels.flash_born_triton`` (the
module name the reference's documentation uses) as an alias of
``quantumdlblocks_amd.kernels.flash_born_triton``.  Call it once, before the
models run; modules imported later pick the new objects up through the
patched ``qdlblocks.kernels``.
"""

from __future__ import annotations

import importlib
import sys
from types import ModuleType

from .kernels import flash_born_triton as _ours

# Names the reference's flash-Born module exports for this path
# (src/qdlblocks/kernels/flash_born.py:20-75, 621-690, 1064-1341).
PATCHED_NAMES = (
    "flash_born_attention",
    "_run_triton_flash_born",
    "_FlashBornAttentionFn",
    "flash_purified_born_attention",
    "_run_triton_flash_purified_born",
    "_FlashPurifiedBornAttentionFn",
    "_apply_window_and_doc_mask",
    "HAS_TRITON",
    "IS_HIP",
    "get_flash_born_launch_meta",
    "get_rdna4_autotune_configs",
)

# Modules that hold their own binding of those names.
TARGET_MODULES = (
    "qdlblocks.kernels.flash_born",
    "qdlblocks.kernels",
    "qdlblocks.layers.attention",
    "qdlblocks",
)


def install(import_targets: bool = True) -> list[str]:
    """Rebind the flash-Born names in QuantumDLBlocks' modules; return the
    names of the modules patched.  With ``import_targets`` the target
    modules are imported first (skipped silently when absent)."""
    patched = []
    sys.modules["qdlblocks.kernels.flash_born_triton"] = _ours
    for name in TARGET_MODULES:
        mod = sys.modules.get(name)
        if mod is None and import_targets:
            try:
                mod = importlib.import_module(name)
            except ImportError:
                mod = None
        if not isinstance(mod, ModuleType):
            continue
        for attr in PATCHED_NAMES:
            if hasattr(mod, attr) or name == "qdlblocks.kernels.flash_born":
                setattr(mod, attr, getattr(_ours, attr))
        patched.append(name)
    parent = sys.modules.get("qdlblocks.kernels")
    if isinstance(parent, ModuleType):
        parent.flash_born_triton = _ours
    return patched
