"""GPU kernels of quantumdlblocks_amd (mirrors ``qdlblocks.kernels`` for the
flash-Born path; reference src/qdlblocks/kernels/__init__.py:3-10)."""

from .flash_born import (
    HAS_HIP_KERNELS,
    HAS_TRITON,
    IS_HIP,
    flash_born_attention,
    flash_purified_born_attention,
    get_flash_born_launch_meta,
    get_mi355x_launch_meta,
    get_rdna4_autotune_configs,
)
from .qk_prologue import flash_born_attention_qk_prologue, fused_qk_rope_l2_normalize

__all__ = [
    "HAS_HIP_KERNELS",
    "HAS_TRITON",
    "IS_HIP",
    "flash_born_attention",
    "flash_born_attention_qk_prologue",
    "flash_purified_born_attention",
    "fused_qk_rope_l2_normalize",
    "get_flash_born_launch_meta",
    "get_mi355x_launch_meta",
    "get_rdna4_autotune_configs",
]
