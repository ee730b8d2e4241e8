"""The module name the reference's documentation gives the flash-Born kernel
(``qdlblocks.kernels.flash_born_triton``, README.md:10 and
docs/BUILDING_BLOCKS.md:17 of Vengo/QuantumDLBlocks).  Same objects as
``quantumdlblocks_amd.kernels.flash_born``."""

from .flash_born import (  # noqa: F401
    HAS_HIP_KERNELS,
    HAS_TRITON,
    IS_HIP,
    _apply_window_and_doc_mask,
    _FlashBornAttentionFn,
    _FlashPurifiedBornAttentionFn,
    _run_hip_flash_born,
    _run_hip_flash_purified_born,
    _run_triton_flash_born,
    _run_triton_flash_purified_born,
    flash_born_attention,
    flash_purified_born_attention,
    get_flash_born_launch_meta,
    get_mi355x_launch_meta,
    get_rdna4_autotune_configs,
)

__all__ = [
    "HAS_HIP_KERNELS",
    "HAS_TRITON",
    "IS_HIP",
    "flash_born_attention",
    "flash_purified_born_attention",
    "get_flash_born_launch_meta",
    "get_mi355x_launch_meta",
    "get_rdna4_autotune_configs",
]
