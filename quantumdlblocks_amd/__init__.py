"""quantumdlblocks_amd: MI355X-native (gfx950 HIP) flash-Born attention.

Drop-in replacement for QuantumDLBlocks' ``flash_born_attention``
(``qdlblocks.kernels.flash_born`` / ``qdlblocks.kernels.flash_born_triton``).
"""

from .functional import apply_unitary_rope, compute_document_ids, l2_normalize
from .kernels import (
    HAS_HIP_KERNELS,
    HAS_TRITON,
    IS_HIP,
    flash_born_attention,
    flash_born_attention_qk_prologue,
    flash_purified_born_attention,
    fused_qk_rope_l2_normalize,
    get_flash_born_launch_meta,
    get_mi355x_launch_meta,
    get_rdna4_autotune_configs,
)

__version__ = "0.1.0"

__all__ = [
    "HAS_HIP_KERNELS",
    "HAS_TRITON",
    "IS_HIP",
    "apply_unitary_rope",
    "compute_document_ids",
    "flash_born_attention",
    "flash_born_attention_qk_prologue",
    "flash_purified_born_attention",
    "fused_qk_rope_l2_normalize",
    "get_flash_born_launch_meta",
    "get_mi355x_launch_meta",
    "get_rdna4_autotune_configs",
    "l2_normalize",
]
