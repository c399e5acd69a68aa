"""MI355X-native selective scan for Vision Mamba.

Public surface mirrors the reference package's ``__init__`` (reference
mlx_vision_mamba/__init__.py:7-33): the scan functions under their reference
names, the Mamba blocks with a ``scan_mode`` that is passed down, and
VisionMamba / PatchEmbed.  Every scan runs the HIP kernels of
``libmvm_scan.so`` (build with ``python -m mlx_vision_mamba_amd.build``).
"""

from .scan import (  # noqa: F401
    SCAN_MODES,
    get_scan_fn,
    selective_scan,
    selective_scan_chunked,
    selective_scan_directions,
    selective_scan_metal,
    selective_scan_metal_fused,
    selective_scan_metal_trainable,
    selective_scan_parallel,
    selective_scan_sequential,
)

from .mamba_block import (  # noqa: F401
    BidirectionalMambaBlock,
    MambaBlock,
    MultiDirectionalMambaBlock,
    ResidualMambaBlock,
)
from .vision_mamba import PatchEmbed4D, VisionMamba  # noqa: F401
from .vit import PatchEmbed, PatchEmbed3D  # noqa: F401

__version__ = "0.1.0"
__all__ = [
    "MambaBlock",
    "BidirectionalMambaBlock",
    "MultiDirectionalMambaBlock",
    "ResidualMambaBlock",
    "VisionMamba",
    "PatchEmbed",
    "PatchEmbed3D",
    "PatchEmbed4D",
    "selective_scan",
    "selective_scan_chunked",
    "selective_scan_parallel",
    "selective_scan_sequential",
    "selective_scan_directions",
    "selective_scan_metal",
    "selective_scan_metal_trainable",
    "selective_scan_metal_fused",
    "SCAN_MODES",
    "get_scan_fn",
]
