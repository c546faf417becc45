"""MI355X (gfx950) implementation of jaxmodules' masked attention hot path.

``masked_attention_via_map`` and the ``block_mask`` machinery, forward and
backward, on hand-written HIP kernels behind the C ABI in ``include/mattn.h``.
"""
from . import blockmap
from .attention import default_kernel, masked_attention_via_map, threshold_kernel

__version__ = "0.1"
__all__ = ["masked_attention_via_map", "default_kernel", "threshold_kernel", "blockmap"]
