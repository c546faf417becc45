"""MI355X (gfx950) implementation of jaxmodules' masked attention hot path.

``masked_attention_via_map`` and the ``block_mask`` machinery, forward and
backward, on hand-written HIP kernels behind the C ABI in ``include/mattn.h``.
"""
from . import block_mask, blockmap, masks
from .attention import (default_kernel, flex_attention, flex_attention_slow, kernel_scale,
                        masked_attention_via_map, threshold_kernel, use_custom_einsum)
from .block_mask import BlockMask, create_block_mask

__version__ = "0.1"
__all__ = ["masked_attention_via_map", "flex_attention", "flex_attention_slow", "default_kernel",
           "threshold_kernel", "use_custom_einsum", "kernel_scale", "blockmap", "masks",
           "block_mask", "BlockMask", "create_block_mask"]
