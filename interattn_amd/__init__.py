"""MI355X-native (gfx950) condition-block sparse decode attention.

The compute path is the HIP library ``libinterattn_amd.so`` (C ABI in
``include/interattn_amd.h``); this package is its torch-facing host side.
"""

from ._native import NativeLibraryMissing, NativeError  # noqa: F401
from .ops import (  # noqa: F401
    append_kv,
    build_block_summaries,
    paged_decode,
    paged_kv,
    select_blocks_topk,
    sequence_scales,
    set_wait_limit,
    sparse_paged_decode,
    sparse_topk_decode,
    update_block_summaries,
    wait_fallbacks,
    workspace_tensor,
)

__version__ = "0.1.0"
