"""ctypes binding of ``libinterattn_amd.so`` (the C ABI in ``include/interattn_amd.h``).

The library is the only compute path: there is no Python or CPU fallback.  If the
shared object is missing, every entry point raises ``NativeLibraryMissing`` with
the build command.
"""

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libinterattn_amd.so")

IA_F32 = 0
IA_BF16 = 1
IA_FP8_E4M3 = 2

IA_SCORE_MEAN_KEY = 0
IA_SCORE_QUEST = 1

IA_NOALLOC_SCRATCH_BYTES = 16 << 20  # library-held scratch of ia_sparse_topk_decode_noalloc

IA_OK = 0
IA_ERR_INVALID = 1
IA_ERR_UNSUPPORTED = 2
IA_ERR_WORKSPACE = 3
IA_ERR_LAUNCH = 4


class NativeLibraryMissing(RuntimeError):
    pass


class NativeError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"interattn_amd error {code}: {msg}")
        self.code = code


class PagedKV(ctypes.Structure):
    _fields_ = [
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("n_pages", ctypes.c_int64),
        ("k_page_stride", ctypes.c_int64),
        ("k_head_stride", ctypes.c_int64),
        ("k_token_stride", ctypes.c_int64),
        ("v_page_stride", ctypes.c_int64),
        ("v_head_stride", ctypes.c_int64),
        ("v_token_stride", ctypes.c_int64),
        ("block_table", ctypes.c_void_p),
        ("bt_stride", ctypes.c_int64),
        ("bt_cols", ctypes.c_int64),
        ("k_scale", ctypes.c_void_p),
        ("v_scale", ctypes.c_void_p),
        ("scale_page_stride", ctypes.c_int64),
        ("seq_scale", ctypes.c_void_p),
        ("seq_scale_b_stride", ctypes.c_int64),
        ("seq_scale_h_stride", ctypes.c_int64),
    ]


class DecodeShape(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32),
        ("n_q_heads", ctypes.c_int32),
        ("n_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("q_batch_stride", ctypes.c_int64),
        ("q_row_stride", ctypes.c_int64),
        ("q_dtype", ctypes.c_int32),
    ]


class BlockSummaries(ctypes.Structure):
    _fields_ = [
        ("k_bar", ctypes.c_void_p),
        ("k_max", ctypes.c_void_p),
        ("k_min", ctypes.c_void_p),
        ("v_bar", ctypes.c_void_p),
        ("k_bar_dtype", ctypes.c_int32),
        ("bounds_dtype", ctypes.c_int32),
        ("v_bar_dtype", ctypes.c_int32),
        ("v_norm_max", ctypes.c_void_p),
        ("v_norm_all", ctypes.c_void_p),
        ("counts", ctypes.c_void_p),
        ("nb", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("bounds_packed", ctypes.c_int32),
    ]


class BlockKeys(ctypes.Structure):
    _fields_ = [
        ("score", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("k_bar", ctypes.c_void_p),
        ("k_max", ctypes.c_void_p),
        ("k_min", ctypes.c_void_p),
        ("batch_stride", ctypes.c_int64),
        ("head_stride", ctypes.c_int64),
    ]


class SuffixKV(ctypes.Structure):
    _fields_ = [
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("k_batch_stride", ctypes.c_int64),
        ("k_head_stride", ctypes.c_int64),
        ("k_token_stride", ctypes.c_int64),
        ("v_batch_stride", ctypes.c_int64),
        ("v_head_stride", ctypes.c_int64),
        ("v_token_stride", ctypes.c_int64),
        ("len", ctypes.c_void_p),
        ("len_stride", ctypes.c_int32),
        ("cap", ctypes.c_int32),
    ]


_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t
_F = ctypes.c_float

# name -> (restype, argtypes); every symbol declared in include/interattn_amd.h
SIGNATURES = {
    "ia_last_error": (ctypes.c_char_p, []),
    "ia_version": (ctypes.c_int, []),
    "ia_build_block_summaries": (
        ctypes.c_int,
        [ctypes.POINTER(PagedKV), _P, _I32, _I32, _I32, _I32, _I32, _P, _I32, _P, _I32, _P, _P, _I32, _P, _P,
         _P, _P],
    ),
    "ia_update_block_summaries": (
        ctypes.c_int,
        [ctypes.POINTER(PagedKV), _P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _P, _I32, _P, _I32, _P, _P, _I32, _P,
         _P, _P, _P],
    ),
    "ia_append_kv": (ctypes.c_int, [ctypes.POINTER(PagedKV), _P, _P, _I64, _I64, _P, _I32, _I32, _I32, _P]),
    "ia_sparse_topk_decode_workspace_size": (_SZ, [_I32, _I32, _I32, _I32, _I32, _I32, _I32]),
    "ia_sparse_topk_decode": (
        ctypes.c_int,
        [ctypes.POINTER(DecodeShape), _P, ctypes.POINTER(PagedKV), _P, ctypes.POINTER(BlockKeys), _I32, _I32, _I32,
         _P, _I32, _I32, _I32, _I32, _F, _P, _I32, _P, _P, _P, _SZ, _P],
    ),
    "ia_sparse_topk_decode_noalloc": (
        ctypes.c_int,
        [ctypes.POINTER(DecodeShape), _P, ctypes.POINTER(PagedKV), _P, ctypes.POINTER(BlockKeys), _I32, _I32, _I32,
         _P, _I32, _I32, _I32, _I32, _F, _P, _I32, _P, _P, _P],
    ),
    "ia_set_wait_limit": (_I64, [_I64]),
    "ia_wait_fallbacks": (_I64, [_I32]),
    "ia_select_topk_workspace_size": (_SZ, [_I32, _I32, _I32]),
    "ia_select_topk": (
        ctypes.c_int,
        [ctypes.POINTER(DecodeShape), _P, ctypes.POINTER(BlockKeys), _P, _I32, _I32, _I32, _P, _I32, _I32, _I32,
         _P, _I32, _P, _P, _P, _SZ, _P],
    ),
    "ia_paged_decode_workspace_size": (_SZ, [_I32, _I32, _I32, _I32, _I32]),
    "ia_sparse_paged_decode": (
        ctypes.c_int,
        [ctypes.POINTER(DecodeShape), _P, ctypes.POINTER(PagedKV), _P, _I32, _P, _I32, _P, _F, _P, _I32, _P,
         _SZ, _P],
    ),
    "ia_paged_decode": (
        ctypes.c_int,
        [ctypes.POINTER(DecodeShape), _P, ctypes.POINTER(PagedKV), _P, _I32, _F, _P, _I32, _P, _SZ, _P],
    ),
    "ia_condition_selection_stats": (
        ctypes.c_int, [ctypes.POINTER(DecodeShape), _P, ctypes.POINTER(BlockSummaries), _I32, _P, _P, _P, _P, _P]),
    "ia_condition_select": (
        ctypes.c_int,
        [ctypes.POINTER(DecodeShape), ctypes.POINTER(BlockSummaries), _P, _P, _P, _F, _I32, _P, _P, _P]),
    "ia_condition_workspace_size": (_SZ, [_I32, _I32, _I32, _I32, _I32, _I32]),
    "ia_condition_decode": (
        ctypes.c_int,
        [ctypes.POINTER(DecodeShape), _P, ctypes.POINTER(BlockSummaries), ctypes.POINTER(PagedKV),
         ctypes.POINTER(SuffixKV), _F, _I32, _P, _F, _P, _I32, _P, _SZ, _P]),
    "ia_condition_decode_fused_workspace_size": (_SZ, [_I32, _I32, _I32, _I32]),
    "ia_condition_decode_fused_items": (
        ctypes.c_int32, [ctypes.POINTER(DecodeShape), ctypes.POINTER(BlockSummaries), _I32, _I32]),
    "ia_condition_decode_fused": (
        ctypes.c_int,
        [ctypes.POINTER(DecodeShape), _P, ctypes.POINTER(BlockSummaries), ctypes.POINTER(PagedKV),
         ctypes.POINTER(SuffixKV), _F, _I32, _P, _F, _P, _I32, _P, _SZ, _P]),
    "ia_fixed_mask_decode_fused": (
        ctypes.c_int,
        [ctypes.POINTER(DecodeShape), _P, ctypes.POINTER(BlockSummaries), _P, ctypes.POINTER(PagedKV),
         ctypes.POINTER(SuffixKV), _F, _P, _I32, _P, _SZ, _P]),
    "ia_fixed_mask_decode": (
        ctypes.c_int,
        [ctypes.POINTER(DecodeShape), _P, ctypes.POINTER(BlockSummaries), _P, ctypes.POINTER(PagedKV),
         ctypes.POINTER(SuffixKV), _F, _P, _I32, _P, _SZ, _P]),
    "ia_topk_block_mask": (ctypes.c_int, [_P, _P, _I32, _I32, _I32, _I32, _P, _P]),
    "ia_sparse_max_items": (_I32, [_I32, _I32, _I32]),
    "ia_dense_max_items": (_I32, [_I32, _I32, _I32]),
}

_lib = None


def lib():
    """Load the library once; raise loudly when it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise NativeLibraryMissing(
                f"{LIB_PATH} is missing; build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                "or `python interattn_amd/build.py`")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(rc):
    if rc != IA_OK:
        msg = lib().ia_last_error().decode("utf-8", "replace")
        if rc in (IA_ERR_INVALID, IA_ERR_UNSUPPORTED, IA_ERR_WORKSPACE):
            raise ValueError(msg)
        raise NativeError(rc, msg)
