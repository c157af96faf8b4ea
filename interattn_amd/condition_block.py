"""The reference's condition-block entry points, on the HIP kernels.

Names, signatures, return values and ``ValueError`` contract checks follow
``llama/script/analysis/condition_block_gen/methods/condition_block_triton_impl/core.py``
(``CBT/core.py`` below) and ``CBG/real_attention_benchmark/fixed_mask.py``, so the
reference's decode loop can call these in place of its Triton launches.  Layout
flags that the reference reads from environment variables
(``CONDITION_BLOCK_MIXED_SUMMARIES``, ``..._K_BAR_DTYPE``, ``..._SUMMARY_DTYPE``) are
keyword arguments here.  Everything launches on the current torch stream; scratch
and outputs live in the caller's ``workspace`` dict (``_workspace_empty``,
CBT/core.py:558-570).
"""

import contextlib
import contextvars
import math
import os
from collections import OrderedDict

import torch
import torch.nn.functional as F

from . import _native as N
from .ops import _code, _require_cuda, _scratch, _stream, workspace_tensor

SELECT_CHUNK = 16  # blocks per selection-stats partial (CBT/core.py:27)

# Whether the attention masks the dense decode hook receives allow a prefix [0, n) of
# the keys (no left padding): set once per generation by the decode loops, which know
# the prompt's mask, so the hook need not check every call (a device-to-host read).
_MASK_PREFIX_HINT = contextvars.ContextVar("interattn_mask_prefix_hint", default=None)


@contextlib.contextmanager
def mask_prefix_hint(is_prefix):
    """Inside the context the dense hook takes every attention mask to allow a prefix
    of the keys (``True``) or not (``False``) without checking it."""
    token = _MASK_PREFIX_HINT.set(bool(is_prefix))
    try:
        yield
    finally:
        _MASK_PREFIX_HINT.reset(token)


def mask_is_prefix(attention_mask):
    """Host decision for a 2-D ``[B, T]`` keep-mask (1 = attend): every row keeps a
    prefix ``[0, n)`` of the positions.  Appending kept decode positions preserves it."""
    m = attention_mask.to(torch.bool)
    n = m.sum(-1, keepdim=True)
    return bool(torch.equal(m, torch.arange(m.shape[-1], device=m.device)[None, :] < n))



# ------------------------------------------------------------------ layout and summaries

def _pad_blocks(x, block_size):
    """``[Hkv, P, *rest] -> ([Hkv, nb, B, *rest], nb)``: the prompt cut into blocks of
    ``block_size`` tokens with the last one zero-filled (CBT/core.py:383-395).  A view
    (no copy) when ``P`` is a multiple of the block size."""
    seq_len = int(x.shape[1])
    n_blocks = -(-seq_len // block_size)
    short = n_blocks * block_size - seq_len
    if short:
        # F.pad lists the trailing dims first: leave them, extend dim 1 at its end
        x = F.pad(x, (0, 0) * (x.dim() - 2) + (0, short))
    return x.unflatten(1, (n_blocks, block_size)), n_blocks


def _ensure_paged_layout(x, block_size):
    """The kernels address a ``[Hkv, nb, B, D]`` view by its head stride plus row-major
    (block, token, dim) offsets, so cache slices are used in place; any other layout
    is copied once (CBT/core.py:397-408)."""
    row_major = (block_size * int(x.shape[-1]), int(x.shape[-1]), 1)
    return x if tuple(x.stride()[1:]) == row_major else x.contiguous()


def summary_storage_dtypes(source_dtype, *, summary_dtype=None, mixed=None, k_bar_dtype=None):
    """Storage dtypes of (k_bar, v_bar, bounds): ``_summary_storage_dtypes``
    (CBT/core.py:411-446).  Arguments left at None read the reference's switches
    ``CONDITION_BLOCK_SUMMARY_DTYPE`` (default float32), ``CONDITION_BLOCK_MIXED_SUMMARIES``
    and ``CONDITION_BLOCK_K_BAR_DTYPE`` (default float32); same ``ValueError``s."""
    if summary_dtype is None:
        name = os.environ.get("CONDITION_BLOCK_SUMMARY_DTYPE", "float32")
        summary_dtype = getattr(torch, name)
    if mixed is None:
        mixed = os.environ.get("CONDITION_BLOCK_MIXED_SUMMARIES") == "1"
    if k_bar_dtype is None:
        name = os.environ.get("CONDITION_BLOCK_K_BAR_DTYPE", "float32")
        if name not in ("float32", "bfloat16"):
            raise ValueError(f"CONDITION_BLOCK_K_BAR_DTYPE must be float32 or bfloat16, got {name!r}.")
        k_bar_dtype = getattr(torch, name)
    if k_bar_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"CONDITION_BLOCK_K_BAR_DTYPE must be float32 or bfloat16, got {k_bar_dtype!r}.")
    if not mixed and k_bar_dtype != torch.float32:
        raise ValueError("CONDITION_BLOCK_K_BAR_DTYPE=bfloat16 requires CONDITION_BLOCK_MIXED_SUMMARIES=1.")
    if not mixed:
        if summary_dtype not in (torch.float32, torch.bfloat16):
            raise ValueError(f"summary dtype must be float32 or bfloat16 on this build, got {summary_dtype!r}.")
        return summary_dtype, summary_dtype, summary_dtype
    if summary_dtype != torch.float32:
        raise ValueError("CONDITION_BLOCK_MIXED_SUMMARIES=1 requires CONDITION_BLOCK_SUMMARY_DTYPE=float32 (or unset).")
    bound = source_dtype if source_dtype in (torch.float32, torch.bfloat16) else torch.float32
    return k_bar_dtype, torch.bfloat16, bound


# the reference's name (CBT/core.py:411), with the layout switches as keyword arguments
_summary_storage_dtypes = summary_storage_dtypes


def _kv_desc(k_block, v_block, block_size):
    """Describe ``[Hkv, nb, B, D]`` prompt views as a pool of ``nb`` pages of ``B`` tokens."""
    kv = N.PagedKV()
    kv.k = k_block.data_ptr()
    kv.v = v_block.data_ptr()
    kv.dtype = _code(k_block.dtype, "prompt K/V")
    kv.page_size = int(block_size)
    kv.n_pages = int(k_block.shape[1])
    kv.k_page_stride, kv.k_head_stride, kv.k_token_stride = int(k_block.stride(1)), int(k_block.stride(0)), int(k_block.stride(2))
    kv.v_page_stride, kv.v_head_stride, kv.v_token_stride = int(v_block.stride(1)), int(v_block.stride(0)), int(v_block.stride(2))
    return kv


def _build_prompt_blocks(k_all, v_all, block_size, *, summary_dtype=None, mixed=None, k_bar_dtype=None):
    """Prompt summaries (CBT/core.py:449-500): the same dict keys, built by the HIP
    summary kernel over the padded block view.  Storage dtypes as
    ``summary_storage_dtypes`` (keywords, else the reference's environment switches);
    with ``CONDITION_BLOCK_TMA_BOUNDS=1`` the bounds are stored as the packed
    ``k_bounds [Hkv, nb, 2D]`` (k_max, k_min interleaved per dimension) and ``k_max`` /
    ``k_min`` become views of it, as the reference does (CBT/core.py:490-499); the
    statistics kernels then read the packed rows."""
    _require_cuda(k_all, v_all)
    if block_size <= 0 or block_size % 16:
        raise ValueError("block_size must be a positive multiple of 16")
    k_block, n_blocks = _pad_blocks(k_all, block_size)
    v_block, _ = _pad_blocks(v_all, block_size)
    k_block = _ensure_paged_layout(k_block, block_size)
    v_block = _ensure_paged_layout(v_block, block_size)
    device = k_all.device
    seq_len = int(k_all.shape[1])
    hkv, d = int(k_all.shape[0]), int(k_all.shape[2])
    k_bar_dt, v_bar_dt, bound_dt = summary_storage_dtypes(k_block.dtype, summary_dtype=summary_dtype, mixed=mixed,
                                                          k_bar_dtype=k_bar_dtype)
    token_idx = torch.arange(n_blocks * block_size, device=device).reshape(n_blocks, block_size)
    valid_token = token_idx < seq_len
    out = {
        "k_bar": torch.empty((1, hkv, n_blocks, d), device=device, dtype=k_bar_dt),
        "v_bar": torch.empty((1, hkv, n_blocks, d), device=device, dtype=v_bar_dt),
        "k_max": torch.empty((1, hkv, n_blocks, d), device=device, dtype=bound_dt),
        "k_min": torch.empty((1, hkv, n_blocks, d), device=device, dtype=bound_dt),
        "v_norm_max": torch.empty((1, hkv, n_blocks), device=device, dtype=torch.float32),
        "v_norm_all": torch.empty((1, hkv), device=device, dtype=torch.float32),
        "counts": torch.empty((1, n_blocks), device=device, dtype=torch.int32),
    }
    seq = torch.full((1,), seq_len, device=device, dtype=torch.int32)
    kv = _kv_desc(k_block, v_block, block_size)
    p = lambda t: t.data_ptr()  # noqa: E731
    if n_blocks > 0:
        rc = N.lib().ia_build_block_summaries(
            kv, p(seq), 1, hkv, d, int(block_size), n_blocks, p(out["k_bar"]), _code(k_bar_dt, "k_bar"),
            p(out["v_bar"]), _code(v_bar_dt, "v_bar"), p(out["k_max"]), p(out["k_min"]), _code(bound_dt, "bounds"),
            p(out["v_norm_max"]), p(out["v_norm_all"]), p(out["counts"]), _stream(k_all))
        N.check(rc)
    counts32 = out["counts"][0]
    res = {
        "k_block_attn": k_block,
        "v_block_attn": v_block,
        "token_idx": token_idx,
        "valid_token": valid_token,
        "k_bar": out["k_bar"][0],
        "v_bar": out["v_bar"][0],
        "k_max": out["k_max"][0],
        "k_min": out["k_min"][0],
        "v_norm_max": out["v_norm_max"][0],
        "v_norm_all": out["v_norm_all"][0],
        "block_valid_counts": counts32.long(),
        "_counts_i32": counts32,
        "_block_size": int(block_size),
    }
    if os.environ.get("CONDITION_BLOCK_TMA_BOUNDS") == "1":
        bounds = torch.stack((res["k_max"], res["k_min"]), dim=-1).flatten(2).contiguous()
        pairs = bounds.view(*res["k_max"].shape, 2)
        res["k_bounds"], res["k_max"], res["k_min"] = bounds, pairs[..., 0], pairs[..., 1]
    return res


def _summaries_desc(prefix, n_kv_heads, head_dim):
    """C-ABI view of a prefix dict (contiguous summary arrays, int32 counts)."""
    sm = N.BlockSummaries()
    keep = []

    def arr(name, required=True):
        t = prefix.get(name)
        if t is None:
            if required:
                raise ValueError(f"prompt prefix lacks {name!r}")
            return None
        if not t.is_contiguous():
            t = t.contiguous()
        keep.append(t)
        return t

    k_bar, v_bar = arr("k_bar"), arr("v_bar")
    nb = int(k_bar.shape[-2])
    if tuple(k_bar.shape) != (n_kv_heads, nb, head_dim):
        raise ValueError(f"k_bar must be [Hkv, nb, D] = {(n_kv_heads, nb, head_dim)}, got {tuple(k_bar.shape)}")
    bounds = prefix.get("k_bounds")
    if bounds is not None:
        # the packed bounds (CBT/core.py:490-499): read in place, k_max / k_min are views
        if tuple(bounds.shape) != (n_kv_heads, nb, 2 * head_dim) or not bounds.is_contiguous():
            raise ValueError(f"k_bounds must be contiguous [Hkv, nb, 2D] = {(n_kv_heads, nb, 2 * head_dim)}")
        keep.append(bounds)
        k_max = k_min = bounds
        sm.bounds_packed = 1
    else:
        k_max, k_min = arr("k_max"), arr("k_min")
        if k_max.dtype != k_min.dtype:
            raise ValueError("k_max and k_min must share a dtype")
    counts = prefix.get("_counts_i32")
    if counts is None:
        counts = prefix["block_valid_counts"].to(torch.int32).contiguous()
        prefix["_counts_i32"] = counts
    keep.append(counts)
    vnm, vna = arr("v_norm_max"), arr("v_norm_all")
    if vnm.dtype != torch.float32 or vna.dtype != torch.float32:
        raise ValueError("v_norm_max and v_norm_all must be float32")
    sm.k_bar, sm.k_max, sm.k_min, sm.v_bar = k_bar.data_ptr(), k_max.data_ptr(), k_min.data_ptr(), v_bar.data_ptr()
    sm.k_bar_dtype = _code(k_bar.dtype, "k_bar")
    sm.bounds_dtype = _code(k_max.dtype, "k_max")
    sm.v_bar_dtype = _code(v_bar.dtype, "v_bar")
    sm.v_norm_max, sm.v_norm_all, sm.counts = vnm.data_ptr(), vna.data_ptr(), counts.data_ptr()
    sm.nb = nb
    sm.block_size = int(prefix.get("_block_size", prefix["k_block_attn"].shape[2]))
    return sm, keep, nb


def _grouped_shape(q_grouped):
    n_kv_heads, group_size, n_query, head_dim = q_grouped.shape
    if n_query != 1:
        raise ValueError("condition-block decode expects q_len=1.")
    rows = n_kv_heads * group_size
    q = q_grouped.reshape(rows, head_dim)
    if q.stride(1) != 1:
        q = q.contiguous()
    sh = N.DecodeShape()
    sh.batch, sh.n_q_heads, sh.n_kv_heads, sh.head_dim = 1, rows, n_kv_heads, head_dim
    sh.q_batch_stride, sh.q_row_stride = int(q.stride(0)) * rows, int(q.stride(0))
    if q.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("q must be float32 or bfloat16")
    sh.q_dtype = _code(q.dtype, "q")
    return q, sh


# ------------------------------------------------------------------ selection

def _run_condition_block_selection_stats(q_grouped, prefix, workspace=None, reduce_globals=True,
                                         term1_mass_exp=False):
    """Selection statistics (CBT/core.py:573-698): returns ``(q [rows, D], s [rows, nb],
    delta [rows, nb], partial [4, rows, n_chunks], global_stats [4, rows] or None,
    n_blocks, n_chunks)``."""
    _require_cuda(q_grouped)
    n_kv_heads, group_size, _, head_dim = q_grouped.shape
    q, sh = _grouped_shape(q_grouped)
    sm, keep, nb = _summaries_desc(prefix, n_kv_heads, head_dim)
    rows = n_kv_heads * group_size
    n_chunks = max(1, math.ceil(nb / SELECT_CHUNK))
    dev = q.device
    s = workspace_tensor(workspace, "selection_s", (rows, nb), device=dev, dtype=torch.float32)
    delta = workspace_tensor(workspace, "selection_delta", (rows, nb), device=dev, dtype=torch.float32)
    partial = workspace_tensor(workspace, "selection_partial", (4, rows, n_chunks), device=dev, dtype=torch.float32)
    glob = None
    if reduce_globals:
        glob = workspace_tensor(workspace, "selection_global", (4, rows), device=dev, dtype=torch.float32)
    rc = N.lib().ia_condition_selection_stats(sh, q.data_ptr(), sm, int(bool(term1_mass_exp)), s.data_ptr(),
                                              delta.data_ptr(), partial.data_ptr(),
                                              None if glob is None else glob.data_ptr(), _stream(q))
    N.check(rc)
    del keep
    return q, s, delta, partial, glob, nb, n_chunks


def _select_prompt_blocks_triton(q_grouped, prefix, eps, term1_mass_exp=False):
    """Selection entry point (CBT/core.py:701-744): ``(selected [Hkv,G,1,nb] bool,
    z_logits [Hkv,G,1,nb], v_bar view [Hkv,G,1,nb,D], size [1,nb], exists [1,nb])``."""
    n_kv_heads, group_size, n_query, head_dim = q_grouped.shape
    q, s, delta, _partial, glob, nb, _n = _run_condition_block_selection_stats(
        q_grouped, prefix, term1_mass_exp=term1_mass_exp)
    _, sh = _grouped_shape(q_grouped)
    sm, keep, _ = _summaries_desc(prefix, n_kv_heads, head_dim)
    rows = n_kv_heads * group_size
    selected = torch.empty((rows, nb), device=q.device, dtype=torch.uint8)
    z = torch.empty((rows, nb), device=q.device, dtype=torch.float32)
    rc = N.lib().ia_condition_select(sh, sm, s.data_ptr(), delta.data_ptr(), glob.data_ptr(), float(eps),
                                     int(bool(term1_mass_exp)), selected.data_ptr(), z.data_ptr(), _stream(q))
    N.check(rc)
    del keep
    size = prefix["block_valid_counts"].view(1, -1)
    v_bar = prefix["v_bar"][:, None, None].expand(n_kv_heads, group_size, 1, nb, head_dim)
    return (selected.view(torch.bool).reshape(n_kv_heads, group_size, 1, nb),
            z.reshape(n_kv_heads, group_size, 1, nb), v_bar, size, size > 0)


# ------------------------------------------------------------------ fused decode

def _suffix_desc(k_suffix, v_suffix, suffix_len_dev, prompt_dtype):
    sfx = N.SuffixKV()
    if k_suffix is None or k_suffix.shape[1] == 0:
        return sfx, []
    _require_cuda(k_suffix, v_suffix, suffix_len_dev)
    if k_suffix.dtype != prompt_dtype or v_suffix.dtype != prompt_dtype:
        raise ValueError("suffix K/V must have the prompt K/V dtype")
    if k_suffix.stride(2) != 1 or v_suffix.stride(2) != 1:
        raise ValueError("suffix rows must be contiguous")
    if suffix_len_dev.dtype != torch.int32 or suffix_len_dev.numel() != 1:
        raise ValueError("suffix_len_dev must be one int32 on the device")
    sfx.k, sfx.v = k_suffix.data_ptr(), v_suffix.data_ptr()
    sfx.k_batch_stride, sfx.k_head_stride, sfx.k_token_stride = 0, int(k_suffix.stride(0)), int(k_suffix.stride(1))
    sfx.v_batch_stride, sfx.v_head_stride, sfx.v_token_stride = 0, int(v_suffix.stride(0)), int(v_suffix.stride(1))
    sfx.len = suffix_len_dev.data_ptr()
    sfx.len_stride = 0
    sfx.cap = int(k_suffix.shape[1])
    return sfx, [k_suffix, v_suffix, suffix_len_dev]


def _one_launch():
    """The condition rule's decode (``ia_condition_decode_fused``) and the fixed-mask
    decode (``ia_fixed_mask_decode_fused``) run as one launch where the call fits one,
    unless ``INTERATTN_CONDITION_ONE_LAUNCH=0`` asks for the multi-launch paths
    (statistics, route, finalize, merge; route, finalize, merge)."""
    return os.environ.get("INTERATTN_CONDITION_ONE_LAUNCH", "1") != "0"


def _condition_decode(q_grouped, prompt_prefix, k_suffix, v_suffix, suffix_len_dev, eps, term1_mass_exp,
                      store_selected, output_dtype, workspace, mask=None):
    _require_cuda(q_grouped)
    n_kv_heads, group_size, _, head_dim = q_grouped.shape
    q, sh = _grouped_shape(q_grouped)
    sm, keep, nb = _summaries_desc(prompt_prefix, n_kv_heads, head_dim)
    rows = n_kv_heads * group_size
    k_block, v_block = prompt_prefix["k_block_attn"], prompt_prefix["v_block_attn"]
    if k_block.stride(3) != 1 or v_block.stride(3) != 1:
        raise ValueError("prompt K/V rows must be contiguous")
    kv = _kv_desc(k_block, v_block, sm.block_size)
    sfx, keep_s = _suffix_desc(k_suffix, v_suffix, suffix_len_dev, k_block.dtype)
    dev = q.device
    lib = N.lib()

    def scratch():  # the four-launch and fixed-mask paths' workspace (no initialisation needed)
        ws_bytes = lib.ia_condition_workspace_size(1, n_kv_heads, group_size, head_dim, nb, sfx.cap)
        return workspace_tensor(workspace, "condition_scratch", (max(int(ws_bytes), 1),), device=dev,
                                dtype=torch.uint8)

    out = workspace_tensor(workspace, "attention_output", (rows, head_dim), device=dev, dtype=output_dtype)
    if output_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("output dtype must be float32 or bfloat16")
    selected = None
    if store_selected:
        selected = workspace_tensor(workspace, "selected_rows", (rows, nb), device=dev, dtype=torch.uint8)
    scale = head_dim ** -0.5
    if mask is None and _one_launch() and lib.ia_condition_decode_fused_items(sh, sm, kv.dtype, sfx.cap) > 0:
        # one launch: its workspace carries per-row counts from call to call (zero-filled
        # once, one per (heads, group, head_dim), whatever the prompt length and eps)
        fws = _scratch(workspace, ("condition_fused_scratch", n_kv_heads, group_size, head_dim),
                       lib.ia_condition_decode_fused_workspace_size(1, n_kv_heads, group_size, head_dim), dev)
        rc = lib.ia_condition_decode_fused(sh, q.data_ptr(), sm, kv, sfx, float(eps), int(bool(term1_mass_exp)),
                                           None if selected is None else selected.data_ptr(), scale,
                                           out.data_ptr(), _code(output_dtype, "out"), fws.data_ptr(), fws.numel(),
                                           _stream(q))
    elif mask is None:
        ws = scratch()
        rc = lib.ia_condition_decode(sh, q.data_ptr(), sm, kv, sfx, float(eps), int(bool(term1_mass_exp)),
                                     None if selected is None else selected.data_ptr(), scale, out.data_ptr(),
                                     _code(output_dtype, "out"), ws.data_ptr(), ws.numel(), _stream(q))
    elif _one_launch() and lib.ia_condition_decode_fused_items(sh, sm, kv.dtype, sfx.cap) > 0:
        fws = _scratch(workspace, ("condition_fused_scratch", n_kv_heads, group_size, head_dim),
                       lib.ia_condition_decode_fused_workspace_size(1, n_kv_heads, group_size, head_dim), dev)
        rc = lib.ia_fixed_mask_decode_fused(sh, q.data_ptr(), sm, mask.data_ptr(), kv, sfx, scale, out.data_ptr(),
                                            _code(output_dtype, "out"), fws.data_ptr(), fws.numel(), _stream(q))
    else:
        ws = scratch()
        rc = lib.ia_fixed_mask_decode(sh, q.data_ptr(), sm, mask.data_ptr(), kv, sfx, scale, out.data_ptr(),
                                      _code(output_dtype, "out"), ws.data_ptr(), ws.numel(), _stream(q))
    N.check(rc)
    del keep, keep_s
    out4 = out.reshape(n_kv_heads, group_size, 1, head_dim)
    if selected is not None:
        return out4, selected.view(torch.bool).reshape(n_kv_heads, group_size, 1, nb)
    return out4, None


def _condition_block_decode_output_fused_triton(*, q_grouped, prompt_prefix, k_suffix, v_suffix, suffix_len_dev,
                                                eps, page_size, store_selected, output_dtype, workspace=None,
                                                term1_mass_exp=False):
    """Fused finalize entry point (CBT/core.py:1035-1155): condition routing, the
    representatives of unselected blocks, the selected blocks' tokens and the exact
    suffix in one online softmax.  Returns ``(out [Hkv,G,1,D], selected or None)``."""
    if int(page_size) != int(prompt_prefix["k_block_attn"].shape[2]):
        raise ValueError("page_size must equal the prompt block size")
    return _condition_decode(q_grouped, prompt_prefix, k_suffix, v_suffix, suffix_len_dev, eps, term1_mass_exp,
                             store_selected, output_dtype, workspace)


_SUFFIX_LEN_RECENT = 4  # uncaptured suffix-length tensors a fixed-mask workspace keeps


def fixed_mask_hybrid_attention(*, q_grouped, prompt_prefix, selected, k_suffix, v_suffix, block_size,
                                output_dtype, workspace=None):
    """Representative + selected-page attention with an external mask
    (CBG/real_attention_benchmark/fixed_mask.py:250-348).  ``selected [Hkv, nb]``."""
    if workspace is None:
        workspace = {}
    n_kv_heads, group_size, n_query, head_dim = q_grouped.shape
    if n_query != 1:
        raise ValueError("fixed-mask attention requires q_len=1")
    n_blocks = int(prompt_prefix["block_valid_counts"].numel())
    if tuple(selected.shape) != (n_kv_heads, n_blocks):
        raise ValueError(f"selected must have shape {(n_kv_heads, n_blocks)}, got {tuple(selected.shape)}")
    if int(block_size) != int(prompt_prefix["k_block_attn"].shape[2]):
        raise ValueError("block_size must equal the prompt block size")
    if (selected.dtype in (torch.bool, torch.uint8) and selected.is_contiguous()
            and selected.device == q_grouped.device):
        mask = selected.view(torch.uint8)  # read in place (one byte per block either way)
    else:
        mask = workspace_tensor(workspace, "fixed_mask", (n_kv_heads, n_blocks), device=q_grouped.device,
                                dtype=torch.uint8)
        mask.copy_(selected)
    # the suffix length lives in device memory: one tensor per length, written once, so
    # a captured call and later calls of another length never share it.  Tensors that a
    # captured graph reads are kept for the workspace's life; the others form a small
    # least-recently-used set (an evicted tensor's memory is reused only by later work on
    # the stream, after the calls that read it)
    s_len = int(k_suffix.shape[1]) if k_suffix is not None else 0
    pinned = workspace.setdefault("suffix_len_captured", {})
    recent = workspace.setdefault("suffix_len_recent", OrderedDict())
    sfx_len = pinned.get(s_len)
    if sfx_len is None:
        sfx_len = recent.get(s_len)
        if sfx_len is None or sfx_len.device != q_grouped.device:
            sfx_len = torch.full((1,), s_len, device=q_grouped.device, dtype=torch.int32)
            recent[s_len] = sfx_len
        recent.move_to_end(s_len)
        if torch.cuda.is_current_stream_capturing():
            pinned[s_len] = recent.pop(s_len)
        while len(recent) > _SUFFIX_LEN_RECENT:
            recent.popitem(last=False)
    out, _ = _condition_decode(q_grouped, prompt_prefix, k_suffix, v_suffix, sfx_len, 0.0, False, False,
                               output_dtype, workspace, mask=mask)
    return out


def _condition_stats(*, selected, size, cluster_exists, prompt_len, suffix_len):
    """Routing statistics of one decode step (CBT/core.py:1441-1456), left on the
    device: each query row attends its selected blocks' tokens, one representative
    per unselected existing block and the exact suffix.  ``selected [Hkv, G, 1, nb]``
    (the fused call's selection output), ``size [1, nb]`` valid tokens per block."""
    picks = selected.reshape(-1, selected.shape[-1])          # [query rows, nb]
    n_rows = int(picks.shape[0])
    tokens = size.reshape(1, -1).long()
    exists = cluster_exists.reshape(1, -1)
    sfx = max(int(suffix_len), 0)
    picked_tokens = torch.where(picks, tokens, 0).sum()
    representatives = (exists & ~picks).sum()
    return {
        "rows": n_rows,
        "clusters": exists.sum() * n_rows,
        "selected_clusters": picks.sum(),
        "selected_tokens": picked_tokens,
        "hybrid_tokens": picked_tokens + representatives + sfx * n_rows,
        "total_available": (int(prompt_len) + sfx) * n_rows,
    }


def _condition_block_decode_output(*, q_grouped, prompt_prefix, k_suffix, v_suffix, suffix_len_dev, block_size, eps,
                                   prompt_len, attention_dtype, workspace=None, term1_mass_exp=False,
                                   collect_stats=True):
    """Dispatcher (CBT/core.py:908-1032): always the fused HIP path (any block size
    that is a multiple of 16); returns ``(output [Hkv,G,1,D], stats or None)``."""
    output, selected = _condition_block_decode_output_fused_triton(
        q_grouped=q_grouped, prompt_prefix=prompt_prefix, k_suffix=k_suffix, v_suffix=v_suffix,
        suffix_len_dev=suffix_len_dev, eps=eps, page_size=int(block_size), store_selected=collect_stats,
        output_dtype=attention_dtype, workspace=workspace, term1_mass_exp=term1_mass_exp)
    stats = None
    if collect_stats:
        size = prompt_prefix["block_valid_counts"].view(1, -1)
        stats = _condition_stats(selected=selected, size=size, cluster_exists=size > 0, prompt_len=prompt_len,
                                 suffix_len=int(k_suffix.shape[1]))
    return output, stats


# ------------------------------------------------------------------ dense fallback

def _sdpa_full_attention_forward(module, query, key, value, attention_mask, scaling, dropout=0.0, **_kwargs):
    """Dense attention with the HF attention-function signature (CBT/core.py:1158-1177):
    ``query [B, Hq, L, D]``, ``key/value [B, Hkv, T, D]`` -> ``([B, L, Hq, D], None)``.
    Single-token decode (L == 1) runs the HIP dense paged decode; the keys it reads
    are ``[0, n_b)`` with ``n_b`` the number of positions ``attention_mask`` allows
    for the query (all T when no mask is given).  A mask whose allowed keys are not
    such a prefix (left-padded batches) is detected on the host and goes to torch
    SDPA with the mask; multi-token calls (prompt prefill) go to transformers' SDPA
    attention function, as in the reference.  Under graph capture the mask must be
    None."""
    if query.shape[2] != 1:
        from transformers.integrations.sdpa_attention import sdpa_attention_forward

        return sdpa_attention_forward(module, query, key, value, attention_mask,
                                      dropout=float(dropout) if getattr(module, "training", False) else 0.0,
                                      scaling=scaling, **_kwargs)
    _require_cuda(query, key, value)
    if key.shape != value.shape or key.dtype != value.dtype:
        raise ValueError("key and value must share shape and dtype")
    if key.stride(3) != 1 or value.stride(3) != 1:
        raise ValueError("key/value rows must be contiguous")
    bsz, hq, _, d = query.shape
    hkv, t_len = int(key.shape[1]), int(key.shape[2])
    if attention_mask is None:
        seq = torch.full((bsz,), t_len, device=query.device, dtype=torch.int32)
    else:
        m = attention_mask[:, 0, -1, :t_len] if attention_mask.dim() == 4 else attention_mask[:, -1, :t_len]
        allowed = m if m.dtype == torch.bool else m > torch.finfo(m.dtype).min / 2
        allowed = allowed.expand(bsz, t_len)
        seq = allowed.sum(-1).to(torch.int32).contiguous()
        # the kernel attends keys [0, n): a mask that is not such a prefix (left
        # padding) goes to transformers' SDPA attention, as the reference's does.  The
        # decode loops say once per generation which kind their masks are
        # (mask_prefix_hint); without that the mask is checked here (a host read)
        if torch.cuda.is_current_stream_capturing():
            raise ValueError("decode under graph capture takes attention_mask=None (keys [0, T) attended)")
        is_prefix = _MASK_PREFIX_HINT.get()
        if is_prefix is None:
            prefix = torch.arange(t_len, device=allowed.device)[None, :] < seq[:, None]
            is_prefix = bool(torch.equal(prefix, allowed))
        if not is_prefix:
            mask = attention_mask[..., :t_len] if attention_mask.dim() == 4 else attention_mask[:, None, :, :t_len]
            mask = mask if mask.dtype == torch.bool else mask.to(query.dtype)
            out = F.scaled_dot_product_attention(query, key, value, attn_mask=mask, scale=scaling,
                                                 enable_gqa=hq != hkv)
            return out.transpose(1, 2).contiguous(), None
    # each sequence is one page of ceil16(T) tokens: page b = batch entry b; the
    # kernel never reads a token at or past seq_len, so the padding is never touched
    kv = N.PagedKV()
    kv.k, kv.v = key.data_ptr(), value.data_ptr()
    kv.dtype = _code(key.dtype, "key")
    kv.page_size = max(16, -(-t_len // 16) * 16)
    kv.n_pages = int(bsz)
    kv.k_page_stride, kv.k_head_stride, kv.k_token_stride = (int(s) for s in key.stride()[:3])
    kv.v_page_stride, kv.v_head_stride, kv.v_token_stride = (int(s) for s in value.stride()[:3])
    table = torch.arange(bsz, device=query.device, dtype=torch.int32).view(bsz, 1)
    kv.block_table, kv.bt_stride, kv.bt_cols = table.data_ptr(), 1, 1
    q = query[:, :, 0]
    if q.stride(2) != 1:
        q = q.contiguous()
    sh = N.DecodeShape()
    sh.batch, sh.n_q_heads, sh.n_kv_heads, sh.head_dim = int(bsz), int(hq), hkv, int(d)
    sh.q_batch_stride, sh.q_row_stride = int(q.stride(0)), int(q.stride(1))
    sh.q_dtype = _code(q.dtype, "query")
    out = torch.empty((bsz, hq, d), device=query.device, dtype=query.dtype)
    lib = N.lib()
    items = lib.ia_dense_max_items(int(bsz), hkv, t_len)
    ws_bytes = lib.ia_paged_decode_workspace_size(int(bsz), hkv, int(hq) // hkv, int(d), items)
    ws = torch.empty((max(int(ws_bytes), 1),), device=query.device, dtype=torch.uint8)
    rc = lib.ia_paged_decode(sh, q.data_ptr(), kv, seq.data_ptr(), t_len, float(scaling), out.data_ptr(),
                             _code(out.dtype, "out"), ws.data_ptr(), ws.numel(), _stream(query))
    N.check(rc)
    return out.unsqueeze(1), None
