"""Paged-pool entry points of the sparse decode-attention path (torch tensors in,
HIP kernels underneath).

Pool layout: ``pool_k, pool_v [n_pages, Hkv, page_size, D]`` (any page/head/token
strides with contiguous rows), ``block_table [batch, max_pages] int32``,
``seq_lens [batch] int32`` on the device.  Logical token ``t`` of sequence ``b`` is
``pool[block_table[b, t // page_size], :, t % page_size]``.  fp8 pools are
``torch.float8_e4m3fn`` with ``scales = (k_scale, v_scale)``, each ``[n_pages, Hkv]``
float32.

Every function launches on the current torch stream and never synchronises, except
where a docstring says otherwise.  Scratch space lives in a caller-owned
``workspace`` dict (the reference's ``_workspace_empty`` convention,
CBT/core.py:558-570): tensors are created on first use and reused while the shapes
match, so steady-state calls allocate nothing (and can be captured in a graph).
"""

import math

import torch

from . import _native as N

_DTYPE_CODE = {torch.float32: N.IA_F32, torch.bfloat16: N.IA_BF16}
if hasattr(torch, "float8_e4m3fn"):
    _DTYPE_CODE[torch.float8_e4m3fn] = N.IA_FP8_E4M3


def _code(dtype, what):
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise ValueError(f"{what}: unsupported dtype {dtype}") from None


def _stream(t):
    return torch.cuda.current_stream(t.device).cuda_stream


def _require_cuda(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("interattn_amd kernels need device (cuda) tensors")


def workspace_tensor(workspace, key, shape, *, device, dtype, zero=False):
    """Reuse ``workspace[key]`` when shape/dtype/device match, else (re)create it.

    Mirrors ``_workspace_empty`` (CBT/core.py:558-570); ``zero=True`` zero-fills a new
    tensor."""
    shape = tuple(int(s) for s in shape)
    make = torch.zeros if zero else torch.empty
    if workspace is None:
        return make(shape, device=device, dtype=dtype)
    t = workspace.get(key)
    if t is None or tuple(t.shape) != shape or t.device != device or t.dtype != dtype:
        t = make(shape, device=device, dtype=dtype)
        workspace[key] = t
    return t


def _scratch(workspace, key, nbytes, device):
    t = workspace_tensor(workspace, key, (max(int(nbytes), 1),), device=device, dtype=torch.uint8, zero=True)
    return t


def _check_i32(t, name, shape=None):
    if t.dtype != torch.int32:
        raise ValueError(f"{name} must be int32, got {t.dtype}")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")


def paged_kv(pool_k, pool_v, block_table=None, scales=None):
    """Describe a pool for the C ABI.  Returns ``(PagedKV, keepalive)``."""
    _require_cuda(pool_k, pool_v, block_table)
    if pool_k.dim() != 4 or pool_v.dim() != 4 or pool_k.shape != pool_v.shape:
        raise ValueError("pool_k/pool_v must both be [n_pages, Hkv, page_size, D]")
    if pool_k.dtype != pool_v.dtype:
        raise ValueError("pool_k and pool_v must share a dtype")
    if pool_k.stride(3) != 1 or pool_v.stride(3) != 1:
        raise ValueError("pool rows (last dim) must be contiguous")
    code = _code(pool_k.dtype, "pool")
    n_pages, hkv, page, d = pool_k.shape
    kv = N.PagedKV()
    kv.k = pool_k.data_ptr()
    kv.v = pool_v.data_ptr()
    kv.dtype = code
    kv.page_size = int(page)
    kv.n_pages = int(n_pages)
    kv.k_page_stride, kv.k_head_stride, kv.k_token_stride = (int(s) for s in pool_k.stride()[:3])
    kv.v_page_stride, kv.v_head_stride, kv.v_token_stride = (int(s) for s in pool_v.stride()[:3])
    keep = [pool_k, pool_v]
    if block_table is not None:
        _check_i32(block_table, "block_table")
        if block_table.dim() != 2 or block_table.stride(1) != 1:
            raise ValueError("block_table must be [batch, max_pages] with contiguous rows")
        kv.block_table = block_table.data_ptr()
        kv.bt_stride = int(block_table.stride(0)) if block_table.shape[0] > 1 else int(block_table.shape[1])
        kv.bt_stride = max(kv.bt_stride, 1)
        kv.bt_cols = int(block_table.shape[1])
        keep.append(block_table)
    if code == N.IA_FP8_E4M3:
        if scales is None:
            raise ValueError("fp8 pools need scales=(k_scale, v_scale), each [n_pages, Hkv] float32")
        if len(scales) not in (2, 3):
            raise ValueError("scales must be (k_scale, v_scale) or (k_scale, v_scale, sequence_scales)")
        ks, vs = scales[0], scales[1]
        seq = scales[2] if len(scales) == 3 else None
        for s_ in (ks, vs):
            _require_cuda(s_)
            if s_.dtype != torch.float32 or tuple(s_.shape) != (n_pages, hkv) or s_.stride(1) != 1:
                raise ValueError("scales must be float32 [n_pages, Hkv] with contiguous rows")
        if ks.stride(0) != vs.stride(0):
            raise ValueError("k_scale and v_scale must share a layout")
        kv.k_scale = ks.data_ptr()
        kv.v_scale = vs.data_ptr()
        kv.scale_page_stride = int(ks.stride(0))
        keep += [ks, vs]
        if seq is not None:
            _require_cuda(seq)
            cols = int(block_table.shape[1]) if block_table is not None else int(n_pages)
            if (seq.dtype != torch.float32 or seq.dim() != 4 or seq.shape[1] != hkv or seq.shape[2] < cols
                    or seq.shape[3] != 2 or seq.stride(3) != 1 or seq.stride(2) != 2):
                raise ValueError("sequence_scales must be float32 [batch, Hkv, >= max_pages, 2] with contiguous "
                                 "(k, v) pairs (see sequence_scales())")
            if seq.stride(0) % 2 or seq.stride(1) % 2 or seq.data_ptr() % 8:
                raise ValueError("sequence_scales pairs must be 8-byte aligned")
            kv.seq_scale = seq.data_ptr()
            kv.seq_scale_b_stride = int(seq.stride(0))
            kv.seq_scale_h_stride = int(seq.stride(1))
            keep.append(seq)
    elif scales is not None and len(scales) == 3:
        raise ValueError("sequence_scales are for fp8 pools only")
    return kv, keep


def sequence_scales(scales, block_table):
    """fp8 pools: the per-page scales gathered per sequence, ``[batch, Hkv, max_pages, 2]``
    float32 holding the (k, v) scale pair of each logical page of each sequence, so that a
    block's consecutive pages share a cache line.  Pass it as the third element of
    ``scales`` (``scales=(k_scale, v_scale, seq)``) to the decode calls: the outputs are
    bit-identical, and the finalize reads one scale line per selected block instead of
    two per page.  Rebuild it whenever the block table or a scale changes (entries past
    a sequence's valid pages are never read)."""
    ks, vs = scales[0], scales[1]
    _check_i32(block_table, "block_table")
    if block_table.dim() != 2:
        raise ValueError("block_table must be [batch, max_pages]")
    pages = block_table.long().clamp(0, max(int(ks.shape[0]) - 1, 0))
    pair = torch.stack((ks[pages], vs[pages]), dim=-1)  # [batch, max_pages, Hkv, 2]
    return pair.permute(0, 2, 1, 3).contiguous()


def _decode_shape(q, hkv):
    if q.dim() != 3 or q.stride(2) != 1:
        raise ValueError("q must be [batch, n_q_heads, D] with contiguous rows")
    b, hq, d = q.shape
    if hq % hkv != 0:
        raise ValueError("n_q_heads must be a multiple of n_kv_heads (grouped query attention)")
    sh = N.DecodeShape()
    sh.batch = int(b)
    sh.n_q_heads = int(hq)
    sh.n_kv_heads = int(hkv)
    sh.head_dim = int(d)
    sh.q_batch_stride = int(q.stride(0))
    sh.q_row_stride = int(q.stride(1))
    if q.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("q must be float32 or bfloat16")
    sh.q_dtype = _code(q.dtype, "q")
    return sh


# --------------------------------------------------------------------------- summaries

def build_block_summaries(pool_k, pool_v, block_table, seq_lens, block_size, *, nb_max, full=False,
                          k_bar_dtype=torch.bfloat16, v_bar_dtype=torch.bfloat16, bounds_dtype=None,
                          scales=None):
    """Per-block summaries of the paged sequences (paged ``_build_prompt_blocks``,
    CBT/core.py:449-500).  Returns a dict with ``k_bar [B, Hkv, nb_max, D]`` and
    ``block_valid_counts [B, nb_max] int32``; with ``full=True`` also ``v_bar, k_max,
    k_min`` (same shape), ``v_norm_max [B, Hkv, nb_max]`` and ``v_norm_all [B, Hkv]``."""
    kv, keep = paged_kv(pool_k, pool_v, block_table, scales)
    _require_cuda(seq_lens)
    _check_i32(seq_lens, "seq_lens")
    b = int(seq_lens.shape[0])
    if block_table is not None and block_table.shape[0] != b:
        raise ValueError("block_table rows must match seq_lens")
    hkv, d = int(pool_k.shape[1]), int(pool_k.shape[3])
    dev = pool_k.device
    if bounds_dtype is None:
        bounds_dtype = torch.float32 if pool_k.dtype == torch.float32 else torch.bfloat16
    out = {
        "k_bar": torch.empty((b, hkv, nb_max, d), device=dev, dtype=k_bar_dtype),
        "block_valid_counts": torch.empty((b, nb_max), device=dev, dtype=torch.int32),
    }
    v_bar = k_max = k_min = vnm = vna = None
    if full:
        out["v_bar"] = v_bar = torch.empty((b, hkv, nb_max, d), device=dev, dtype=v_bar_dtype)
        out["k_max"] = k_max = torch.empty((b, hkv, nb_max, d), device=dev, dtype=bounds_dtype)
        out["k_min"] = k_min = torch.empty((b, hkv, nb_max, d), device=dev, dtype=bounds_dtype)
        out["v_norm_max"] = vnm = torch.empty((b, hkv, nb_max), device=dev, dtype=torch.float32)
        out["v_norm_all"] = vna = torch.empty((b, hkv), device=dev, dtype=torch.float32)
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    rc = N.lib().ia_build_block_summaries(
        kv, seq_lens.data_ptr(), b, hkv, d, int(block_size), int(nb_max),
        p(out["k_bar"]), _code(k_bar_dtype, "k_bar"), p(v_bar), _code(v_bar_dtype, "v_bar"),
        p(k_max), p(k_min), _code(bounds_dtype, "bounds"), p(vnm), p(vna),
        out["block_valid_counts"].data_ptr(), _stream(pool_k))
    N.check(rc)
    del keep
    return out


def update_block_summaries(summ, pool_k, pool_v, block_table, old_seq_lens, seq_lens, block_size, *,
                           max_new_tokens, scales=None):
    """Refresh ``summ`` (a ``build_block_summaries`` dict, holding the summaries at
    ``old_seq_lens``) in place for sequences grown to ``seq_lens``; only the blocks
    the new tokens touch are recomputed (``max_new_tokens`` bounds the growth).
    Equal to a full rebuild at ``seq_lens``."""
    kv, keep = paged_kv(pool_k, pool_v, block_table, scales)
    _require_cuda(old_seq_lens, seq_lens)
    _check_i32(old_seq_lens, "old_seq_lens")
    _check_i32(seq_lens, "seq_lens", tuple(old_seq_lens.shape))
    b = int(seq_lens.shape[0])
    hkv, d = int(pool_k.shape[1]), int(pool_k.shape[3])
    kb = summ["k_bar"]
    if kb.dim() != 4 or tuple(kb.shape[:2]) != (b, hkv) or kb.shape[3] != d or not kb.is_contiguous():
        raise ValueError("summ['k_bar'] must be a contiguous [batch, Hkv, nb_max, D] tensor")
    nb_max = int(kb.shape[2])
    get = lambda k: summ.get(k)  # noqa: E731
    v_bar, k_max, k_min, vnm, vna = get("v_bar"), get("k_max"), get("k_min"), get("v_norm_max"), get("v_norm_all")
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    rc = N.lib().ia_update_block_summaries(
        kv, old_seq_lens.data_ptr(), seq_lens.data_ptr(), b, hkv, d, int(block_size), nb_max, int(max_new_tokens),
        kb.data_ptr(), _code(kb.dtype, "k_bar"), p(v_bar), _code(v_bar.dtype if v_bar is not None else kb.dtype, "v_bar"),
        p(k_max), p(k_min), _code(k_max.dtype if k_max is not None else kb.dtype, "bounds"), p(vnm), p(vna),
        summ["block_valid_counts"].data_ptr(), _stream(pool_k))
    N.check(rc)
    del keep
    return summ


def append_kv(pool_k, pool_v, block_table, seq_lens, k_new, v_new):
    """Write one token per sequence (``k_new, v_new [batch, Hkv, D]``) at position
    ``seq_lens[b]`` of the paged pool and advance ``seq_lens`` in place, on the
    device (capturable in a graph)."""
    kv, keep = paged_kv(pool_k, pool_v, block_table)
    _require_cuda(seq_lens, k_new, v_new)
    _check_i32(seq_lens, "seq_lens")
    b = int(seq_lens.shape[0])
    hkv, d = int(pool_k.shape[1]), int(pool_k.shape[3])
    for t in (k_new, v_new):
        if tuple(t.shape) != (b, hkv, d) or t.stride(2) != 1 or t.dtype != pool_k.dtype:
            raise ValueError("k_new/v_new must be [batch, Hkv, D] of the pool dtype with contiguous rows")
    if k_new.stride()[:2] != v_new.stride()[:2]:
        raise ValueError("k_new and v_new must share strides")
    rc = N.lib().ia_append_kv(kv, k_new.data_ptr(), v_new.data_ptr(), int(k_new.stride(0)), int(k_new.stride(1)),
                              seq_lens.data_ptr(), b, hkv, d, _stream(pool_k))
    N.check(rc)
    del keep
    return seq_lens


# --------------------------------------------------------------------------- top-k selection

SCORES = {"mean": N.IA_SCORE_MEAN_KEY, "quest": N.IA_SCORE_QUEST}


def _block_keys(k_bar, score):
    """C-ABI block keys.  ``score="mean"``: ``k_bar [B, Hkv, nb_max, D]``; ``"quest"``:
    ``k_bar = (k_max, k_min)``, both ``[B, Hkv, nb_max, D]`` of one dtype and layout.
    Returns ``(BlockKeys, (B, Hkv, nb_max, D), dtype, keepalive)``."""
    if score not in SCORES:
        raise ValueError(f"score must be one of {sorted(SCORES)}, got {score!r}")
    arrays = tuple(k_bar) if score == "quest" else (k_bar,)
    if score == "quest" and len(arrays) != 2:
        raise ValueError("score='quest' takes k_bar=(k_max, k_min)")
    ref = arrays[0]
    _require_cuda(*arrays)
    for t in arrays:
        if t.dim() != 4 or t.stride(3) != 1 or t.stride(2) != t.shape[3]:
            raise ValueError("block keys must be [B, Hkv, nb_max, D] with contiguous blocks")
        if t.shape != ref.shape or t.stride() != ref.stride() or t.dtype != ref.dtype:
            raise ValueError("k_max and k_min must share shape, strides and dtype")
    keys = N.BlockKeys()
    keys.score = SCORES[score]
    keys.dtype = _code(ref.dtype, "block keys")
    if score == "quest":
        keys.k_max, keys.k_min = arrays[0].data_ptr(), arrays[1].data_ptr()
    else:
        keys.k_bar = ref.data_ptr()
    keys.batch_stride, keys.head_stride = int(ref.stride(0)), int(ref.stride(1))
    return keys, tuple(int(x) for x in ref.shape), ref.dtype, arrays


def set_wait_limit(ticks):
    """Bound (100 MHz clock ticks) of every wait between the workgroups of a one-launch
    call (default 20,000 = 200 us); a negative value restores the default.  A wait that
    reaches it makes the waiting workgroup compute the missing data itself (same
    results).  Returns the previous bound."""
    return int(N.lib().ia_set_wait_limit(int(ticks)))


def wait_fallbacks(reset=False):
    """Diagnostic: waits of the one-launch calls on the current device that reached their
    bound since the process started or the last ``reset`` (each one's workgroup computed
    the missing scores or statistics itself).  Nonzero in normal operation means the
    launches' workgroups were not all resident together (other work on the GPU).  Reads
    device memory synchronously."""
    return int(N.lib().ia_wait_fallbacks(1 if reset else 0))

def select_blocks_topk(q, k_bar, seq_lens, k, *, block_size, forced_first=0, forced_last=0,
                       forced_in_k=False, k_cap=None, k_per_seq=None, return_scores=False, score="mean",
                       workspace=None):
    """Top-k block selection per (sequence, kv head).

    ``q [B, Hq, D]``.  ``score="mean"``: ``k_bar [B, Hkv, nb_max, D]`` (bf16/fp32
    summaries), score = group-mean ``q . k_bar / sqrt(D)``; ``score="quest"``:
    ``k_bar = (k_max, k_min)``, score = group-mean ``sum_d max(q_d k_max_d, q_d k_min_d)``
    (CBG/methods/quest.py:91-103).  Returns ``(idx [B, Hkv, k_cap] int32, n_sel [B, Hkv]
    int32[, scores [B, Hkv, nb_max] f32])``; ``idx[b, h, :n_sel[b, h]]`` are the chosen
    blocks in ascending order (forced first ``forced_first`` / last ``forced_last``
    blocks included; ``forced_in_k`` counts them inside ``k``).  Ties at the k-th score
    go to the lower block index.  ``k_per_seq`` (int32 ``[B]`` on the device) overrides
    ``k`` per sequence; ``k_cap`` must then cover its largest entry plus the forced
    blocks."""
    keys, (b, hkv, nb_max, d), _, keep = _block_keys(k_bar, score)
    _require_cuda(q, seq_lens)
    sh = _decode_shape(q, hkv)
    if q.shape[0] != b or q.shape[2] != d:
        raise ValueError("q and the block keys disagree on batch or head_dim")
    _check_i32(seq_lens, "seq_lens", (b,))
    if k < 0 or forced_first < 0 or forced_last < 0:
        raise ValueError("k and forced block counts must be >= 0")
    if k_per_seq is not None:
        _require_cuda(k_per_seq)
        _check_i32(k_per_seq, "k_per_seq", (b,))
        if k_cap is None:
            raise ValueError("k_per_seq needs an explicit k_cap")
    if k_cap is None:
        k_cap = max(int(k), forced_first + forced_last) if forced_in_k else int(k) + forced_first + forced_last
    k_cap = max(int(k_cap), 1)
    dev = q.device
    idx = workspace_tensor(workspace, "topk_idx", (b, hkv, k_cap), device=dev, dtype=torch.int32)
    n_sel = workspace_tensor(workspace, "topk_n_sel", (b, hkv), device=dev, dtype=torch.int32)
    scores = None
    if return_scores:
        scores = workspace_tensor(workspace, "topk_scores", (b, hkv, nb_max), device=dev, dtype=torch.float32)
    lib = N.lib()
    ws_bytes = lib.ia_select_topk_workspace_size(b, hkv, nb_max)
    ws = _scratch(workspace if workspace is not None else {}, "topk_scratch", ws_bytes, dev)
    rc = lib.ia_select_topk(
        sh, q.data_ptr(), keys, seq_lens.data_ptr(), int(block_size), nb_max, int(k),
        None if k_per_seq is None else k_per_seq.data_ptr(), int(forced_first),
        int(forced_last), int(bool(forced_in_k)), idx.data_ptr(), k_cap, n_sel.data_ptr(),
        None if scores is None else scores.data_ptr(), ws.data_ptr(), ws.numel(), _stream(q))
    N.check(rc)
    del keep
    if return_scores:
        return idx, n_sel, scores
    return idx, n_sel


# --------------------------------------------------------------------------- decode

def _out_tensor(q, out, out_dtype, workspace):
    dtype = q.dtype if out_dtype is None else out_dtype
    if out is None:
        out = workspace_tensor(workspace, "attention_output", tuple(q.shape), device=q.device, dtype=dtype)
    if tuple(out.shape) != tuple(q.shape) or not out.is_contiguous():
        raise ValueError("out must be a contiguous [batch, n_q_heads, D] tensor")
    if out.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("out must be float32 or bfloat16")
    return out


def sparse_paged_decode(q, pool_k, pool_v, block_table, seq_lens, idx, n_sel, *, block_size, scale=None,
                        scales=None, include_representatives=False, summaries=None, out=None, out_dtype=None,
                        workspace=None):
    """Attention over the selected blocks only: for each query row, softmax(q.K^T*scale)
    over the valid tokens of blocks ``idx[b, h, :n_sel[b, h]]``, applied to V.  The
    top-k form of the finalize stage (CBT/page_attention.py:206-255 + the split-K merge
    of CBT/legacy.py:765-794).  Returns ``[B, Hq, D]`` (``out`` when given).

    ``include_representatives=True`` adds one representative per unselected non-empty
    block in the same softmax: logit ``q.k_bar/sqrt(D) + log(count)`` (q, k_bar rounded
    to bf16 for bf16 caches) and value ``v_bar``, the external-mask semantics of
    fixed_mask_hybrid_attention (CBG/real_attention_benchmark/fixed_mask.py:38-239).
    It needs ``summaries`` from ``build_block_summaries(..., full=True)`` at the same
    ``block_size`` (valid tokens per block are the summaries' counts) and bf16 or fp32
    K/V."""
    if include_representatives:
        return _sparse_decode_with_representatives(q, pool_k, pool_v, block_table, seq_lens, idx, n_sel,
                                                   block_size=block_size, scale=scale, scales=scales,
                                                   summaries=summaries, out=out, out_dtype=out_dtype,
                                                   workspace=workspace)
    kv, keep = paged_kv(pool_k, pool_v, block_table, scales)
    _require_cuda(q, seq_lens, idx, n_sel)
    hkv, d = int(pool_k.shape[1]), int(pool_k.shape[3])
    sh = _decode_shape(q, hkv)
    b = int(q.shape[0])
    if q.shape[2] != d:
        raise ValueError("q head_dim does not match the pool")
    _check_i32(seq_lens, "seq_lens", (b,))
    _check_i32(n_sel, "n_sel", (b, hkv))
    if idx.dim() != 3 or tuple(idx.shape[:2]) != (b, hkv) or not idx.is_contiguous():
        raise ValueError("idx must be a contiguous [B, Hkv, k_cap] int32 tensor")
    _check_i32(idx, "idx")
    if block_table is not None and block_table.shape[0] != b:
        raise ValueError("block_table rows must match the batch")
    if not n_sel.is_contiguous():
        raise ValueError("n_sel must be contiguous")
    k_cap = int(idx.shape[2])
    scale = d ** -0.5 if scale is None else float(scale)
    out = _out_tensor(q, out, out_dtype, workspace)
    lib = N.lib()
    g = int(q.shape[1]) // hkv
    items = lib.ia_sparse_max_items(b, hkv, k_cap)
    ws_bytes = lib.ia_paged_decode_workspace_size(b, hkv, g, d, items)
    ws = _scratch(workspace if workspace is not None else {}, "decode_scratch", ws_bytes, q.device)
    rc = lib.ia_sparse_paged_decode(
        sh, q.data_ptr(), kv, seq_lens.data_ptr(), int(block_size), idx.data_ptr(), k_cap, n_sel.data_ptr(),
        scale, out.data_ptr(), _code(out.dtype, "out"), ws.data_ptr(), ws.numel(), _stream(q))
    N.check(rc)
    del keep
    return out


def _paged_summaries_desc(summaries, b, hkv, d, block_size):
    """C-ABI view of ``build_block_summaries(..., full=True)`` output ([B, Hkv, nb, D])."""
    if summaries is None:
        raise ValueError("include_representatives needs summaries=build_block_summaries(..., full=True)")
    need = ("k_bar", "v_bar", "block_valid_counts", "v_norm_max", "v_norm_all")
    miss = [k for k in need if summaries.get(k) is None]
    if miss:
        raise ValueError(f"summaries lack {miss}: build them with full=True")
    k_bar, v_bar = summaries["k_bar"], summaries["v_bar"]
    nb = int(k_bar.shape[2]) if k_bar.dim() == 4 else -1
    for name in ("k_bar", "v_bar"):
        t = summaries[name]
        if t.dim() != 4 or tuple(t.shape) != (b, hkv, nb, d) or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous [B, Hkv, nb, D] tensor")
    _check_i32(summaries["block_valid_counts"], "block_valid_counts", (b, nb))
    vnm, vna = summaries["v_norm_max"], summaries["v_norm_all"]
    if vnm.dtype != torch.float32 or vna.dtype != torch.float32 or not vnm.is_contiguous():
        raise ValueError("v_norm_max and v_norm_all must be contiguous float32")
    sm = N.BlockSummaries()
    sm.k_bar, sm.v_bar = k_bar.data_ptr(), v_bar.data_ptr()
    sm.k_max = summaries["k_max"].data_ptr() if summaries.get("k_max") is not None else None
    sm.k_min = summaries["k_min"].data_ptr() if summaries.get("k_min") is not None else None
    sm.k_bar_dtype = _code(k_bar.dtype, "k_bar")
    sm.v_bar_dtype = _code(v_bar.dtype, "v_bar")
    bounds = summaries.get("k_max")
    sm.bounds_dtype = _code(bounds.dtype if bounds is not None else torch.float32, "bounds")
    sm.v_norm_max, sm.v_norm_all = vnm.data_ptr(), vna.data_ptr()
    sm.counts = summaries["block_valid_counts"].data_ptr()
    sm.nb = nb
    sm.block_size = int(block_size)
    return sm, nb


def _sparse_decode_with_representatives(q, pool_k, pool_v, block_table, seq_lens, idx, n_sel, *, block_size,
                                        scale, scales, summaries, out, out_dtype, workspace):
    if pool_k.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("representatives need bf16 or fp32 K/V")
    kv, keep = paged_kv(pool_k, pool_v, block_table, scales)
    _require_cuda(q, seq_lens, idx, n_sel)
    hkv, d = int(pool_k.shape[1]), int(pool_k.shape[3])
    sh = _decode_shape(q, hkv)
    b = int(q.shape[0])
    if q.shape[2] != d:
        raise ValueError("q head_dim does not match the pool")
    _check_i32(n_sel, "n_sel", (b, hkv))
    if idx.dim() != 3 or tuple(idx.shape[:2]) != (b, hkv) or not idx.is_contiguous():
        raise ValueError("idx must be a contiguous [B, Hkv, k_cap] int32 tensor")
    _check_i32(idx, "idx")
    if not n_sel.is_contiguous():
        raise ValueError("n_sel must be contiguous")
    if block_table is not None and block_table.shape[0] != b:
        raise ValueError("block_table rows must match the batch")
    sm, nb = _paged_summaries_desc(summaries, b, hkv, d, block_size)
    scale = d ** -0.5 if scale is None else float(scale)
    out = _out_tensor(q, out, out_dtype, workspace)
    ws_dict = workspace if workspace is not None else {}
    mask = workspace_tensor(ws_dict, "topk_block_mask", (b, hkv, max(nb, 1)), device=q.device, dtype=torch.uint8)
    lib = N.lib()
    N.check(lib.ia_topk_block_mask(idx.data_ptr(), n_sel.data_ptr(), int(idx.shape[2]), b, hkv, nb,
                                   mask.data_ptr(), _stream(q)))
    g = int(q.shape[1]) // hkv
    ws_bytes = lib.ia_condition_workspace_size(b, hkv, g, d, nb, 0)
    ws = _scratch(ws_dict, "hybrid_scratch", ws_bytes, q.device)
    sfx = N.SuffixKV()
    rc = lib.ia_fixed_mask_decode(sh, q.data_ptr(), sm, mask.data_ptr(), kv, sfx, scale, out.data_ptr(),
                                  _code(out.dtype, "out"), ws.data_ptr(), ws.numel(), _stream(q))
    N.check(rc)
    del keep
    return out


def paged_decode(q, pool_k, pool_v, block_table, seq_lens, *, max_seq_len=None, scale=None, scales=None,
                 out=None, out_dtype=None, workspace=None):
    """Dense paged decode (the fallback path): softmax(q.K^T*scale).V over all
    ``seq_lens[b]`` tokens.  ``max_seq_len`` must bound ``seq_lens``; when omitted it is
    read back from the device (one host synchronisation)."""
    kv, keep = paged_kv(pool_k, pool_v, block_table, scales)
    _require_cuda(q, seq_lens)
    hkv, d = int(pool_k.shape[1]), int(pool_k.shape[3])
    sh = _decode_shape(q, hkv)
    b = int(q.shape[0])
    _check_i32(seq_lens, "seq_lens", (b,))
    if block_table is not None and block_table.shape[0] != b:
        raise ValueError("block_table rows must match the batch")
    if max_seq_len is None:
        max_seq_len = int(seq_lens.max().item()) if b else 0
    scale = d ** -0.5 if scale is None else float(scale)
    out = _out_tensor(q, out, out_dtype, workspace)
    lib = N.lib()
    g = int(q.shape[1]) // hkv
    items = lib.ia_dense_max_items(b, hkv, int(max_seq_len))
    ws_bytes = lib.ia_paged_decode_workspace_size(b, hkv, g, d, items)
    ws = _scratch(workspace if workspace is not None else {}, "dense_scratch", ws_bytes, q.device)
    rc = lib.ia_paged_decode(sh, q.data_ptr(), kv, seq_lens.data_ptr(), int(max_seq_len), scale,
                             out.data_ptr(), _code(out.dtype, "out"), ws.data_ptr(), ws.numel(), _stream(q))
    N.check(rc)
    del keep
    return out


FUSED_MAX_BLOCKS = 4096  # score rows the fused top-k decode stages in LDS
FUSED_MAX_K_CAP = 512


def sparse_topk_decode(q, pool_k, pool_v, block_table, seq_lens, k_bar, k, *, block_size, forced_first=0,
                       forced_last=0, forced_in_k=False, k_cap=None, k_per_seq=None, scale=None, scales=None,
                       out=None, out_dtype=None, return_selection=False, score="mean", workspace=None):
    """One decode-attention layer call of the top-k path: the selection of
    ``select_blocks_topk`` (``score`` and ``k_bar`` as there) followed by
    ``sparse_paged_decode``.  Up to 4096 blocks per sequence and ``k_cap <= 512`` it is
    one launch (``ia_sparse_topk_decode``: each (sequence, kv head) row's items score
    their share of the blocks, exchange scores, select, stream their share of the
    chosen blocks and merge); beyond that the two calls.  The launch's workspace
    (``workspace[("topk_decode_scratch", *shape)]``, one per call shape) is zero-filled
    when it is created and must not be shared by overlapping calls.  With ``return_selection`` returns
    ``(out, idx, n_sel)``."""
    keys, (b, hkv, nb_max, d), _, keep_k = _block_keys(k_bar, score)
    _require_cuda(q, seq_lens)
    if k < 0 or forced_first < 0 or forced_last < 0:
        raise ValueError("k and forced block counts must be >= 0")
    if k_per_seq is not None:
        _require_cuda(k_per_seq)
        _check_i32(k_per_seq, "k_per_seq", (b,))
        if k_cap is None:
            raise ValueError("k_per_seq needs an explicit k_cap")
    if k_cap is None:
        k_cap = max(int(k), forced_first + forced_last) if forced_in_k else int(k) + forced_first + forced_last
    k_cap = max(int(k_cap), 1)
    if nb_max > FUSED_MAX_BLOCKS or k_cap > FUSED_MAX_K_CAP:
        idx, n_sel = select_blocks_topk(q, k_bar, seq_lens, k, block_size=block_size, forced_first=forced_first,
                                        forced_last=forced_last, forced_in_k=forced_in_k, k_cap=k_cap,
                                        k_per_seq=k_per_seq, score=score, workspace=workspace)
        res = sparse_paged_decode(q, pool_k, pool_v, block_table, seq_lens, idx, n_sel, block_size=block_size,
                                  scale=scale, scales=scales, out=out, out_dtype=out_dtype, workspace=workspace)
        return (res, idx, n_sel) if return_selection else res
    kv, keep = paged_kv(pool_k, pool_v, block_table, scales)
    if int(pool_k.shape[1]) != hkv or int(pool_k.shape[3]) != d:
        raise ValueError("the block keys and the pool disagree on Hkv or head_dim")
    sh = _decode_shape(q, hkv)
    if q.shape[0] != b or q.shape[2] != d:
        raise ValueError("q and the block keys disagree on batch or head_dim")
    _check_i32(seq_lens, "seq_lens", (b,))
    if block_table is not None and block_table.shape[0] != b:
        raise ValueError("block_table rows must match the batch")
    scale = d ** -0.5 if scale is None else float(scale)
    out = _out_tensor(q, out, out_dtype, workspace)
    dev = q.device
    idx = n_sel = None
    if return_selection:
        idx = workspace_tensor(workspace, "topk_idx", (b, hkv, k_cap), device=dev, dtype=torch.int32)
        n_sel = workspace_tensor(workspace, "topk_n_sel", (b, hkv), device=dev, dtype=torch.int32)
    lib = N.lib()
    g = int(q.shape[1]) // hkv
    ws_bytes = lib.ia_sparse_topk_decode_workspace_size(b, hkv, g, d, nb_max, k_cap, int(block_size))
    # the launch keeps per-row counts in its workspace from call to call: one
    # zero-filled buffer per call shape
    ws = _scratch(workspace if workspace is not None else {},
                  ("topk_decode_scratch", b, hkv, g, d, nb_max, k_cap, int(block_size)), ws_bytes, dev)
    rc = lib.ia_sparse_topk_decode(
        sh, q.data_ptr(), kv, seq_lens.data_ptr(), keys, int(block_size), nb_max, int(k),
        None if k_per_seq is None else k_per_seq.data_ptr(), int(forced_first), int(forced_last),
        int(bool(forced_in_k)), k_cap, scale, out.data_ptr(), _code(out.dtype, "out"),
        None if idx is None else idx.data_ptr(), None if n_sel is None else n_sel.data_ptr(), ws.data_ptr(),
        ws.numel(), _stream(q))
    N.check(rc)
    del keep, keep_k
    return (out, idx, n_sel) if return_selection else out


def nb_for(seq_len, block_size):
    return int(math.ceil(int(seq_len) / int(block_size)))
