"""Decode attention (test infrastructure only).

* ``dense_decode``        -- textbook SDPA decode with GQA: the dense fallback
  (``_sdpa_full_attention_forward``, CBT/core.py:1158-1177; ``run_full_sdpa``,
  CBG/condition_block_stage_latency.py:461-478).
* ``sparse_decode``       -- attention over the tokens of the selected blocks only
  (top-k mode: no representatives, as the Quest rule attends selected pages only,
  CBG/methods/quest.py:105-127).
* ``hybrid_decode_dense`` -- ``_condition_block_decode_output_dense``
  (CBT/legacy.py:797-868): selected tokens + representatives of unselected
  existing blocks (logit z, value v_bar) + the exact suffix, one global softmax.
* ``fixed_mask_hybrid``   -- the external-mask finalize
  (CBG/real_attention_benchmark/fixed_mask.py:38-239): representative logit
  recomputed as bf16(q).bf16(k_bar)/sqrt(D) + log(count).
* ``splitk_merge``        -- ``_condition_block_stage2_reduce_kernel`` (CBT/legacy.py:765-794).

Row convention: query head ``h*G + g`` attends kv head ``h`` (GQA grouping,
``q_grouped = query.reshape(Hkv, G, 1, D)``, CBT/core.py:1313).
"""

import math

import numpy as np

from .numerics import bf16_round


def _softmax_attend(logits, values):
    """logits [..., n], values [..., n, D] -> [..., D]; -inf logits contribute 0."""
    m = np.max(logits, axis=-1, keepdims=True)
    m = np.where(np.isneginf(m), 0.0, m)
    e = np.exp(logits - m)
    num = np.einsum("...n,...nd->...d", e, values)
    den = e.sum(axis=-1)[..., None]
    return num / np.maximum(den, 1e-30)


def dense_decode(q, k, v, scale=None):
    """``q [Hq, D]``, ``k, v [Hkv, L, D]`` -> ``[Hq, D]`` float64."""
    hq, d = q.shape
    hkv = k.shape[0]
    g = hq // hkv
    scale = d ** -0.5 if scale is None else scale
    qg = q.astype(np.float64).reshape(hkv, g, d)
    logits = np.einsum("hgd,htd->hgt", qg, k.astype(np.float64)) * scale
    out = _softmax_attend(logits, np.broadcast_to(v.astype(np.float64)[:, None], (hkv, g) + v.shape[1:]))
    return out.reshape(hq, d)


def block_token_mask(idx_per_head, seq_len, block):
    """Boolean ``[Hkv, L]``: token t is attended iff its block t//block is selected."""
    hkv = len(idx_per_head)
    mask = np.zeros((hkv, seq_len), dtype=bool)
    for h, idx in enumerate(idx_per_head):
        for j in np.asarray(idx, dtype=np.int64):
            mask[h, j * block:min((j + 1) * block, seq_len)] = True
    return mask


def sparse_decode(q, k, v, idx_per_head, block, scale=None, p_bf16=False):
    """Attention over the selected blocks' valid tokens.

    ``p_bf16`` rounds the softmax weights to bfloat16 before the weighted sum of V
    (the cast point of CBT/page_attention.py:248-252), while the normalizer keeps the
    float32 weights (CBT/page_attention.py:253).
    """
    hq, d = q.shape
    hkv, seq_len, _ = k.shape
    g = hq // hkv
    scale = d ** -0.5 if scale is None else scale
    mask = block_token_mask(idx_per_head, seq_len, block)
    qg = q.astype(np.float64).reshape(hkv, g, d)
    logits = np.einsum("hgd,htd->hgt", qg, k.astype(np.float64)) * scale
    logits = np.where(mask[:, None, :], logits, -np.inf)
    m = logits.max(axis=-1, keepdims=True)
    m = np.where(np.isneginf(m), 0.0, m)
    e = np.exp(logits - m)
    den = e.sum(axis=-1)
    w = bf16_round(e.astype(np.float32)).astype(np.float64) if p_bf16 else e
    num = np.einsum("hgt,htd->hgd", w, v.astype(np.float64))
    out = num / np.maximum(den, 1e-30)[..., None]
    return out.reshape(hq, d)


def hybrid_decode_dense(q_grouped, k_block, v_block, valid_token, token_idx, pos,
                        prompt_len, k_suffix, v_suffix, selected, z, v_bar, exists):
    """Restates ``_condition_block_decode_output_dense`` (CBT/legacy.py:797-868).

    ``q_grouped [Hkv,G,1,D]``; ``k_block, v_block [Hkv, nb, B, D]``; ``valid_token,
    token_idx [nb, B]``; ``k_suffix, v_suffix [Hkv, S, D]``; ``selected, z
    [Hkv,G,1,nb]``; ``v_bar [Hkv, nb, D]``; ``exists [nb]``.  Returns ``[Hkv,G,1,D]``.
    """
    hkv, g, nq, d = q_grouped.shape
    scale = math.sqrt(d)
    q = q_grouped.astype(np.float64)
    visible = valid_token[None, None, None] & (token_idx[None, None, None] <= pos)   # legacy.py:814-820
    token_active = selected[..., None] & visible                                      # legacy.py:821
    tl_ = np.einsum("gsqd,gbtd->gsqbt", q, k_block.astype(np.float64)) / scale         # legacy.py:824
    tl_ = np.where(token_active, tl_, -np.inf)
    cluster_active = (~selected) & exists[None, None, None]                           # legacy.py:827
    cl_ = np.where(cluster_active, z, -np.inf)
    parts = [tl_.reshape(hkv, g, nq, -1).max(axis=-1), cl_.max(axis=-1)]
    s_len = k_suffix.shape[1]
    if s_len > 0:
        suffix_pos = np.arange(prompt_len, prompt_len + s_len)
        suf_active = np.broadcast_to(suffix_pos[None, None, None] <= pos, (hkv, g, nq, s_len))
        sl_ = np.einsum("grqd,gtd->grqt", q, k_suffix.astype(np.float64)) / scale
        sl_ = np.where(suf_active, sl_, -np.inf)
        parts.append(sl_.max(axis=-1))
    mx = np.max(np.stack(parts), axis=0)
    mx_safe = np.where(np.isneginf(mx), 0.0, mx)
    with np.errstate(invalid="ignore"):
        te = np.where(token_active, np.exp(tl_ - mx_safe[..., None, None]), 0.0)
        ce = np.where(cluster_active, np.exp(cl_ - mx_safe[..., None]), 0.0)
    norm = te.reshape(hkv, g, nq, -1).sum(-1) + ce.sum(-1)
    num = np.einsum("gsqbt,gbtd->gsqd", te, v_block.astype(np.float64))
    num = num + np.einsum("gsqb,gbd->gsqd", ce, v_bar.astype(np.float64))
    if s_len > 0:
        with np.errstate(invalid="ignore"):
            se = np.where(suf_active, np.exp(sl_ - mx_safe[..., None]), 0.0)
        norm = norm + se.sum(-1)
        num = num + np.einsum("grqt,gtd->grqd", se, v_suffix.astype(np.float64))
    return num / np.maximum(norm, 1e-30)[..., None]


def fixed_mask_hybrid(q_grouped, k_block, v_block, counts, k_bar, v_bar, selected,
                      k_suffix, v_suffix, emulate_bf16=True):
    """External-mask hybrid attention (CBG/real_attention_benchmark/fixed_mask.py:38-239).

    ``selected [Hkv, nb]`` per kv head.  Representative logit =
    ``bf16(q) . bf16(k_bar) / sqrt(D) + log(max(count,1))`` (fixed_mask.py:102-107);
    value ``bf16(v_bar)``; page and suffix tokens use ``bf16(q) . K`` (fixed_mask.py:86-90).
    Returns ``[Hkv, G, 1, D]`` float64.
    """
    hkv, g, nq, d = q_grouped.shape
    nb, blk = k_block.shape[1], k_block.shape[2]
    rnd = (lambda x: bf16_round(np.asarray(x, np.float32)).astype(np.float64)) if emulate_bf16 \
        else (lambda x: np.asarray(x, np.float64))
    q = rnd(q_grouped[:, :, 0])                                       # [hkv, g, d]
    counts = np.asarray(counts).astype(np.int64)
    active = counts > 0
    sel = np.asarray(selected, dtype=bool) & active[None]
    rep = (~sel) & active[None]
    scale = d ** -0.5
    rep_logit = np.einsum("hgd,hbd->hgb", q, rnd(k_bar)) * scale + np.log(np.maximum(counts, 1))[None, None]
    tok_valid = (np.arange(blk)[None, :] < counts[:, None])           # [nb, blk]
    tok_logit = np.einsum("hgd,hbtd->hgbt", q, rnd(k_block)) * scale
    tok_mask = sel[:, None, :, None] & tok_valid[None, None]
    logits = [np.where(rep[:, None], rep_logit, -np.inf), np.where(tok_mask, tok_logit, -np.inf).reshape(hkv, g, -1)]
    values = [np.broadcast_to(rnd(v_bar)[:, None], (hkv, g, nb, d)),
              np.broadcast_to(rnd(v_block).reshape(hkv, 1, nb * blk, d), (hkv, g, nb * blk, d))]
    if k_suffix.shape[1] > 0:
        logits.append(np.einsum("hgd,htd->hgt", q, rnd(k_suffix)) * scale)
        values.append(np.broadcast_to(rnd(v_suffix)[:, None], (hkv, g) + v_suffix.shape[1:]))
    out = _softmax_attend(np.concatenate(logits, axis=-1), np.concatenate(values, axis=-2))
    return out[:, :, None, :]


def splitk_merge(acc, m, l):
    """``acc [C, rows, D]``, ``m, l [C, rows]`` -> ``[rows, D]`` (CBT/legacy.py:765-794)."""
    gm = m.max(axis=0)
    with np.errstate(invalid="ignore"):
        w = np.where(np.isneginf(m), 0.0, np.exp(m - gm[None]))
    den = (w * l).sum(axis=0)
    num = (acc * w[..., None]).sum(axis=0)
    return num / np.maximum(den, 1e-30)[:, None]


def splitk_partials(q, k, v, token_mask, chunk_bounds, scale=None):
    """Split-K partials of masked attention: one (acc, m, l) per token range.

    Used to pin ``splitk_merge``: merging the partials of any chunking equals the
    unchunked softmax.  ``q [Hq, D]``, ``k, v [Hkv, L, D]``, ``token_mask [Hkv, L]``.
    """
    hq, d = q.shape
    hkv = k.shape[0]
    g = hq // hkv
    scale = d ** -0.5 if scale is None else scale
    qg = q.astype(np.float64).reshape(hkv, g, d)
    logits = np.einsum("hgd,htd->hgt", qg, k.astype(np.float64)) * scale
    logits = np.where(token_mask[:, None], logits, -np.inf)
    accs, ms, ls = [], [], []
    for lo, hi in chunk_bounds:
        lg = logits[..., lo:hi]
        m = lg.max(axis=-1) if hi > lo else np.full((hkv, g), -np.inf)
        ms_ = np.where(np.isneginf(m), 0.0, m)
        e = np.exp(lg - ms_[..., None]) if hi > lo else np.zeros((hkv, g, 0))
        accs.append(np.einsum("hgt,htd->hgd", e, v[:, lo:hi].astype(np.float64)).reshape(hq, d))
        ms.append(m.reshape(hq))
        ls.append(e.sum(-1).reshape(hq))
    return np.stack(accs), np.stack(ms), np.stack(ls)
