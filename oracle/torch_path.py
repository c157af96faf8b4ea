"""torch CPU restatements of one decode-attention layer call, top-k and condition(eps)
(test infrastructure and the timed CPU baselines of ``bench.py``; never imported by
``interattn_amd``).

The reference's CPU PyTorch path for a top-k step is the Quest convention
(CBG/methods/quest.py:91-103: group-mean page score, ``torch.topk``, attention over
the selected pages in fp32) with the cached block summaries of
``_build_prompt_blocks`` (CBT/core.py:449-500) as the block representatives, and the
fp32 attention of the dense oracle (CBT/legacy.py:797-868).  This module runs that
path on CPU tensors, one sequence at a time, reading K/V out of the paged pool
through the block table (the gather is part of the work), so that ``bench.py`` can
time it on the host cores next to the GPU path.

The condition(eps) call restates the reference's own CPU path for its rule,
``_select_prompt_blocks_eager`` (CBT/core.py:509-555) followed by
``_condition_block_decode_output_dense`` (CBT/legacy.py:797-868), in float32 torch.

Pinned against the numpy oracle (``oracle.select`` / ``oracle.attention``) by
``tests/test_oracle.py::test_torch_path_matches_numpy_oracle`` (top-k) and against
the reference-written golden vectors and the numpy oracle by
``tests/test_golden.py::test_torch_condition_path_matches_reference`` (condition).
"""

import math

import torch


def block_scores(q, k_bar, nb, group, mode="mean"):
    """``q [Hq, D]``, ``k_bar [Hkv, nb_max, D]`` -> ``[Hkv, nb]`` float32.

    ``mode="mean"``: ``mean_g(q_g . k_bar_b) / sqrt(D)`` (the group mean of
    CBG/methods/quest.py:101 with the mean key as representative).
    ``mode="quest"`` takes ``k_bar`` as the pair ``(k_max, k_min)`` and scores
    ``mean_g sum_d max(q_gd k_max_bd, q_gd k_min_bd)`` (CBG/methods/quest.py:97-101).
    """
    hq, d = q.shape
    hkv = hq // group
    qg = q.float().view(hkv, group, d)
    if mode == "quest":
        k_max, k_min = k_bar
        a = qg[:, :, None, :] * k_max[:, None, :nb].float()
        b = qg[:, :, None, :] * k_min[:, None, :nb].float()
        return torch.maximum(a, b).sum(-1).mean(1)
    s = torch.matmul(qg, k_bar[:, :nb].float().transpose(1, 2)) / math.sqrt(d)
    return s.mean(1)


def select_topk(scores, k, forced_first=0, forced_last=0, forced_in_k=False):
    """Chosen block ids (ascending) of one ``[nb]`` score row: the forced first/last
    blocks plus the ``k_eff`` best others, ties to the lower index (a stable sort,
    where ``torch.topk`` leaves exact ties unspecified)."""
    nb = int(scores.shape[0])
    forced = set(range(min(forced_first, nb))) | set(range(max(nb - forced_last, 0), nb))
    k_eff = max(int(k) - len(forced), 0) if forced_in_k else int(k)
    mask = torch.ones(nb, dtype=torch.bool)
    if forced:
        mask[list(forced)] = False
    cand = torch.nonzero(mask).flatten()
    order = torch.sort(scores[cand], descending=True, stable=True).indices
    chosen = cand[order[:k_eff]]
    out = torch.cat([chosen, torch.tensor(sorted(forced), dtype=torch.long)])
    return torch.sort(out).values


def gather_blocks(pool, table_row, seq_len, blocks, block, page, head, scale=None):
    """Rows ``[T, D]`` float32 of the valid tokens of ``blocks`` (kv head ``head``),
    read through the block table; fp8 pools multiply by ``scale[page, head]``."""
    tok = (blocks[:, None] * block + torch.arange(block)[None, :]).flatten()
    tok = tok[tok < seq_len]
    pages = table_row[torch.div(tok, page, rounding_mode="floor")].long()
    rows = pool[pages, head, tok % page].float()
    if scale is not None:
        rows = rows * scale[pages, head][:, None]
    return rows


def topk_layer_call(q, pool_k, pool_v, table_row, seq_len, k_bar, *, block, page, k, forced_first=0,
                    forced_last=0, forced_in_k=False, scales=None, score_mode="mean"):
    """One sequence of a top-k layer call.  ``q [Hq, D]``; ``pool_* [n_pages, Hkv,
    page, D]`` (bf16, fp32 or float8_e4m3fn with ``scales=(k_scale, v_scale)``
    ``[n_pages, Hkv]``); ``table_row [max_pages]``; ``k_bar [Hkv, nb_max, D]`` (or
    ``(k_max, k_min)`` for ``score_mode="quest"``).  Returns ``(out [Hq, D] float32,
    chosen block ids per kv head)``."""
    hq, d = q.shape
    hkv = pool_k.shape[1]
    g = hq // hkv
    nb = -(-int(seq_len) // block)
    scores = block_scores(q, k_bar, nb, g, score_mode)
    qf = q.float().view(hkv, g, d)
    out = torch.empty((hkv, g, d), dtype=torch.float32)
    chosen_all = []
    ks, vs = (None, None) if scales is None else scales
    for h in range(hkv):
        chosen = select_topk(scores[h], k, forced_first, forced_last, forced_in_k)
        chosen_all.append(chosen)
        kk = gather_blocks(pool_k, table_row, seq_len, chosen, block, page, h, ks)
        vv = gather_blocks(pool_v, table_row, seq_len, chosen, block, page, h, vs)
        logits = torch.matmul(qf[h], kk.t()) / math.sqrt(d)
        out[h] = torch.matmul(torch.softmax(logits, dim=-1), vv)
    return out.view(hq, d), chosen_all


# ------------------------------------------------------------- condition(eps) rule

def condition_select(q_grouped, prefix, eps):
    """The eager selection rule of ``_select_prompt_blocks_eager`` (CBT/core.py:509-555)
    on CPU tensors in float32.  ``q_grouped [Hkv, G, 1, D]``; ``prefix`` holds
    ``k_bar, k_max, k_min [Hkv, nb, D]``, ``v_norm_max [Hkv, nb]`` and
    ``block_valid_counts [nb]``.  Returns ``(selected [Hkv, G, 1, nb] bool, z
    [Hkv, G, 1, nb])``: per block s = q.k_bar/sqrt(D), the range bound delta from the
    elementwise extrema, z = log(count) + s, p = softmax(z), and the condition
    p (2 B_all (cosh delta - 1) / sum_b p cosh delta + 2 b_c tanh(delta/2)) averaged
    over the group against eps."""
    q = q_grouped.float()
    hkv, g, nq, d = q.shape
    inv = 1.0 / math.sqrt(d)
    count = prefix["block_valid_counts"].long()
    live = count > 0
    s = torch.matmul(q, prefix["k_bar"].float().transpose(1, 2)[:, None]) * inv     # [hkv, g, nq, nb]
    hi = q[..., None, :] * prefix["k_max"].float()[:, None, None]
    lo = q[..., None, :] * prefix["k_min"].float()[:, None, None]
    upper = torch.maximum(hi, lo).sum(-1) * inv
    lower = torch.minimum(hi, lo).sum(-1) * inv
    delta = torch.maximum((upper - s).abs(), (lower - s).abs()).masked_fill(~live, 0.0)
    b_c = prefix["v_norm_max"].float()[:, None, None, :].masked_fill(~live, 0.0)
    b_all = b_c.amax(-1, keepdim=True)
    z = (s + count.clamp_min(1).float().log()).masked_fill(~live, float("-inf"))
    p = torch.softmax(z, dim=-1)
    ch = torch.cosh(delta)
    mass = (p * ch).sum(-1, keepdim=True).clamp_min(1e-30)
    cond = p * (2.0 * b_all * (ch - 1.0) / mass + 2.0 * b_c * torch.tanh(0.5 * delta))
    chosen = (cond.mean(1, keepdim=True) > eps) & live
    return chosen.expand(hkv, g, nq, -1), z


def condition_attend(q_grouped, k_block, v_block, counts, z, selected, v_bar, k_suffix, v_suffix):
    """The dense hybrid attention of ``_condition_block_decode_output_dense``
    (CBT/legacy.py:797-868) on CPU tensors in float32, for a decode step that sees the
    whole prompt and suffix: the selected blocks' valid tokens (``k_block, v_block
    [Hkv, nb, B, D]``, the first ``counts[b]`` tokens of block b valid), one
    representative per unselected non-empty block (logit z, value ``v_bar [Hkv, nb,
    D]``) and the exact suffix ``[Hkv, S, D]``, one softmax over all of them.
    Returns ``[Hkv, G, 1, D]``."""
    q = q_grouped.float()[:, :, 0]                                                  # [hkv, g, d]
    hkv, g, d = q.shape
    nb, blk = k_block.shape[1], k_block.shape[2]
    inv = 1.0 / math.sqrt(d)
    live = counts.long() > 0
    sel = selected[:, 0, 0] & live                                                  # [hkv, nb]
    tok_ok = torch.arange(blk)[None, :] < counts.long()[:, None]                    # [nb, blk]
    tok_logit = torch.matmul(q, k_block.float().reshape(hkv, nb * blk, d).transpose(1, 2)) * inv
    tok_mask = (sel[:, :, None] & tok_ok[None]).reshape(hkv, 1, nb * blk)
    tok_logit = tok_logit.masked_fill(~tok_mask, float("-inf"))
    rep_logit = z.float()[:, :, 0].masked_fill(~((~sel) & live)[:, None, :], float("-inf"))
    logits = [tok_logit, rep_logit]
    values = [v_block.float().reshape(hkv, nb * blk, d), v_bar.float()]
    if k_suffix.shape[1] > 0:
        logits.append(torch.matmul(q, k_suffix.float().transpose(1, 2)) * inv)
        values.append(v_suffix.float())
    lg = torch.cat(logits, dim=-1)
    top = lg.amax(-1, keepdim=True)
    w = torch.exp(lg - torch.where(torch.isinf(top), torch.zeros_like(top), top))
    num = torch.matmul(w, torch.cat(values, dim=1))
    return (num / w.sum(-1, keepdim=True).clamp_min(1e-30))[:, :, None, :]


def condition_layer_call(q_grouped, prefix, k_block, v_block, k_suffix, v_suffix, eps):
    """One layer call of the reference's CPU path for its own rule: the eager selection
    then the dense hybrid attention.  Returns ``(out [Hkv, G, 1, D], selected)``."""
    selected, z = condition_select(q_grouped, prefix, eps)
    out = condition_attend(q_grouped, k_block, v_block, prefix["block_valid_counts"], z, selected,
                           prefix["v_bar"], k_suffix, v_suffix)
    return out, selected
