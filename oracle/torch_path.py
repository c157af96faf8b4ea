"""torch CPU restatement of one top-k decode-attention layer call (test infrastructure
and the timed CPU baseline of ``bench.py``; never imported by ``interattn_amd``).

The reference's CPU PyTorch path for a top-k step is the Quest convention
(CBG/methods/quest.py:91-103: group-mean page score, ``torch.topk``, attention over
the selected pages in fp32) with the cached block summaries of
``_build_prompt_blocks`` (CBT/core.py:449-500) as the block representatives, and the
fp32 attention of the dense oracle (CBT/legacy.py:797-868).  This module runs that
path on CPU tensors, one sequence at a time, reading K/V out of the paged pool
through the block table (the gather is part of the work), so that ``bench.py`` can
time it on the host cores next to the GPU path.

Pinned against the numpy oracle (``oracle.select`` / ``oracle.attention``) by
``tests/test_oracle.py::test_torch_path_matches_numpy_oracle``.
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
