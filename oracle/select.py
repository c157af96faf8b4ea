"""Block selection (test infrastructure only).

Two rules live behind the one selection boundary:

* **top-k** (BASELINE configs): ``score_b = mean_g(q_g . k_bar_b) / sqrt(D)`` per
  (sequence, kv-head); the group-mean convention and ``torch.topk`` follow the
  Quest baseline (CBG/methods/quest.py:91-103).  Forced sink/local blocks are
  added on top of (or inside) ``k``; ties break toward the lower block index.
* **condition(eps)** (reference parity): the eager rule of
  ``_select_prompt_blocks_eager`` (CBT/core.py:509-555) and its chunked Triton
  form (CBT/core.py:747-905, CBT/page_attention.py:72-171).
"""

import math

import numpy as np


# --------------------------------------------------------------------------- top-k

def topk_block_scores(q, k_bar, counts, group):
    """``q [Hq, D]``, ``k_bar [Hkv, nb, D]``, ``counts [nb]`` -> ``[Hkv, nb]`` float64.

    Group-mean representative score (CBG/methods/quest.py:101, ``score.mean(dim=0)``
    over the GQA group), with the mean key as the representative.  Empty blocks
    (count 0) score -inf.
    """
    hq, d = q.shape
    hkv = k_bar.shape[0]
    qg = q.astype(np.float64).reshape(hkv, group, d)
    s = np.einsum("hgd,hbd->hgb", qg, k_bar.astype(np.float64)) / math.sqrt(d)
    s = s.mean(axis=1)
    s[:, np.asarray(counts) <= 0] = -np.inf
    return s


def quest_block_scores(q, k_max, k_min, group):
    """``q [Hq, D]``, ``k_max, k_min [Hkv, nb, D]`` -> ``[Hkv, nb]`` float64.

    The Quest page score (CBG/methods/quest.py:97-101): per query head,
    ``sum_d max(q_d * k_max_d, q_d * k_min_d)`` (an upper bound of ``q . k_t`` over the
    block's tokens, no ``1/sqrt(D)``), then the mean over the GQA group.  Blocks with
    no valid token (``k_max = -inf``) score -inf.
    """
    hq, d = q.shape
    hkv = k_max.shape[0]
    qg = q.astype(np.float64).reshape(hkv, group, 1, d)
    kx = k_max.astype(np.float64)[:, None]
    kn = k_min.astype(np.float64)[:, None]
    with np.errstate(invalid="ignore"):
        s = np.maximum(qg * kx, qg * kn).sum(-1).mean(axis=1)
    s[~np.isfinite(k_max.astype(np.float64)).all(-1)] = -np.inf
    return s


def forced_blocks(nb_valid, forced_first, forced_last):
    f = set(range(min(int(forced_first), nb_valid)))
    f |= set(range(max(nb_valid - int(forced_last), 0), nb_valid))
    return sorted(f)


def select_topk(scores, nb_valid, k, forced_first=0, forced_last=0, forced_in_k=False):
    """Sorted block indices chosen for one (sequence, kv-head).

    ``forced`` = the first ``forced_first`` and last ``forced_last`` valid blocks.
    ``k_eff = k - len(forced)`` when ``forced_in_k`` (C1: "top-8 always including the
    last block") else ``k`` (C2: "top-64 plus the first block and the last 2").
    The remaining blocks are ranked by score, descending, ties to the lower index
    (a stable order; ``torch.topk`` leaves exact ties unspecified).
    """
    nb_valid = int(nb_valid)
    forced = forced_blocks(nb_valid, forced_first, forced_last)
    k_eff = int(k) - len(forced) if forced_in_k else int(k)
    k_eff = max(k_eff, 0)
    fset = set(forced)
    cand = np.array([j for j in range(nb_valid) if j not in fset], dtype=np.int64)
    if len(cand) and k_eff > 0:
        sc = np.asarray(scores, dtype=np.float64)[cand]
        order = np.lexsort((cand, -sc))            # primary: score desc, then index asc
        chosen = cand[order[:k_eff]]
    else:
        chosen = np.zeros(0, dtype=np.int64)
    return np.array(sorted(set(chosen.tolist()) | fset), dtype=np.int32)


def topk_threshold(scores, nb_valid, k, forced_first=0, forced_last=0, forced_in_k=False):
    """Score of the last block admitted by rank (None when selection is not rank-limited)."""
    forced = set(forced_blocks(int(nb_valid), forced_first, forced_last))
    k_eff = int(k) - len(forced) if forced_in_k else int(k)
    cand = [j for j in range(int(nb_valid)) if j not in forced]
    if k_eff <= 0 or k_eff >= len(cand):
        return None
    sc = np.sort(np.asarray(scores, dtype=np.float64)[cand])[::-1]
    return float(sc[k_eff - 1])


# ---------------------------------------------------------------- condition(eps)

def select_condition_eager(q_grouped, prefix, eps, term1_mass_exp=False):
    """Restates ``_select_prompt_blocks_eager`` (CBT/core.py:509-555) in float64.

    ``q_grouped [Hkv, G, 1, D]``.  Returns ``(selected [Hkv,G,1,nb] bool, z [Hkv,G,1,nb])``.
    ``term1_mass_exp`` switches term 1 to ``2 B softmax(z + delta)``
    (CBT/page_attention.py:127-141, CBT/core.py:886-889).
    """
    hkv, g, nq, d = q_grouped.shape
    scale = math.sqrt(d)
    size = np.asarray(prefix["block_valid_counts"]).astype(np.int64)
    exists = size > 0
    size_f = np.maximum(size, 1).astype(np.float64)
    q = q_grouped.astype(np.float64)
    k_bar = prefix["k_bar"].astype(np.float64)
    k_max = prefix["k_max"].astype(np.float64)
    k_min = prefix["k_min"].astype(np.float64)
    s_c = np.einsum("gsqd,gbd->gsqb", q, k_bar) / scale                       # core.py:523
    qb = q[:, :, :, None, :]
    a = qb * k_max[:, None, None]
    b = qb * k_min[:, None, None]
    upper = np.maximum(a, b).sum(-1) / scale                                   # core.py:525-528
    lower = np.minimum(a, b).sum(-1) / scale                                   # core.py:529-532
    delta = np.maximum(np.abs(upper - s_c), np.abs(lower - s_c))               # core.py:533
    delta = np.where(exists, delta, 0.0)
    b_c = np.broadcast_to(prefix["v_norm_max"].astype(np.float64)[:, None, None, :], delta.shape)
    b_c = np.where(exists, b_c, 0.0)
    b_all = b_c.max(axis=-1)                                                   # core.py:538
    z = np.log(size_f) + s_c                                                   # core.py:540
    z = np.where(exists, z, -np.inf)
    zmax = z.max(axis=-1, keepdims=True)
    ez = np.exp(z - zmax)
    p = ez / ez.sum(axis=-1, keepdims=True)                                    # core.py:542
    if term1_mass_exp:
        zc = z + delta
        cm = zc.max(axis=-1, keepdims=True)
        ec = np.exp(zc - cm)
        term1 = 2.0 * b_all[..., None] * ec / ec.sum(axis=-1, keepdims=True)
    else:
        denom = np.maximum((p * np.cosh(delta)).sum(axis=-1), 1e-30)           # core.py:543
        term1 = 2.0 * b_all[..., None] * (np.cosh(delta) - 1.0) / denom[..., None] * p
    cond = term1 + p * 2.0 * b_c * np.tanh(delta / 2.0)                         # core.py:544-547
    cond = np.where(exists, cond, 0.0)
    sel = (cond.mean(axis=1, keepdims=True) > eps) & exists                    # core.py:549
    sel = np.broadcast_to(sel, (hkv, g, nq, len(size))).copy()
    return sel, z


def selection_stats_chunked(q, prefix, group, chunk=16, term1_mass_exp=False):
    """Restates ``_condition_block_selection_stats_kernel`` (CBT/core.py:751-814) and
    ``_condition_block_selection_reduce_kernel`` (CBT/core.py:821-847).

    ``q [rows, D]`` with rows = Hkv*G.  Returns a dict with ``s, delta [rows, nb]``
    (0 where the block is empty), ``partial [4, rows, n_chunks]`` = (z_m, z_l, c_m, c_l)
    per chunk and ``globals [4, rows]``.
    """
    rows, d = q.shape
    hkv = rows // group
    scale = d ** -0.5
    counts = np.asarray(prefix["block_valid_counts"]).astype(np.int64)
    nb = len(counts)
    active = counts > 0
    qf = q.astype(np.float64).reshape(hkv, group, d)
    kb = prefix["k_bar"].astype(np.float64)
    kh = prefix["k_max"].astype(np.float64)
    kl = prefix["k_min"].astype(np.float64)
    s = np.einsum("hgd,hbd->hgb", qf, kb) * scale
    pos = qf[:, :, None, :] >= 0.0
    upper_k = np.where(pos, kh[:, None], kl[:, None])                         # core.py:788
    lower_k = np.where(pos, kl[:, None], kh[:, None])                         # core.py:789
    upper = (qf[:, :, None, :] * upper_k).sum(-1) * scale
    lower = (qf[:, :, None, :] * lower_k).sum(-1) * scale
    delta = np.maximum(np.abs(upper - s), np.abs(lower - s))
    z = s + np.log(np.maximum(counts, 1).astype(np.float64))[None, None]
    z = np.where(active[None, None], z, -np.inf)
    if term1_mass_exp:
        zc = z + delta
    else:
        zc = z + np.log(0.5 * (np.exp(delta) + np.exp(-delta)))
    s = np.where(active[None, None], s, 0.0).reshape(rows, nb)
    delta = np.where(active[None, None], delta, 0.0).reshape(rows, nb)
    z = z.reshape(rows, nb)
    zc = zc.reshape(rows, nb)
    n_chunks = int(math.ceil(nb / chunk))
    part = np.zeros((4, rows, n_chunks))
    for c in range(n_chunks):
        sl = slice(c * chunk, min((c + 1) * chunk, nb))
        for i, arr in ((0, z), (2, zc)):
            m = arr[:, sl].max(axis=1)
            with np.errstate(invalid="ignore"):
                l = np.exp(arr[:, sl] - m[:, None]).sum(axis=1)
            l = np.where(np.isneginf(m), 0.0, l)       # an all-empty chunk contributes nothing
            part[i, :, c] = m
            part[i + 1, :, c] = l
    glob = np.zeros((4, rows))
    for i in (0, 2):
        gm = part[i].max(axis=1)
        glob[i] = gm
        with np.errstate(invalid="ignore"):
            w = np.where(np.isneginf(part[i]), 0.0, np.exp(part[i] - gm[:, None]))
        glob[i + 1] = (part[i + 1] * w).sum(axis=1)
    return {"s": s, "delta": delta, "z": z, "partial": part, "globals": glob, "n_chunks": n_chunks}


def selection_finalize(stats, prefix, group, eps, term1_mass_exp=False):
    """Restates ``_condition_block_selection_finalize_kernel`` (CBT/core.py:858-905) and the
    inline condition of the fused kernel (CBT/page_attention.py:126-165).

    Returns ``selected [rows, nb]`` (broadcast over the group) and ``z [rows, nb]``.
    """
    mean, z = condition_group_mean(stats, prefix, group, term1_mass_exp)
    active = np.asarray(prefix["block_valid_counts"]).astype(np.int64) > 0
    sel = (mean > eps) & active[None]
    return np.repeat(sel, group, axis=0), z


def condition_group_mean(stats, prefix, group, term1_mass_exp=False):
    """The group-mean condition ``[Hkv, nb]`` that ``selection_finalize`` thresholds
    (0 for empty blocks), and ``z [rows, nb]``."""
    s, delta = stats["s"], stats["delta"]
    rows, nb = s.shape
    hkv = rows // group
    counts = np.asarray(prefix["block_valid_counts"]).astype(np.int64)
    active = counts > 0
    z = s + np.log(np.maximum(counts, 1).astype(np.float64))[None]
    zm, zl, cm, cl = stats["globals"]
    b_c = np.where(active[None], prefix["v_norm_max"].astype(np.float64), 0.0)    # [hkv, nb]
    b_c = np.repeat(b_c, group, axis=0)
    b_all = np.repeat(prefix["v_norm_all"].astype(np.float64), group)[:, None]
    if term1_mass_exp:
        tanh_half = (1.0 - np.exp(-delta)) / (1.0 + np.exp(-delta))
        term1 = 2.0 * b_all * np.exp(z + delta - cm[:, None]) / cl[:, None]
    else:
        cosh = 0.5 * (np.exp(delta) + np.exp(-delta))
        tanh_half = 2.0 / (1.0 + np.exp(-delta)) - 1.0
        term1 = 2.0 * b_all * np.exp(z - cm[:, None]) * (cosh - 1.0) / cl[:, None]
    term2 = 2.0 * b_c * np.exp(z - zm[:, None]) * tanh_half / zl[:, None]
    cond = np.where(active[None], term1 + term2, 0.0)
    return cond.reshape(hkv, group, nb).sum(axis=1) / group, z


def condition_stats(selected, counts, prompt_len, suffix_len):
    """Restates ``_condition_stats`` (CBT/core.py:1441-1456) for one query position.

    ``selected [Hkv, G, 1, nb]`` bool, ``counts [nb]``.  Returns the reference's keys:
    rows, clusters, selected_clusters, selected_tokens, hybrid_tokens, total_available.
    """
    hkv, g, nq, nb = selected.shape
    counts = np.asarray(counts).astype(np.int64)
    exists = counts > 0
    sel = np.asarray(selected, dtype=bool)
    selected_tokens = int((sel.astype(np.int64) * counts[None, None, None]).sum())
    cluster_active = (~sel) & exists[None, None, None]
    rows = hkv * g * nq
    return {
        "rows": rows,
        "clusters": int(exists.sum()) * hkv * g,
        "selected_clusters": int(sel.sum()),
        "selected_tokens": selected_tokens,
        "hybrid_tokens": selected_tokens + int(cluster_active.sum()) + max(int(suffix_len), 0) * hkv * g,
        "total_available": (int(prompt_len) + max(int(suffix_len), 0)) * rows,
    }
