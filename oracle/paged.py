"""Paged KV pool helpers for the oracle (test infrastructure only).

The reference keeps prompt K/V as one contiguous padded view per sequence,
``[Hkv, nb, B, D]`` addressed as ``head*head_stride + (page*B + t)*D``
(CBT/core.py:383-408, CBT/page_attention.py:223-230).  The BASELINE configs add
a vLLM-style pool: ``pool[n_pages, Hkv, page_size, D]`` plus a per-sequence
block table, so logical token ``t`` of sequence ``i`` lives at
``pool[block_table[i, t // page_size], :, t % page_size, :]``.  The oracle of
every paged function is "gather the pages by the table, then run the
contiguous restatement".
"""

import math

import numpy as np


def pages_for(seq_len, page_size):
    return int(math.ceil(int(seq_len) / int(page_size)))


def paged_gather(pool, block_table_row, seq_len, page_size):
    """Gather one sequence's ``[Hkv, seq_len, D]`` view out of the pool."""
    n = pages_for(seq_len, page_size)
    if n == 0:
        return np.zeros((pool.shape[1], 0, pool.shape[3]), dtype=pool.dtype)
    pages = pool[np.asarray(block_table_row[:n], dtype=np.int64)]      # [n, Hkv, P, D]
    seq = np.transpose(pages, (1, 0, 2, 3)).reshape(pool.shape[1], n * page_size, pool.shape[3])
    return seq[:, : int(seq_len)]


def build_pool(seqs, page_size, rng, n_pages=None, fill=0.0):
    """Scatter contiguous per-sequence ``[Hkv, L, D]`` arrays into a permuted pool.

    Returns ``(pool, block_table)``; each sequence takes ``ceil(L/page)`` pages
    from one shared ``rng.permutation`` of the pool (the C2-C4 page recipe).
    Unused pool pages keep ``fill``; unused block-table slots are -1.
    """
    hkv, d = seqs[0].shape[0], seqs[0].shape[2]
    need = [pages_for(s.shape[1], page_size) for s in seqs]
    total = sum(need)
    if n_pages is None:
        n_pages = max(total, 1)
    if total > n_pages:
        raise ValueError("pool too small")
    perm = rng.permutation(n_pages)
    pool = np.full((n_pages, hkv, page_size, d), fill, dtype=seqs[0].dtype)
    max_pages = max(max(need), 1)
    table = np.full((len(seqs), max_pages), -1, dtype=np.int32)
    cursor = 0
    for i, s in enumerate(seqs):
        n = need[i]
        ids = perm[cursor:cursor + n]
        cursor += n
        table[i, :n] = ids
        padded = np.zeros((hkv, n * page_size, d), dtype=s.dtype)
        padded[:, : s.shape[1]] = s
        pool[ids] = np.transpose(padded.reshape(hkv, n, page_size, d), (1, 0, 2, 3))
    return pool, table
