"""The top-k selection rule on adversarial score rows, exactly.

The workgroup selection (bucketed threshold search with exact ranks in the
threshold bucket, radix-select fallback, ordered compaction) must pick exactly
the blocks of the oracle's rule -- score descending, ties to the lowest index,
forced first/last blocks always in -- applied to the kernel's own scores (no
near-tie allowance: the scores are the same numbers).  The rows are built from
repeated k_bar rows so that exact ties are frequent:

* ``dup5``: five distinct rows, massive ties at every score;
* ``zero``: every score equal (the whole row is one tie);
* ``crowd``: random rows plus 400 copies of the best one (a crowded threshold
  bucket: the radix fallback and its tie scan);
* ``crowd100``: 100 copies of the best row (a threshold bucket of 65..128 members,
  ranked through LDS);
* ``crowd40``: 40 copies of the best row at three nearby scales (a threshold bucket
  of at most 64 members, ranked from registers in every wave; ties and distinct
  keys);
* ``inf``: positive queries and rows of +-3e38 (scores of +-inf, the non-finite
  fallback);
* ``far``: random rows plus a few scaled by 1e6 (a huge range, most candidates in
  one bucket);
* ``random``: plain random rows (the bucket fast path).
Both the standalone selector (one workgroup) and the fused layer call (one wave of
the finalize prologue) are checked; the standalone one also on 20000-block rows,
whose ties sit in the second compaction chunk, the fused one on 4000-block rows.
"""

import math

import numpy as np
import pytest
import torch

import interattn_amd as ia
from oracle import select as S
from tests._util import announce

pytestmark = pytest.mark.gpu

HQ, HKV, D, BLOCK, PAGE = 8, 2, 64, 16, 16
PATTERNS = ["dup5", "zero", "crowd", "inf", "far", "random", "crowd100", "crowd40"]
RULES = [(37, 0, 0, False), (37, 2, 3, False), (40, 1, 2, True)]


def _rows(pattern, nb, rng):
    kb = rng.standard_normal((HKV, nb, D)).astype(np.float32)
    q = rng.standard_normal((HQ, D)).astype(np.float32)
    if pattern == "dup5":
        base = rng.standard_normal((HKV, 5, D)).astype(np.float32)
        kb = base[:, rng.integers(0, 5, nb)]
    elif pattern == "zero":
        kb[:] = 0.0
    elif pattern in ("crowd", "crowd100", "crowd40"):
        m = {"crowd": 400, "crowd100": 100, "crowd40": 40}[pattern]
        qm = q.reshape(HKV, HQ // HKV, D).sum(1)
        for h in range(HKV):
            best = kb[h, np.argmax(kb[h] @ qm[h])].copy()
            pick = rng.choice(nb, m, replace=False)
            scale = rng.choice([1.0, 1.0 - 1.0 / 128, 1.0 - 1.0 / 64], m) if pattern == "crowd40" else np.ones(m)
            kb[h, pick] = best[None] * scale[:, None].astype(np.float32)
    elif pattern == "inf":
        q = np.abs(q) + 0.1
        pick = rng.choice(nb, 60, replace=False)
        kb[:, pick[:30]] = 3.0e38
        kb[:, pick[30:]] = -3.0e38
    elif pattern == "far":
        kb[:, rng.choice(nb, 5, replace=False)] *= 1.0e6
    return q, kb


def _to_dev(q, kb, device):
    q_t = torch.from_numpy(np.ascontiguousarray(q[None])).to(device=device, dtype=torch.bfloat16)
    kb_t = torch.from_numpy(np.ascontiguousarray(kb[None])).to(device=device, dtype=torch.bfloat16)
    return q_t, kb_t


def _check(idx, n_sel, scores, nb, rule):
    k, ff, fl, in_k = rule
    for h in range(HKV):
        ref = S.select_topk(scores[h, :nb], nb, k, ff, fl, in_k)
        got = idx[h, :n_sel[h]]
        assert np.array_equal(got, ref), (h, got[:10], ref[:10], len(got), len(ref))


@pytest.mark.parametrize("rule", RULES, ids=["k37", "k37_f2_3", "k40_in"])
@pytest.mark.parametrize("pattern", PATTERNS)
def test_selection_rule_exact(pattern, rule, device):
    announce(f"selection rule {pattern} {rule}")
    rng = np.random.default_rng(4242 + PATTERNS.index(pattern))
    nb = 1500
    L = nb * BLOCK - 5
    q, kb = _rows(pattern, nb, rng)
    q_t, kb_t = _to_dev(q, kb, device)
    seq = torch.tensor([L], device=device, dtype=torch.int32)
    k, ff, fl, in_k = rule
    idx, n_sel, scores = ia.select_blocks_topk(q_t, kb_t, seq, k, block_size=BLOCK, forced_first=ff,
                                               forced_last=fl, forced_in_k=in_k, return_scores=True)
    # the fused call on a small pool (values irrelevant to the selection)
    n_pages = math.ceil(L / PAGE)
    pool_k = torch.randn((n_pages, HKV, PAGE, D), device=device, dtype=torch.bfloat16)
    pool_v = torch.randn((n_pages, HKV, PAGE, D), device=device, dtype=torch.bfloat16)
    table = torch.arange(n_pages, device=device, dtype=torch.int32)[None]
    _, idx_f, n_f = ia.sparse_topk_decode(q_t, pool_k, pool_v, table, seq, kb_t, k, block_size=BLOCK,
                                          forced_first=ff, forced_last=fl, forced_in_k=in_k,
                                          return_selection=True, workspace={})
    torch.cuda.synchronize()
    sc = scores[0].float().cpu().numpy()
    _check(idx[0].cpu().numpy(), n_sel[0].cpu().numpy(), sc, nb, rule)
    _check(idx_f[0].cpu().numpy(), n_f[0].cpu().numpy(), sc, nb, rule)


@pytest.mark.parametrize("pattern", ["late_ties", "zero", "random"])
def test_selection_rule_long_rows(pattern, device):
    """20000 blocks: the standalone selector's scans run over more than one chunk."""
    announce(f"selection rule long rows {pattern}")
    rng = np.random.default_rng(99)
    nb = 20000
    L = nb * BLOCK
    q, kb = _rows("random" if pattern == "late_ties" else pattern, nb, rng)
    if pattern == "late_ties":
        kb[:, :17000] *= 0.01
        qm = q.reshape(HKV, HQ // HKV, D).sum(1)
        for h in range(HKV):
            kb[h, 17000:] = 10.0 * qm[h] / np.linalg.norm(qm[h])
    q_t, kb_t = _to_dev(q, kb, device)
    seq = torch.tensor([L], device=device, dtype=torch.int32)
    rule = (37, 2, 3, False)
    idx, n_sel, scores = ia.select_blocks_topk(q_t, kb_t, seq, rule[0], block_size=BLOCK, forced_first=rule[1],
                                               forced_last=rule[2], return_scores=True)
    torch.cuda.synchronize()
    _check(idx[0].cpu().numpy(), n_sel[0].cpu().numpy(), scores[0].float().cpu().numpy(), nb, rule)


@pytest.mark.parametrize("pattern", ["dup5", "zero", "crowd", "crowd40", "random"])
def test_fused_selection_rule_4000(pattern, device):
    """The fused call's one-wave selection on 4000-block rows (63 chunks of 64)."""
    announce(f"fused selection rule 4000 {pattern}")
    rng = np.random.default_rng(7 + PATTERNS.index(pattern))
    nb = 4000
    L = nb * BLOCK - 3
    q, kb = _rows(pattern, nb, rng)
    q_t, kb_t = _to_dev(q, kb, device)
    seq = torch.tensor([L], device=device, dtype=torch.int32)
    rule = (300, 2, 3, False)
    _, _, scores = ia.select_blocks_topk(q_t, kb_t, seq, rule[0], block_size=BLOCK, forced_first=rule[1],
                                         forced_last=rule[2], return_scores=True)
    n_pages = math.ceil(L / PAGE)
    pool_k = torch.randn((n_pages, HKV, PAGE, D), device=device, dtype=torch.bfloat16)
    pool_v = torch.randn((n_pages, HKV, PAGE, D), device=device, dtype=torch.bfloat16)
    table = torch.arange(n_pages, device=device, dtype=torch.int32)[None]
    _, idx_f, n_f = ia.sparse_topk_decode(q_t, pool_k, pool_v, table, seq, kb_t, rule[0], block_size=BLOCK,
                                          forced_first=rule[1], forced_last=rule[2], return_selection=True,
                                          workspace={})
    torch.cuda.synchronize()
    _check(idx_f[0].cpu().numpy(), n_f[0].cpu().numpy(), scores[0].float().cpu().numpy(), nb, rule)
