"""GPU parity of the balanced launch plan: one flat grid whose workgroups each take a
subtile range of one (sequence, kv head) row, rows receiving items in proportion to
their work.  Rows of very different lengths, empty rows, idle workgroups, rows past
the plan's LDS stage (more than 2048 rows) and merges of one to many items must all
give the oracle's outputs, and the fused top-k call must stay bit-identical to the
two-step call (both plan from the same unit counts).  Bars as in test_gpu_paged.py.
"""

import math

import numpy as np
import pytest
import torch

import interattn_amd as ia
from oracle import attention as A
from oracle import select as S
from oracle.cases import make_case
from tests._util import announce, check_indices, oracle_summaries, to_dev

pytestmark = pytest.mark.gpu


def _run(case, device, hq, hkv, block, kvec, sample, dense_sample):
    dev = to_dev(case, device)
    lens = [int(x) for x in case["seq_lens"]]
    b = len(lens)
    nb_max = max(1, max(math.ceil(L / block) for L in lens))
    kb, counts, _ = oracle_summaries(case, block)
    kb_t = torch.from_numpy(kb).to(device=device, dtype=torch.bfloat16)
    k_cap = int(max(kvec))
    kv_t = torch.tensor(kvec, device=device, dtype=torch.int32)
    idx, n_sel = ia.select_blocks_topk(dev["q"], kb_t, dev["seq_lens"], 0, block_size=block, k_per_seq=kv_t,
                                       k_cap=k_cap, forced_last=1, forced_in_k=True)
    two = ia.sparse_paged_decode(dev["q"], dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"], idx,
                                 n_sel, block_size=block, workspace={})
    fused, idx2, n2 = ia.sparse_topk_decode(dev["q"], dev["pool_k"], dev["pool_v"], dev["block_table"],
                                            dev["seq_lens"], kb_t, 0, block_size=block, k_per_seq=kv_t, k_cap=k_cap,
                                            forced_last=1, forced_in_k=True, return_selection=True, workspace={})
    dense = ia.paged_decode(dev["q"], dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"],
                            max_seq_len=max(lens), workspace={})
    torch.cuda.synchronize()
    assert torch.equal(n2, n_sel)
    assert torch.equal(fused, two), "fused top-k decode differs from select + decode"
    idx_h, n_h = idx.cpu().numpy(), n_sel.cpu().numpy()
    got, gd = two.float().cpu().numpy(), dense.float().cpu().numpy()
    g = hq // hkv
    for i in sample:
        nb = math.ceil(lens[i] / block)
        sc = S.topk_block_scores(case["q"][i].astype(np.float64), kb[i], counts[i], g)
        sel = []
        for h in range(hkv):
            check_indices(idx_h[i, h], n_h[i, h], sc[h, :nb], nb, kvec[i], 0, 1, True)
            sel.append(idx_h[i, h, :n_h[i, h]])
        if lens[i]:
            ref = A.sparse_decode(case["q"][i], case["k"][i], case["v"][i], sel, block, p_bf16=True)
        else:  # an empty sequence: zero output
            ref = np.zeros_like(got[i])
        err = float(np.abs(got[i] - ref).max())
        assert err <= 2e-2, f"sparse seq {i} (len {lens[i]}): max abs err {err}"
    for i in dense_sample:
        ref = A.dense_decode(case["q"][i], case["k"][i], case["v"][i]) if lens[i] else np.zeros_like(gd[i])
        err = float(np.abs(gd[i] - ref).max())
        assert err <= 2e-2, f"dense seq {i} (len {lens[i]}): max abs err {err}"


def test_plan_extreme_ragged(device):
    """Rows from 0 to 12000 tokens: from one item per row up to many, with empty rows
    and idle workgroups at the end of the grid."""
    announce("balanced plan: extreme ragged batch")
    lens = [0, 1, 17, 129, 4096, 12000, 100, 65, 8000, 33]
    hq, hkv, d, block = 32, 8, 128, 64
    case = make_case(seed=4242, batch=len(lens), hq=hq, hkv=hkv, d=d, seq_lens=lens, page_size=16)
    kvec = [max(1, math.ceil(L / block) // 3) for L in lens]
    _run(case, device, hq, hkv, block, kvec, sample=range(len(lens)), dense_sample=range(len(lens)))


def test_plan_rows_past_lds_stage(device):
    """2400 (sequence, kv head) rows: the plan re-reads the unit counts of rows past
    its 2048-row LDS stage from global memory."""
    announce("balanced plan: 2400 rows")
    rng = np.random.default_rng(5150)
    b, hq, hkv, d, block = 300, 8, 8, 64, 16
    lens = rng.integers(0, 200, size=b).tolist()
    lens[7] = 1500  # one long row among many short ones
    case = make_case(seed=5151, batch=b, hq=hq, hkv=hkv, d=d, seq_lens=lens, page_size=16)
    kvec = [3] * b
    kvec[7] = 40
    sample = [0, 1, 7, 150, 298, 299]
    _run(case, device, hq, hkv, block, kvec, sample=sample, dense_sample=sample)


def test_plan_one_long_row(device):
    """A single (sequence, kv head) row spread over many items (merge of many slots)
    next to rows of one item each."""
    announce("balanced plan: one long row")
    lens = [30000, 20, 40]
    hq, hkv, d, block = 4, 1, 128, 32
    case = make_case(seed=31337, batch=len(lens), hq=hq, hkv=hkv, d=d, seq_lens=lens, page_size=16)
    kvec = [400, 1, 2]
    _run(case, device, hq, hkv, block, kvec, sample=range(len(lens)), dense_sample=range(len(lens)))


def test_dense_reads_nothing_past_max_seq_len(device):
    """A sequence longer than the launch's max_seq_len: the dense plan caps its tiles
    at ceil(max_seq_len / 128), so the call reads (and attends) the first 1024 tokens
    only and every row keeps its items within the partial stride."""
    announce("balanced plan: dense past max_seq_len")
    lens = [700, 5000]
    hq, hkv, d = 8, 2, 128
    case = make_case(seed=6060, batch=2, hq=hq, hkv=hkv, d=d, seq_lens=lens, page_size=16)
    dev = to_dev(case, device)
    out = ia.paged_decode(dev["q"], dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"],
                          max_seq_len=1000, workspace={})
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    ref0 = A.dense_decode(case["q"][0], case["k"][0], case["v"][0])
    ref1 = A.dense_decode(case["q"][1], case["k"][1][:, :1024], case["v"][1][:, :1024])
    assert np.abs(got[0] - ref0).max() <= 2e-2
    assert np.abs(got[1] - ref1).max() <= 2e-2
