"""Serving-pool maintenance on the GPU: incremental block summaries, the paged K/V
append, and one whole decode step (append, summary refresh, top-k select,
finalize) captured in a graph and replayed.

Bars: an incremental refresh equals a full rebuild bit for bit (same kernel, same
blocks); the append writes exactly the given rows and advances only mapped
sequences; every graph replay equals the eager step on the same state bit for bit,
and the eager step matches the oracle (2e-2 abs, bf16).
"""

import math
import zlib

import numpy as np
import pytest
import torch

import interattn_amd as ia
from oracle import attention as A
from oracle import select as S
from oracle.cases import make_case
from oracle.paged import paged_gather
from tests._util import announce, check_indices, to_dev

pytestmark = pytest.mark.gpu

SUMMARY_KEYS = ("k_bar", "v_bar", "k_max", "k_min", "v_norm_max", "v_norm_all", "block_valid_counts")


def _full(dev, lens, block, nb_max, dtype):
    seq = torch.tensor(lens, device=dev["pool_k"].device, dtype=torch.int32)
    return ia.build_block_summaries(dev["pool_k"], dev["pool_v"], dev["block_table"], seq, block, nb_max=nb_max,
                                    full=True, k_bar_dtype=dtype, v_bar_dtype=dtype, scales=dev["scales"])


# old lengths -> new lengths (the pool holds the new lengths' tokens)
UPDATE_CASES = [
    ("one_token_partial", [1000, 333], [1001, 334], 64, "bf16"),
    ("one_token_new_block", [1024, 320], [1025, 321], 64, "bf16"),
    ("fill_block", [1023, 319], [1024, 320], 64, "bf16"),
    ("many_tokens", [500, 10], [900, 700], 32, "bf16"),
    ("from_empty", [0, 0], [77, 128], 128, "bf16"),
    ("f32_pool", [200, 64], [260, 65], 16, "f32"),
    ("fp8_pool", [511, 100], [530, 130], 64, "fp8"),
]


@pytest.mark.parametrize("c", UPDATE_CASES, ids=[c[0] for c in UPDATE_CASES])
def test_update_equals_rebuild(c, device):
    name, old, new, block, dt = c
    announce(f"summary update {name}")
    case = make_case(seed=zlib.crc32(name.encode()) % 10000, batch=2, hq=16, hkv=4, d=128, seq_lens=new, page_size=16,
                     dtype="f32" if dt == "f32" else "bf16", fp8=(dt == "fp8"))
    dev = to_dev(case, device, dtype=torch.float32 if dt == "f32" else torch.bfloat16, fp8=(dt == "fp8"))
    nb_max = max(math.ceil(L / block) for L in new) + 1
    sdt = torch.float32 if dt == "f32" else torch.bfloat16
    ref = _full(dev, new, block, nb_max, sdt)
    got = _full(dev, old, block, nb_max, sdt)
    old_t = torch.tensor(old, device=device, dtype=torch.int32)
    new_t = torch.tensor(new, device=device, dtype=torch.int32)
    ia.update_block_summaries(got, dev["pool_k"], dev["pool_v"], dev["block_table"], old_t, new_t, block,
                              max_new_tokens=max(n - o for n, o in zip(new, old)), scales=dev["scales"])
    torch.cuda.synchronize()
    for key in SUMMARY_KEYS:
        assert torch.equal(got[key], ref[key]), key


def _pool(device, n_seq, hkv, d, page, pages_per_seq, dtype, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    n_pages = n_seq * pages_per_seq + 3
    pool_k = torch.randn((n_pages, hkv, page, d), generator=g).to(device=device, dtype=dtype)
    pool_v = torch.randn((n_pages, hkv, page, d), generator=g).to(device=device, dtype=dtype)
    perm = torch.randperm(n_pages, generator=g)[:n_seq * pages_per_seq].view(n_seq, pages_per_seq)
    return pool_k, pool_v, perm.to(device=device, dtype=torch.int32)


def test_append_kv_writes_rows(device):
    announce("append_kv")
    hkv, d, page = 4, 128, 16
    pool_k, pool_v, table = _pool(device, 3, hkv, d, page, 4, torch.bfloat16, 5)
    lens = torch.tensor([0, 17, 64], device=device, dtype=torch.int32)  # 64 = capacity of 4 pages: not mapped
    k_new = torch.randn((3, hkv, d), device=device).to(torch.bfloat16)
    v_new = torch.randn((3, hkv, d), device=device).to(torch.bfloat16)
    before_k = pool_k.clone()
    ia.append_kv(pool_k, pool_v, table, lens, k_new, v_new)
    torch.cuda.synchronize()
    assert lens.tolist() == [1, 18, 64]
    for b, pos in ((0, 0), (1, 17)):
        pg = int(table[b, pos // page])
        assert torch.equal(pool_k[pg, :, pos % page], k_new[b])
        assert torch.equal(pool_v[pg, :, pos % page], v_new[b])
    # nothing else changed
    diff = (pool_k != before_k).any(dim=3)  # [n_pages, Hkv, page]: one row per head per token
    assert int(diff.sum()) == 2 * hkv


def _check_step_vs_oracle(pool_k, pool_v, table, lens, q, k_bar, block, k, page, out):
    """The GPU selection of the final state matches the oracle's (near-tie rule) and
    the output matches the oracle's attention over the GPU's selection (float64)."""
    idx, n_sel = ia.select_blocks_topk(q, k_bar, lens, k, block_size=block)
    torch.cuda.synchronize()
    pk, pv = pool_k.float().cpu().numpy(), pool_v.float().cpu().numpy()
    tb, ln = table.cpu().numpy(), lens.cpu().numpy()
    qh, kb = q.float().cpu().numpy(), k_bar.float().cpu().numpy()
    idx_h, ns_h = idx.cpu().numpy(), n_sel.cpu().numpy()
    hq, hkv = q.shape[1], pool_k.shape[1]
    for b in range(q.shape[0]):
        L = int(ln[b])
        nb = math.ceil(L / block)
        counts = np.array([min(block, L - j * block) for j in range(nb)])
        sc = S.topk_block_scores(qh[b].astype(np.float64), kb[b, :, :nb], counts, hq // hkv)
        sel = []
        for h in range(hkv):
            check_indices(idx_h[b, h], ns_h[b, h], sc[h], nb, k, 0, 0, False)
            sel.append(idx_h[b, h, :ns_h[b, h]])
        kk = paged_gather(pk, tb[b], L, page)
        vv = paged_gather(pv, tb[b], L, page)
        exp = A.sparse_decode(qh[b], kk, vv, sel, block, p_bf16=True)
        np.testing.assert_allclose(out[b].float().cpu().numpy(), exp, atol=2e-2, rtol=0)


def test_graph_captured_serving_step(device):
    """append -> summary refresh -> select -> finalize, captured once, replayed 4 times."""
    announce("graph-captured serving step")
    hkv, hq, d, page, block, k = 4, 16, 128, 16, 64, 4
    n_seq, pages_per_seq = 2, 40
    pool_k, pool_v, table = _pool(device, n_seq, hkv, d, page, pages_per_seq, torch.bfloat16, 9)
    lens0 = torch.tensor([300, 511], device=device, dtype=torch.int32)
    nb_max = pages_per_seq * page // block
    summ = ia.build_block_summaries(pool_k, pool_v, table, lens0, block, nb_max=nb_max, k_bar_dtype=torch.bfloat16)
    steps = 5
    gen = torch.Generator(device="cpu").manual_seed(3)
    qs = [torch.randn((n_seq, hq, d), generator=gen).to(device=device, dtype=torch.bfloat16) for _ in range(steps)]
    ks = [torch.randn((n_seq, hkv, d), generator=gen).to(device=device, dtype=torch.bfloat16) for _ in range(steps)]
    vs = [torch.randn((n_seq, hkv, d), generator=gen).to(device=device, dtype=torch.bfloat16) for _ in range(steps)]

    state0 = (pool_k.clone(), pool_v.clone(), lens0.clone(), {kk: v.clone() for kk, v in summ.items()})
    q_in = torch.empty_like(qs[0])
    k_in = torch.empty_like(ks[0])
    v_in = torch.empty_like(vs[0])
    lens = lens0.clone()
    old = torch.empty_like(lens)
    ws = {}
    out = torch.empty_like(q_in)

    def step():
        old.copy_(lens)
        ia.append_kv(pool_k, pool_v, table, lens, k_in, v_in)
        ia.update_block_summaries(summ, pool_k, pool_v, table, old, lens, block, max_new_tokens=1)
        ia.sparse_topk_decode(q_in, pool_k, pool_v, table, lens, summ["k_bar"], k, block_size=block,
                              out=out, workspace=ws)

    # eager reference run of all steps, from the initial state
    eager_outs = []
    for i in range(steps):
        q_in.copy_(qs[i]); k_in.copy_(ks[i]); v_in.copy_(vs[i])
        step()
        eager_outs.append(out.clone())
    torch.cuda.synchronize()
    eager_state = (pool_k.clone(), lens.clone(), summ["k_bar"].clone())
    _check_step_vs_oracle(pool_k, pool_v, table, lens, qs[-1], summ["k_bar"], block, k, page, eager_outs[-1])

    # restore the initial state, run step 0 eagerly (workspaces), capture step 1, replay the rest
    pool_k.copy_(state0[0]); pool_v.copy_(state0[1]); lens.copy_(state0[2])
    for kk, v in state0[3].items():
        summ[kk].copy_(v)
    q_in.copy_(qs[0]); k_in.copy_(ks[0]); v_in.copy_(vs[0])
    step()
    torch.cuda.synchronize()
    assert torch.equal(out, eager_outs[0])
    q_in.copy_(qs[1]); k_in.copy_(ks[1]); v_in.copy_(vs[1])
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph):
            step()
    torch.cuda.current_stream().wait_stream(s)
    # capture records without running: step 1 runs on the first replay
    for i in range(1, steps):
        q_in.copy_(qs[i]); k_in.copy_(ks[i]); v_in.copy_(vs[i])
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager_outs[i]), f"replay {i}"
    assert torch.equal(pool_k, eager_state[0])
    assert torch.equal(lens, eager_state[1])
    assert torch.equal(summ["k_bar"], eager_state[2])
