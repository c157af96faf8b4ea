"""Pins the CPU oracle (CPU only).

Each check compares an oracle function with an independent computation: a torch
library routine, a brute-force loop, a closed form or an invariant, chosen so that a
dropped term, a wrong index or a transposed operand fails.
"""

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import numerics as Nm
from oracle import paged as P
from oracle import select as S
from oracle import summaries as Su
from oracle.cases import make_case


# ------------------------------------------------------------------ numerics

def test_bf16_round_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 20000),
        np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 3.0e38, -3.0e38, 1e-40, np.inf, -np.inf], np.float32),
    ]).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    got = Nm.bf16_round(x)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_bf16_round_ties_to_even():
    # 1 + 2^-8 is exactly halfway between bf16 neighbours 1 and 1 + 2^-7: ties to even (1.0)
    assert Nm.bf16_round(np.float32(1.0 + 2.0 ** -8)) == np.float32(1.0)
    assert Nm.bf16_round(np.float32(1.0 + 3 * 2.0 ** -8)) == np.float32(1.0 + 2.0 ** -6)


@pytest.mark.skipif(not hasattr(torch, "float8_e4m3fn"), reason="torch without float8")
def test_e4m3_decode_table_matches_torch():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    got = Nm.e4m3_decode(codes)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], ref[~nan])
    assert np.nanmax(Nm.E4M3_VALUES) == 448.0


@pytest.mark.skipif(not hasattr(torch, "float8_e4m3fn"), reason="torch without float8")
def test_e4m3_encode_matches_torch():
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.uniform(-448, 448, 20000), rng.standard_normal(20000) * 0.01,
        Nm.E4M3_VALUES[:127], -Nm.E4M3_VALUES[:127],
        (Nm.E4M3_VALUES[1:127] + Nm.E4M3_VALUES[:126]) / 2,     # exact midpoints: ties to even
    ]).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = Nm.e4m3_encode(x)
    # +0/-0 encode differently only in sign; compare decoded values
    assert np.array_equal(Nm.e4m3_decode(got), Nm.e4m3_decode(ref))


# ------------------------------------------------------------------ paging

def test_paged_gather_brute_force_and_permutation_invariance():
    rng = np.random.default_rng(2)
    seqs = [rng.standard_normal((2, L, 8)).astype(np.float32) for L in (37, 64, 1, 100)]
    for seed in (3, 4):
        pool, table = P.build_pool(seqs, 16, np.random.default_rng(seed), n_pages=40)
        for i, s in enumerate(seqs):
            g = P.paged_gather(pool, table[i], s.shape[1], 16)
            brute = np.zeros_like(s)
            for t in range(s.shape[1]):
                brute[:, t] = pool[table[i, t // 16], :, t % 16]
            assert np.array_equal(g, s)
            assert np.array_equal(brute, s)


# ------------------------------------------------------------------ summaries

def _brute_summaries(k, v, block):
    hkv, L, d = k.shape
    nb = math.ceil(L / block)
    out = {n: np.zeros((hkv, nb, d)) for n in ("k_bar", "v_bar", "k_max", "k_min")}
    vnm = np.full((hkv, nb), -np.inf)
    counts = np.zeros(nb, np.int64)
    for j in range(nb):
        toks = list(range(j * block, min((j + 1) * block, L)))
        counts[j] = len(toks)
        for h in range(hkv):
            for t in toks:
                out["k_bar"][h, j] += k[h, t]
                out["v_bar"][h, j] += v[h, t]
                vnm[h, j] = max(vnm[h, j], math.sqrt(float(np.dot(v[h, t].astype(np.float64), v[h, t]))))
            out["k_bar"][h, j] /= max(len(toks), 1)
            out["v_bar"][h, j] /= max(len(toks), 1)
            out["k_max"][h, j] = np.max(k[h, toks], axis=0)
            out["k_min"][h, j] = np.min(k[h, toks], axis=0)
    return out, vnm, counts


@pytest.mark.parametrize("L,block", [(64, 16), (70, 16), (33, 32), (5, 64)])
def test_summaries_brute_force(L, block):
    rng = np.random.default_rng(L)
    k = rng.standard_normal((2, L, 8)).astype(np.float32)
    v = rng.standard_normal((2, L, 8)).astype(np.float32)
    got = Su.build_block_summaries(k, v, block)
    ref, vnm, counts = _brute_summaries(k, v, block)
    assert np.array_equal(got["block_valid_counts"], counts)
    for n in ref:
        np.testing.assert_allclose(got[n], ref[n], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(got["v_norm_max"], vnm, rtol=1e-6)
    assert np.array_equal(got["v_norm_all"], got["v_norm_max"].max(axis=1))
    assert np.all(got["k_min"] <= got["k_bar"] + 1e-6) and np.all(got["k_bar"] <= got["k_max"] + 1e-6)


def test_summaries_bf16_storage_rounds_the_fp32_mean():
    rng = np.random.default_rng(9)
    k = rng.standard_normal((2, 50, 8)).astype(np.float32)
    a = Su.build_block_summaries(k, k, 16)
    b = Su.build_block_summaries(k, k, 16, k_bar_dtype="bf16")
    assert np.array_equal(b["k_bar"], Nm.bf16_round(a["k_bar"]))


# ------------------------------------------------------------------ top-k selection

def test_topk_scores_brute_force():
    rng = np.random.default_rng(5)
    q = rng.standard_normal((8, 16)).astype(np.float32)
    kb = rng.standard_normal((2, 6, 16)).astype(np.float32)
    counts = np.array([16, 16, 16, 16, 3, 0])
    got = S.topk_block_scores(q, kb, counts, 4)
    for h in range(2):
        for j in range(6):
            if counts[j] == 0:
                assert got[h, j] == -np.inf
                continue
            s = sum(float(np.dot(q[h * 4 + g].astype(np.float64), kb[h, j])) for g in range(4)) / 4
            assert abs(got[h, j] - s / 4.0) < 1e-9


def test_quest_scores_bound_and_closed_forms():
    """The Quest page score is pinned by what it must satisfy, not by its formula:
    (1) it bounds the group-mean q . k_t of every token of the block from above;
    (2) a one-token block (k_max = k_min = k) scores exactly mean_g q_g . k;
    (3) a group whose queries are all >= 0 scores mean_g q_g . k_max, all <= 0
    mean_g q_g . k_min; (4) empty blocks score -inf."""
    rng = np.random.default_rng(21)
    hq, hkv, d, block, L = 8, 2, 16, 8, 45
    g = hq // hkv
    q = rng.standard_normal((hq, d))
    # float32 keys: the summaries hold float32 extrema, so every comparison is exact
    k = (rng.standard_normal((hkv, L, d)) * np.exp(rng.standard_normal((hkv, 1, d)))).astype(np.float32)
    k = k.astype(np.float64)
    pre = Su.build_block_summaries(k, k, block)
    got = S.quest_block_scores(q, pre["k_max"], pre["k_min"], g)
    qm = q.reshape(hkv, g, d).mean(1)
    for h in range(hkv):
        for t in range(L):
            assert float(qm[h] @ k[h, t]) <= got[h, t // block] + 1e-9
    one = Su.build_block_summaries(k, k, 1)
    got1 = S.quest_block_scores(q, one["k_max"], one["k_min"], g)
    np.testing.assert_allclose(got1, np.einsum("hd,htd->ht", qm, k), rtol=1e-12, atol=1e-12)
    qp = np.abs(q)
    np.testing.assert_allclose(S.quest_block_scores(qp, pre["k_max"], pre["k_min"], g),
                               np.einsum("hd,hbd->hb", qp.reshape(hkv, g, d).mean(1), pre["k_max"]), rtol=1e-6)
    np.testing.assert_allclose(S.quest_block_scores(-qp, pre["k_max"], pre["k_min"], g),
                               np.einsum("hd,hbd->hb", -qp.reshape(hkv, g, d).mean(1), pre["k_min"]), rtol=1e-6)
    kx = pre["k_max"].copy()
    kx[:, 2] = -np.inf
    assert np.all(S.quest_block_scores(q, kx, pre["k_min"], g)[:, 2] == -np.inf)


def _brute_topk(scores, nb, k, ff, fl, in_k):
    forced = sorted(set(range(min(ff, nb))) | set(range(max(nb - fl, 0), nb)))
    keff = k - len(forced) if in_k else k
    rest = sorted((j for j in range(nb) if j not in forced), key=lambda j: (-scores[j], j))
    return sorted(set(forced) | set(rest[:max(keff, 0)]))


@pytest.mark.parametrize("nb,k,ff,fl,in_k", [
    (32, 8, 0, 1, True),     # C1: top-8 always including the last block
    (50, 10, 1, 2, False),   # C2 shape: top-k plus first and last two
    (12, 20, 1, 2, False),   # k >= candidates: everything
    (9, 0, 1, 1, False),     # k = 0: forced only
    (40, 16, 0, 0, False),   # C3/C4: plain top-k
    (3, 3, 2, 2, True),      # overlapping forced sets
])
def test_select_topk_brute_force(nb, k, ff, fl, in_k):
    rng = np.random.default_rng(nb * 7 + k)
    for trial in range(20):
        sc = rng.standard_normal(nb)
        if trial % 3 == 0:
            sc = np.round(sc, 1)      # many exact ties
        got = S.select_topk(sc, nb, k, ff, fl, in_k).tolist()
        assert got == _brute_topk(sc, nb, k, ff, fl, in_k)
        assert got == sorted(got)


def test_select_topk_forced_counts():
    sc = np.arange(32.0)[::-1]       # block 0 best, block 31 worst
    got = S.select_topk(sc, 32, 8, 0, 1, True)
    assert len(got) == 8 and 31 in got and list(got[:7]) == list(range(7))
    got = S.select_topk(np.arange(512.0), 512, 64, 1, 2, False)    # best blocks are the last ones
    assert len(got) == 67 and 0 in got and 510 in got and 511 in got
    assert list(got[1:]) == list(range(446, 512))   # 64 best of 1..509 plus forced 510, 511


# ------------------------------------------------------------------ attention

def test_dense_decode_matches_torch_sdpa():
    rng = np.random.default_rng(6)
    q = rng.standard_normal((8, 32))
    k = rng.standard_normal((2, 77, 32))
    v = rng.standard_normal((2, 77, 32))
    got = A.dense_decode(q, k, v)
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q)[None, :, None], torch.from_numpy(k)[None], torch.from_numpy(v)[None],
        enable_gqa=True)[0, :, 0].numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)


def test_sparse_decode_all_blocks_equals_dense_and_brute_force_mask():
    rng = np.random.default_rng(7)
    q = rng.standard_normal((8, 16))
    k = rng.standard_normal((2, 100, 16))
    v = rng.standard_normal((2, 100, 16))
    nb = math.ceil(100 / 32)
    all_idx = [np.arange(nb)] * 2
    np.testing.assert_allclose(A.sparse_decode(q, k, v, all_idx, 32), A.dense_decode(q, k, v), rtol=1e-12)
    idx = [np.array([0, 3]), np.array([1])]
    got = A.sparse_decode(q, k, v, idx, 32)
    for h, sel in enumerate(idx):
        toks = [t for j in sel for t in range(j * 32, min((j + 1) * 32, 100))]
        for g in range(4):
            row = torch.from_numpy(q[h * 4 + g])
            lg = torch.from_numpy(k[h, toks]) @ row / 4.0
            ref = torch.softmax(lg, 0) @ torch.from_numpy(v[h, toks])
            np.testing.assert_allclose(got[h * 4 + g], ref.numpy(), rtol=1e-12, atol=1e-12)


def test_splitk_merge_chunking_invariance():
    rng = np.random.default_rng(8)
    q = rng.standard_normal((4, 16))
    k = rng.standard_normal((1, 90, 16)) * 3
    v = rng.standard_normal((1, 90, 16))
    mask = rng.random((1, 90)) < 0.7
    full = A.splitk_partials(q, k, v, mask, [(0, 90)])
    one = A.splitk_merge(*full)
    np.testing.assert_allclose(one, full[0][0] / full[2][0][:, None], rtol=1e-12)
    chunked = A.splitk_merge(*A.splitk_partials(q, k, v, mask, [(0, 7), (7, 7), (7, 50), (50, 90)]))
    np.testing.assert_allclose(chunked, one, rtol=1e-12, atol=1e-12)
    logits = np.where(mask[:, None], np.einsum("hgd,htd->hgt", q.reshape(1, 4, 16), k) / 4.0, -np.inf)
    w = np.exp(logits - logits.max(-1, keepdims=True))
    ref = (np.einsum("hgt,htd->hgd", w, v) / w.sum(-1)[..., None]).reshape(4, 16)
    np.testing.assert_allclose(one, ref, rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------------ condition selection

def _prefix(seed, L=300, block=32, hkv=2, d=16):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((hkv, L, d)).astype(np.float32)
    v = rng.standard_normal((hkv, L, d)).astype(np.float32)
    return k, v, Su.build_block_summaries(k, v, block)


@pytest.mark.parametrize("mass_exp", [False, True])
def test_condition_eps_extremes(mass_exp):
    k, v, pre = _prefix(10)
    q = np.random.default_rng(11).standard_normal((2, 4, 1, 16))
    sel, z = S.select_condition_eager(q, pre, 0.0, mass_exp)
    assert sel.all()            # eps = 0: every existing block (condition > 0 when delta > 0)
    sel, _ = S.select_condition_eager(q, pre, 1e9, mass_exp)
    assert not sel.any()
    z_ref = np.einsum("hgd,hbd->hgb", q[:, :, 0], pre["k_bar"].astype(np.float64)) / 4.0
    z_ref = z_ref + np.log(pre["block_valid_counts"].astype(np.float64))
    np.testing.assert_allclose(z[:, :, 0], z_ref, rtol=1e-12)


@pytest.mark.parametrize("mass_exp", [False, True])
def test_condition_chunked_equals_eager(mass_exp):
    """The chunked-LSE form (Triton kernels) and the softmax form (eager) agree."""
    k, v, pre = _prefix(12, L=1000, block=16)
    q = np.random.default_rng(13).standard_normal((2, 4, 1, 16)) * 2
    sel_e, z_e = S.select_condition_eager(q, pre, 0.0, mass_exp)
    st = S.selection_stats_chunked(q.reshape(8, 16), pre, 4, chunk=16, term1_mass_exp=mass_exp)
    # global LSE from chunks == direct LSE
    for i in (0,):
        lse_direct = np.log(np.exp(st["z"] - st["z"].max(1, keepdims=True)).sum(1)) + st["z"].max(1)
        lse_chunk = np.log(st["globals"][1]) + st["globals"][0]
        np.testing.assert_allclose(lse_chunk, lse_direct, rtol=1e-12)
    for eps in (0.0, 1e-4, 1e-3, 1e-2):
        sel_e, _ = S.select_condition_eager(q, pre, eps, mass_exp)
        sel_t, z_t = S.selection_finalize(st, pre, 4, eps, mass_exp)
        assert np.array_equal(sel_t, sel_e.reshape(8, -1))
    np.testing.assert_allclose(z_t, z_e.reshape(8, -1), rtol=1e-12)


def test_condition_delta_is_a_sound_bound():
    k, v, pre = _prefix(14, L=256, block=32)
    q = np.random.default_rng(15).standard_normal((8, 16))
    st = S.selection_stats_chunked(q, pre, 4)
    for h in range(2):
        for g in range(4):
            for j in range(8):
                toks = k[h, j * 32:(j + 1) * 32]
                dev = np.abs(toks @ q[h * 4 + g] - q[h * 4 + g] @ pre["k_bar"][h, j]) / 4.0
                assert dev.max() <= st["delta"][h * 4 + g, j] + 1e-9


def test_hybrid_dense_special_cases():
    rng = np.random.default_rng(16)
    hkv, g, d, block, L = 2, 4, 16, 16, 70
    k = rng.standard_normal((hkv, L, d))
    v = rng.standard_normal((hkv, L, d))
    pre = Su.build_block_summaries(k, v, block)
    nb = pre["block_valid_counts"].shape[0]
    kp = np.concatenate([k, np.zeros((hkv, nb * block - L, d))], 1).reshape(hkv, nb, block, d)
    vp = np.concatenate([v, np.zeros((hkv, nb * block - L, d))], 1).reshape(hkv, nb, block, d)
    tok = np.arange(nb * block).reshape(nb, block)
    valid = tok < L
    q = rng.standard_normal((hkv, g, 1, d))
    exists = pre["block_valid_counts"] > 0
    z = np.einsum("hgqd,hbd->hgqb", q, pre["k_bar"]) / 4.0 + np.log(pre["block_valid_counts"])
    empty = np.zeros((hkv, 0, d))
    all_sel = np.ones((hkv, g, 1, nb), bool)
    out = A.hybrid_decode_dense(q, kp, vp, valid, tok, L - 1, L, empty, empty, all_sel, z, pre["v_bar"], exists)
    np.testing.assert_allclose(out[:, :, 0].reshape(-1, d), A.dense_decode(q[:, :, 0].reshape(-1, d), k, v),
                               rtol=1e-12, atol=1e-12)
    none = np.zeros_like(all_sel)
    out = A.hybrid_decode_dense(q, kp, vp, valid, tok, L - 1, L, empty, empty, none, z, pre["v_bar"], exists)
    w = np.exp(z - z.max(-1, keepdims=True))
    ref = np.einsum("hgqb,hbd->hgqd", w, pre["v_bar"]) / w.sum(-1)[..., None]
    np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-12)
    # representative of a block with count c and mean key k_bar stands for c copies of k_bar
    ks = rng.standard_normal((hkv, 3, d))
    vs = rng.standard_normal((hkv, 3, d))
    out = A.hybrid_decode_dense(q, kp, vp, valid, tok, L + 2, L, ks, vs, none, z, pre["v_bar"], exists)
    logits = np.concatenate([z, np.einsum("hgqd,htd->hgqt", q, ks) / 4.0], -1)
    vals = np.concatenate([pre["v_bar"], vs], 1)
    w = np.exp(logits - logits.max(-1, keepdims=True))
    ref = np.einsum("hgqn,hnd->hgqd", w, vals) / w.sum(-1)[..., None]
    np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-12)


def test_fixed_mask_hybrid_matches_hybrid_dense_without_rounding():
    rng = np.random.default_rng(17)
    hkv, g, d, block, L = 2, 4, 16, 16, 64
    k = rng.standard_normal((hkv, L, d))
    v = rng.standard_normal((hkv, L, d))
    pre = Su.build_block_summaries(k, v, block)
    nb = 4
    kp, vp = k.reshape(hkv, nb, block, d), v.reshape(hkv, nb, block, d)
    q = rng.standard_normal((hkv, g, 1, d))
    sel_kv = rng.random((hkv, nb)) < 0.5
    z = np.einsum("hgqd,hbd->hgqb", q, pre["k_bar"].astype(np.float64)) / 4.0 + np.log(pre["block_valid_counts"])
    empty = np.zeros((hkv, 0, d))
    ref = A.hybrid_decode_dense(q, kp, vp, np.ones((nb, block), bool), np.arange(L).reshape(nb, block), L - 1,
                                L, empty, empty, np.broadcast_to(sel_kv[:, None, None], (hkv, g, 1, nb)), z,
                                pre["v_bar"], pre["block_valid_counts"] > 0)
    got = A.fixed_mask_hybrid(q, kp, vp, pre["block_valid_counts"], pre["k_bar"], pre["v_bar"], sel_kv,
                              empty, empty, emulate_bf16=False)
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-6)


def test_case_generator_is_reproducible():
    a = make_case(seed=3, batch=2, hq=8, hkv=2, d=16, seq_lens=[40, 17], page_size=16)
    b = make_case(seed=3, batch=2, hq=8, hkv=2, d=16, seq_lens=[40, 17], page_size=16)
    assert np.array_equal(a["pool_k"], b["pool_k"]) and np.array_equal(a["block_table"], b["block_table"])
    for i, L in enumerate([40, 17]):
        assert np.array_equal(P.paged_gather(a["pool_k"], a["block_table"][i], L, 16), a["k"][i])


@pytest.mark.parametrize("fp8", [False, True])
def test_torch_path_matches_numpy_oracle(fp8):
    """The timed torch CPU restatement (oracle.torch_path) equals the numpy oracle:
    same chosen blocks (mean-key and Quest scores), outputs within float32 rounding."""
    from oracle import torch_path as T

    hq, hkv, d, page, block, k = 16, 4, 32, 16, 32, 3
    lens = [200, 77]
    case = make_case(seed=11, batch=2, hq=hq, hkv=hkv, d=d, seq_lens=lens, page_size=page, k_outlier=True,
                     fp8=fp8)
    if fp8:
        pk = torch.from_numpy(case["pool_k_codes"]).view(torch.float8_e4m3fn)
        pv = torch.from_numpy(case["pool_v_codes"]).view(torch.float8_e4m3fn)
        scales = (torch.from_numpy(case["k_scale"]), torch.from_numpy(case["v_scale"]))
    else:
        pk, pv, scales = torch.from_numpy(case["pool_k"]), torch.from_numpy(case["pool_v"]), None
    table = torch.from_numpy(case["block_table"])
    for b, L in enumerate(lens):
        pre = Su.build_block_summaries(case["k"][b], case["v"][b], block)
        nb = pre["block_valid_counts"].shape[0]
        for mode in ("mean", "quest"):
            if mode == "mean":
                ref_sc = S.topk_block_scores(case["q"][b], pre["k_bar"], pre["block_valid_counts"], hq // hkv)
                kb = torch.from_numpy(pre["k_bar"])
            else:
                ref_sc = S.quest_block_scores(case["q"][b], pre["k_max"], pre["k_min"], hq // hkv)
                kb = (torch.from_numpy(pre["k_max"]), torch.from_numpy(pre["k_min"]))
            out, chosen = T.topk_layer_call(torch.from_numpy(case["q"][b]), pk, pv, table[b], L, kb, block=block,
                                            page=page, k=k, forced_last=1, scales=scales, score_mode=mode)
            ref_idx = [S.select_topk(ref_sc[h], nb, k, 0, 1, False) for h in range(hkv)]
            for h in range(hkv):
                assert np.array_equal(chosen[h].numpy(), ref_idx[h]), (b, mode, h)
            ref = A.sparse_decode(case["q"][b], case["k"][b], case["v"][b], ref_idx, block)
            np.testing.assert_allclose(out.numpy(), ref, rtol=1e-5, atol=1e-5)
