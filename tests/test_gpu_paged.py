"""GPU parity of the paged top-k path against the CPU oracle at oracle-sized shapes.

Bars: selected block indices equal except near-ties (scores
within 1e-3 relative of the k-th admitted score); outputs within 2e-2 abs for bf16
and 1e-4 abs for fp32.  fp8 K/V: within 2e-3 abs of the oracle run on the
dequantised values (the kernel's products are exact; only accumulation order and
the bf16 output rounding differ) and within 6e-2 abs of the bf16 result.
"""

import math
import zlib

import numpy as np
import pytest
import torch

import interattn_amd as ia
from oracle import attention as A
from oracle import select as S
from oracle import summaries as Su
from oracle.cases import make_case
from oracle.paged import paged_gather
from tests._util import announce, check_indices, oracle_summaries, to_dev

pytestmark = pytest.mark.gpu

TOL = {"bf16": 2e-2, "f32": 1e-4}

# name, batch, hq, hkv, d, seq_lens, page, block, dtype, (k, forced_first, forced_last, in_k), outlier
CASES = [
    ("c1_f32", 1, 8, 2, 64, [2048], 64, 64, "f32", (8, 0, 1, True), False),
    ("c2_small", 1, 32, 8, 128, [4133], 16, 64, "bf16", (16, 1, 2, False), True),
    ("ragged_b3", 3, 32, 8, 128, [1000, 64, 3333], 16, 64, "bf16", (8, 0, 0, False), False),
    ("g8_d64", 2, 16, 2, 64, [500, 777], 32, 32, "bf16", (5, 1, 1, False), False),
    ("g2_b16", 2, 4, 2, 128, [300, 129], 16, 16, "bf16", (6, 0, 2, True), False),
    ("g1_b128", 1, 2, 2, 128, [1257], 64, 128, "bf16", (3, 1, 0, False), False),
    ("block256", 1, 8, 2, 128, [2000], 16, 256, "bf16", (2, 0, 1, False), False),
    ("c4_small", 2, 32, 8, 128, [8192, 6000], 16, 128, "bf16", (16, 0, 0, False), False),
    ("f32_d128", 2, 8, 2, 128, [700, 333], 32, 32, "f32", (4, 1, 1, False), False),
    ("f32_g8_d128", 2, 16, 2, 128, [900, 517], 16, 32, "f32", (5, 1, 1, False), False),
]
IDS = [c[0] for c in CASES]


def _build(c, fp8=False):
    name, b, hq, hkv, d, lens, page, block, dt, sel, outlier = c
    case = make_case(seed=zlib.crc32(name.encode()) % 10000, batch=b, hq=hq, hkv=hkv, d=d, seq_lens=lens, page_size=page,
                     dtype=dt, k_outlier=outlier, fp8=fp8)
    return case


def _k_cap(sel):
    k, ff, fl, in_k = sel
    return max(k, ff + fl) if in_k else k + ff + fl


def _torch_dtype(dt):
    return torch.float32 if dt == "f32" else torch.bfloat16


@pytest.mark.parametrize("c", CASES, ids=IDS)
def test_summaries_match_oracle(c, device):
    name, b, hq, hkv, d, lens, page, block, dt, sel, _ = c
    announce(f"summaries {name}")
    case = _build(c)
    dev = to_dev(case, device, _torch_dtype(dt))
    nb_max = max(math.ceil(L / block) for L in lens)
    kb_dtype = torch.float32 if dt == "f32" else torch.bfloat16
    got = ia.build_block_summaries(dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"], block,
                                   nb_max=nb_max, full=True, k_bar_dtype=kb_dtype, v_bar_dtype=kb_dtype)
    torch.cuda.synchronize()
    for i, L in enumerate(lens):
        ref = Su.build_block_summaries(case["k"][i], case["v"][i], block)
        n = ref["block_valid_counts"].shape[0]
        assert np.array_equal(got["block_valid_counts"][i, :n].cpu().numpy(), ref["block_valid_counts"])
        assert np.all(got["block_valid_counts"][i, n:].cpu().numpy() == 0)
        tol = 1e-5 if dt == "f32" else 2 ** -7
        for key in ("k_bar", "v_bar"):
            g = got[key][i, :, :n].float().cpu().numpy()
            np.testing.assert_allclose(g, ref[key], rtol=tol, atol=1e-5, err_msg=key)
        for key in ("k_max", "k_min"):
            assert np.array_equal(got[key][i, :, :n].float().cpu().numpy(), ref[key]), key
        np.testing.assert_allclose(got["v_norm_max"][i, :, :n].cpu().numpy(), ref["v_norm_max"], rtol=1e-5)
        np.testing.assert_allclose(got["v_norm_all"][i].cpu().numpy(), ref["v_norm_all"], rtol=1e-5)
        if n < nb_max:
            assert torch.isneginf(got["v_norm_max"][i, :, n:]).all()


@pytest.mark.parametrize("c", CASES, ids=IDS)
def test_select_topk_matches_oracle(c, device):
    name, b, hq, hkv, d, lens, page, block, dt, sel, _ = c
    k, ff, fl, in_k = sel
    announce(f"select_topk {name}")
    case = _build(c)
    kb, counts, _ = oracle_summaries(case, block, k_bar_dtype="f32" if dt == "f32" else "bf16")
    q = torch.from_numpy(case["q"]).to(device=device, dtype=_torch_dtype(dt))
    kb_t = torch.from_numpy(kb).to(device=device, dtype=_torch_dtype(dt))
    seq_lens = torch.from_numpy(case["seq_lens"]).to(device)
    idx, n_sel, scores = ia.select_blocks_topk(q, kb_t, seq_lens, k, block_size=block, forced_first=ff,
                                               forced_last=fl, forced_in_k=in_k, return_scores=True)
    torch.cuda.synchronize()
    idx, n_sel, scores = idx.cpu().numpy(), n_sel.cpu().numpy(), scores.cpu().numpy()
    qf = case["q"].astype(np.float64)
    for i, L in enumerate(lens):
        nb = math.ceil(L / block)
        ref_sc = S.topk_block_scores(qf[i], kb[i], counts[i], hq // hkv)
        np.testing.assert_allclose(scores[i, :, :nb], ref_sc[:, :nb], rtol=1e-5, atol=1e-5)
        assert np.all(np.isneginf(scores[i, :, nb:]))
        for h in range(hkv):
            check_indices(idx[i, h], n_sel[i, h], ref_sc[h, :nb], nb, k, ff, fl, in_k)


def _oracle_idx(case, block, sel, hkv, group, kb_dtype):
    k, ff, fl, in_k = sel
    kb, counts, _ = oracle_summaries(case, block, k_bar_dtype=kb_dtype)
    out = []
    for i, L in enumerate(case["seq_lens"]):
        nb = math.ceil(int(L) / block)
        sc = S.topk_block_scores(case["q"][i].astype(np.float64), kb[i], counts[i], group)
        out.append([S.select_topk(sc[h, :nb], nb, k, ff, fl, in_k) for h in range(hkv)])
    return out


def _pack_idx(per_seq, k_cap, device):
    b, hkv = len(per_seq), len(per_seq[0])
    idx = np.full((b, hkv, k_cap), -1, np.int32)
    n = np.zeros((b, hkv), np.int32)
    for i in range(b):
        for h in range(hkv):
            s = per_seq[i][h]
            idx[i, h, :len(s)] = s
            n[i, h] = len(s)
    return torch.from_numpy(idx).to(device), torch.from_numpy(n).to(device)


@pytest.mark.parametrize("out_f32", [False, True])
@pytest.mark.parametrize("c", CASES, ids=IDS)
def test_sparse_decode_matches_oracle(c, out_f32, device):
    name, b, hq, hkv, d, lens, page, block, dt, sel, _ = c
    announce(f"sparse_decode {name} out_f32={out_f32}")
    case = _build(c)
    dev = to_dev(case, device, _torch_dtype(dt))
    per_seq = _oracle_idx(case, block, sel, hkv, hq // hkv, "f32" if dt == "f32" else "bf16")
    idx, n_sel = _pack_idx(per_seq, _k_cap(sel), device)
    out = ia.sparse_paged_decode(dev["q"], dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"],
                                 idx, n_sel, block_size=block, out_dtype=torch.float32 if out_f32 else None)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    tol = TOL[dt]
    for i, L in enumerate(lens):
        ref = A.sparse_decode(case["q"][i], case["k"][i], case["v"][i], per_seq[i], block, p_bf16=(dt == "bf16"))
        err = np.abs(got[i] - ref).max()
        assert err <= tol, f"seq {i}: max abs err {err}"


@pytest.mark.parametrize("c", CASES, ids=IDS)
def test_dense_decode_matches_oracle(c, device):
    name, b, hq, hkv, d, lens, page, block, dt, sel, _ = c
    announce(f"dense_decode {name}")
    case = _build(c)
    dev = to_dev(case, device, _torch_dtype(dt))
    out = ia.paged_decode(dev["q"], dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"],
                          max_seq_len=max(lens))
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    for i, L in enumerate(lens):
        ref = A.dense_decode(case["q"][i], case["k"][i], case["v"][i])
        err = np.abs(got[i] - ref).max()
        assert err <= TOL[dt], f"seq {i}: max abs err {err}"


FP8_CASES = [
    ("c5_small", 2, 32, 8, 128, [4096, 3000], 16, 128, "bf16", (8, 0, 0, False), False),
    ("fp8_d64_g8", 2, 16, 2, 64, [777, 64], 32, 32, "bf16", (4, 1, 1, False), False),
]


@pytest.mark.skipif(not hasattr(torch, "float8_e4m3fn"), reason="torch without float8")
@pytest.mark.parametrize("c", FP8_CASES, ids=[c[0] for c in FP8_CASES])
def test_fp8_paths_match_oracle(c, device):
    name, b, hq, hkv, d, lens, page, block, dt, sel, _ = c
    announce(f"fp8 {name}")
    case = _build(c, fp8=True)
    dev = to_dev(case, device, fp8=True)
    per_seq = _oracle_idx(case, block, sel, hkv, hq // hkv, "bf16")
    idx, n_sel = _pack_idx(per_seq, _k_cap(sel), device)
    out = ia.sparse_paged_decode(dev["q"], dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"],
                                 idx, n_sel, block_size=block, scales=dev["scales"])
    dense = ia.paged_decode(dev["q"], dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"],
                            max_seq_len=max(lens), scales=dev["scales"])
    # the same scales gathered per sequence (one line per block): the same bits
    s3 = (*dev["scales"], ia.sequence_scales(dev["scales"], dev["block_table"]))
    out3 = ia.sparse_paged_decode(dev["q"], dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"],
                                  idx, n_sel, block_size=block, scales=s3)
    dense3 = ia.paged_decode(dev["q"], dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"],
                             max_seq_len=max(lens), scales=s3)
    torch.cuda.synchronize()
    assert torch.equal(out3, out) and torch.equal(dense3, dense)
    # the bf16 reference: same inputs before quantisation
    case_bf = _build(c)
    dev_bf = to_dev(case_bf, device, torch.bfloat16)
    out_bf = ia.sparse_paged_decode(dev_bf["q"], dev_bf["pool_k"], dev_bf["pool_v"], dev_bf["block_table"],
                                    dev_bf["seq_lens"], idx, n_sel, block_size=block)
    torch.cuda.synchronize()
    got, gd, gbf = out.float().cpu().numpy(), dense.float().cpu().numpy(), out_bf.float().cpu().numpy()
    for i, L in enumerate(lens):
        # Q.K is exact on the dequantised values; P.V uses bf16(p * v_scale) weights on the
        # codes, within 2^-8 relative of the oracle's bf16(p) weights on dequantised V
        vmax = float(np.abs(case["v"][i]).max())
        ref = A.sparse_decode(case["q"][i], case["k"][i], case["v"][i], per_seq[i], block, p_bf16=True)
        assert np.abs(got[i] - ref).max() <= 2e-3 + 2 ** -8 * vmax
        refd = A.dense_decode(case["q"][i], case["k"][i], case["v"][i])
        assert np.abs(gd[i] - refd).max() <= 2e-3 + 2 ** -8 * vmax
        assert np.abs(got[i] - gbf[i]).max() <= 6e-2


def test_fp8_codec_on_device(device):
    """v_cvt_pk_f32_fp8 decodes OCP e4m3fn: a kernel that sees every code once."""
    if not hasattr(torch, "float8_e4m3fn"):
        pytest.skip("torch without float8")
    announce("fp8 codec")
    codes = torch.arange(256, dtype=torch.uint8)
    codes = codes[(codes & 0x7F) != 0x7F]          # drop NaN codes
    n = codes.numel()                               # 254 codes
    page, d = 16, 128
    pool = torch.zeros((1, 1, page, d), dtype=torch.uint8)
    flat = pool.view(-1)
    flat[:n] = codes
    pool_k = pool.to(device).view(torch.float8_e4m3fn)
    pool_v = torch.zeros_like(pool_k)
    one = torch.ones((1, 1), device=device, dtype=torch.float32)
    seq = torch.tensor([page], device=device, dtype=torch.int32)
    s = ia.build_block_summaries(pool_k, pool_v, None, seq, 16, nb_max=1, full=True,
                                 k_bar_dtype=torch.float32, bounds_dtype=torch.float32, scales=(one, one))
    torch.cuda.synchronize()
    vals = torch.from_numpy(pool.numpy()).view(torch.float8_e4m3fn).float().view(page, d)
    assert torch.equal(s["k_max"][0, 0, 0].cpu(), vals.max(0).values)
    assert torch.equal(s["k_min"][0, 0, 0].cpu(), vals.min(0).values)
    # with max, min and the (exact) mean of the two non-zero codes per dim, every code is pinned
    assert torch.equal(s["k_bar"][0, 0, 0].cpu(), vals.sum(0) / page)


def test_fp8_decode_widening_on_device(device):
    """The finalize widens e4m3 codes to bf16 with v_cvt_scalef32_pk_bf16_fp8: with K = 0
    every token weighs 1, so each output dim is the one non-zero V code / 16, exactly."""
    if not hasattr(torch, "float8_e4m3fn"):
        pytest.skip("torch without float8")
    announce("fp8 decode widening")
    codes = torch.arange(256, dtype=torch.uint8)
    codes = codes[(codes & 0x7F) != 0x7F]          # drop NaN codes: 254 codes
    page, d = 16, 128
    one = torch.ones((2, 1), device=device, dtype=torch.float32)
    pool_v = torch.zeros((2, 1, page, d), dtype=torch.uint8)
    pool_v[0, 0, 0, :] = codes[:d]
    pool_v[1, 0, 0, :codes.numel() - d] = codes[d:]
    pool_v = pool_v.to(device).view(torch.float8_e4m3fn)
    pool_k = torch.zeros_like(pool_v)
    q = torch.zeros((2, 1, d), device=device, dtype=torch.bfloat16)
    table = torch.tensor([[0], [1]], device=device, dtype=torch.int32)
    seq = torch.tensor([page, page], device=device, dtype=torch.int32)
    out = ia.paged_decode(q, pool_k, pool_v, table, seq, max_seq_len=page, scales=(one, one), out_dtype=torch.float32)
    torch.cuda.synchronize()
    vals = pool_v[:, 0, 0, :].cpu().float()
    assert torch.equal(out[:, 0].cpu(), vals / 16)


def test_edge_cases(device):
    announce("edge cases")
    hq, hkv, d, page, block = 8, 2, 128, 16, 32
    case = make_case(seed=99, batch=4, hq=hq, hkv=hkv, d=d, seq_lens=[0, 1, 40, 96], page_size=page)
    dev = to_dev(case, device)
    # sequence 3: poison its last page id (out of range) -> that page is skipped
    bt = dev["block_table"].clone()
    bt[3, 5] = 10 ** 6
    kb, counts, _ = oracle_summaries(case, block)
    kb_t = torch.from_numpy(kb).to(device=device, dtype=torch.bfloat16)
    idx, n_sel = ia.select_blocks_topk(dev["q"], kb_t, dev["seq_lens"], 2, block_size=block, forced_last=1)
    out = ia.sparse_paged_decode(dev["q"], dev["pool_k"], dev["pool_v"], bt, dev["seq_lens"], idx, n_sel,
                                 block_size=block)
    zero_k = ia.sparse_paged_decode(dev["q"], dev["pool_k"], dev["pool_v"], bt, dev["seq_lens"], idx,
                                    torch.zeros_like(n_sel), block_size=block)
    dense = ia.paged_decode(dev["q"], dev["pool_k"], dev["pool_v"], bt, dev["seq_lens"], max_seq_len=96)
    torch.cuda.synchronize()
    n_sel = n_sel.cpu().numpy()
    assert n_sel[0].tolist() == [0, 0]                      # empty sequence selects nothing
    assert n_sel[1].tolist() == [1, 1]
    assert torch.all(out[0] == 0) and torch.all(zero_k == 0) and torch.all(dense[0] == 0)
    got = out.float().cpu().numpy()
    idx = idx.cpu().numpy()
    for i in (1, 2):
        sel = [idx[i, h, :n_sel[i, h]] for h in range(hkv)]
        ref = A.sparse_decode(case["q"][i], case["k"][i], case["v"][i], sel, block, p_bf16=True)
        assert np.abs(got[i] - ref).max() <= 2e-2
    # seq 3 without its 6th page (tokens 80..95)
    k3, v3 = case["k"][3][:, :80], case["v"][3][:, :80]
    ref = A.dense_decode(case["q"][3], k3, v3)
    assert np.abs(dense[3].float().cpu().numpy() - ref).max() <= 2e-2


def test_workspace_reuse(device):
    """Repeated calls on one workspace give identical results."""
    announce("workspace reuse")
    c = CASES[7]
    case = _build(c)
    dev = to_dev(case, device)
    block = c[7]
    kb, counts, _ = oracle_summaries(case, block)
    kb_t = torch.from_numpy(kb).to(device=device, dtype=torch.bfloat16)
    ws = {}
    outs = []
    for _ in range(3):
        o = ia.sparse_topk_decode(dev["q"], dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"],
                                  kb_t, 16, block_size=block, workspace=ws)
        outs.append(o.clone())
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2])


@pytest.mark.parametrize("return_scores", [False, True])
def test_select_topk_long_rows_use_global_scores(return_scores, device):
    """nb > 8192 blocks per row: scores do not fit the LDS stage and round-trip
    through global memory inside the selecting workgroup."""
    announce(f"select long rows return_scores={return_scores}")
    rng = np.random.default_rng(77)
    hq, hkv, d, block = 8, 2, 64, 16
    lens = [140000, 9000]
    nb_max = math.ceil(max(lens) / block)
    kb = rng.standard_normal((2, hkv, nb_max, d)).astype(np.float32)
    kb_t = torch.from_numpy(kb).to(device=device, dtype=torch.bfloat16)
    kb = kb_t.float().cpu().numpy()
    q = rng.standard_normal((2, hq, d)).astype(np.float32)
    q_t = torch.from_numpy(q).to(device=device, dtype=torch.bfloat16)
    q = q_t.float().cpu().numpy()
    seq = torch.tensor(lens, device=device, dtype=torch.int32)
    res = ia.select_blocks_topk(q_t, kb_t, seq, 33, block_size=block, forced_first=2, forced_last=3,
                                return_scores=return_scores)
    torch.cuda.synchronize()
    idx, n_sel = res[0].cpu().numpy(), res[1].cpu().numpy()
    for i, L in enumerate(lens):
        nb = math.ceil(L / block)
        counts = np.full(nb_max, block)
        counts[nb:] = 0
        sc = S.topk_block_scores(q[i].astype(np.float64), kb[i], counts, hq // hkv)
        if return_scores:
            np.testing.assert_allclose(res[2][i, :, :nb].cpu().numpy(), sc[:, :nb], rtol=1e-5, atol=1e-5)
        for h in range(hkv):
            check_indices(idx[i, h], n_sel[i, h], sc[h, :nb], nb, 33, 2, 3, False)


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("c", CASES, ids=IDS)
def test_fused_topk_decode_equals_two_step(c, fp8, device):
    """ia_sparse_topk_decode (scorer + finalize selecting in its prologue) returns the
    same selection and the same output, bit for bit, as select_topk + sparse decode."""
    name, b, hq, hkv, d, lens, page, block, dt, sel, _ = c
    if fp8 and dt == "f32":
        pytest.skip("fp8 pools take bf16 q")
    k, ff, fl, in_k = sel
    announce(f"fused topk decode {name} fp8={fp8}")
    case = _build(c, fp8=fp8)
    dev = to_dev(case, device, _torch_dtype(dt), fp8=fp8)
    nb_max = max(math.ceil(L / block) for L in lens) + 2
    kb_dtype = torch.float32 if dt == "f32" else torch.bfloat16
    summ = ia.build_block_summaries(dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"], block,
                                    nb_max=nb_max, k_bar_dtype=kb_dtype, scales=dev["scales"])
    kw = dict(block_size=block, forced_first=ff, forced_last=fl, forced_in_k=in_k)
    idx, n_sel = ia.select_blocks_topk(dev["q"], summ["k_bar"], dev["seq_lens"], k, **kw)
    ref = ia.sparse_paged_decode(dev["q"], dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"], idx,
                                 n_sel, block_size=block, scales=dev["scales"])
    out, idx2, n_sel2 = ia.sparse_topk_decode(dev["q"], dev["pool_k"], dev["pool_v"], dev["block_table"],
                                              dev["seq_lens"], summ["k_bar"], k, scales=dev["scales"],
                                              return_selection=True, workspace={}, **kw)
    torch.cuda.synchronize()
    assert torch.equal(n_sel2, n_sel)
    for i in range(b):
        for h in range(hkv):
            n = int(n_sel[i, h])
            assert torch.equal(idx2[i, h, :n], idx[i, h, :n]), (i, h)
    assert torch.equal(out, ref)
    if fp8:  # the scales gathered per sequence: the same bits
        s3 = (*dev["scales"], ia.sequence_scales(dev["scales"], dev["block_table"]))
        out3 = ia.sparse_topk_decode(dev["q"], dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"],
                                     summ["k_bar"], k, scales=s3, workspace={}, **kw)
        torch.cuda.synchronize()
        assert torch.equal(out3, ref)


def test_fused_topk_decode_k_per_seq_and_fallback(device):
    """Per-sequence k (C3's rule) through the fused path, and the two-step fallback
    past the fused limits (more than 4096 blocks)."""
    announce("fused topk decode k_per_seq + fallback")
    lens = [3000, 700, 1900]
    case = make_case(seed=77, batch=3, hq=32, hkv=8, d=128, seq_lens=lens, page_size=16)
    dev = to_dev(case, device)
    block = 64
    nb_max = max(math.ceil(L / block) for L in lens)
    kvec = torch.tensor([max(2, math.ceil(L / block) // 8) for L in lens], device=device, dtype=torch.int32)
    k_cap = int(kvec.max())
    summ = ia.build_block_summaries(dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"], block,
                                    nb_max=nb_max)
    idx, n_sel = ia.select_blocks_topk(dev["q"], summ["k_bar"], dev["seq_lens"], 0, block_size=block,
                                       k_per_seq=kvec, k_cap=k_cap)
    ref = ia.sparse_paged_decode(dev["q"], dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"], idx,
                                 n_sel, block_size=block)
    out = ia.sparse_topk_decode(dev["q"], dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"],
                                summ["k_bar"], 0, block_size=block, k_per_seq=kvec, k_cap=k_cap, workspace={})
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    # a k_bar row of more than 4096 blocks runs as the two calls
    wide = torch.zeros((3, 8, 4100, 128), device=device, dtype=torch.bfloat16)
    wide[:, :, :nb_max] = summ["k_bar"]
    out2 = ia.sparse_topk_decode(dev["q"], dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"],
                                 wide, 0, block_size=block, k_per_seq=kvec, k_cap=k_cap, workspace={})
    torch.cuda.synchronize()
    assert torch.equal(out2, ref)


@pytest.mark.parametrize("hq,hkv,page,lens", [
    (8, 2, 16, [1, 17, 2049]),     # G = 4: a one-token sequence, a partial subtile
    (16, 2, 32, [300, 4133, 64]),  # G = 8, two-subtile pages
    (16, 8, 16, [999, 33, 5000]),  # G = 2
    (8, 8, 64, [1250, 4096]),      # G = 1, pages of four subtiles
], ids=["g4_p16", "g8_p32", "g2_p16", "g1_p64"])
def test_key_row_instance_equals_two_step(hq, hkv, page, lens, device):
    """Launches with per-sequence k at head_dim 128 run the instance that loads keys as
    whole rows and passes them through LDS to the MFMA operand layout; the words that
    reach the products are the ones the operand-layout loads give, so the output equals
    the two-step path bit for bit, for every group size, page size and ragged length
    (one-token sequences and partial subtiles included)."""
    announce(f"key-row instance: G={hq // hkv} page={page} lens={lens}")
    case = make_case(seed=31 + page + hq, batch=len(lens), hq=hq, hkv=hkv, d=128, seq_lens=lens, page_size=page)
    dev = to_dev(case, device)
    block = 64
    nb_max = max(math.ceil(L / block) for L in lens)
    kvec = torch.tensor([max(1, math.ceil(L / block) // 4) for L in lens], device=device, dtype=torch.int32)
    k_cap = int(kvec.max()) + 2
    summ = ia.build_block_summaries(dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"], block,
                                    nb_max=nb_max)
    idx, n_sel = ia.select_blocks_topk(dev["q"], summ["k_bar"], dev["seq_lens"], 0, block_size=block,
                                       k_per_seq=kvec, k_cap=k_cap, forced_first=1, forced_last=1)
    ref = ia.sparse_paged_decode(dev["q"], dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"], idx,
                                 n_sel, block_size=block)
    ws = {}
    for _ in range(2):  # a second call on the same workspace
        out = ia.sparse_topk_decode(dev["q"], dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"],
                                    summ["k_bar"], 0, block_size=block, k_per_seq=kvec, k_cap=k_cap,
                                    forced_first=1, forced_last=1, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
    assert torch.isfinite(out.float()).all()


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_sparse_decode_with_representatives(dt, device):
    """Top-k finalize with representatives for the unselected blocks (logit
    q.k_bar/sqrt(D) + log count, value v_bar: the external-mask hybrid of
    fixed_mask.py:38-239) on a ragged paged batch, against the oracle's
    fixed_mask_hybrid per sequence; with every block selected it equals the plain
    top-k finalize."""
    announce(f"sparse decode with representatives {dt}")
    hq, hkv, d, page, block, k = 8, 2, 128, 16, 64, 5
    lens = [1000, 3000, 70]
    case = make_case(seed=515, batch=3, hq=hq, hkv=hkv, d=d, seq_lens=lens, page_size=page, dtype=dt)
    tdt = _torch_dtype(dt)
    dev = to_dev(case, device, dtype=tdt)
    nb_max = max(math.ceil(L / block) for L in lens)
    sdt = torch.float32 if dt == "f32" else torch.bfloat16
    summ = ia.build_block_summaries(dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"], block,
                                    nb_max=nb_max, full=True, k_bar_dtype=sdt, v_bar_dtype=sdt)
    idx, n_sel = ia.select_blocks_topk(dev["q"], summ["k_bar"], dev["seq_lens"], k, block_size=block, forced_last=1)
    out = ia.sparse_paged_decode(dev["q"], dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"], idx,
                                 n_sel, block_size=block, include_representatives=True, summaries=summ,
                                 out_dtype=torch.float32, workspace={})
    # every block selected: no representative remains
    all_idx = torch.arange(nb_max, device=device, dtype=torch.int32).expand(3, hkv, nb_max).contiguous()
    all_n = torch.tensor([[math.ceil(L / block)] * hkv for L in lens], device=device, dtype=torch.int32)
    full_r = ia.sparse_paged_decode(dev["q"], dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"],
                                    all_idx, all_n, block_size=block, include_representatives=True, summaries=summ,
                                    out_dtype=torch.float32, workspace={})
    full_p = ia.sparse_paged_decode(dev["q"], dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"],
                                    all_idx, all_n, block_size=block, out_dtype=torch.float32)
    torch.cuda.synchronize()
    np.testing.assert_allclose(full_r.cpu().numpy(), full_p.cpu().numpy(), atol=TOL[dt], rtol=0)
    host = {key: summ[key].float().cpu().numpy() for key in ("k_bar", "v_bar")}
    counts = summ["block_valid_counts"].cpu().numpy()
    idx_h, n_h = idx.cpu().numpy(), n_sel.cpu().numpy()
    got = out.cpu().numpy()
    g = hq // hkv
    for b, L in enumerate(lens):
        nb = math.ceil(L / block)
        kb = np.zeros((hkv, nb * block, d), np.float32)
        vb = np.zeros((hkv, nb * block, d), np.float32)
        kb[:, :L], vb[:, :L] = case["k"][b], case["v"][b]
        sel = np.zeros((hkv, nb), bool)
        for h in range(hkv):
            sel[h, idx_h[b, h, :n_h[b, h]]] = True
        ref = A.fixed_mask_hybrid(case["q"][b].reshape(hkv, g, 1, d), kb.reshape(hkv, nb, block, d),
                                  vb.reshape(hkv, nb, block, d), counts[b, :nb], host["k_bar"][b, :, :nb],
                                  host["v_bar"][b, :, :nb], sel, np.zeros((hkv, 0, d), np.float32),
                                  np.zeros((hkv, 0, d), np.float32), emulate_bf16=(dt == "bf16"))
        np.testing.assert_allclose(got[b], ref[:, :, 0].reshape(hq, d), atol=TOL[dt], rtol=0)


@pytest.mark.parametrize("c", CASES, ids=IDS)
def test_quest_score_selection_and_decode(c, device):
    """The Quest page score (CBG/methods/quest.py:97-101) on the device: scores equal
    the oracle's (float64, 1e-5), indices equal the oracle's top-k of them (near-tie
    rule), the fused layer call equals select + decode bit for bit, and the output
    equals exact attention over the chosen blocks."""
    name, b, hq, hkv, d, lens, page, block, dt, sel, _ = c
    k, ff, fl, in_k = sel
    announce(f"quest score {name}")
    case = _build(c)
    dev = to_dev(case, device, _torch_dtype(dt))
    nb_max = max(math.ceil(L / block) for L in lens)
    summ = ia.build_block_summaries(dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"], block,
                                    nb_max=nb_max, full=True)
    keys = (summ["k_max"], summ["k_min"])
    kw = dict(block_size=block, forced_first=ff, forced_last=fl, forced_in_k=in_k, score="quest")
    idx, n_sel, scores = ia.select_blocks_topk(dev["q"], keys, dev["seq_lens"], k, return_scores=True, **kw)
    ref = ia.sparse_paged_decode(dev["q"], dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"], idx,
                                 n_sel, block_size=block)
    out, idx2, n_sel2 = ia.sparse_topk_decode(dev["q"], dev["pool_k"], dev["pool_v"], dev["block_table"],
                                              dev["seq_lens"], keys, k, return_selection=True, workspace={}, **kw)
    torch.cuda.synchronize()
    assert torch.equal(n_sel2, n_sel) and torch.equal(out, ref)
    g = hq // hkv
    got = out.float().cpu().numpy()
    for i, L in enumerate(lens):
        nb = math.ceil(L / block)
        kx = summ["k_max"][i, :, :nb].double().cpu().numpy()
        kn = summ["k_min"][i, :, :nb].double().cpu().numpy()
        sc = S.quest_block_scores(case["q"][i], kx, kn, g)
        np.testing.assert_allclose(scores[i, :, :nb].cpu().numpy(), sc, rtol=1e-5, atol=1e-5)
        chosen = []
        for h in range(hkv):
            n = int(n_sel[i, h])
            check_indices(idx[i, h].cpu().numpy(), n, sc[h], nb, k, ff, fl, in_k)
            assert torch.equal(idx2[i, h, :n], idx[i, h, :n])
            chosen.append(idx[i, h, :n].cpu().numpy())
        exp = A.sparse_decode(case["q"][i], case["k"][i], case["v"][i], chosen, block, p_bf16=dt == "bf16")
        assert np.abs(got[i] - exp).max() <= TOL[dt]


@pytest.mark.parametrize("name", ["c2_small", "c4_small", "ragged_b3", "g8_d64"])
def test_fused_handoff_fallback_is_exact(name, device):
    """With a wait bound of 0 every item that finds a partner's scores missing scores
    that range itself: the result (selection and output) equals the waiting run's bit
    for bit.  One workspace serves calls on different queries back to back, so flags
    left set by a call would show up as a wrong selection in the next."""
    c = CASES[IDS.index(name)]
    _, b, hq, hkv, d, lens, page, block, dt, sel, _ = c
    k, ff, fl, in_k = sel
    announce(f"fused hand-off fallback {name}")
    case = _build(c)
    dev = to_dev(case, device, _torch_dtype(dt))
    nb_max = max(math.ceil(L / block) for L in lens)
    kb_dtype = torch.float32 if dt == "f32" else torch.bfloat16
    summ = ia.build_block_summaries(dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"], block,
                                    nb_max=nb_max, k_bar_dtype=kb_dtype)
    kw = dict(block_size=block, forced_first=ff, forced_last=fl, forced_in_k=in_k)
    gen = torch.Generator(device=device).manual_seed(5)
    qs = [dev["q"]] + [torch.randn(dev["q"].shape, device=device, generator=gen).to(dev["q"].dtype) for _ in range(2)]
    refs = []
    for q in qs:
        idx, n_sel = ia.select_blocks_topk(q, summ["k_bar"], dev["seq_lens"], k, **kw)
        refs.append(ia.sparse_paged_decode(q, dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"],
                                           idx, n_sel, block_size=block).clone())
    ws = {}
    ia.wait_fallbacks(reset=True)
    previous = ia.set_wait_limit(0)
    try:
        got0 = [ia.sparse_topk_decode(q, dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"],
                                      summ["k_bar"], k, workspace=ws, **kw).clone() for q in qs]
    finally:
        ia.set_wait_limit(previous)
    torch.cuda.synchronize()
    n0 = ia.wait_fallbacks(reset=True)
    got = [ia.sparse_topk_decode(q, dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"],
                                 summ["k_bar"], k, workspace=ws, **kw).clone() for q in qs]
    torch.cuda.synchronize()
    for r, a, b_ in zip(refs, got0, got):
        assert torch.equal(a, r) and torch.equal(b_, r)
    # the diagnostic counts the bound-0 run's fallbacks (none when every row scores
    # itself), and none at the default bound with every workgroup resident
    print(f"[{name}] wait fallbacks at bound 0: {n0}", flush=True)
    assert n0 >= 0 and ia.wait_fallbacks() == 0


@pytest.mark.parametrize("rows", [(4, 32, 8), (7, 16, 4)], ids=["32rows", "28rows"])
def test_fused_merge_item_boundary(rows, device):
    """Uniform launches whose rows get about budget / rows items: 32 rows of 8 items on
    a 256-workgroup launch (the tagged partials' merge, up to 8 items) and 28 rows of 9
    (the untagged merge, more than 8).  Selection and output equal the two-step path's
    bit for bit, also with a wait bound of 0 (every missing score computed by the
    waiting item; the merge still waits for finished items' stores)."""
    b, hq, hkv = rows
    announce(f"fused merge item boundary: batch {b}, {hkv} kv heads")
    lens = [4096] * b
    case = make_case(seed=31 + b, batch=b, hq=hq, hkv=hkv, d=128, seq_lens=lens, page_size=16, dtype="bf16",
                     k_outlier=False, fp8=False)
    dev = to_dev(case, device, torch.bfloat16)
    block, k = 64, 16
    summ = ia.build_block_summaries(dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"], block,
                                    nb_max=4096 // block, k_bar_dtype=torch.bfloat16)
    idx, n_sel = ia.select_blocks_topk(dev["q"], summ["k_bar"], dev["seq_lens"], k, block_size=block)
    ref = ia.sparse_paged_decode(dev["q"], dev["pool_k"], dev["pool_v"], dev["block_table"], dev["seq_lens"], idx,
                                 n_sel, block_size=block)
    ws = {}
    outs = []
    for limit in (None, 0):
        previous = ia.set_wait_limit(limit) if limit is not None else None
        try:
            for _ in range(2):  # the second call reuses the workspace's counts and epochs
                out, idx2, n_sel2 = ia.sparse_topk_decode(dev["q"], dev["pool_k"], dev["pool_v"], dev["block_table"],
                                                          dev["seq_lens"], summ["k_bar"], k, block_size=block,
                                                          return_selection=True, workspace=ws)
                torch.cuda.synchronize()
                assert torch.equal(idx2, idx) and torch.equal(n_sel2, n_sel)
                outs.append(out.clone())
        finally:
            if previous is not None:
                ia.set_wait_limit(previous)
    for o in outs:
        assert torch.equal(o, ref)
    assert torch.isfinite(ref).all()


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("c", [CASES[7], CASES[2]], ids=[CASES[7][0], CASES[2][0]])
def test_paired_kv_layout_equals_split(c, fp8, device):
    """K and V of a (page, kv head) adjacent in one buffer [n_pages, Hkv, 2, page, D]
    (pool_k / pool_v are its views, bench.py --kv-layout paired): the one-launch call
    and the summaries equal those of separate pools bit for bit."""
    name, b, hq, hkv, d, lens, page, block, dt, sel, _ = c
    k, ff, fl, in_k = sel
    announce(f"paired kv layout {name} fp8={fp8}")
    case = _build(c, fp8=fp8)
    dev = to_dev(case, device, _torch_dtype(dt), fp8=fp8)
    buf = torch.empty((dev["pool_k"].shape[0], hkv, 2, page, d), device=device, dtype=dev["pool_k"].dtype)
    buf[:, :, 0].copy_(dev["pool_k"])
    buf[:, :, 1].copy_(dev["pool_v"])
    pk, pv = buf[:, :, 0], buf[:, :, 1]
    nb_max = max(math.ceil(L / block) for L in lens)
    kw = dict(block_size=block, forced_first=ff, forced_last=fl, forced_in_k=in_k)
    outs = []
    for pool_k, pool_v in ((dev["pool_k"], dev["pool_v"]), (pk, pv)):
        summ = ia.build_block_summaries(pool_k, pool_v, dev["block_table"], dev["seq_lens"], block, nb_max=nb_max,
                                        k_bar_dtype=torch.bfloat16, scales=dev["scales"])
        out, idx, n_sel = ia.sparse_topk_decode(dev["q"], pool_k, pool_v, dev["block_table"], dev["seq_lens"],
                                                summ["k_bar"], k, scales=dev["scales"], return_selection=True,
                                                workspace={}, **kw)
        outs.append((summ["k_bar"].clone(), out.clone(), idx.clone(), n_sel.clone()))
    torch.cuda.synchronize()
    (kb0, o0, i0, n0), (kb1, o1, i1, n1) = outs
    assert torch.equal(kb0, kb1)
    assert torch.equal(n0, n1) and torch.equal(o0, o1)
    for i in range(b):
        for h in range(hkv):
            n = int(n0[i, h])
            assert torch.equal(i0[i, h, :n], i1[i, h, :n])
