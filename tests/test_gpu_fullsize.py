"""Parity at the BASELINE configs' full sizes (C2, C3, C4, C5 shapes, one GPU).

* the fused layer call equals select + decode bit for bit (indices and output);
* the selected blocks equal the oracle's top-k of the same k_bar scores (near-tie
  rule) and the output equals exact attention over the selected tokens (float64,
  2e-2 abs: bf16 weights): every sequence of C2, C3 and C4;
* the device summaries of one full sequence of C4 (block 128) and of C3 (block 64)
  equal the oracle's (counts, extrema exact; means within bf16 storage rounding);
* C2: one 32768-token sequence, block 64, top-64 plus the first block and the last
  two (67 blocks), keys scaled per (kv head, channel) by exp(N(0,1));
* C3: 16 ragged sequences whose pages are drawn from one shared pool of 4M tokens in
  random order;
* C5: fp8 K/V against the oracle on the dequantised values (2e-3 + 2^-8 max|v|) on
  every sequence, and within 6e-2 abs of the bf16 result on the same selection;
* the dense fallback over a whole 128K context equals float64 attention (2e-2).
"""

import math

import numpy as np
import pytest
import torch

import interattn_amd as ia
from oracle import attention as A
from oracle import select as S
from oracle import summaries as Su
from tests._util import announce, check_indices

pytestmark = pytest.mark.gpu

HQ, HKV, D, PAGE = 32, 8, 128, 16


def _make(device, lens, seed, k_outlier=False, pool_tokens=0):
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    pages = [math.ceil(L / PAGE) for L in lens]
    # the sequences' pages come from one permutation of a pool of at least pool_tokens
    n_pages = max(sum(pages), pool_tokens // PAGE)
    perm = torch.randperm(n_pages, device=device, generator=gen).to(torch.int32)
    table = torch.full((len(lens), max(pages)), -1, device=device, dtype=torch.int32)
    off = 0
    for b, n in enumerate(pages):
        table[b, :n] = perm[off:off + n]
        off += n
    pool_k = torch.randn((n_pages, HKV, PAGE, D), device=device, dtype=torch.bfloat16, generator=gen)
    pool_v = torch.randn((n_pages, HKV, PAGE, D), device=device, dtype=torch.bfloat16, generator=gen)
    if k_outlier:
        # per-(kv head, channel) key scale exp(N(0,1)) ("RoPE'd keys")
        outlier = torch.randn((HKV, D), device=device, generator=gen).exp()
        pool_k.mul_(outlier[None, :, None, :].to(torch.bfloat16))
    q = torch.randn((len(lens), HQ, D), device=device, dtype=torch.bfloat16, generator=gen)
    seq = torch.tensor(lens, device=device, dtype=torch.int32)
    return pool_k, pool_v, table, seq, q


def _gather_head(pool, table_row, blocks, block, L, h, scale=None):
    """[tokens, D] float64 of the given logical blocks of one sequence and kv head (one
    indexed read on the device; fp8 pools times their per-(page, head) scale)."""
    blocks = torch.as_tensor(np.asarray(blocks, dtype=np.int64), device=pool.device)
    tok = (blocks[:, None] * block + torch.arange(block, device=pool.device)[None]).flatten()
    tok = tok[tok < L]
    pg = table_row.long()[tok // PAGE]
    x = pool[pg, h, tok % PAGE].float().double()
    if scale is not None:
        x = x * scale[pg, h].double()[:, None]
    return x.cpu().numpy()


def _check_summaries(pool_k, pool_v, table, seq, b, block, k_bar):
    """The full summaries of sequence b (one build over its block-table row) against
    the oracle's, per kv head; the k_bar that the top-k scored is the same array."""
    L = int(seq[b])
    nb = math.ceil(L / block)
    got = ia.build_block_summaries(pool_k, pool_v, table[b:b + 1].contiguous(), seq[b:b + 1].contiguous(), block,
                                   nb_max=nb, full=True, k_bar_dtype=torch.bfloat16, v_bar_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(got["k_bar"][0], k_bar[b, :, :nb])
    pg = table[b, :math.ceil(L / PAGE)].long()
    for h in range(HKV):
        kk = pool_k[pg, h].reshape(-1, D)[:L].float().cpu().numpy()[None]
        vv = pool_v[pg, h].reshape(-1, D)[:L].float().cpu().numpy()[None]
        ref = Su.build_block_summaries(kk, vv, block, k_bar_dtype="bf16", v_bar_dtype="bf16")
        assert np.array_equal(got["block_valid_counts"][0, :nb].cpu().numpy(), ref["block_valid_counts"])
        for key in ("k_bar", "v_bar"):
            np.testing.assert_allclose(got[key][0, h:h + 1, :nb].float().cpu().numpy(), ref[key], rtol=2 ** -7,
                                       atol=1e-5, err_msg=f"{key} head {h}")
        for key in ("k_max", "k_min"):
            assert np.array_equal(got[key][0, h:h + 1, :nb].float().cpu().numpy(), ref[key]), (key, h)
        np.testing.assert_allclose(got["v_norm_max"][0, h:h + 1, :nb].cpu().numpy(), ref["v_norm_max"], rtol=1e-5)
        np.testing.assert_allclose(got["v_norm_all"][0, h:h + 1].cpu().numpy(), ref["v_norm_all"], rtol=1e-5)


def _check_sample(q, pool_k, pool_v, table, seq, k_bar, idx, n_sel, out, block, k, sample, k_per_seq=None,
                  ff=0, fl=0):
    g = HQ // HKV
    for b in sample:
        L = int(seq[b])
        nb = math.ceil(L / block)
        counts = np.array([min(block, L - j * block) for j in range(nb)])
        qb = q[b].double().cpu().numpy()
        sc = S.topk_block_scores(qb, k_bar[b, :, :nb].double().cpu().numpy(), counts, g)
        kb_ = int(k_per_seq[b]) if k_per_seq is not None else k
        for h in range(HKV):
            n = int(n_sel[b, h])
            chosen = idx[b, h, :n].cpu().numpy()
            check_indices(chosen, n, sc[h], nb, kb_, ff, fl, False)
            kk = _gather_head(pool_k, table[b], chosen, block, L, h)
            vv = _gather_head(pool_v, table[b], chosen, block, L, h)
            ref = A.dense_decode(qb[h * g:(h + 1) * g], kk[None], vv[None])
            got = out[b, h * g:(h + 1) * g].double().cpu().numpy()
            assert np.abs(got - ref).max() <= 2e-2, (b, h)


@pytest.fixture(scope="module")
def c4(device):
    announce("full-size C4 pool (16 x 131072, bf16)")
    lens = [131072] * 16
    pool_k, pool_v, table, seq, q = _make(device, lens, 1237)
    summ = ia.build_block_summaries(pool_k, pool_v, table, seq, 128, nb_max=1024, k_bar_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    yield dict(pool_k=pool_k, pool_v=pool_v, table=table, seq=seq, q=q, k_bar=summ["k_bar"])


def test_c4_fullsize(c4, device):
    announce("C4 full size: fused == two-step, sampled oracle")
    p = c4
    out, idx, n_sel = ia.sparse_topk_decode(p["q"], p["pool_k"], p["pool_v"], p["table"], p["seq"], p["k_bar"], 64,
                                            block_size=128, return_selection=True, workspace={})
    idx2, n_sel2 = ia.select_blocks_topk(p["q"], p["k_bar"], p["seq"], 64, block_size=128)
    out2 = ia.sparse_paged_decode(p["q"], p["pool_k"], p["pool_v"], p["table"], p["seq"], idx2, n_sel2,
                                  block_size=128)
    torch.cuda.synchronize()
    assert torch.equal(n_sel, n_sel2) and torch.equal(idx, idx2) and torch.equal(out, out2)
    assert bool((n_sel == 64).all())
    _check_sample(p["q"], p["pool_k"], p["pool_v"], p["table"], p["seq"], p["k_bar"], idx, n_sel, out, 128, 64,
                  sample=range(16))


def test_c4_fullsize_summaries(c4, device):
    announce("C4 full size: summaries of sequence 5 against the oracle")
    p = c4
    _check_summaries(p["pool_k"], p["pool_v"], p["table"], p["seq"], 5, 128, p["k_bar"])


def test_c5_fullsize_fp8(c4, device):
    announce("C5 full size: fp8 K/V vs the oracle (every sequence) and vs bf16 on the same selection")
    p = c4
    pk, pv = p["pool_k"], p["pool_v"]
    ks = (pk.abs().amax(dim=(2, 3)).float().clamp_min(1e-12) / 448.0).contiguous()
    vs = (pv.abs().amax(dim=(2, 3)).float().clamp_min(1e-12) / 448.0).contiguous()
    k8 = (pk.float() / ks[:, :, None, None]).to(torch.float8_e4m3fn)
    v8 = (pv.float() / vs[:, :, None, None]).to(torch.float8_e4m3fn)
    idx, n_sel = ia.select_blocks_topk(p["q"], p["k_bar"], p["seq"], 64, block_size=128)
    ref = ia.sparse_paged_decode(p["q"], pk, pv, p["table"], p["seq"], idx, n_sel, block_size=128)
    got = ia.sparse_paged_decode(p["q"], k8, v8, p["table"], p["seq"], idx, n_sel, block_size=128, scales=(ks, vs))
    # the fused fp8 layer call selects from the same k_bar: same blocks, same output
    fused = ia.sparse_topk_decode(p["q"], k8, v8, p["table"], p["seq"], p["k_bar"], 64, block_size=128,
                                  scales=(ks, vs), workspace={})
    # and with the scales gathered per sequence (the bench's C5 form): the same bits
    fused3 = ia.sparse_topk_decode(p["q"], k8, v8, p["table"], p["seq"], p["k_bar"], 64, block_size=128,
                                   scales=(ks, vs, ia.sequence_scales((ks, vs), p["table"])), workspace={})
    torch.cuda.synchronize()
    assert torch.equal(fused, got) and torch.equal(fused3, got)
    err = (got.float() - ref.float()).abs().max().item()
    assert err <= 6e-2, err
    g = HQ // HKV
    for b in range(16):
        L = int(p["seq"][b])
        qb = p["q"][b].double().cpu().numpy()
        for h in range(HKV):
            chosen = idx[b, h, :int(n_sel[b, h])].cpu().numpy()
            kk = _gather_head(k8, p["table"][b], chosen, 128, L, h, ks)
            vv = _gather_head(v8, p["table"][b], chosen, 128, L, h, vs)
            # Q.K is exact on the dequantised values; P.V uses bf16(p * v_scale) weights on
            # the codes, within 2^-8 relative of the oracle's bf16(p) weights on dequantised V
            r = A.sparse_decode(qb[h * g:(h + 1) * g], kk[None], vv[None], [np.arange(64)], 128, p_bf16=True)
            vmax = float(np.abs(vv).max())
            e = np.abs(got[b, h * g:(h + 1) * g].double().cpu().numpy() - r).max()
            assert e <= 2e-3 + 2 ** -8 * vmax, (b, h, e)
    del k8, v8


def test_dense_fullsize_128k(c4, device):
    announce("dense decode over 128K, two sequences")
    p = c4
    seq2 = p["seq"][:2].contiguous()
    out = ia.paged_decode(p["q"][:2].contiguous(), p["pool_k"], p["pool_v"], p["table"][:2].contiguous(), seq2,
                          max_seq_len=131072)
    torch.cuda.synchronize()
    b = 1
    pg = p["table"][b].long()
    kk = p["pool_k"][pg].permute(1, 0, 2, 3).reshape(HKV, -1, D).double().cpu().numpy()
    vv = p["pool_v"][pg].permute(1, 0, 2, 3).reshape(HKV, -1, D).double().cpu().numpy()
    ref = A.dense_decode(p["q"][b].double().cpu().numpy(), kk, vv)
    assert np.abs(out[b].double().cpu().numpy() - ref).max() <= 2e-2


def test_c3_fullsize_ragged(device):
    announce("C3 full size: ragged batch over a shared 4M-token pool, k = max(16, nb/16)")
    lens = [int(x) for x in np.random.default_rng(1236).integers(8192, 65537, size=16)]
    pool_k, pool_v, table, seq, q = _make(device, lens, 1236, pool_tokens=4 << 20)
    assert pool_k.shape[0] == (4 << 20) // PAGE
    nb_max = max(math.ceil(L / 64) for L in lens)
    summ = ia.build_block_summaries(pool_k, pool_v, table, seq, 64, nb_max=nb_max, k_bar_dtype=torch.bfloat16)
    kvec = torch.tensor([max(16, math.ceil(L / 64) // 16) for L in lens], device=device, dtype=torch.int32)
    k_cap = int(kvec.max())
    out, idx, n_sel = ia.sparse_topk_decode(q, pool_k, pool_v, table, seq, summ["k_bar"], 0, block_size=64,
                                            k_per_seq=kvec, k_cap=k_cap, return_selection=True, workspace={})
    idx2, n_sel2 = ia.select_blocks_topk(q, summ["k_bar"], seq, 0, block_size=64, k_per_seq=kvec, k_cap=k_cap)
    out2 = ia.sparse_paged_decode(q, pool_k, pool_v, table, seq, idx2, n_sel2, block_size=64)
    torch.cuda.synchronize()
    assert torch.equal(n_sel, n_sel2) and torch.equal(out, out2)
    assert n_sel.cpu().tolist() == [[int(k)] * HKV for k in kvec.cpu().tolist()]
    _check_sample(q, pool_k, pool_v, table, seq, summ["k_bar"], idx, n_sel, out, 64, 0, sample=range(16),
                  k_per_seq=kvec.cpu().numpy())
    announce("C3 full size: summaries of the longest sequence against the oracle")
    _check_summaries(pool_k, pool_v, table, seq, int(np.argmax(lens)), 64, summ["k_bar"])
    del pool_k, pool_v


def test_c2_fullsize(device):
    """BASELINE config 2 at its workload: batch 1, 32768 tokens, block 64 (512 blocks),
    top-64 plus the first block and the last two, K with per-channel outliers."""
    announce("C2 full size: batch 1, 32K, block 64, top-64 + first + last 2, key outliers")
    lens = [32768]
    pool_k, pool_v, table, seq, q = _make(device, lens, 1235, k_outlier=True)
    summ = ia.build_block_summaries(pool_k, pool_v, table, seq, 64, nb_max=512, k_bar_dtype=torch.bfloat16)
    out, idx, n_sel = ia.sparse_topk_decode(q, pool_k, pool_v, table, seq, summ["k_bar"], 64, block_size=64,
                                            forced_first=1, forced_last=2, return_selection=True, workspace={})
    idx2, n_sel2 = ia.select_blocks_topk(q, summ["k_bar"], seq, 64, block_size=64, forced_first=1, forced_last=2)
    out2 = ia.sparse_paged_decode(q, pool_k, pool_v, table, seq, idx2, n_sel2, block_size=64)
    torch.cuda.synchronize()
    assert torch.equal(n_sel, n_sel2) and torch.equal(idx, idx2) and torch.equal(out, out2)
    assert bool((n_sel == 67).all())
    assert bool((idx[0, :, 0] == 0).all()) and bool((idx[0, :, 65:67] == torch.tensor([510, 511], device=device)).all())
    _check_sample(q, pool_k, pool_v, table, seq, summ["k_bar"], idx, n_sel, out, 64, 64, sample=(0,), ff=1, fl=2)
