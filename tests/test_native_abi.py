"""The C ABI library loads and exports every symbol ``include/interattn_amd.h`` declares,
and rejects bad arguments before touching the GPU (CPU only: no compute calls)."""

import ctypes
import os
import re

import pytest

from interattn_amd import _native as N

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "interattn_amd.h")


def header_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"IA_API\s+[\w\s\*]*?\b(ia_\w+)\s*\(", text)))


def test_header_declares_the_bound_symbols():
    syms = header_symbols()
    assert syms, "no IA_API declarations found"
    assert set(syms) == set(N.SIGNATURES), "ctypes signatures and header declarations differ"


def test_library_exports_every_header_symbol():
    lib = N.lib()
    for name in header_symbols():
        assert hasattr(lib, name), name
    assert lib.ia_version() >= 1


def test_struct_layouts_match_the_header():
    # ia_paged_kv: 2 pointers, 2 int32, 7 int64, pointer, 2 int64, 2 pointers, int64, pointer, 2 int64
    assert ctypes.sizeof(N.PagedKV) == 8 * 2 + 4 * 2 + 8 * 7 + 8 + 8 * 2 + 8 * 2 + 8 + 8 + 8 * 2
    assert ctypes.sizeof(N.DecodeShape) == 4 * 4 + 8 * 2 + 8
    # ia_block_summaries: 4 pointers, 3 int32 (+pad), 3 pointers, 3 int32 (+pad)
    assert ctypes.sizeof(N.BlockSummaries) == 8 * 4 + 4 * 4 + 8 * 3 + 4 * 4
    # ia_suffix_kv: 2 pointers, 6 int64, pointer, 2 int32
    assert ctypes.sizeof(N.SuffixKV) == 8 * 2 + 8 * 6 + 8 + 4 * 2
    # ia_block_keys: 2 int32, 3 pointers, 2 int64
    assert ctypes.sizeof(N.BlockKeys) == 4 * 2 + 8 * 3 + 8 * 2


def test_workspace_sizes_are_consistent():
    lib = N.lib()
    assert lib.ia_select_topk_workspace_size(16, 8, 1024) >= 16 * 8 * 1024 * 4
    items = lib.ia_sparse_max_items(16, 8, 64)
    assert 1 <= items <= 64
    need = lib.ia_paged_decode_workspace_size(16, 8, 4, 128, items)
    assert need >= 16 * 8 * items * 4 * 128 * 4
    assert lib.ia_dense_max_items(1, 8, 0) == 1


def test_invalid_arguments_are_rejected_without_launching():
    lib = N.lib()
    sh = N.DecodeShape(batch=1, n_q_heads=6, n_kv_heads=4, head_dim=128, q_batch_stride=0, q_row_stride=128,
                       q_dtype=N.IA_BF16)
    kv = N.PagedKV()
    rc = lib.ia_sparse_paged_decode(sh, None, kv, None, 64, None, 8, None, 1.0, None, N.IA_BF16, None, 0, None)
    assert rc != 0
    assert lib.ia_last_error()
    sh.n_q_heads = 32
    sh.n_kv_heads = 8
    sh.head_dim = 96
    keys = N.BlockKeys(score=N.IA_SCORE_MEAN_KEY, dtype=N.IA_BF16)
    rc = lib.ia_select_topk(sh, None, keys, None, 64, 8, 4, None, 0, 0, 0, None, 4, None, None, None, 0, None)
    assert rc != 0
    with pytest.raises(ValueError):
        N.check(rc)
    # an unknown score, and a Quest score without its k_max / k_min rows
    sh.head_dim = 128
    for bad in (N.BlockKeys(score=7, dtype=N.IA_BF16, k_bar=256),
                N.BlockKeys(score=N.IA_SCORE_QUEST, dtype=N.IA_BF16, k_bar=256)):
        rc = lib.ia_select_topk(sh, 256, bad, 256, 64, 8, 4, None, 0, 0, 0, 256, 4, 256, None, None, 0, None)
        assert rc == N.IA_ERR_INVALID, lib.ia_last_error()
        rc = lib.ia_sparse_topk_decode(sh, 256, kv, 256, bad, 64, 8, 4, None, 0, 0, 0, 4, 1.0, 256, N.IA_BF16, None,
                                       None, None, 0, None)
        assert rc == N.IA_ERR_INVALID
    previous = lib.ia_set_wait_limit(5)
    assert lib.ia_set_wait_limit(-1) == 5 and previous > 0
    assert lib.ia_set_wait_limit(-1) == previous
    rc = lib.ia_build_block_summaries(kv, None, 1, 8, 128, 64, 4, None, 1, None, 1, None, None, 1, None, None, None,
                                      None)
    assert rc == N.IA_ERR_INVALID


def test_noalloc_scratch_bound_matches_the_header():
    text = open(HEADER).read()
    m = re.search(r"#define IA_NOALLOC_SCRATCH_BYTES \((\d+)u << (\d+)\)", text)
    assert m, "IA_NOALLOC_SCRATCH_BYTES not found"
    assert int(m.group(1)) << int(m.group(2)) == N.IA_NOALLOC_SCRATCH_BYTES


def test_noalloc_rejects_bad_arguments_before_its_scratch():
    lib = N.lib()
    sh = N.DecodeShape(batch=1, n_q_heads=32, n_kv_heads=8, head_dim=128, q_batch_stride=32 * 128, q_row_stride=128,
                       q_dtype=N.IA_BF16)
    kv = N.PagedKV()
    keys = N.BlockKeys(score=N.IA_SCORE_MEAN_KEY, dtype=N.IA_BF16, k_bar=256)
    for block_size, nb_max, k_cap in ((40, 8, 4), (64, -1, 4), (64, 8, 0)):
        rc = lib.ia_sparse_topk_decode_noalloc(sh, 256, kv, 256, keys, block_size, nb_max, 4, None, 0, 0, 0, k_cap,
                                               1.0, 256, N.IA_BF16, None, None, None)
        assert rc == N.IA_ERR_INVALID, lib.ia_last_error()
    sh.n_q_heads = 30  # not a multiple of the kv heads
    rc = lib.ia_sparse_topk_decode_noalloc(sh, 256, kv, 256, keys, 64, 8, 4, None, 0, 0, 0, 4, 1.0, 256, N.IA_BF16,
                                           None, None, None)
    assert rc != 0


def test_noalloc_rejects_calls_beyond_its_scratch_before_launching():
    # more (sequence, kv head) rows than the scratch's fixed row lines, then rows that
    # fit but a score row too long for the bytes: both rejected before any launch
    lib = N.lib()
    keys = N.BlockKeys(score=N.IA_SCORE_MEAN_KEY, dtype=N.IA_BF16, k_bar=256)
    kv = N.PagedKV()
    for batch, nb_max, what in ((300, 64, "rows"), (256, 4096, "bytes")):
        sh = N.DecodeShape(batch=batch, n_q_heads=32, n_kv_heads=8, head_dim=128, q_batch_stride=32 * 128,
                           q_row_stride=128, q_dtype=N.IA_BF16)
        rc = lib.ia_sparse_topk_decode_noalloc(sh, 256, kv, 256, keys, 128, nb_max, 16, None, 0, 0, 0, 64, 0.1, 256,
                                               N.IA_BF16, None, None, None)
        assert rc == N.IA_ERR_WORKSPACE, (what, lib.ia_last_error())
        assert "scratch" in lib.ia_last_error().decode(), what


def test_sequence_scales_are_checked_before_launching():
    # per-sequence scale pairs on a bf16 pool, and odd (unaligned) pair strides on an
    # fp8 pool: both rejected by the argument checks
    lib = N.lib()
    sh = N.DecodeShape(batch=1, n_q_heads=32, n_kv_heads=8, head_dim=128, q_batch_stride=32 * 128, q_row_stride=128,
                       q_dtype=N.IA_BF16)
    kv = N.PagedKV(k=256, v=256, dtype=N.IA_BF16, page_size=16, n_pages=4, k_page_stride=8 * 16 * 128,
                   k_head_stride=16 * 128, k_token_stride=128, v_page_stride=8 * 16 * 128, v_head_stride=16 * 128,
                   v_token_stride=128, seq_scale=256, seq_scale_b_stride=64, seq_scale_h_stride=8)
    rc = lib.ia_paged_decode(sh, 256, kv, 256, 64, 0.1, 256, N.IA_BF16, 256, 1 << 20, None)
    assert rc == N.IA_ERR_INVALID and b"seq_scale" in lib.ia_last_error()
    kv.dtype = N.IA_FP8_E4M3
    kv.k_scale = kv.v_scale = 256
    kv.scale_page_stride = 8
    kv.seq_scale_h_stride = 3
    rc = lib.ia_paged_decode(sh, 256, kv, 256, 64, 0.1, 256, N.IA_BF16, 256, 1 << 20, None)
    assert rc == N.IA_ERR_INVALID and b"seq_scale" in lib.ia_last_error()


def test_sequence_scales_gather_the_page_scales():
    import torch

    import interattn_amd as ia

    g = torch.Generator().manual_seed(3)
    ks, vs = torch.rand(10, 4, generator=g), torch.rand(10, 4, generator=g)
    table = torch.tensor([[3, 7, 1, -1], [0, 9, 2, 5]], dtype=torch.int32)
    seq = ia.sequence_scales((ks, vs), table)
    assert seq.shape == (2, 4, 4, 2) and seq.is_contiguous()
    for b in range(2):
        for lp in range(4):
            pg = int(table[b, lp])
            if pg < 0:
                continue  # never read: the finalize skips invalid pages
            for h in range(4):
                assert float(seq[b, h, lp, 0]) == float(ks[pg, h]) and float(seq[b, h, lp, 1]) == float(vs[pg, h])
