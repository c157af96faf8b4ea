"""ia_sparse_topk_decode_noalloc (library-held scratch, no workspace argument) against
ia_sparse_topk_decode (caller workspace), through the C ABI.

The two entry points run the same launch, so the bar is bit equality of the output,
the selected block ids and their counts.  Calls in a row on one device: a C4-shaped
call (two 8K/6K sequences, 32/8 heads, block 128, top-16), then a smaller one (one
sequence, fewer blocks: a new call shape, so the scratch is cleared first), then the
first shape again, then a call too large for the scratch (a clear error, nothing
launched).
"""

import ctypes
import math

import pytest
import torch

import interattn_amd as ia
from interattn_amd import _native as N
from interattn_amd import ops
from tests._util import announce

pytestmark = pytest.mark.gpu


def _inputs(device, seed, batch, lens, hq=32, hkv=8, d=128, page=16, block=128):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    pages = [math.ceil(L / page) for L in lens]
    n_pages = sum(pages)
    pool_k = torch.randn((n_pages, hkv, page, d), device=device, generator=g).to(torch.bfloat16)
    pool_v = torch.randn((n_pages, hkv, page, d), device=device, generator=g).to(torch.bfloat16)
    perm = torch.randperm(n_pages, device=device, generator=g).to(torch.int32)
    table = torch.full((batch, max(pages)), -1, device=device, dtype=torch.int32)
    off = 0
    for i, n in enumerate(pages):
        table[i, :n] = perm[off:off + n]
        off += n
    seq = torch.tensor(lens, device=device, dtype=torch.int32)
    q = torch.randn((batch, hq, d), device=device, generator=g).to(torch.bfloat16)
    nb_max = max(math.ceil(L / block) for L in lens)
    summ = ia.build_block_summaries(pool_k, pool_v, table, seq, block, nb_max=nb_max)
    return dict(q=q, pool_k=pool_k, pool_v=pool_v, table=table, seq=seq, k_bar=summ["k_bar"], block=block)


def _noalloc(x, k, k_cap):
    """One ia_sparse_topk_decode_noalloc call; returns (rc, out, idx, n_sel)."""
    lib = N.lib()
    b, hq, d = x["q"].shape
    hkv = int(x["pool_k"].shape[1])
    keys, _, _, keep_k = ops._block_keys(x["k_bar"], "mean")
    kv, keep = ops.paged_kv(x["pool_k"], x["pool_v"], x["table"])
    sh = ops._decode_shape(x["q"], hkv)
    out = torch.empty_like(x["q"])
    idx = torch.full((b, hkv, k_cap), -7, device=x["q"].device, dtype=torch.int32)
    n_sel = torch.full((b, hkv), -7, device=x["q"].device, dtype=torch.int32)
    nb_max = int(x["k_bar"].shape[2])
    rc = lib.ia_sparse_topk_decode_noalloc(
        sh, x["q"].data_ptr(), kv, x["seq"].data_ptr(), keys, x["block"], nb_max, k, None, 0, 0, 0, k_cap,
        d ** -0.5, out.data_ptr(), N.IA_BF16, idx.data_ptr(), n_sel.data_ptr(),
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    del keep, keep_k
    return rc, out, idx, n_sel


def _reference(x, k, k_cap):
    return ia.sparse_topk_decode(x["q"], x["pool_k"], x["pool_v"], x["table"], x["seq"], x["k_bar"], k,
                                 block_size=x["block"], k_cap=k_cap, return_selection=True, workspace={})


def _check(x, k, k_cap, what):
    announce(f"no-alloc decode {what}")
    rc, out, idx, n_sel = _noalloc(x, k, k_cap)
    N.check(rc)
    ref, ref_idx, ref_n = _reference(x, k, k_cap)
    torch.cuda.synchronize()
    assert torch.equal(n_sel, ref_n), what
    b, hkv = n_sel.shape
    for i in range(b):
        for h in range(hkv):
            n = int(ref_n[i, h])
            assert torch.equal(idx[i, h, :n], ref_idx[i, h, :n]), (what, i, h)
    assert torch.equal(out, ref), what


def test_noalloc_equals_workspace_call(device):
    big = _inputs(device, 11, 2, [8192, 6000])
    small = _inputs(device, 12, 1, [3000], block=64)
    _check(big, 16, 16, "first call (2 x 8K/6K, block 128)")
    _check(small, 8, 10, "second call, smaller (1 x 3K, block 64)")
    _check(big, 16, 16, "first shape again")
    _check(big, 16, 16, "same shape, no clear")


def test_noalloc_rejects_calls_beyond_its_scratch(device):
    announce("no-alloc decode: scratch bound")
    lib = N.lib()
    x = _inputs(device, 13, 1, [1024])
    # a 4096-block row for 512 sequences x 8 heads needs far more than the scratch
    sh = ops._decode_shape(x["q"], 8)
    sh.batch = 512
    keys, _, _, keep_k = ops._block_keys(x["k_bar"], "mean")
    kv, keep = ops.paged_kv(x["pool_k"], x["pool_v"], x["table"])
    need = lib.ia_sparse_topk_decode_workspace_size(512, 8, 4, 128, 4096, 64, 128)
    assert need > N.IA_NOALLOC_SCRATCH_BYTES
    rc = lib.ia_sparse_topk_decode_noalloc(sh, x["q"].data_ptr(), kv, x["seq"].data_ptr(), keys, 128, 4096, 16, None,
                                           0, 0, 0, 64, 0.1, x["q"].data_ptr(), N.IA_BF16, None, None, None)
    assert rc == N.IA_ERR_WORKSPACE
    assert "scratch" in lib.ia_last_error().decode()
    del keep, keep_k
