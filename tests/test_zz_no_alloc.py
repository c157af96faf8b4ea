"""ia_sparse_topk_decode_noalloc (library-held scratch, no workspace argument) against
ia_sparse_topk_decode (caller workspace), through the C ABI.

The two entry points run the same launch, so the bar is bit equality of the output,
the selected block ids and their counts, on every call.  The scratch keeps per-row
epochs and tagged words from call to call, so the calls change shape and query
between them: rows of 2 items (whole-row scoring, tagged merge), of 8 items (score
hand-off, tagged merge) and of 16 or 32 items (untagged merge) follow each other, a
shape is re-entered with a new query, and a graph holding the call is replayed with a
new query each time between eager calls of other shapes, both when its capture holds
the scratch's first clear (the first test of this file: the process's first
allocation-free call) and when it does not.  A call too large for the scratch fails
with a clear error and launches nothing.
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


def _expect(x, k, k_cap, got, what):
    """Bit equality of a no-alloc result (out, idx, n_sel) with the workspace call."""
    out, idx, n_sel = got
    ref, ref_idx, ref_n = _reference(x, k, k_cap)
    torch.cuda.synchronize()
    assert torch.equal(n_sel, ref_n), what
    b, hkv = n_sel.shape
    for i in range(b):
        for h in range(hkv):
            n = int(ref_n[i, h])
            assert torch.equal(idx[i, h, :n], ref_idx[i, h, :n]), (what, i, h)
    assert torch.equal(out, ref), what


def _check(x, k, k_cap, what):
    announce(f"no-alloc decode {what}")
    rc, out, idx, n_sel = _noalloc(x, k, k_cap)
    N.check(rc)
    _expect(x, k, k_cap, (out, idx, n_sel), what)


def _new_q(x, seed):
    g = torch.Generator(device=x["q"].device)
    g.manual_seed(seed)
    y = dict(x)
    y["q"] = torch.randn(x["q"].shape, device=x["q"].device, generator=g).to(x["q"].dtype)
    return y


# rows of 8 items each (4 sequences x 8 kv heads over 256 resident workgroups: score
# hand-off and tagged merge), of 2 items (16 x 8, equal rows: whole-row scoring and
# tagged merge), of 16 items (2 x 8: untagged merge)
def _shape_hand_off(device, seed):
    return _inputs(device, seed, 4, [5000, 8192, 3000, 6500])


def _shape_two_items(device, seed):
    return _inputs(device, seed, 16, [4096] * 16, block=64)


def _shape_many_items(device, seed):
    return _inputs(device, seed, 2, [8192, 6000])


def _graph_of_noalloc(x, k, k_cap):
    """A graph holding one no-alloc call on static q/out/idx/n_sel tensors."""
    lib = N.lib()
    b, hq, d = x["q"].shape
    hkv = int(x["pool_k"].shape[1])
    keys, _, _, keep_k = ops._block_keys(x["k_bar"], "mean")
    kv, keep = ops.paged_kv(x["pool_k"], x["pool_v"], x["table"])
    sh = ops._decode_shape(x["q"], hkv)
    st = dict(q=x["q"].clone(), out=torch.empty_like(x["q"]),
              idx=torch.full((b, hkv, k_cap), -7, device=x["q"].device, dtype=torch.int32),
              n_sel=torch.full((b, hkv), -7, device=x["q"].device, dtype=torch.int32))
    nb_max = int(x["k_bar"].shape[2])
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = lib.ia_sparse_topk_decode_noalloc(
            sh, st["q"].data_ptr(), kv, x["seq"].data_ptr(), keys, x["block"], nb_max, k, None, 0, 0, 0, k_cap,
            d ** -0.5, st["out"].data_ptr(), N.IA_BF16, st["idx"].data_ptr(), st["n_sel"].data_ptr(),
            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    N.check(rc)
    st["_keep"] = (keep, keep_k, kv, keys, sh)
    return graph, st


def _replays(graph, st, x, k, k_cap, others, seeds, what):
    """Replay the graph with a new query each time; eager no-alloc calls of other
    shapes (with new queries too) run between the replays.  Every result is checked."""
    for n, seed in enumerate(seeds):
        xq = _new_q(x, seed)
        st["q"].copy_(xq["q"])
        announce(f"no-alloc decode {what}: replay {n}")
        graph.replay()
        torch.cuda.synchronize()
        _expect(xq, k, k_cap, (st["out"], st["idx"], st["n_sel"]), f"{what}: replay {n}")
        for m, (y, ky, kcy, name) in enumerate(others):
            _check(_new_q(y, seed * 10 + m), ky, kcy, f"{what}: {name} after replay {n}")


def test_noalloc_graph_holding_the_first_clear(device):
    a = _shape_hand_off(device, 21)
    b2 = _shape_two_items(device, 22)
    c = _shape_many_items(device, 23)
    # the library's lazy set-up (occupancy, kernel attributes) outside the capture,
    # through the workspace entry point only: the graph's call is the process's first
    # allocation-free call, so its capture holds the clear of the scratch
    _reference(a, 16, 16)
    torch.cuda.synchronize()
    announce("no-alloc decode: capture (8-item rows)")
    graph, st = _graph_of_noalloc(a, 16, 16)
    _replays(graph, st, a, 16, 16, [(b2, 8, 8, "2-item rows"), (c, 16, 16, "16-item rows")], [31, 32, 33],
             "graph holding the clear")


def test_noalloc_equals_workspace_call(device):
    big = _inputs(device, 11, 2, [8192, 6000])
    small = _inputs(device, 12, 1, [3000], block=64)
    _check(big, 16, 16, "first call (2 x 8K/6K, block 128)")
    _check(small, 8, 10, "second call, smaller (1 x 3K, block 64)")
    _check(big, 16, 16, "first shape again")
    _check(big, 16, 16, "same shape, no clear")


def test_noalloc_shape_changes_with_new_queries(device):
    a = _shape_hand_off(device, 41)
    b2 = _shape_two_items(device, 42)
    c = _shape_many_items(device, 43)
    _check(a, 16, 16, "A: 8-item rows")
    _check(b2, 8, 8, "B: 2-item rows")
    _check(_new_q(a, 44), 16, 16, "A' (new q) after B")
    _check(c, 16, 16, "C: 16-item rows")
    _check(_new_q(b2, 45), 8, 8, "B' (new q) after C")
    _check(_new_q(a, 46), 16, 16, "A'' (new q) after B'")
    _check(_new_q(b2, 47), 8, 8, "B'' (new q) after A''")


def test_noalloc_graph_replays_between_other_shapes(device):
    a = _shape_hand_off(device, 51)
    b2 = _shape_two_items(device, 52)
    _check(b2, 8, 8, "B before the capture")
    announce("no-alloc decode: capture (2-item rows after another shape)")
    graph, st = _graph_of_noalloc(_new_q(b2, 53), 8, 8)
    _replays(graph, st, b2, 8, 8, [(a, 16, 16, "8-item rows")], [61, 62, 63], "graph of 2-item rows")


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
