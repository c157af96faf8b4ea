"""The one-launch condition call (``ia_condition_decode_fused``) beyond the parity
cases that ``tests/test_gpu_condition.py`` runs on both implementations:

* which calls fit one launch (GQA groups up to 4, rows x items within the device's
  resident workgroups);
* the statistics hand-off: with a wait limit of 0 every item computes the other
  items' partials itself, and selection and output equal the default run bit for
  bit (the result never depends on which workgroups run together);
* one zero-filled workspace serving prompts of different lengths in turn, and a
  captured call replayed with a new query each time between eager calls of another
  length: every result equals a call on a fresh workspace bit for bit;
* a batch of two sequences through the C ABI against the oracle (the routing per
  sequence, the selected flags of every query row, the output);
* the reference's published configuration (32 query / 8 KV heads, block 64,
  mixed summaries with bf16 k_bar, 128K tokens): one launch against the four-launch
  path (selection equal up to eps-boundary blocks, output within the bf16 bar).
"""

import ctypes
import math

import numpy as np
import pytest
import torch

from interattn_amd import _native as N
from interattn_amd import condition_block as cb
from tests._util import announce
from tests.test_gpu_condition import CASES, TOL, _check_selected, _expected, _make, _np, _oracle_stats, _prefix_np

pytestmark = pytest.mark.gpu


@pytest.fixture
def one_launch(monkeypatch):
    monkeypatch.setenv("INTERATTN_CONDITION_ONE_LAUNCH", "1")


def _items(batch, hkv, g, d, nb, block, sfx_cap=1, dtype=N.IA_BF16):
    sh = N.DecodeShape(batch=batch, n_q_heads=hkv * g, n_kv_heads=hkv, head_dim=d, q_batch_stride=hkv * g * d,
                       q_row_stride=d, q_dtype=dtype)
    sm = N.BlockSummaries(nb=nb, block_size=block)
    return int(N.lib().ia_condition_decode_fused_items(sh, sm, dtype, sfx_cap))


def test_one_launch_eligibility(device):
    announce("one-launch condition call: which calls fit")
    n = _items(1, 8, 4, 128, 2048, 64)
    assert 4 <= n <= 64, n                          # the reference's 128K configuration
    assert _items(1, 8, 4, 128, 512, 64) >= 1     # 32K
    assert _items(1, 8, 8, 128, 512, 64) == 0     # G = 8 takes the four-launch path
    assert _items(1, 8, 4, 96, 512, 64) == 0      # head_dim
    assert _items(64, 8, 4, 128, 2048, 64) == 0   # 512 rows x 4 items of 512 blocks: not resident at once
    assert _items(1, 2, 4, 128, 3, 64) <= 3       # never more items than blocks


def _call(q, prefix, ks, vs, sfx_len, b, eps, p, ws, stats=False):
    return cb._condition_block_decode_output(q_grouped=q, prompt_prefix=prefix, k_suffix=ks, v_suffix=vs,
                                             suffix_len_dev=sfx_len, block_size=b, eps=eps, prompt_len=p,
                                             attention_dtype=torch.float32, workspace=ws, collect_stats=stats)


@pytest.mark.parametrize("name", ["bf16_c1_like", "f32_b64_g4", "bf16_mixed_b32_mass"])
def test_one_launch_handoff_fallback_is_exact(name, device, one_launch):
    c = next(x for x in CASES if x[0] == name)
    _, seed, hkv, g, d, b, p, s, dt, mixed, kbd, mass = c
    announce(f"one-launch condition call: hand-off fallback {name}")
    host, dev = _make(c, device)
    kbt = torch.bfloat16 if kbd == "bf16" else torch.float32
    prefix = cb._build_prompt_blocks(dev["k"], dev["v"], b, mixed=mixed, k_bar_dtype=kbt)
    pre = _prefix_np(prefix)
    _, mean, _ = _oracle_stats(host["q"][:, :, 0].reshape(-1, d), pre, g, mass)
    vals = np.unique(mean[mean > 0])
    eps = float(0.5 * (vals[int(0.9 * len(vals))] + vals[int(0.9 * len(vals)) + 1]))
    sfx_len = torch.full((1,), s, device=device, dtype=torch.int32)
    lib = N.lib()
    res = []
    lib.ia_wait_fallbacks(1)
    counts = []
    for limit in (-1, 0):  # default bound, then 0: every item computes every partial itself
        prev = lib.ia_set_wait_limit(limit)
        try:
            ws = {}
            out, _ = cb._condition_block_decode_output(
                q_grouped=dev["q"], prompt_prefix=prefix, k_suffix=dev["ks"], v_suffix=dev["vs"],
                suffix_len_dev=sfx_len, block_size=b, eps=eps, prompt_len=p, attention_dtype=torch.float32,
                workspace=ws, term1_mass_exp=mass)
            torch.cuda.synchronize()
        finally:
            lib.ia_set_wait_limit(prev)
        counts.append(lib.ia_wait_fallbacks(1))
        res.append((out.clone(), ws["selected_rows"].clone()))
    assert torch.equal(res[0][1], res[1][1]), "selection depends on the hand-off"
    assert torch.equal(res[0][0], res[1][0]), "output depends on the hand-off"
    # the diagnostic: no fallback at the default bound with every workgroup resident
    print(f"[{name}] wait fallbacks: default bound {counts[0]}, bound 0 {counts[1]}", flush=True)
    assert counts[0] == 0


def test_one_launch_workspace_across_lengths_and_graph_replays(device, one_launch):
    """One workspace dict (one zero-filled scratch for the heads/group/head_dim) over
    prompts of 3000 and 20000 tokens in turn; a call captured on it is replayed with a
    new query each time, with eager calls of the other length between replays."""
    announce("one-launch condition call: shared workspace and graph replays")
    ca = ("wsA", 51, 4, 4, 128, 64, 3000, 5, "bf16", True, "bf16", False)
    cbb = ("wsB", 52, 4, 4, 128, 64, 20000, 9, "bf16", True, "bf16", False)
    _, dev_a = _make(ca, device)
    _, dev_b = _make(cbb, device)
    pa = cb._build_prompt_blocks(dev_a["k"], dev_a["v"], 64, mixed=True, k_bar_dtype=torch.bfloat16)
    pb = cb._build_prompt_blocks(dev_b["k"], dev_b["v"], 64, mixed=True, k_bar_dtype=torch.bfloat16)
    la = torch.full((1,), 5, device=device, dtype=torch.int32)
    lb = torch.full((1,), 9, device=device, dtype=torch.int32)
    eps = 0.02
    gen = torch.Generator(device=device)
    gen.manual_seed(5)

    def fresh(q, prefix, ks, vs, ln, p):
        o, _ = _call(q, prefix, ks, vs, ln, 64, eps, p, {})
        return o.clone()

    ws = {}
    q_static = dev_a["q"].clone()
    _call(q_static, pa, dev_a["ks"], dev_a["vs"], la, 64, eps, 3000, ws)
    _call(dev_b["q"], pb, dev_b["ks"], dev_b["vs"], lb, 64, eps, 20000, ws)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_g, _ = _call(q_static, pa, dev_a["ks"], dev_a["vs"], la, 64, eps, 3000, ws)
    for n in range(3):
        qa = torch.randn(dev_a["q"].shape, device=device, generator=gen).to(torch.bfloat16)
        qb = torch.randn(dev_b["q"].shape, device=device, generator=gen).to(torch.bfloat16)
        q_static.copy_(qa)
        graph.replay()
        torch.cuda.synchronize()
        got = out_g.clone()
        assert torch.equal(got, fresh(qa, pa, dev_a["ks"], dev_a["vs"], la, 3000)), f"replay {n}"
        ob, _ = _call(qb, pb, dev_b["ks"], dev_b["vs"], lb, 64, eps, 20000, ws)
        ob = ob.clone()
        torch.cuda.synchronize()
        assert torch.equal(ob, fresh(qb, pb, dev_b["ks"], dev_b["vs"], lb, 20000)), f"other length after replay {n}"


def test_one_launch_batch_of_two_through_the_c_abi(device):
    """Two sequences of different lengths in one call (block table over one pool),
    each against the oracle: selected flags of every query row near the threshold
    only, output on the GPU's own selection within the bf16 bar."""
    announce("one-launch condition call: batch 2 through the C ABI")
    hkv, g, d, b = 4, 4, 128, 64
    cases = [("bA", 61, hkv, g, d, b, 6000, 3, "bf16", True, "bf16", False),
             ("bB", 62, hkv, g, d, b, 9000, 3, "bf16", True, "bf16", False)]
    hosts, devs, prefixes = [], [], []
    for c in cases:
        h_, d_ = _make(c, device)
        hosts.append(h_)
        devs.append(d_)
        prefixes.append(cb._build_prompt_blocks(d_["k"], d_["v"], b, mixed=True, k_bar_dtype=torch.bfloat16))
    nbs = [int(pf["block_valid_counts"].numel()) for pf in prefixes]
    nb = max(nbs)
    # one pool of pages (one block each): sequence i's blocks at pages [off_i, off_i + nb_i)
    kpool = torch.cat([pf["k_block_attn"].transpose(0, 1) for pf in prefixes]).contiguous()  # [pages, Hkv, B, D]
    vpool = torch.cat([pf["v_block_attn"].transpose(0, 1) for pf in prefixes]).contiguous()
    table = torch.full((2, nb), -1, device=device, dtype=torch.int32)
    table[0, :nbs[0]] = torch.arange(nbs[0], device=device, dtype=torch.int32)
    table[1, :nbs[1]] = torch.arange(nbs[0], nbs[0] + nbs[1], device=device, dtype=torch.int32)

    def stack(key, dtype=None):
        parts = []
        for pf in prefixes:
            x = pf[key]
            pad = nb - x.shape[-2] if x.dim() == 3 else nb - x.shape[-1]
            if x.dim() == 3:
                x = torch.cat([x, x.new_zeros((x.shape[0], pad, x.shape[2]))], 1)
            elif x.dim() == 2:
                x = torch.cat([x, x.new_full((x.shape[0], pad), float("-inf"))], 1)
            else:
                x = torch.cat([x, x.new_zeros((pad,))])
            parts.append(x)
        out = torch.stack(parts).contiguous()
        return out if dtype is None else out.to(dtype)

    kb, kx, kn, vb = stack("k_bar"), stack("k_max"), stack("k_min"), stack("v_bar")
    vnm = stack("v_norm_max").float().contiguous()
    vna = torch.stack([pf["v_norm_all"] for pf in prefixes]).float().contiguous()
    cnt = stack("block_valid_counts").to(torch.int32).contiguous()
    sm = N.BlockSummaries()
    sm.k_bar, sm.k_max, sm.k_min, sm.v_bar = kb.data_ptr(), kx.data_ptr(), kn.data_ptr(), vb.data_ptr()
    sm.k_bar_dtype = N.IA_BF16 if kb.dtype == torch.bfloat16 else N.IA_F32
    sm.bounds_dtype = N.IA_BF16 if kx.dtype == torch.bfloat16 else N.IA_F32
    sm.v_bar_dtype = N.IA_BF16 if vb.dtype == torch.bfloat16 else N.IA_F32
    sm.v_norm_max, sm.v_norm_all, sm.counts = vnm.data_ptr(), vna.data_ptr(), cnt.data_ptr()
    sm.nb, sm.block_size = nb, b
    kv = N.PagedKV()
    kv.k, kv.v, kv.dtype, kv.page_size, kv.n_pages = kpool.data_ptr(), vpool.data_ptr(), N.IA_BF16, b, int(kpool.shape[0])
    kv.k_page_stride, kv.k_head_stride, kv.k_token_stride = (int(x) for x in kpool.stride()[:3])
    kv.v_page_stride, kv.v_head_stride, kv.v_token_stride = (int(x) for x in vpool.stride()[:3])
    kv.block_table, kv.bt_stride, kv.bt_cols = table.data_ptr(), nb, nb
    ks = torch.stack([d_["ks"] for d_ in devs]).contiguous()  # [2, Hkv, S, D]
    vs = torch.stack([d_["vs"] for d_ in devs]).contiguous()
    slen = torch.full((2,), 3, device=device, dtype=torch.int32)
    sfx = N.SuffixKV()
    sfx.k, sfx.v = ks.data_ptr(), vs.data_ptr()
    sfx.k_batch_stride, sfx.k_head_stride, sfx.k_token_stride = (int(x) for x in ks.stride()[:3])
    sfx.v_batch_stride, sfx.v_head_stride, sfx.v_token_stride = (int(x) for x in vs.stride()[:3])
    sfx.len, sfx.len_stride, sfx.cap = slen.data_ptr(), 1, 3
    q = torch.stack([d_["q"].reshape(hkv * g, d) for d_ in devs]).contiguous()  # [2, Hq, D]
    sh = N.DecodeShape(batch=2, n_q_heads=hkv * g, n_kv_heads=hkv, head_dim=d, q_batch_stride=hkv * g * d,
                       q_row_stride=d, q_dtype=N.IA_BF16)
    lib = N.lib()
    assert lib.ia_condition_decode_fused_items(sh, sm, N.IA_BF16, 3) > 0
    nbytes = lib.ia_condition_decode_fused_workspace_size(2, hkv, g, d)
    ws = torch.zeros((nbytes,), device=device, dtype=torch.uint8)
    out = torch.empty((2, hkv * g, d), device=device, dtype=torch.float32)
    selected = torch.full((2, hkv * g, nb), 7, device=device, dtype=torch.uint8)
    means = []
    for i in range(2):
        pre = _prefix_np(prefixes[i])
        _, mean, _ = _oracle_stats(hosts[i]["q"][:, :, 0].reshape(-1, d), pre, g, False)
        means.append(mean)
    eps = 0.02
    N.check(lib.ia_condition_decode_fused(sh, q.data_ptr(), sm, kv, sfx, eps, 0, selected.data_ptr(), d ** -0.5,
                                          out.data_ptr(), N.IA_F32, ws.data_ptr(), ws.numel(),
                                          ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()
    for i in range(2):
        pre = _prefix_np(prefixes[i])
        n_i = nbs[i]
        sel_gpu = _np(selected[i, :, :n_i]).astype(bool).reshape(hkv, g, 1, n_i)
        ref_sel = np.repeat((means[i] > eps) & (pre["block_valid_counts"] > 0)[None], g, 0).reshape(hkv, g, 1, -1)
        _check_selected(sel_gpu, ref_sel, means[i], eps, f"sequence {i}")
        _, _, z = _oracle_stats(hosts[i]["q"][:, :, 0].reshape(-1, d), pre, g, False)
        exp = _expected(hosts[i]["q"], hosts[i]["k"], hosts[i]["v"], hosts[i]["ks"], hosts[i]["vs"], b, pre, sel_gpu,
                        z)
        np.testing.assert_allclose(_np(out[i]).reshape(exp.shape), exp, atol=TOL["bf16"], rtol=0,
                                   err_msg=f"sequence {i}")


def test_one_launch_matches_four_launch_at_128k(device, monkeypatch):
    """The reference's published configuration: 32 query / 8 KV heads, block 64, mixed
    summaries (bf16 k_bar), 131072 tokens, one suffix token, ~1% of blocks selected."""
    announce("one-launch condition call: 128K, against the four-launch path")
    hkv, g, d, b, p, s = 8, 4, 128, 64, 131072, 1
    gen = torch.Generator(device=device)
    gen.manual_seed(1238)
    k = torch.randn((hkv, p, d), device=device, dtype=torch.bfloat16, generator=gen)
    v = torch.randn((hkv, p, d), device=device, dtype=torch.bfloat16, generator=gen)
    ks = torch.randn((hkv, s, d), device=device, dtype=torch.bfloat16, generator=gen)
    vs = torch.randn((hkv, s, d), device=device, dtype=torch.bfloat16, generator=gen)
    q = torch.randn((hkv, g, 1, d), device=device, dtype=torch.bfloat16, generator=gen)
    prefix = cb._build_prompt_blocks(k, v, b, mixed=True, k_bar_dtype=torch.bfloat16)
    pre = _prefix_np(prefix)
    _, mean, _ = _oracle_stats(_np(q)[:, :, 0].reshape(-1, d), pre, g, False)
    vals = np.sort(mean.reshape(-1))
    eps = float(vals[int(0.99 * len(vals))])  # ~1% of the blocks above it
    sfx_len = torch.full((1,), s, device=device, dtype=torch.int32)
    res = {}
    for mode in ("1", "0"):
        monkeypatch.setenv("INTERATTN_CONDITION_ONE_LAUNCH", mode)
        ws = {}
        out, _ = cb._condition_block_decode_output(
            q_grouped=q, prompt_prefix=prefix, k_suffix=ks, v_suffix=vs, suffix_len_dev=sfx_len, block_size=b,
            eps=eps, prompt_len=p, attention_dtype=torch.bfloat16, workspace=ws)
        torch.cuda.synchronize()
        res[mode] = (_np(out), _np(ws["selected_rows"]).astype(bool).reshape(hkv, g, 1, -1))
    _check_selected(res["1"][1], res["0"][1], mean, eps, "one launch vs four launches")
    frac = float(res["1"][1].mean())
    assert 0.002 < frac < 0.05, frac
    if np.array_equal(res["1"][1], res["0"][1]):
        assert np.abs(res["1"][0] - res["0"][0]).max() <= TOL["bf16"]
