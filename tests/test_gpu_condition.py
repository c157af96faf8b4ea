"""GPU parity of the condition (eps-threshold) path through the reference-API mirror
``interattn_amd.condition_block`` against the golden vectors of the reference's own
functions and against the CPU oracle.

Bars: block selection equal to the reference's except for blocks whose group-mean
condition lies within 1e-3 relative (plus 1e-5 absolute) of eps; outputs within
1e-4 abs for float32 K/V and 2e-2 abs for bfloat16 K/V of the float64 restatement of
``_condition_block_decode_output_dense`` (CBT/legacy.py:797-868) evaluated on the
GPU's own selection; statistics and routing counts exact.

The decode tests run both implementations of the fused and fixed-mask entry points:
the one-launch calls (``ia_condition_decode_fused``, ``ia_fixed_mask_decode_fused``,
the default where a call fits one launch) and the multi-launch paths (statistics,
route, finalize, merge; route, finalize, merge).
"""

import glob
import math
import os

import numpy as np
import pytest
import torch

from interattn_amd import condition_block as cb
from oracle import attention as A
from oracle import select as S
from oracle import summaries as Su
from oracle.numerics import bf16_round
from tests._util import announce

pytestmark = pytest.mark.gpu

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURES = sorted(glob.glob(os.path.join(HERE, "cond_*.npz")))
TOL = {"bf16": 2e-2, "f32": 1e-4}


@pytest.fixture(params=["one_launch", "four_launch"])
def path(request, monkeypatch):
    """Which implementation the reference-API mirror's decode call takes."""
    monkeypatch.setenv("INTERATTN_CONDITION_ONE_LAUNCH", "1" if request.param == "one_launch" else "0")
    return request.param


def _load(path):
    f = np.load(path, allow_pickle=False)
    return {k: f[k] for k in f.files}


def _np(t):
    return t.detach().float().cpu().numpy() if t.is_floating_point() else t.detach().cpu().numpy()


def _prefix_np(prefix):
    keys = ("k_bar", "v_bar", "k_max", "k_min", "v_norm_max", "v_norm_all", "block_valid_counts")
    return {k: _np(prefix[k]) for k in keys}


def _padded(x, b):
    hkv, p, d = x.shape
    nb = math.ceil(p / b)
    return np.concatenate([x, np.zeros((hkv, nb * b - p, d), x.dtype)], 1).reshape(hkv, nb, b, d)


def _check_selected(got, ref, mean, eps, what):
    """``got/ref [Hkv, G, 1, nb]`` bool; ``mean [Hkv, nb]`` oracle group-mean condition."""
    diff = got != ref
    if diff.any():
        hh, _, _, jj = np.nonzero(diff)
        margin = np.abs(mean[hh, jj] - eps)
        tol = 1e-3 * abs(eps) + 1e-5
        assert np.all(margin <= tol), f"{what}: {int(diff.sum())} selections differ beyond the threshold band"
    # the group decision is broadcast over the group
    assert np.all(got == got[:, :1]), f"{what}: selection differs within a group"
    return int(diff.any(axis=(1, 2)).sum())


def _oracle_stats(q_rows, pre, g, mass_exp):
    st = S.selection_stats_chunked(q_rows.astype(np.float64), pre, g, term1_mass_exp=mass_exp)
    mean, z = S.condition_group_mean(st, pre, g, mass_exp)
    return st, mean, z


def _expected(q, k, v, ks, vs, b, pre, selected, z):
    hkv, g, _, d = q.shape
    p = k.shape[1]
    nb = pre["block_valid_counts"].shape[0]
    tok = np.arange(nb * b).reshape(nb, b)
    return A.hybrid_decode_dense(q, _padded(k, b), _padded(v, b), tok < p, tok, p + ks.shape[1] - 1, p, ks, vs,
                                 selected, z.reshape(hkv, g, 1, nb), pre["v_bar"], pre["block_valid_counts"] > 0)


# ------------------------------------------------------------------ golden vectors

@pytest.mark.parametrize("fixture", FIXTURES, ids=[os.path.basename(p)[:-4] for p in FIXTURES])
def test_golden_condition_path(fixture, path, device):
    fx = _load(fixture)
    hkv, g, d, b, p, s = (int(x) for x in fx["meta"])
    dt = "bf16" if "bf16" in os.path.basename(fixture) else "f32"
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    announce(f"golden {os.path.basename(fixture)} ({path}) hkv={hkv} g={g} d={d} block={b} P={p} S={s}")
    k = torch.from_numpy(fx["k"]).to(device, tdt)
    v = torch.from_numpy(fx["v"]).to(device, tdt)
    q = torch.from_numpy(fx["q"]).to(device, torch.float32)
    ks = torch.from_numpy(fx["k_suffix"]).to(device, tdt)
    vs = torch.from_numpy(fx["v_suffix"]).to(device, tdt)

    prefix = cb._build_prompt_blocks(k, v, b)
    torch.cuda.synchronize()
    got = _prefix_np(prefix)
    assert np.array_equal(got["block_valid_counts"], fx["prefix_block_valid_counts"])
    for key in ("k_bar", "v_bar", "v_norm_max", "v_norm_all"):
        np.testing.assert_allclose(got[key], fx["prefix_" + key], rtol=2e-6, atol=2e-6, err_msg=key)
    for key in ("k_max", "k_min"):
        assert np.array_equal(got[key], fx["prefix_" + key]), key

    pre = {kk[len("prefix_"):]: fx[kk] for kk in fx if kk.startswith("prefix_")}
    _, mean, _ = _oracle_stats(fx["q"][:, :, 0].reshape(-1, d), pre, g, False)
    sfx_len = torch.full((1,), s, device=device, dtype=torch.int32)
    ws = {}
    keys = [str(kk) for kk in fx["stats_keys"]]
    for i, eps in enumerate(fx["eps"]):
        sel, z, _vb, size, exists = cb._select_prompt_blocks_triton(q, prefix, float(eps))
        torch.cuda.synchronize()
        ref_sel = fx[f"selected_{i}"]
        _check_selected(_np(sel), ref_sel, mean, float(eps), f"select eps={eps}")
        np.testing.assert_allclose(_np(z), fx[f"z_{i}"], rtol=1e-5, atol=1e-4)

        out, stats = cb._condition_block_decode_output(
            q_grouped=q, prompt_prefix=prefix, k_suffix=ks, v_suffix=vs, suffix_len_dev=sfx_len, block_size=b,
            eps=float(eps), prompt_len=p, attention_dtype=torch.float32, workspace=ws)
        torch.cuda.synchronize()
        sel_gpu = _np(ws["selected_rows"]).astype(bool).reshape(hkv, g, 1, -1)
        n_diff = _check_selected(sel_gpu, ref_sel, mean, float(eps), f"decode eps={eps}")
        if n_diff == 0:
            np.testing.assert_allclose(_np(out), fx[f"out_{i}"], atol=TOL[dt], rtol=0, err_msg=f"eps={eps}")
            assert [int(stats[kk]) for kk in keys] == fx[f"stats_{i}"].tolist()
        exp = _expected(fx["q"], fx["k"], fx["v"], fx["k_suffix"], fx["v_suffix"], b, pre, sel_gpu, fx[f"z_{i}"])
        np.testing.assert_allclose(_np(out), exp, atol=TOL[dt], rtol=0, err_msg=f"oracle eps={eps}")


# ------------------------------------------------------------------ oracle cases

# name, seed, Hkv, G, D, block, P, S, dtype, mixed, k_bar dtype, mass_exp
CASES = [
    ("f32_b64_g4", 11, 2, 4, 64, 64, 1027, 33, "f32", False, "f32", False),
    ("bf16_b128_d128", 12, 2, 4, 128, 128, 9000, 17, "bf16", False, "f32", False),
    ("bf16_mixed_g8_2chunks", 13, 2, 8, 128, 64, 20000, 100, "bf16", True, "bf16", False),
    ("bf16_mixed_b32_mass", 14, 2, 2, 128, 32, 5000, 0, "bf16", True, "f32", True),
    ("bf16_b16_g1_many_chunks", 15, 2, 1, 64, 16, 70000, 300, "bf16", False, "f32", False),
    ("f32_b256_mass", 16, 1, 8, 128, 256, 3000, 5, "f32", False, "f32", True),
    ("bf16_c1_like", 17, 8, 4, 128, 64, 32768, 1, "bf16", True, "bf16", False),
]
IDS = [c[0] for c in CASES]


def _make(c, device):
    name, seed, hkv, g, d, b, p, s, dt, mixed, kbd, mass = c
    rng = np.random.default_rng(seed)
    rnd = bf16_round if dt == "bf16" else (lambda x: x.astype(np.float32))
    # a few heavy key directions make the condition spread over several decades
    k = rng.standard_normal((hkv, p, d), dtype=np.float32)
    k[:, rng.integers(0, p, size=max(1, p // 500))] *= 4.0
    k = rnd(k + 0.5 * rng.standard_normal((hkv, 1, d), dtype=np.float32))
    v = rnd(rng.standard_normal((hkv, p, d), dtype=np.float32))
    q = rnd(rng.standard_normal((hkv, g, 1, d), dtype=np.float32))
    ks = rnd(rng.standard_normal((hkv, s, d), dtype=np.float32))
    vs = rnd(rng.standard_normal((hkv, s, d), dtype=np.float32))
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    dev = {
        "k": torch.from_numpy(k).to(device, tdt), "v": torch.from_numpy(v).to(device, tdt),
        "q": torch.from_numpy(q).to(device, tdt),
        "ks": torch.from_numpy(ks).to(device, tdt), "vs": torch.from_numpy(vs).to(device, tdt),
    }
    return {"k": k, "v": v, "q": q, "ks": ks, "vs": vs}, dev


def _eps_list(mean):
    """eps values between distinct condition values: all, ~60%, ~15%, ~2% and none selected."""
    vals = np.unique(mean[mean > 0])
    out = [0.0]
    for frac in (0.4, 0.85, 0.98):
        i = min(int(frac * len(vals)), len(vals) - 2)
        out.append(float(0.5 * (vals[i] + vals[i + 1])))
    out.append(1e30)
    return out


@pytest.mark.parametrize("c", CASES, ids=IDS)
def test_condition_decode_vs_oracle(c, path, device):
    name, seed, hkv, g, d, b, p, s, dt, mixed, kbd, mass = c
    announce(f"condition {name} ({path}): hkv={hkv} g={g} d={d} block={b} P={p} S={s} {dt} mixed={mixed} "
             f"mass={mass}")
    host, dev = _make(c, device)
    kbt = torch.bfloat16 if kbd == "bf16" else torch.float32
    prefix = cb._build_prompt_blocks(dev["k"], dev["v"], b, mixed=mixed, k_bar_dtype=kbt)
    torch.cuda.synchronize()
    pre = _prefix_np(prefix)
    ref = Su.build_block_summaries(host["k"], host["v"], b, k_bar_dtype=kbd if mixed else "f32",
                                   v_bar_dtype="bf16" if mixed else "f32")
    assert np.array_equal(pre["block_valid_counts"], ref["block_valid_counts"])
    for key in ("k_max", "k_min"):
        assert np.array_equal(pre[key], ref[key]), key
    for key in ("k_bar", "v_bar"):
        bf = (key == "k_bar" and mixed and kbd == "bf16") or (key == "v_bar" and mixed)
        np.testing.assert_allclose(pre[key], ref[key], rtol=8e-3 if bf else 2e-6, atol=1e-6, err_msg=key)
    np.testing.assert_allclose(pre["v_norm_max"], ref["v_norm_max"], rtol=2e-6, atol=2e-6)

    q_rows = host["q"][:, :, 0].reshape(-1, d)
    st, mean, z = _oracle_stats(q_rows, pre, g, mass)
    q_s, s_t, delta_t, part_t, glob_t, nb, n_chunks = cb._run_condition_block_selection_stats(
        dev["q"], prefix, term1_mass_exp=mass)
    torch.cuda.synchronize()
    assert n_chunks == st["n_chunks"]
    np.testing.assert_allclose(_np(s_t), st["s"], rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(_np(delta_t), st["delta"], rtol=1e-4, atol=1e-4)
    gm = _np(glob_t)
    for i in (0, 2):
        np.testing.assert_allclose(gm[i], st["globals"][i], rtol=1e-4, atol=1e-4)
        np.testing.assert_allclose(gm[i + 1], st["globals"][i + 1], rtol=1e-3)
    pt = _np(part_t)
    fin = np.isfinite(st["partial"][0])
    assert np.array_equal(np.isfinite(pt[0]), fin)
    np.testing.assert_allclose(pt[0][fin], st["partial"][0][fin], rtol=1e-4, atol=1e-4)

    sfx_len = torch.full((1,), s, device=device, dtype=torch.int32)
    ws = {}
    for eps in _eps_list(mean):
        announce(f"condition {name}: eps={eps:.6g}")
        sel, z_t, _vb, _size, _ex = cb._select_prompt_blocks_triton(dev["q"], prefix, eps, term1_mass_exp=mass)
        torch.cuda.synchronize()
        ref_sel = np.repeat((mean > eps) & (pre["block_valid_counts"] > 0)[None], g, 0).reshape(hkv, g, 1, -1)
        _check_selected(_np(sel), ref_sel, mean, eps, f"select eps={eps}")
        fz = np.isfinite(z)
        np.testing.assert_allclose(_np(z_t).reshape(z.shape)[fz], z[fz], rtol=1e-5, atol=1e-4)

        out, stats = cb._condition_block_decode_output(
            q_grouped=dev["q"], prompt_prefix=prefix, k_suffix=dev["ks"], v_suffix=dev["vs"], suffix_len_dev=sfx_len,
            block_size=b, eps=eps, prompt_len=p, attention_dtype=torch.float32, workspace=ws, term1_mass_exp=mass)
        torch.cuda.synchronize()
        sel_gpu = _np(ws["selected_rows"]).astype(bool).reshape(hkv, g, 1, -1)
        _check_selected(sel_gpu, ref_sel, mean, eps, f"decode eps={eps}")
        if path == "four_launch":  # the same statistics kernel: the same bits
            assert np.array_equal(sel_gpu, _np(sel)), "fused and standalone selection disagree"
        else:  # the row statistics summed in another order: equal up to eps-boundary blocks
            _check_selected(sel_gpu, _np(sel), mean, eps, f"one launch vs standalone eps={eps}")
        exp = _expected(host["q"], host["k"], host["v"], host["ks"], host["vs"], b, pre, sel_gpu, z)
        np.testing.assert_allclose(_np(out), exp, atol=TOL[dt], rtol=0, err_msg=f"eps={eps}")
        ref_stats = S.condition_stats(sel_gpu, pre["block_valid_counts"], p, s)
        assert {k_: int(v_) for k_, v_ in stats.items()} == ref_stats


@pytest.mark.parametrize("name", ["f32_b64_g4", "bf16_mixed_b32_mass", "bf16_c1_like"])
def test_packed_bounds_equal_separate(name, path, device, monkeypatch):
    """The reference's packed bounds (CONDITION_BLOCK_TMA_BOUNDS=1: k_bounds [Hkv, nb,
    2D] with k_max / k_min as views, CBT/core.py:490-499) read in place by the
    statistics: statistics, selection and output equal the separate rows' bit for bit."""
    c = next(x for x in CASES if x[0] == name)
    _, seed, hkv, g, d, b, p, s, dt, mixed, kbd, mass = c
    announce(f"packed bounds {name} ({path})")
    host, dev = _make(c, device)
    kbt = torch.bfloat16 if kbd == "bf16" else torch.float32
    monkeypatch.delenv("CONDITION_BLOCK_TMA_BOUNDS", raising=False)
    sep = cb._build_prompt_blocks(dev["k"], dev["v"], b, mixed=mixed, k_bar_dtype=kbt)
    monkeypatch.setenv("CONDITION_BLOCK_TMA_BOUNDS", "1")
    packed = cb._build_prompt_blocks(dev["k"], dev["v"], b, mixed=mixed, k_bar_dtype=kbt)
    monkeypatch.delenv("CONDITION_BLOCK_TMA_BOUNDS")
    assert "k_bounds" in packed and not packed["k_max"].is_contiguous()
    assert packed["k_max"].data_ptr() == packed["k_bounds"].data_ptr()
    assert torch.equal(packed["k_max"], sep["k_max"]) and torch.equal(packed["k_min"], sep["k_min"])
    pre = _prefix_np(sep)
    _, mean, _ = _oracle_stats(host["q"][:, :, 0].reshape(-1, d), pre, g, mass)
    vals = np.unique(mean[mean > 0])
    eps = float(0.5 * (vals[int(0.85 * len(vals))] + vals[int(0.85 * len(vals)) + 1]))
    st = [cb._run_condition_block_selection_stats(dev["q"], pf, term1_mass_exp=mass) for pf in (sep, packed)]
    for a, b_ in zip(st[0][1:5], st[1][1:5]):
        assert torch.equal(a, b_), "statistics depend on the bounds layout"
    sfx_len = torch.full((1,), s, device=device, dtype=torch.int32)
    res = []
    for pf in (sep, packed):
        ws = {}
        out, _ = cb._condition_block_decode_output(
            q_grouped=dev["q"], prompt_prefix=pf, k_suffix=dev["ks"], v_suffix=dev["vs"], suffix_len_dev=sfx_len,
            block_size=b, eps=eps, prompt_len=p, attention_dtype=torch.float32, workspace=ws, term1_mass_exp=mass)
        torch.cuda.synchronize()
        res.append((out.clone(), ws["selected_rows"].clone()))
    assert torch.equal(res[0][1], res[1][1]) and torch.equal(res[0][0], res[1][0])


def test_condition_suffix_length_on_device(path, device):
    """The suffix length is read on the device: one buffer of capacity 64 serves
    lengths 0, 1 and 40 (the captured decode step advances it in place)."""
    c = ("sfx", 21, 2, 4, 128, 64, 3000, 64, "bf16", False, "f32", False)
    name, seed, hkv, g, d, b, p, cap, dt, *_ = c
    announce(f"condition suffix-on-device ({path})")
    host, dev = _make(c, device)
    prefix = cb._build_prompt_blocks(dev["k"], dev["v"], b)
    pre = _prefix_np(prefix)
    st, mean, z = _oracle_stats(host["q"][:, :, 0].reshape(-1, d), pre, g, False)
    eps = _eps_list(mean)[2]
    sfx_len = torch.zeros((1,), device=device, dtype=torch.int32)
    ws = {}
    for n in (0, 1, 40):
        sfx_len.fill_(n)
        out, _ = cb._condition_block_decode_output(
            q_grouped=dev["q"], prompt_prefix=prefix, k_suffix=dev["ks"], v_suffix=dev["vs"], suffix_len_dev=sfx_len,
            block_size=b, eps=eps, prompt_len=p, attention_dtype=torch.bfloat16, workspace=ws, collect_stats=False)
        torch.cuda.synchronize()
        sel = np.repeat((mean > eps) & (pre["block_valid_counts"] > 0)[None], g, 0).reshape(hkv, g, 1, -1)
        exp = _expected(host["q"], host["k"], host["v"], host["ks"][:, :n], host["vs"][:, :n], b, pre, sel, z)
        np.testing.assert_allclose(_np(out), exp, atol=TOL["bf16"], rtol=0, err_msg=f"suffix {n}")


@pytest.mark.parametrize("case", ["few_selected", "all_selected"])
def test_condition_decode_ignores_workspace_contents(case, device, monkeypatch):
    """Split-K slots of finalize items that get no units are written whole (their
    accumulators too, which the merge weighs by 0): a workspace full of NaN bytes
    gives the same output as a zeroed one."""
    from interattn_amd import _native as N

    monkeypatch.setenv("INTERATTN_CONDITION_ONE_LAUNCH", "0")  # the four-launch path's workspace
    # 16 blocks and one suffix tile: 17 finalize items and one route chunk, so the merge
    # reads every slot in one round trip (empty ones included)
    c = ("ws_nan", 23, 2, 4, 128, 64, 1000, 3, "bf16", False, "f32", False)
    name, seed, hkv, g, d, b, p, s, *_ = c
    announce(f"condition workspace contents: {case}")
    host, dev = _make(c, device)
    prefix = cb._build_prompt_blocks(dev["k"], dev["v"], b)
    pre = _prefix_np(prefix)
    _, mean, _ = _oracle_stats(host["q"][:, :, 0].reshape(-1, d), pre, g, False)
    eps = _eps_list(mean)[3] if case == "few_selected" else 0.0
    sfx_len = torch.full((1,), s, device=device, dtype=torch.int32)
    nb = int(pre["block_valid_counts"].shape[0])
    ws_bytes = int(N.lib().ia_condition_workspace_size(1, hkv, g, d, nb, s))
    outs = []
    for fill in (0, 0xFF):  # 0xFFFFFFFF is a NaN as float32
        ws = {"condition_scratch": torch.full((max(ws_bytes, 1),), fill, device=device, dtype=torch.uint8)}
        out, _ = cb._condition_block_decode_output(
            q_grouped=dev["q"], prompt_prefix=prefix, k_suffix=dev["ks"], v_suffix=dev["vs"], suffix_len_dev=sfx_len,
            block_size=b, eps=eps, prompt_len=p, attention_dtype=torch.float32, workspace=ws, collect_stats=False)
        torch.cuda.synchronize()
        assert ws["condition_scratch"].numel() == max(ws_bytes, 1), "the prefilled workspace was not used"
        outs.append(out.clone())
    assert torch.isfinite(outs[1]).all(), "NaN from an uninitialised workspace reached the output"
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_fixed_mask_hybrid_vs_oracle(dt, path, device):
    c = ("mask", 31, 4, 4, 128, 64, 10000, 7, dt, False, "f32", False)
    name, seed, hkv, g, d, b, p, s, *_ = c
    announce(f"fixed-mask {dt} ({path})")
    host, dev = _make(c, device)
    prefix = cb._build_prompt_blocks(dev["k"], dev["v"], b)
    pre = _prefix_np(prefix)
    nb = pre["block_valid_counts"].shape[0]
    rng = np.random.default_rng(7)
    for frac in (0.0, 0.3, 1.0):
        mask = rng.random((hkv, nb)) < frac
        out = cb.fixed_mask_hybrid_attention(q_grouped=dev["q"], prompt_prefix=prefix,
                                             selected=torch.from_numpy(mask).to(device), k_suffix=dev["ks"],
                                             v_suffix=dev["vs"], block_size=b, output_dtype=torch.float32)
        torch.cuda.synchronize()
        exp = A.fixed_mask_hybrid(host["q"], _padded(host["k"], b), _padded(host["v"], b),
                                  pre["block_valid_counts"], pre["k_bar"], pre["v_bar"], mask, host["ks"],
                                  host["vs"], emulate_bf16=(dt == "bf16"))
        np.testing.assert_allclose(_np(out), exp, atol=TOL[dt], rtol=0,
                                   err_msg=f"mask frac {frac}")


def test_fixed_mask_suffix_length_tensors_are_bounded(device):
    """One workspace over many suffix lengths keeps a few uncaptured suffix-length
    tensors; one read by a captured graph stays, and every call is still right."""
    c = ("sfxcache", 33, 2, 4, 128, 64, 3000, 9, "bf16", False, "f32", False)
    name, seed, hkv, g, d, b, p, s, *_ = c
    announce("fixed-mask: suffix-length tensors of one workspace")
    host, dev = _make(c, device)
    prefix = cb._build_prompt_blocks(dev["k"], dev["v"], b)
    nb = int(prefix["block_valid_counts"].numel())
    mask = torch.zeros((hkv, nb), dtype=torch.bool, device=device)
    mask[:, ::3] = True
    ws = {}

    def call(n):
        return cb.fixed_mask_hybrid_attention(q_grouped=dev["q"], prompt_prefix=prefix, selected=mask,
                                              k_suffix=dev["ks"][:, :n], v_suffix=dev["vs"][:, :n], block_size=b,
                                              output_dtype=torch.float32, workspace=ws)

    refs = {}
    for n in range(1, 10):
        refs[n] = call(n).clone()
        torch.cuda.synchronize()
        assert len(ws["suffix_len_recent"]) <= 4
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = call(2)
    assert 2 in ws["suffix_len_captured"] and 2 not in ws["suffix_len_recent"]
    for n in (5, 6, 7, 8, 9, 1, 3):  # churn the uncaptured set between replays
        assert torch.equal(call(n), refs[n])
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, refs[2])


def test_fixed_mask_clustered_selection(path, device):
    """Clustered selections (all selected blocks contiguous inside one 256-block
    route chunk, a different chunk per kv head) are split over the finalize's items
    by count like spread ones: parity with the oracle for clustered, spread and
    single-block masks over three route chunks."""
    c = ("cluster", 41, 4, 4, 128, 64, 40000, 3, "bf16", False, "f32", False)
    name, seed, hkv, g, d, b, p, s, *_ = c
    announce(f"fixed-mask clustered selections ({path})")
    host, dev = _make(c, device)
    prefix = cb._build_prompt_blocks(dev["k"], dev["v"], b)
    pre = _prefix_np(prefix)
    nb = pre["block_valid_counts"].shape[0]
    assert nb > 2 * 256
    masks = {}
    m = np.zeros((hkv, nb), bool)
    for h in range(hkv):
        start = 30 + 256 * (h % 3)
        m[h, start:start + 60] = True
    masks["clustered"] = m
    masks["spread"] = np.zeros((hkv, nb), bool)
    masks["spread"][:, ::10] = True
    masks["single"] = np.zeros((hkv, nb), bool)
    masks["single"][:, nb - 1] = True
    for label, mask in masks.items():
        out = cb.fixed_mask_hybrid_attention(q_grouped=dev["q"], prompt_prefix=prefix,
                                             selected=torch.from_numpy(mask).to(device), k_suffix=dev["ks"],
                                             v_suffix=dev["vs"], block_size=b, output_dtype=torch.float32)
        torch.cuda.synchronize()
        exp = A.fixed_mask_hybrid(host["q"], _padded(host["k"], b), _padded(host["v"], b),
                                  pre["block_valid_counts"], pre["k_bar"], pre["v_bar"], mask, host["ks"],
                                  host["vs"], emulate_bf16=True)
        np.testing.assert_allclose(_np(out), exp, atol=TOL["bf16"], rtol=0, err_msg=label)


def test_condition_contract_errors(device):
    announce("condition contract errors")
    k = torch.zeros((2, 100, 64), device=device, dtype=torch.bfloat16)
    prefix = cb._build_prompt_blocks(k, k, 32)
    q = torch.zeros((2, 4, 2, 64), device=device)
    with pytest.raises(ValueError):
        cb._select_prompt_blocks_triton(q, prefix, 1.0)
    q = torch.zeros((2, 3, 1, 64), device=device)
    with pytest.raises(ValueError):
        cb._select_prompt_blocks_triton(q, prefix, 1.0)
    q = torch.zeros((2, 4, 1, 64), device=device)
    with pytest.raises(ValueError):
        cb._condition_block_decode_output_fused_triton(
            q_grouped=q, prompt_prefix=prefix, k_suffix=None, v_suffix=None, suffix_len_dev=None, eps=1.0,
            page_size=64, store_selected=False, output_dtype=torch.float32)
    with pytest.raises(ValueError):
        cb._build_prompt_blocks(k, k, 24)


@pytest.mark.parametrize("bsz,hq,hkv,t_len,dt", [(1, 32, 8, 4133, "bf16"), (3, 8, 2, 1000, "bf16"),
                                                 (2, 4, 4, 77, "f32")])
def test_sdpa_full_attention_forward(bsz, hq, hkv, t_len, dt, device):
    announce(f"dense sdpa b={bsz} hq={hq} hkv={hkv} T={t_len} {dt}")
    rng = np.random.default_rng(t_len)
    rnd = bf16_round if dt == "bf16" else (lambda x: x.astype(np.float32))
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    d = 128
    q = rnd(rng.standard_normal((bsz, hq, 1, d), dtype=np.float32))
    k = rnd(rng.standard_normal((bsz, hkv, t_len, d), dtype=np.float32))
    v = rnd(rng.standard_normal((bsz, hkv, t_len, d), dtype=np.float32))
    tq, tk, tv = (torch.from_numpy(x).to(device, tdt) for x in (q, k, v))
    out, w = cb._sdpa_full_attention_forward(None, tq, tk, tv, None, d ** -0.5)
    torch.cuda.synchronize()
    assert w is None and tuple(out.shape) == (bsz, 1, hq, d)
    for bi in range(bsz):
        exp = A.dense_decode(q[bi, :, 0], k[bi], v[bi])
        np.testing.assert_allclose(_np(out[bi, 0]), exp, atol=TOL[dt], rtol=0)


def test_sdpa_full_attention_forward_masks(device):
    """A prefix mask (keys [0, n) allowed) runs the HIP dense decode over those keys;
    a left-padded mask (keys not a prefix) is detected and gives the masked attention
    as well (transformers' SDPA), never a silently wrong prefix."""
    announce("dense sdpa with prefix and left-padded masks")
    rng = np.random.default_rng(77)
    bsz, hq, hkv, t_len, d = 2, 8, 2, 300, 128
    q = rng.standard_normal((bsz, hq, 1, d), dtype=np.float32)
    k = rng.standard_normal((bsz, hkv, t_len, d), dtype=np.float32)
    v = rng.standard_normal((bsz, hkv, t_len, d), dtype=np.float32)
    tq, tk, tv = (torch.from_numpy(x).to(device) for x in (q, k, v))
    for name, allowed in (("prefix", np.arange(t_len)[None, :] < np.array([[250], [300]])),
                          ("left-pad", np.arange(t_len)[None, :] >= np.array([[40], [0]]))):
        mask = torch.zeros((bsz, 1, 1, t_len), dtype=torch.float32)
        mask[torch.from_numpy(~allowed)[:, None, None, :]] = torch.finfo(torch.float32).min
        out, _ = cb._sdpa_full_attention_forward(None, tq, tk, tv, mask.to(device), d ** -0.5)
        torch.cuda.synchronize()
        for bi in range(bsz):
            keep = allowed[bi]
            exp = A.dense_decode(q[bi, :, 0], k[bi][:, keep], v[bi][:, keep])
            np.testing.assert_allclose(_np(out[bi, 0]), exp, atol=1e-4, rtol=0, err_msg=name)
