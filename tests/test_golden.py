"""The oracle against golden vectors written by the reference's own CPU functions
(``tests/golden/make_fixtures.py``): ``_build_prompt_blocks``, ``_select_prompt_blocks_eager``,
``_condition_block_decode_output_dense`` and ``_condition_stats`` (CPU only)."""

import glob
import math
import os

import numpy as np
import pytest

from oracle import attention as A
from oracle import select as S
from oracle import summaries as Su

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURES = sorted(glob.glob(os.path.join(HERE, "cond_*.npz")))


def load(path):
    f = np.load(path, allow_pickle=False)
    return {k: f[k] for k in f.files}


def prefix_of(fx):
    return {k[len("prefix_"):]: fx[k] for k in fx if k.startswith("prefix_")}


def padded_blocks(x, b):
    hkv, p, d = x.shape
    nb = math.ceil(p / b)
    pad = np.zeros((hkv, nb * b - p, d), x.dtype)
    return np.concatenate([x, pad], 1).reshape(hkv, nb, b, d)


def condition_mean(q, pre, group):
    """Group-mean condition per (kv head, block), for near-threshold margins."""
    st = S.selection_stats_chunked(q[:, :, 0].reshape(-1, q.shape[-1]), pre, group)
    s, delta = st["s"], st["delta"]
    counts = np.asarray(pre["block_valid_counts"]).astype(np.int64)
    z = s + np.log(np.maximum(counts, 1))[None]
    zm, zl, cm, cl = st["globals"]
    b_c = np.repeat(np.where(counts > 0, pre["v_norm_max"], 0.0), group, axis=0)
    b_all = np.repeat(pre["v_norm_all"], group)[:, None]
    term1 = 2 * b_all * np.exp(z - cm[:, None]) * (np.cosh(delta) - 1) / cl[:, None]
    term2 = 2 * b_c * np.exp(z - zm[:, None]) * np.tanh(delta / 2) / zl[:, None]
    return (term1 + term2).reshape(q.shape[0], group, -1).mean(axis=1)


def test_fixtures_present():
    assert len(FIXTURES) >= 3


@pytest.mark.parametrize("path", FIXTURES, ids=[os.path.basename(p) for p in FIXTURES])
def test_summaries_match_reference(path):
    fx = load(path)
    hkv, g, d, b, p, s = fx["meta"]
    got = Su.build_block_summaries(fx["k"], fx["v"], int(b))
    ref = prefix_of(fx)
    assert np.array_equal(got["block_valid_counts"], ref["block_valid_counts"])
    for key in ("k_bar", "v_bar", "v_norm_max", "v_norm_all"):
        np.testing.assert_allclose(got[key], ref[key], rtol=2e-6, atol=2e-6, err_msg=key)
    for key in ("k_max", "k_min"):
        assert np.array_equal(got[key], ref[key]), key


@pytest.mark.parametrize("path", FIXTURES, ids=[os.path.basename(p) for p in FIXTURES])
def test_condition_selection_matches_reference(path):
    fx = load(path)
    hkv, g, d, b, p, s = (int(x) for x in fx["meta"])
    pre = prefix_of(fx)
    cm = condition_mean(fx["q"].astype(np.float64), pre, g)
    for i, eps in enumerate(fx["eps"]):
        sel, z = S.select_condition_eager(fx["q"], pre, float(eps))
        ref = fx[f"selected_{i}"]
        diff = sel != ref
        if diff.any():
            # only blocks whose condition sits on the threshold (float32 vs float64 rounding) may differ
            hh, _, _, jj = np.nonzero(diff)
            assert np.all(np.abs(cm[hh, jj] - eps) <= 1e-5 * max(abs(eps), 1.0)), (i, eps)
        np.testing.assert_allclose(z, fx[f"z_{i}"], rtol=1e-5, atol=1e-5)
        st = S.condition_stats(ref, pre["block_valid_counts"], p, s)
        keys = [str(k) for k in fx["stats_keys"]]
        assert [st[k] for k in keys] == fx[f"stats_{i}"].tolist()


@pytest.mark.parametrize("path", FIXTURES, ids=[os.path.basename(p) for p in FIXTURES])
def test_hybrid_dense_output_matches_reference(path):
    fx = load(path)
    hkv, g, d, b, p, s = (int(x) for x in fx["meta"])
    pre = prefix_of(fx)
    nb = pre["block_valid_counts"].shape[0]
    tok = np.arange(nb * b).reshape(nb, b)
    for i, eps in enumerate(fx["eps"]):
        out = A.hybrid_decode_dense(
            fx["q"], padded_blocks(fx["k"], b), padded_blocks(fx["v"], b), tok < p, tok, p + s - 1, p,
            fx["k_suffix"], fx["v_suffix"], fx[f"selected_{i}"], fx[f"z_{i}"], pre["v_bar"],
            pre["block_valid_counts"] > 0)
        np.testing.assert_allclose(out, fx[f"out_{i}"], rtol=1e-5, atol=2e-6)


@pytest.mark.parametrize("path", FIXTURES, ids=[os.path.basename(p) for p in FIXTURES])
def test_torch_condition_path_matches_reference(path):
    """The timed torch CPU restatement of the reference's own CPU path for its rule
    (oracle.torch_path.condition_layer_call: eager selection + dense hybrid attention)
    against the reference-written selections and outputs, and against the numpy
    oracle on the same inputs."""
    import torch

    from oracle import torch_path as T

    fx = load(path)
    hkv, g, d, b, p, s = (int(x) for x in fx["meta"])
    pre = prefix_of(fx)
    cm = condition_mean(fx["q"].astype(np.float64), pre, g)
    tpre = {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in pre.items()}
    kb, vb = padded_blocks(fx["k"], b), padded_blocks(fx["v"], b)
    nb = pre["block_valid_counts"].shape[0]
    tok = np.arange(nb * b).reshape(nb, b)
    for i, eps in enumerate(fx["eps"]):
        out, sel = T.condition_layer_call(torch.from_numpy(fx["q"]), tpre, torch.from_numpy(kb),
                                          torch.from_numpy(vb), torch.from_numpy(fx["k_suffix"]),
                                          torch.from_numpy(fx["v_suffix"]), float(eps))
        sel = sel.numpy()
        diff = sel != fx[f"selected_{i}"]
        if diff.any():
            hh, _, _, jj = np.nonzero(diff)
            assert np.all(np.abs(cm[hh, jj] - eps) <= 1e-5 * max(abs(eps), 1.0)), (i, eps)
        # the output on the reference's own selection
        _, z = T.condition_select(torch.from_numpy(fx["q"]), tpre, float(eps))
        ref_sel = torch.from_numpy(fx[f"selected_{i}"])
        got = T.condition_attend(torch.from_numpy(fx["q"]), torch.from_numpy(kb), torch.from_numpy(vb),
                                 tpre["block_valid_counts"], z, ref_sel, tpre["v_bar"],
                                 torch.from_numpy(fx["k_suffix"]), torch.from_numpy(fx["v_suffix"]))
        np.testing.assert_allclose(got.numpy(), fx[f"out_{i}"], rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(z.numpy(), fx[f"z_{i}"], rtol=1e-5, atol=1e-5)
        ref = A.hybrid_decode_dense(fx["q"], kb, vb, tok < p, tok, p + s - 1, p, fx["k_suffix"], fx["v_suffix"],
                                    sel, z.numpy(), pre["v_bar"], pre["block_valid_counts"] > 0)
        np.testing.assert_allclose(out.numpy(), ref, rtol=1e-5, atol=1e-5)
