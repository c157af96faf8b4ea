"""Shared helpers for the GPU parity tests: upload oracle cases, compare indices with
the near-tie rule, and print the case name before each GPU step."""

import sys

import numpy as np
import torch

from oracle import select as S
from oracle import summaries as Su


def announce(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def to_dev(case, device, dtype=torch.bfloat16, fp8=False):
    """Upload a ``make_case`` dict.  Returns a dict of device tensors."""
    out = {
        "q": torch.from_numpy(case["q"]).to(device=device, dtype=dtype if dtype != "fp8" else torch.bfloat16),
        "block_table": torch.from_numpy(case["block_table"]).to(device),
        "seq_lens": torch.from_numpy(case["seq_lens"]).to(device),
    }
    if fp8:
        out["q"] = torch.from_numpy(case["q"]).to(device=device, dtype=torch.bfloat16)
        out["pool_k"] = torch.from_numpy(case["pool_k_codes"]).to(device).view(torch.float8_e4m3fn)
        out["pool_v"] = torch.from_numpy(case["pool_v_codes"]).to(device).view(torch.float8_e4m3fn)
        out["scales"] = (torch.from_numpy(case["k_scale"]).to(device), torch.from_numpy(case["v_scale"]).to(device))
    else:
        out["pool_k"] = torch.from_numpy(case["pool_k"]).to(device=device, dtype=dtype)
        out["pool_v"] = torch.from_numpy(case["pool_v"]).to(device=device, dtype=dtype)
        out["scales"] = None
    return out


def oracle_summaries(case, block, k_bar_dtype="bf16"):
    """Per-sequence oracle summaries, stacked to [B, Hkv, nb_max, D] / [B, nb_max]."""
    sums = [Su.build_block_summaries(k, v, block, k_bar_dtype=k_bar_dtype) for k, v in zip(case["k"], case["v"])]
    nb_max = max(s["block_valid_counts"].shape[0] for s in sums)
    hkv, d = case["k"][0].shape[0], case["k"][0].shape[2]
    kb = np.zeros((len(sums), hkv, nb_max, d), np.float32)
    counts = np.zeros((len(sums), nb_max), np.int64)
    for i, s in enumerate(sums):
        n = s["block_valid_counts"].shape[0]
        kb[i, :, :n] = s["k_bar"]
        counts[i, :n] = s["block_valid_counts"]
    return kb, counts, sums


def check_indices(gpu_idx, gpu_n, scores, nb, k, ff, fl, in_k, rel=1e-3):
    """GPU selection == oracle selection except for blocks whose scores are within
    ``rel`` (relative) of the k-th admitted score (the north-star near-tie rule)."""
    ref = S.select_topk(scores, nb, k, ff, fl, in_k)
    got = np.asarray(gpu_idx[:gpu_n])
    assert len(got) == len(ref), (len(got), len(ref))
    assert np.all(np.diff(got) > 0), "indices must be strictly ascending"
    diff = set(got.tolist()) ^ set(ref.tolist())
    if diff:
        thr = S.topk_threshold(scores, nb, k, ff, fl, in_k)
        assert thr is not None, f"mismatch {sorted(diff)} without a rank limit"
        tol = rel * max(abs(thr), 1e-6)
        for j in diff:
            assert abs(scores[j] - thr) <= tol, f"block {j}: score {scores[j]} vs threshold {thr}"
    return len(diff)
