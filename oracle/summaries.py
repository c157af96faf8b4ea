"""Per-block summaries (test infrastructure only).

Restates ``_pad_blocks`` / ``_build_prompt_blocks`` (CBT/core.py:383-395,
:449-500): for each block of ``block`` tokens, over the valid tokens only,

* ``counts``      = number of valid tokens (CBT/core.py:460),
* ``k_bar/v_bar`` = float32 sum / max(count, 1)   (CBT/core.py:461-466, :481-482),
* ``k_max/k_min`` = elementwise extrema, masked with -inf/+inf (CBT/core.py:467-468, :477-478),
* ``v_norm_max``  = max over tokens of ||v_t||_2, -inf for an empty block (CBT/core.py:469-470, :485),
* ``v_norm_all``  = max over blocks of v_norm_max (CBT/core.py:486).

Sums are taken in float64 here; the reference sums in float32 (``dtype=torch.float32``),
so the two agree to float32 rounding, which every consumer's tolerance covers.
``k_bar_dtype``/``v_bar_dtype`` "bf16" apply the storage rounding of the reference's
mixed-summary layout (CBT/core.py:411-446).
"""

import math

import numpy as np

from .numerics import bf16_round


def build_block_summaries(k, v, block, k_bar_dtype="f32", v_bar_dtype="f32"):
    """``k, v``: ``[Hkv, L, D]`` (float values).  Returns the reference's prefix dict
    (``k_bar, v_bar, k_max, k_min`` as ``[Hkv, nb, D]``, ``v_norm_max [Hkv, nb]``,
    ``v_norm_all [Hkv]``, ``block_valid_counts [nb]``) as float32/int64 arrays."""
    hkv, seq_len, d = k.shape
    nb = int(math.ceil(seq_len / block))
    pad = nb * block - seq_len
    kp = np.concatenate([k, np.zeros((hkv, pad, d), k.dtype)], axis=1).astype(np.float64)
    vp = np.concatenate([v, np.zeros((hkv, pad, d), v.dtype)], axis=1).astype(np.float64)
    kb = kp.reshape(hkv, nb, block, d)
    vb = vp.reshape(hkv, nb, block, d)
    token_idx = np.arange(nb * block).reshape(nb, block)
    valid = token_idx < seq_len
    counts = valid.sum(axis=1).astype(np.int64)
    denom = np.maximum(counts, 1).astype(np.float64)
    vm = valid[None, :, :, None]
    k_bar = (kb * vm).sum(axis=2) / denom[None, :, None]
    v_bar = (vb * vm).sum(axis=2) / denom[None, :, None]
    k_max = np.where(vm, kb, -np.inf).max(axis=2)
    k_min = np.where(vm, kb, np.inf).min(axis=2)
    v_norm = np.sqrt((vb * vb).sum(axis=-1))
    v_norm = np.where(valid[None], v_norm, -np.inf)
    v_norm_max = v_norm.max(axis=2)
    k_bar = k_bar.astype(np.float32)
    v_bar = v_bar.astype(np.float32)
    if k_bar_dtype == "bf16":
        k_bar = bf16_round(k_bar)
    if v_bar_dtype == "bf16":
        v_bar = bf16_round(v_bar)
    return {
        "k_bar": k_bar,
        "v_bar": v_bar,
        "k_max": k_max.astype(np.float32),
        "k_min": k_min.astype(np.float32),
        "v_norm_max": v_norm_max.astype(np.float32),
        "v_norm_all": (v_norm_max.max(axis=-1) if nb else np.full(hkv, -np.inf)).astype(np.float32),
        "block_valid_counts": counts,
    }
