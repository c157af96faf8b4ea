"""Seeded synthetic inputs for parity tests and smoke runs (test infrastructure only).

Inputs are drawn with numpy PCG64 (``np.random.default_rng(seed)``) in float32 and
then rounded to the working dtype, so any machine regenerates them bit-exactly.
The recipes follow the BASELINE configs: q/K/V ~ N(0,1); optional per-(kv head,
channel) key outlier scale exp(N(0,1)) (C2, "RoPE'd keys"); a paged pool whose page
order is one random permutation (C2-C4).
"""

import numpy as np

from .numerics import bf16_round, e4m3_encode, e4m3_decode, E4M3_MAX
from .paged import build_pool


def make_case(*, seed, batch, hq, hkv, d, seq_lens, page_size, dtype="bf16", k_outlier=False,
              n_pages=None, fp8=False):
    """Return a dict of numpy arrays: q [B,Hq,D]; per-sequence k/v [Hkv,L,D] (already
    rounded to ``dtype``); pool_k/pool_v [n_pages,Hkv,page,D]; block_table; seq_lens.
    With ``fp8`` the pool holds e4m3 codes (uint8) with per-(page, kv head) scales
    amax/448 and k/v hold the dequantised values."""
    rng = np.random.default_rng(seed)
    rnd = bf16_round if dtype == "bf16" else (lambda x: np.asarray(x, np.float32))
    q = rnd(rng.standard_normal((batch, hq, d), dtype=np.float32))
    outlier = None
    if k_outlier:
        outlier = np.exp(rng.standard_normal((hkv, 1, d))).astype(np.float32)
    ks, vs = [], []
    for L in seq_lens:
        k = rng.standard_normal((hkv, int(L), d), dtype=np.float32)
        if outlier is not None:
            k = k * outlier
        v = rng.standard_normal((hkv, int(L), d), dtype=np.float32)
        ks.append(rnd(k))
        vs.append(rnd(v))
    case = {"q": q, "seq_lens": np.asarray(seq_lens, dtype=np.int32), "page_size": page_size}
    perm_rng = np.random.default_rng(seed + 7919)
    pool_k, table = build_pool(ks, page_size, perm_rng, n_pages=n_pages)
    perm_rng = np.random.default_rng(seed + 7919)
    pool_v, table_v = build_pool(vs, page_size, perm_rng, n_pages=n_pages)
    assert np.array_equal(table, table_v)
    case["block_table"] = table
    if fp8:
        ksc = np.maximum(np.abs(pool_k).max(axis=(2, 3)), 1e-12) / E4M3_MAX   # [n_pages, Hkv]
        vsc = np.maximum(np.abs(pool_v).max(axis=(2, 3)), 1e-12) / E4M3_MAX
        kc = e4m3_encode(pool_k / ksc[:, :, None, None])
        vc = e4m3_encode(pool_v / vsc[:, :, None, None])
        case["k_scale"] = ksc.astype(np.float32)
        case["v_scale"] = vsc.astype(np.float32)
        pool_k = e4m3_decode(kc) * case["k_scale"][:, :, None, None]
        pool_v = e4m3_decode(vc) * case["v_scale"][:, :, None, None]
        case["pool_k_codes"], case["pool_v_codes"] = kc, vc
        # the dequantised sequences are the oracle's K/V
        from .paged import paged_gather
        ks = [paged_gather(pool_k, table[i], L, page_size) for i, L in enumerate(seq_lens)]
        vs = [paged_gather(pool_v, table[i], L, page_size) for i, L in enumerate(seq_lens)]
    case["pool_k"], case["pool_v"] = pool_k.astype(np.float32), pool_v.astype(np.float32)
    case["k"], case["v"] = ks, vs
    return case
