"""Generate golden vectors for the condition-block path from the reference's own CPU
functions.  Run in the build container only (the reference is not present on GPU boxes):

    PYTHONPATH=/root/reference python tests/golden/make_fixtures.py

Inputs are drawn with numpy PCG64 (np.random.default_rng(seed)) in float32 and
rounded to the case dtype; outputs come from the reference's
``_build_prompt_blocks`` (CBT/core.py:449-500), ``_select_prompt_blocks_eager``
(CBT/core.py:509-555), ``_condition_block_decode_output_dense`` (CBT/legacy.py:797-868)
and ``_condition_stats`` (CBT/core.py:1441-1456), with
CBT = llama/script/analysis/condition_block_gen/methods/condition_block_triton_impl.
Only data (inputs and expected outputs) is written, as .npz files beside this script.
"""

import os

import numpy as np
import torch

from llama.script.analysis.condition_block_gen.methods.condition_block_triton_impl import core, legacy

HERE = os.path.dirname(os.path.abspath(__file__))

# name, seed, Hkv, G, D, B, P, S, dtype, eps list (chosen to select all, ~75%, ~40%,
# ~10% and none of the blocks for these inputs)
CASES = [
    ("cond_f32_b64", 1234, 2, 4, 64, 64, 1027, 33, "f32", (0.0, 2.3, 2.6, 2.9, 1e6)),
    ("cond_bf16_b32", 1235, 2, 4, 128, 32, 515, 1, "bf16", (0.0, 2.8, 3.4, 3.8, 1e9)),
    ("cond_f32_b16_g8", 1236, 1, 8, 64, 16, 300, 7, "f32", (0.0, 1.7, 2.1, 3.3, 1e6)),
]


def rnd(x, dtype):
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    return t.to(torch.bfloat16) if dtype == "bf16" else t


def main():
    for name, seed, hkv, g, d, b, p, s, dtype, eps_list in CASES:
        rng = np.random.default_rng(seed)
        k = rnd(rng.standard_normal((hkv, p, d), dtype=np.float32), dtype)
        v = rnd(rng.standard_normal((hkv, p, d), dtype=np.float32), dtype)
        q = rnd(rng.standard_normal((hkv, g, 1, d), dtype=np.float32), dtype)
        ks = rnd(rng.standard_normal((hkv, s, d), dtype=np.float32), dtype)
        vs = rnd(rng.standard_normal((hkv, s, d), dtype=np.float32), dtype)
        prefix = core._build_prompt_blocks(k, v, b)
        out = {
            "k": k.float().numpy(), "v": v.float().numpy(), "q": q.float().numpy(),
            "k_suffix": ks.float().numpy(), "v_suffix": vs.float().numpy(),
            "meta": np.array([hkv, g, d, b, p, s], dtype=np.int64),
            "eps": np.array(eps_list, dtype=np.float64),
        }
        for key in ("k_bar", "v_bar", "k_max", "k_min", "v_norm_max", "v_norm_all", "block_valid_counts"):
            out["prefix_" + key] = prefix[key].float().numpy() if key != "block_valid_counts" else prefix[key].numpy()
        qf = q.float()
        pos = torch.tensor([p + s - 1], dtype=torch.long)
        for i, eps in enumerate(eps_list):
            sel, z, v_bar, size, exists = core._select_prompt_blocks_eager(qf, prefix, eps)
            dense = legacy._condition_block_decode_output_dense(
                q_grouped=qf, pos_tensor=pos, prompt_prefix=prefix, k_suffix=ks.float(), v_suffix=vs.float(),
                block_size=b, prompt_len=p, selected=sel, z_logits=z, v_bar=v_bar, cluster_exists=exists)
            stats = core._condition_stats(selected=sel, size=size, cluster_exists=exists, prompt_len=p,
                                          suffix_len=s)
            out[f"selected_{i}"] = sel.numpy()
            out[f"z_{i}"] = z.numpy()
            out[f"out_{i}"] = dense.numpy()
            out[f"stats_{i}"] = np.array([int(stats[kk]) for kk in sorted(stats)], dtype=np.int64)
            out["stats_keys"] = np.array(sorted(stats))
            print(f"{name} eps={eps}: selected {sel[:, 0, 0].float().mean().item():.3f} of blocks")
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **out)


if __name__ == "__main__":
    main()
