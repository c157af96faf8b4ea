"""Register budget of the built kernels, from the compiler's kernel-resource-usage
remarks that ``interattn_amd.build`` keeps in ``_build/kernel_resources.json``: no
instance spills to scratch memory (per-lane private memory, which would put every
spilled value through the cache hierarchy), and every paged-finalize instance runs
two waves per SIMD, which its one 512-thread workgroup per CU needs."""
import json
import os

import pytest

PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "_build", "kernel_resources.json")


def _resources():
    if not os.path.exists(PATH):
        pytest.skip("the library has not been built in this tree")
    with open(PATH) as f:
        return json.load(f)


def test_no_kernel_uses_scratch():
    res = _resources()
    assert len(res) > 200, "the report should cover every kernel instance"
    spilled = {name: r["scratch_bytes"] for name, r in res.items() if r.get("scratch_bytes", 0) > 0}
    assert not spilled, spilled


def test_finalize_instances_run_two_waves_per_simd():
    res = _resources()
    fin = {name: r for name, r in res.items() if "ia_condition_block_paged_finalize" in name}
    assert len(fin) >= 100
    low = {name: (r.get("vgprs"), r.get("occupancy")) for name, r in fin.items() if r.get("occupancy", 0) < 2}
    assert not low, low
