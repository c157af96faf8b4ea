"""Build the gfx950 HIP library ``libinterattn_amd.so`` in-tree.

Each ``csrc/*.hip`` file is compiled to an object in parallel under
``_build/`` and the objects are linked into ``interattn_amd/libinterattn_amd.so``.
The library exports only the C ABI declared in ``include/interattn_amd.h``.
"""

import concurrent.futures
import json
import os
import shutil
import subprocess
import sys
import time

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(ROOT, "_build")
LIB = os.path.join(PKG, "libinterattn_amd.so")
ARCH = os.environ.get("IA_OFFLOAD_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    # keep packed fp32 (v_pk_*_f32) out of the generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
    # per-kernel register, scratch and occupancy report, kept in _build/kernel_resources.json
    "-Rpass-analysis=kernel-resource-usage",
]
RESOURCES = os.path.join(BUILD, "kernel_resources.json")


def _resources(stderr, src):
    """Per-kernel figures from the kernel-resource-usage remarks of one compile."""
    out, name = {}, None
    for line in stderr.splitlines():
        if "remark:" not in line:
            continue
        body = line.split("remark:", 1)[1].strip()
        body = body.split(" [-Rpass-analysis")[0]
        if body.startswith("Function Name:"):
            name = body.split(":", 1)[1].strip()
            out.setdefault(name, {"source": os.path.basename(src)})
        elif name is not None and ":" in body:
            key, val = body.rsplit(":", 1)
            key = {"VGPRs": "vgprs", "AGPRs": "agprs", "ScratchSize [bytes/lane]": "scratch_bytes",
                   "Occupancy [waves/SIMD]": "occupancy", "LDS Size [bytes/block]": "lds_bytes"}.get(key.strip())
            if key and val.strip().isdigit():
                out[name][key] = int(val.strip())
    return out


def _compile(src):
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    t0 = time.time()
    res = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l and "remark:" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    return obj, time.time() - t0, _resources(res.stderr, src)


def build(verbose=True):
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    jobs = min(len(srcs), max(1, (os.cpu_count() or 2)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        results = list(ex.map(_compile, srcs))
    resources = {}
    for obj, dt, res in results:
        resources.update(res)
        if verbose:
            print(f"[build] {os.path.basename(obj)} {dt:.1f}s", flush=True)
    with open(RESOURCES, "w") as f:
        json.dump(resources, f, indent=1, sort_keys=True)
    for name, r in sorted(resources.items()):
        if r.get("scratch_bytes", 0) > 0:
            print(f"[build] warning: {name} uses {r['scratch_bytes']} bytes of scratch per lane", flush=True)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *[o for o, _, _ in results]]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("link failed:\n" + res.stderr)
    os.replace(tmp, LIB)
    if verbose:
        print(f"[build] wrote {LIB}", flush=True)
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
