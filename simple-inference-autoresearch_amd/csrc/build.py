"""Build libsia_attention.so for gfx950 with hipcc (in-tree, parallel).

    python simple-inference-autoresearch_amd/csrc/build.py [--jobs N] [--verbose]

Every source in this folder (*.hip, *.cpp) is compiled as HIP for gfx950 into
``_build/`` next to the package and linked into
``simple-inference-autoresearch_amd/libsia_attention.so``.  The library is
always rebuilt from scratch: it is small and the objects are independent.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
ROOT = os.path.dirname(PKG)
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(ROOT, "_build")
LIB_NAME = "libsia_attention.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON_FLAGS = [
    "-x", "hip", f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-I", INCLUDE, "-I", HERE,
    # packed fp32 instructions stay off on this target (see the build notes)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable", "-Wno-unused-result",
]


def sources():
    return sorted(f for f in os.listdir(HERE) if f.endswith((".hip", ".cpp")))


# Extra flags per source: the decode kernels keep their MFMA accumulators in
# VGPRs (no AGPR round trips around the online-softmax rescale).
EXTRA_FLAGS = {
    "decode_f16.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "decode_bf16.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "decode_i8.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def compile_one(src: str, verbose: bool):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, *EXTRA_FLAGS.get(src, []), "-c", os.path.join(HERE, src), "-o", obj]
    t0 = time.time()
    r = subprocess.run(cmd, capture_output=True, text=True)
    dt = time.time() - t0
    out = (r.stdout + r.stderr).strip()
    # hipcc's host pass does not know the packed-fp32 feature: drop that note
    lines = [l for l in out.splitlines() if "packed-fp32-ops" not in l or "error" in l]
    return src, obj, r.returncode, "\n".join(lines), dt, cmd


def build(jobs: int | None = None, verbose: bool = False) -> str:
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    shutil.rmtree(BUILD, ignore_errors=True)
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, min(16, os.cpu_count() or 1)))
    objs = []
    failed = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for src, obj, rc, log, dt, cmd in ex.map(lambda s: compile_one(s, verbose), srcs):
            if verbose or rc:
                print(f"[build] {src}: rc={rc} {dt:.1f}s", flush=True)
                if log:
                    print(log, flush=True)
            if rc:
                failed.append(src)
            objs.append(obj)
    if failed:
        raise RuntimeError(f"hipcc failed for: {', '.join(failed)}")
    lib = os.path.join(PKG, LIB_NAME)
    tmp = lib + ".tmp"
    # -z defs: every symbol must resolve at link time (a kernel whose host-side
    # launch stub was not emitted fails here instead of at load time)
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-z,defs", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, lib)
    if verbose:
        print(f"[build] wrote {lib}", flush=True)
    return lib


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__)
    p.add_argument("--jobs", type=int, default=None)
    p.add_argument("--verbose", action="store_true")
    args = p.parse_args(argv)
    t0 = time.time()
    lib = build(args.jobs, args.verbose)
    print(f"built {lib} in {time.time() - t0:.1f}s")


if __name__ == "__main__":
    sys.exit(main())
