"""Build libsia_attention.so for gfx950 with hipcc, and its torch extension (in-tree, parallel).

    python simple-inference-autoresearch_amd/csrc/build.py [--jobs N] [--verbose]

Every source in this folder (*.hip, *.cpp) is compiled as HIP for gfx950 into
``_build/`` next to the package and linked into
``simple-inference-autoresearch_amd/libsia_attention.so``.  The thin torch
extension ``torch_ext/sia_ops.cpp`` (host C++ only: it calls the C ABI) is
compiled with g++ against torch's headers at the same time and linked into
``simple-inference-autoresearch_amd/_sia_ops.so`` with the library found next
to it (rpath $ORIGIN).  Everything is always rebuilt from scratch.
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


EXT_SRC = os.path.join(PKG, "torch_ext", "sia_ops.cpp")
EXT_NAME = "_sia_ops"


def torch_ext_flags():
    """Include paths and defines of a torch C++ extension on this (ROCm) torch build."""
    import sysconfig

    import torch
    import torch.utils.cpp_extension as ce

    inc = [*ce.include_paths(), sysconfig.get_paths()["include"], "/opt/rocm/include", INCLUDE]
    defs = ["-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-DTORCH_EXTENSION_NAME={EXT_NAME}",
            "-DTORCH_API_INCLUDE_EXTENSION_H", f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}"]
    return [f for d in inc for f in ("-I", d)] + defs, ce.library_paths()


def compile_ext(verbose: bool):
    obj = os.path.join(BUILD, EXT_NAME + ".o")
    flags, _ = torch_ext_flags()
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function", *flags, "-c", EXT_SRC, "-o", obj]
    t0 = time.time()
    r = subprocess.run(cmd, capture_output=True, text=True)
    return os.path.basename(EXT_SRC), obj, r.returncode, (r.stdout + r.stderr).strip(), time.time() - t0, cmd


def link_ext(obj: str) -> str:
    _, libdirs = torch_ext_flags()
    out = os.path.join(PKG, EXT_NAME + ".so")
    tmp = out + ".tmp"
    cmd = ["g++", "-shared", "-fPIC", "-o", tmp, obj, *[f"-L{d}" for d in libdirs],
           "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python",
           f"-L{PKG}", "-lsia_attention", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError("extension link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, out)
    return out


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
    with cf.ThreadPoolExecutor(max_workers=jobs + 1) as ex:
        ext_job = ex.submit(compile_ext, verbose)   # the slowest unit: start it first
        for src, obj, rc, log, dt, cmd in ex.map(lambda s: compile_one(s, verbose), srcs):
            if verbose or rc:
                print(f"[build] {src}: rc={rc} {dt:.1f}s", flush=True)
                if log:
                    print(log, flush=True)
            if rc:
                failed.append(src)
            objs.append(obj)
        esrc, ext_obj, erc, elog, edt, _ = ext_job.result()
        if verbose or erc:
            print(f"[build] {esrc}: rc={erc} {edt:.1f}s", flush=True)
            if elog:
                print(elog, flush=True)
        if erc:
            failed.append(esrc)
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
    ext = link_ext(ext_obj)
    if verbose:
        print(f"[build] wrote {lib} and {ext}", flush=True)
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
