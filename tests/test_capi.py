"""CPU checks of the C ABI: the library loads and exports every declared symbol.

No kernel is launched here (there may be no GPU); only pure host functions
(ABI version, status strings, workspace sizing, argument validation) run.
"""

from __future__ import annotations

import ctypes
import glob
import os
import re
import subprocess
import sys

import pytest
import torch  # noqa: F401  (torch's HIP runtime must be loaded before the library)

from conftest import ROOT, load_pkg

HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def declared_symbols():
    names = set()
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"\b(sia_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


@pytest.fixture(scope="module")
def lib():
    pkg = load_pkg()
    path = pkg.library_path()
    if not os.path.exists(path):  # build on the CPU (hipcc cross-compiles gfx950)
        build = os.path.join(ROOT, "simple-inference-autoresearch_amd", "csrc", "build.py")
        subprocess.run([sys.executable, build], check=True)
    return pkg.load_library()


def test_header_declares_entry_points():
    names = declared_symbols()
    for must in ("sia_attention_flash_decode", "sia_attention_flash_decode_int8",
                 "sia_paged_attention_flash_decode", "sia_gqa_int8_flash_decode",
                 "sia_paged_gqa_int8_flash_decode", "sia_decode_workspace_size"):
        assert must in names


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_header():
    pkg = load_pkg()
    assert sorted(pkg.exported_symbols()) == declared_symbols()


def test_host_only_functions(lib):
    assert lib.sia_abi_version() == 1
    assert lib.sia_status_string(0) == b"ok"
    assert lib.sia_status_string(-1) == b"invalid argument"
    n = ctypes.c_size_t(0)
    assert lib.sia_decode_workspace_size(64, 32, 8, 128, ctypes.byref(n)) == 0
    assert n.value > 64 * 8 * 4 * 130 * 4  # at least one fp32 partial per (sequence, kv head)
    assert lib.sia_decode_workspace_size(2, 7, 2, 128, ctypes.byref(n)) == -1   # 7 % 2 != 0
    assert b"multiple" in lib.sia_last_error_message()


def test_null_arguments_are_rejected_without_launching(lib):
    rc = lib.sia_attention_flash_decode(None, None, None, None, ctypes.c_float(0.1), None, None, 0, None, None)
    assert rc == -1


def test_prefill_f16_v_rows_checked_on_the_host(lib):
    """float16 V at head_dim 128 is read in place, so its token stride is
    checked like K's, on the host, before any device query: rows closer than
    one row's bytes are refused (SIA_ERR_UNSUPPORTED).  The same descriptors in
    bfloat16 pass that check (V is repacked) and stop at the missing workspace."""
    from importlib import import_module
    lm = import_module("simple-inference-autoresearch_amd._lib")

    def d(dtype, shape, stride, addr):
        t = lm.SiaTensor()
        t.data, t.dtype, t.ndim = addr, dtype, 4
        for i in range(4):
            t.shape[i], t.stride[i] = shape[i], stride[i]
        return t

    for dtype, want in ((0, -2), (1, -3)):   # SIA_F16: unsupported; SIA_BF16: workspace
        q = d(dtype, (1, 8, 4, 128), (4096, 512, 128, 1), 0x10000)
        k = d(dtype, (1, 2, 4, 128), (1024, 512, 128, 1), 0x20000)
        v = d(dtype, (1, 2, 4, 128), (1024, 512, 64, 1), 0x30000)    # rows 128 bytes apart, 256 long
        o = d(dtype, (1, 8, 4, 128), (4096, 512, 128, 1), 0x40000)
        rc = lib.sia_attention_flash_fwd(ctypes.byref(q), ctypes.byref(k), ctypes.byref(v), 1, ctypes.c_float(0.1),
                                         ctypes.byref(o), None, 0, None)
        assert rc == want, (dtype, rc, lib.sia_last_error_message())
        if dtype == 0:
            assert b"v token stride" in lib.sia_last_error_message()


def test_no_cpu_fallback(monkeypatch):
    """Without the HIP library (or without a GPU) the product path raises."""
    pkg = load_pkg()
    from importlib import import_module
    lib_mod = import_module("simple-inference-autoresearch_amd._lib")
    monkeypatch.setattr(lib_mod, "LIB_PATH", "/nonexistent/libsia_attention.so")
    monkeypatch.setattr(lib_mod, "_lib", None)
    monkeypatch.setattr(lib_mod, "_ops", None)
    monkeypatch.setattr(lib_mod, "_gpu_checked", False)
    q = torch.zeros(1, 8, 1, 128, dtype=torch.bfloat16)
    k = torch.zeros(1, 2, 16, 128, dtype=torch.bfloat16)
    with pytest.raises(pkg.LibraryMissing):
        pkg.attention_flash_decode(q, k, k, torch.tensor([16], dtype=torch.int32))


def test_torch_extension_loads_and_binds_the_library(lib):
    """The thin torch extension loads on the CPU, links the same C ABI and exposes one op per path."""
    from importlib import import_module
    lib_mod = import_module("simple-inference-autoresearch_amd._lib")
    ops = lib_mod.ops()
    assert ops.abi_version() == lib.sia_abi_version() == 1
    for name in ("decode", "prefill", "prefill_rope", "quantize_kv_int8", "kv_write", "rope_kv_write", "rope_qk",
                 "decode_workspace_size", "prefill_workspace_size"):
        assert callable(getattr(ops, name)), name
    n = ctypes.c_size_t(0)
    assert lib.sia_decode_workspace_size(64, 32, 8, 128, ctypes.byref(n)) == 0
    assert ops.decode_workspace_size(64, 32, 8, 128) == n.value
    with pytest.raises(ValueError, match="multiple"):
        ops.decode_workspace_size(2, 7, 2, 128)
    with pytest.raises(NotImplementedError):
        ops.prefill_workspace_size(1, 8, 100, 48)


def test_torch_extension_rejects_host_tensors(lib):
    """Host tensors never reach the kernels: the extension raises before any launch."""
    from importlib import import_module
    ops = import_module("simple-inference-autoresearch_amd._lib").ops()
    q = torch.zeros(1, 8, 1, 128, dtype=torch.bfloat16)
    k = torch.zeros(1, 2, 16, 128, dtype=torch.bfloat16)
    kl = torch.tensor([16], dtype=torch.int32)
    with pytest.raises(ValueError, match="GPU"):
        ops.decode(0, q, k, k, None, None, None, kl, 0, 0.1, 0, 0, 0)
    with pytest.raises(ValueError, match="GPU"):
        ops.prefill(q, k, k, True, 0.1, False)
    with pytest.raises(ValueError, match="GPU"):
        ops.kv_write(k, k, k, k, None, None, None, None, 0, 0)
