"""Loading of ``libsia_attention.so`` (the gfx950 C ABI in include/sia_attention.h).

Two bindings of the same library:

* ``ops()`` -- the thin torch extension ``_sia_ops.so`` (built from
  ``torch_ext/sia_ops.cpp``), which every kernel call of this package goes
  through: it checks devices, describes the tensors, takes outputs and
  workspace from torch's caching allocator and calls the C ABI on torch's
  current stream, in C++.
* ``load_library()`` -- a ctypes handle on the C ABI itself, for the ABI
  version check, status strings and symbol checks, and as the template of an
  FFI binding from another host language.

Both are loaded lazily, after ``import torch`` so that the library shares
torch's HIP runtime (both resolve ``libamdhip64.so.7``).  There is no
fallback: when either is missing every kernel call raises ``LibraryMissing``.
"""

from __future__ import annotations

import ctypes
import importlib.machinery
import importlib.util
import os
import threading

import torch

LIB_NAME = "libsia_attention.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
EXT_NAME = "_sia_ops"
EXT_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), EXT_NAME + ".so")

SIA_MAX_DIMS = 5
SIA_F16, SIA_BF16, SIA_F32, SIA_I8, SIA_I32, SIA_I64, SIA_U8 = range(7)

SIA_OK = 0
SIA_ERR_INVALID_ARGUMENT = -1
SIA_ERR_UNSUPPORTED = -2
SIA_ERR_WORKSPACE = -3
SIA_ERR_LAUNCH = -4
SIA_ERR_DEVICE = -5

_DTYPE_CODES = {
    torch.float16: SIA_F16,
    torch.bfloat16: SIA_BF16,
    torch.float32: SIA_F32,
    torch.int8: SIA_I8,
    torch.int32: SIA_I32,
    torch.int64: SIA_I64,
    torch.uint8: SIA_U8,
}


class LibraryMissing(RuntimeError):
    """The HIP library is not built or cannot be loaded (no CPU fallback exists)."""


class SiaError(RuntimeError):
    """A launch or device failure reported by the library."""


class SiaTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("ndim", ctypes.c_int32),
        ("shape", ctypes.c_int64 * SIA_MAX_DIMS),
        ("stride", ctypes.c_int64 * SIA_MAX_DIMS),
    ]


class DecodeOptions(ctypes.Structure):
    _fields_ = [
        ("tiles_per_split", ctypes.c_int32),
        ("reserved0", ctypes.c_int32),
        ("main_begin_event", ctypes.c_void_p),
        ("main_end_event", ctypes.c_void_p),
        ("reserved", ctypes.c_int64 * 4),
    ]


_P = ctypes.POINTER(SiaTensor)
_VP = ctypes.c_void_p
_SZ = ctypes.c_size_t
_F = ctypes.c_float
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64

# name -> argtypes (restype is int for every entry point)
_SIGNATURES = {
    "sia_abi_version": [],
    "sia_status_string": [ctypes.c_int],
    "sia_last_error_message": [],
    "sia_decode_workspace_size": [_I64, _I64, _I64, _I64, ctypes.POINTER(_SZ)],
    "sia_attention_flash_decode": [_P, _P, _P, _P, _F, _P, _VP, _SZ, ctypes.POINTER(DecodeOptions), _VP],
    "sia_attention_flash_decode_int8": [_P, _P, _P, _P, _P, _P, _F, _P, _VP, _SZ,
                                        ctypes.POINTER(DecodeOptions), _VP],
    "sia_gqa_int8_flash_decode": [_P, _P, _P, _P, _P, _P, _F, _P, _VP, _SZ,
                                  ctypes.POINTER(DecodeOptions), _VP],
    "sia_paged_attention_flash_decode": [_P, _P, _P, _P, _P, _I32, _F, _P, _VP, _SZ,
                                         ctypes.POINTER(DecodeOptions), _VP],
    "sia_paged_gqa_int8_flash_decode": [_P, _P, _P, _P, _P, _P, _P, _I32, _F, _P, _VP, _SZ,
                                        ctypes.POINTER(DecodeOptions), _VP],
    "sia_paged_gqa_int8_flash_decode_noalloc": [_P, _P, _P, _P, _P, _P, _P, _I32, _F, _P,
                                                ctypes.POINTER(DecodeOptions), _VP],
    "sia_attention_flash_fwd": [_P, _P, _P, _I32, _F, _P, _VP, _SZ, _VP],
    "sia_attention_flash_fwd_rope": [_P, _P, _P, _P, _P, _I32, _P, _I32, _I32, _F, _P, _VP, _SZ, _VP],
    "sia_prefill_workspace_size": [_I64, _I64, _I64, _I64, ctypes.POINTER(_SZ)],
    "sia_quantize_kv_int8": [_P, _P, _P, _VP],
    "sia_kv_write": [_P, _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _VP],
    "sia_rope_qk": [_P, _P, _P, _P, _I32, _P, _P, _VP],
    "sia_rope_kv_write": [_P, _P, _P, _P, _P, _I32, _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _VP],
}
_STRING_RESULT = {"sia_status_string", "sia_last_error_message"}

_lock = threading.Lock()
_lib = None
_ops = None
_gpu_checked = False


def library_path() -> str:
    return LIB_PATH


def exported_symbols():
    """Names of the C entry points this binding expects the library to export."""
    return sorted(_SIGNATURES)


def load_library():
    """Load (once) and return the ctypes handle; raise LibraryMissing if absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise LibraryMissing(
                f"{LIB_NAME} is not built (expected at {LIB_PATH}); run __graft_entry__.build() "
                "or python simple-inference-autoresearch_amd/csrc/build.py")
        try:
            h = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_LOCAL)
        except OSError as exc:  # pragma: no cover - depends on the host
            raise LibraryMissing(f"cannot load {LIB_PATH}: {exc}") from exc
        for name, argtypes in _SIGNATURES.items():
            fn = getattr(h, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_char_p if name in _STRING_RESULT else ctypes.c_int
        if h.sia_abi_version() != 1:
            raise LibraryMissing("libsia_attention.so ABI version mismatch; rebuild it")
        _lib = h
        return _lib


def require_library():
    """Raise unless the library is loaded and a GPU is visible to torch."""
    h = load_library()
    if not torch.cuda.is_available():
        raise LibraryMissing("no GPU is visible; the attention kernels run on MI355X (gfx950) only")
    return h


def ops():
    """The torch extension module (loaded once, after the library); raises LibraryMissing."""
    global _ops
    if _ops is not None:
        return _ops
    load_library()
    with _lock:
        if _ops is not None:
            return _ops
        if not os.path.exists(EXT_PATH):
            raise LibraryMissing(
                f"{EXT_NAME}.so is not built (expected at {EXT_PATH}); run __graft_entry__.build() "
                "or python simple-inference-autoresearch_amd/csrc/build.py")
        try:
            loader = importlib.machinery.ExtensionFileLoader(EXT_NAME, EXT_PATH)
            spec = importlib.util.spec_from_file_location(EXT_NAME, EXT_PATH, loader=loader)
            mod = importlib.util.module_from_spec(spec)
            loader.exec_module(mod)
        except ImportError as exc:  # pragma: no cover - depends on the host
            raise LibraryMissing(f"cannot load {EXT_PATH}: {exc}") from exc
        if mod.abi_version() != 1:
            raise LibraryMissing("_sia_ops.so was built against another ABI version; rebuild it")
        mod.set_error_class(SiaError)
        _ops = mod
        return _ops


def gpu_ops():
    """``ops()`` once a GPU has been seen (checked on the first call only)."""
    global _gpu_checked
    if not _gpu_checked:
        require_library()
        _gpu_checked = True
    return ops()


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dt]
    except KeyError:
        raise ValueError(f"dtype {dt} is not supported by the attention kernels") from None


def desc(t: torch.Tensor, device: torch.device | None = None) -> SiaTensor:
    """Describe a device tensor (pointer, dtype, shape, element strides) for a ctypes call.

    The tensor must be a GPU tensor, on ``device`` when given: a host tensor
    would hand a host address to the kernels.
    """
    if not t.is_cuda or (device is not None and t.device != device):
        raise ValueError(f"tensor on {t.device}: the attention kernels need every tensor on "
                         f"{device if device is not None else 'the GPU'}")
    if t.dim() > SIA_MAX_DIMS:
        raise ValueError(f"tensor with {t.dim()} dims; at most {SIA_MAX_DIMS} supported")
    d = SiaTensor()
    d.data = t.data_ptr()
    d.dtype = dtype_code(t.dtype)
    d.ndim = t.dim()
    for i, (n, s) in enumerate(zip(t.shape, t.stride())):
        d.shape[i] = n
        d.stride[i] = s
    return d


def check(rc: int) -> None:
    """Map a library status to the exception the reference's wrappers would raise."""
    if rc == SIA_OK:
        return
    h = load_library()
    msg = (h.sia_last_error_message() or b"").decode(errors="replace")
    kind = (h.sia_status_string(rc) or b"").decode(errors="replace")
    text = f"{kind}: {msg}" if msg else kind
    if rc == SIA_ERR_INVALID_ARGUMENT:
        raise ValueError(text)
    if rc == SIA_ERR_UNSUPPORTED:
        raise NotImplementedError(text)
    raise SiaError(text)


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
