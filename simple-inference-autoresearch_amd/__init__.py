"""MI355X-native (gfx950) attention hot path for simple-inference-autoresearch.

Drop-in replacements for the reference engine's attention functions, backed by
hand-written HIP kernels in ``libsia_attention.so`` (C ABI:
``include/sia_attention.h``).  The package directory name contains hyphens, so
import it with ``importlib.import_module("simple-inference-autoresearch_amd")``.

Importing the package never needs a GPU; calling a kernel does, and raises
``LibraryMissing`` when the HIP library is not built (there is no CPU path).
"""

from __future__ import annotations

import torch  # noqa: F401  (load torch's HIP runtime before the library)

from ._lib import LibraryMissing, SiaError, exported_symbols, library_path, load_library, require_library
from .decode import (
    attention_flash_decode,
    attention_flash_decode_int8,
    decode_options,
    decode_workspace_size,
    gqa_int8_flash_decode,
    paged_attention_flash_decode,
    paged_gqa_int8_flash_decode,
)
from .prefill import attention_flash_triton, prefill_workspace_size, rope_attention_flash_triton
from .kv_cache import KVCache, kv_write, quantize_kv_int8, rope_kv_write
from .paged_kv_cache import PagedKVCache
from .rope import RopeFrequencies, apply_rope, rope_triton
from .attention import DecodeCtx, decode_step_attention, gqa_attention, rope_decode_step_attention
from . import plugins  # noqa: F401  (cache builders, transformers attention hook)

__all__ = [
    "DecodeCtx",
    "KVCache",
    "LibraryMissing",
    "PagedKVCache",
    "RopeFrequencies",
    "apply_rope",
    "rope_decode_step_attention",
    "rope_kv_write",
    "rope_triton",
    "decode_step_attention",
    "gqa_attention",
    "kv_write",
    "quantize_kv_int8",
    "attention_flash_triton",
    "rope_attention_flash_triton",
    "SiaError",
    "attention_flash_decode",
    "attention_flash_decode_int8",
    "decode_options",
    "decode_workspace_size",
    "exported_symbols",
    "gqa_int8_flash_decode",
    "library_path",
    "load_library",
    "paged_attention_flash_decode",
    "paged_gqa_int8_flash_decode",
    "prefill_workspace_size",
    "require_library",
]
