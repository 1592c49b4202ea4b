"""GPU checks of the drop-in boundary: every tensor argument must live on the
call's GPU (a host tensor would hand a host address to the kernels), and the
error types follow the reference wrappers (ValueError for a bad argument).
Nothing here launches a kernel with a bad argument: each call raises before
any launch.
"""

from __future__ import annotations

import importlib

import pytest
import torch

from helpers import announce

pytestmark = pytest.mark.gpu

DEV = "cuda"
syn = importlib.import_module("simple-inference-autoresearch_amd.synthetic")


def test_decode_rejects_host_tensors(gpu_pkg):
    announce("decode with host tensors")
    case = syn.paged_case([40, 17], Hq=8, Hkv=2, D=128, page=16, seed=1, device=DEV, kv="int8")
    args = dict(q=case.q, k_pool=case.k_pool, v_pool=case.v_pool, k_scale_pool=case.k_scale,
                v_scale_pool=case.v_scale, block_table=case.block_table, kv_len=case.kv_len, page_size=16)
    for name in ("q", "k_pool", "v_pool", "k_scale_pool", "v_scale_pool", "block_table", "kv_len"):
        bad = dict(args)
        bad[name] = args[name].cpu()
        with pytest.raises(ValueError):
            gpu_pkg.paged_gqa_int8_flash_decode(**bad)
    # the good call still works afterwards
    out = gpu_pkg.paged_gqa_int8_flash_decode(**args)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()


def test_prefill_and_writes_reject_host_tensors(gpu_pkg):
    announce("prefill / kv_write / rope with host tensors")
    q = torch.randn(1, 8, 64, 128, device=DEV).to(torch.bfloat16)
    k = torch.randn(1, 2, 64, 128, device=DEV).to(torch.bfloat16)
    with pytest.raises(ValueError):
        gpu_pkg.attention_flash_triton(q, k.cpu(), k, causal=True)
    cache = gpu_pkg.KVCache(1, 2, 512, 2, 128, device=DEV)          # int8 pools (max_seq_len > 256)
    kn = torch.randn(2, 2, 1, 128, device=DEV).to(torch.bfloat16)
    with pytest.raises(ValueError):
        cache.write_decode(0, torch.tensor([3, 4], dtype=torch.int32), kn, kn)   # host positions
    cos = torch.ones(16, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        gpu_pkg.rope_triton(torch.randn(1, 4, 8, 128, device=DEV).to(torch.bfloat16),
                            torch.randn(1, 4, 2, 128, device=DEV).to(torch.bfloat16), cos, cos)
    with pytest.raises(ValueError):
        gpu_pkg.quantize_kv_int8(torch.randn(4, 128))
    with pytest.raises(ValueError):                                 # host rotary tables
        gpu_pkg.rope_attention_flash_triton(q, k, k, torch.ones(64, 128, dtype=torch.bfloat16),
                                            torch.ones(64, 128, dtype=torch.bfloat16), causal=True)
    with pytest.raises(ValueError):                                 # host start positions
        cg = torch.ones(64, 128, dtype=torch.bfloat16, device=DEV)
        gpu_pkg.rope_attention_flash_triton(q, k, k, cg, cg, causal=True,
                                            start_pos=torch.zeros(1, dtype=torch.int32))
