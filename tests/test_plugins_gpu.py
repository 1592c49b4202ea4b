"""GPU checks of the plugin boundary: llama cache builder and the Qwen3.5 attention interface.

* ``sia_attention_forward`` against the float64 oracle (2e-3 before one output rounding).
* A small randomly initialised Qwen3.5 text model whose layers are all full
  attention (head_dim 256, 8 query / 2 KV heads): run on the GPU in bf16
  through the registered kernels, and as the reference on the CPU in fp32 with
  transformers' eager attention.  Prefill and three cached decode steps must
  agree to the reference's own gate, max-abs < 5e-2 relative to the logit
  scale (benchmarks/benchmark_kernel/bench_attention_compare.py:71-91).
"""

from __future__ import annotations

import copy
from importlib import import_module

import numpy as np
import pytest
import torch

from helpers import announce, assert_close
from oracle import attention as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def f64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _plugins():
    return import_module("simple-inference-autoresearch_amd.plugins")


class _Module:
    is_causal = True


@pytest.mark.parametrize("T,S,D", [(37, 37, 256), (1, 300, 256), (64, 100, 128)])
def test_attention_function_matches_oracle(gpu_pkg, T, S, D):
    announce(f"sia_attention_forward T={T} S={S} D={D}")
    g = torch.Generator(device=DEV).manual_seed(T + S)
    q = (torch.randn(2, 8, T, D, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
    k = (torch.randn(2, 2, S, D, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
    v = (torch.randn(2, 2, S, D, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
    out, w = _plugins().sia_attention_forward(_Module(), q, k, v, None, scaling=D ** -0.5)
    torch.cuda.synchronize()
    assert w is None and out.shape == (2, T, 8, D)
    ref = O.flash_attention(f64(q), f64(k), f64(v), True, D ** -0.5)     # (B, Hq, T, D)
    assert_close(out.transpose(1, 2), ref, 2e-3, f"T={T} S={S} D={D}")


def test_attention_function_rejects_padding(gpu_pkg):
    q = torch.zeros(1, 2, 4, 64, dtype=torch.bfloat16, device=DEV)
    k = torch.zeros(1, 2, 4, 64, dtype=torch.bfloat16, device=DEV)
    mask = torch.tensor([[0, 1, 1, 1]], device=DEV)
    with pytest.raises(NotImplementedError):
        _plugins().sia_attention_forward(_Module(), q, k, k, mask, scaling=0.125)
    # any mask the registered builder returns marks padding: rejected without reading it
    with pytest.raises(NotImplementedError):
        _plugins().sia_attention_forward(_Module(), q, k, k, torch.ones(1, 4, dtype=torch.bool, device=DEV),
                                         scaling=0.125)
    with pytest.raises(NotImplementedError):
        _plugins().sia_attention_forward(_Module(), q, k, k, None, dropout=0.1)


def test_attention_function_decode_step_in_hip_graph(gpu_pkg):
    """A Qwen3.5 decode step (Tq = 1, head_dim 256, 8/2 heads) through sia_attention_forward,
    captured once in a HIP graph and replayed with new query and cache contents: every
    replay equals the eager call bit for bit and the oracle within 2e-3 before one rounding."""
    announce("sia_attention_forward decode step under HIP-graph capture")
    B, Hq, Hkv, S, D = 2, 8, 2, 300, 256
    g = torch.Generator(device=DEV).manual_seed(77)
    q = (torch.randn(B, Hq, 1, D, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
    k = (torch.randn(B, Hkv, S, D, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
    v = (torch.randn(B, Hkv, S, D, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
    fwd = _plugins().sia_attention_forward
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fwd(_Module(), q, k, v, None, scaling=D ** -0.5)          # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out, _ = fwd(_Module(), q, k, v, None, scaling=D ** -0.5)
    for i in range(3):
        q.copy_((torch.randn(B, Hq, 1, D, generator=g, device=DEV) * 0.5).to(torch.bfloat16))
        v[:, :, 17 * i] = (torch.randn(B, Hkv, D, generator=g, device=DEV)).to(torch.bfloat16)
        graph.replay()
        torch.cuda.synchronize()
        eager, _ = fwd(_Module(), q, k, v, None, scaling=D ** -0.5)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs from the eager call"
        ref = O.flash_attention(f64(q), f64(k), f64(v), True, D ** -0.5)
        assert_close(out.transpose(1, 2), ref, 2e-3, f"replay {i}")


def test_qwen35_full_attention_model(gpu_pkg):
    announce("Qwen3.5 text model through the registered attention")
    from transformers import DynamicCache, Qwen3_5ForCausalLM, Qwen3_5TextConfig

    torch.manual_seed(0)
    cfg = Qwen3_5TextConfig(vocab_size=512, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                            num_attention_heads=8, num_key_value_heads=2, head_dim=256,
                            layer_types=["full_attention", "full_attention"], max_position_embeddings=4096)
    cfg._attn_implementation = "eager"
    ref_model = Qwen3_5ForCausalLM(cfg).eval()                   # fp32 reference on the CPU
    gpu_model = copy.deepcopy(ref_model)
    _plugins().use_for(gpu_model.config)
    for layer in gpu_model.model.layers:
        layer.self_attn.config._attn_implementation = gpu_model.config._attn_implementation
    gpu_model = gpu_model.to(DEV, torch.bfloat16)

    ids = torch.randint(0, 512, (2, 40), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        rc, gc = DynamicCache(config=cfg), DynamicCache(config=gpu_model.config)
        ref = ref_model(input_ids=ids, past_key_values=rc, use_cache=True).logits[:, -1:]
        got = gpu_model(input_ids=ids.to(DEV), past_key_values=gc, use_cache=True).logits[:, -1:]
        torch.cuda.synchronize()
        steps = [(ref, got)]
        for i in range(3):
            nxt = ref[:, -1].argmax(-1, keepdim=True)
            ref = ref_model(input_ids=nxt, past_key_values=rc, use_cache=True).logits
            got = gpu_model(input_ids=nxt.to(DEV), past_key_values=gc, use_cache=True).logits
            torch.cuda.synchronize()
            steps.append((ref, got))
    for i, (r, g_) in enumerate(steps):
        r, g_ = r.double(), g_.double().cpu()
        err = (r - g_).abs().max().item()
        scale = r.abs().max().item()
        assert err <= 5e-2 * max(1.0, scale), f"step {i}: max abs err {err:.3e} (logit scale {scale:.3f})"


def test_llama_cache_builders(gpu_pkg):
    announce("llama cache builders")

    class Cfg:
        num_hidden_layers, num_key_value_heads, head_dim = 3, 8, 128

    pl = _plugins()
    c = pl.llama_cache_builder(Cfg, max_batch=2, max_seq_len=512, dtype=torch.bfloat16, device=DEV)
    assert c.is_int8 and c.k_cache.shape == (3, 2, 8, 512, 128) and c.k_scale.dtype == torch.float16
    c = pl.llama_cache_builder(Cfg, max_batch=2, max_seq_len=128, dtype=torch.bfloat16, device=DEV)
    assert not c.is_int8 and c.k_cache.dtype == torch.bfloat16
    p = pl.llama_paged_cache_builder(Cfg, max_batch=2, max_seq_len=100, dtype=torch.bfloat16, device=DEV,
                                     kv_dtype=torch.int8)
    assert p.k_pool.shape == (3, 2 * 7, 8, 16, 128) and p.k_scale_pool.dtype == torch.float32
