"""Seeded synthetic inputs for the five BASELINE configurations.

There are no checkpoints or datasets offline, so every benchmark and parity
case uses random inputs of the configured shapes.  Lengths, block tables and
(for configs 1/4) the tensors themselves come from CPU ``torch.Generator``s;
the large K/V pools of the decode configs are drawn on the target device from a
seeded device generator (fast, reproducible on the same device type).

Config  seed  definition
------  ----  --------------------------------------------------------------
1       0     q (1,32,1,64), k,v (1,8,512,64) fp32 N(0,1); scale 1/8; CPU
2       1     B16, 32/8 heads, D128, page 16, ctx ~ U[256,4096], fp16 N(0,1)
3       2     B64, 32/8, D128, page 16, ctx 8192; K/V N(0,1) -> int8 with
              per-token-per-head fp32 scales absmax/127; q bf16 N(0,1)
4       3     q (4,32,2048,128), k,v (4,8,2048,128) bf16 N(0,1)*0.5, causal
5       4     B256, 64/8, D128, page 16, ctx = clip(round(exp(N(ln 2048, 1))),
              128, 32768); int8 as config 3; split-K + reduction
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch


def quantize_per_vector(x: torch.Tensor, scale_dtype=torch.float32):
    """Symmetric per-vector int8 over the last dim (model/kv_cache.py:58-67 recipe)."""
    amax = x.abs().amax(dim=-1, keepdim=True).clamp_min(1e-8).float()
    scale = amax / 127.0
    xi = torch.round(x.float() / scale).clamp_(-127, 127).to(torch.int8)
    return xi, scale.squeeze(-1).to(scale_dtype)


@dataclass
class PagedCase:
    """A paged decode batch resident on one device."""

    q: torch.Tensor
    k_pool: torch.Tensor
    v_pool: torch.Tensor
    block_table: torch.Tensor
    kv_len: torch.Tensor
    page_size: int
    ctx: list
    k_scale: torch.Tensor | None = None
    v_scale: torch.Tensor | None = None
    meta: dict = field(default_factory=dict)

    @property
    def is_int8(self) -> bool:
        return self.k_pool.dtype == torch.int8


def paged_case(ctx, *, Hq: int, Hkv: int, D: int, page: int, seed: int, device, kv: str,
               q_dtype=torch.bfloat16, scale_dtype=torch.float32, per_seq_len: bool = True,
               chunk_pages: int = 4096) -> PagedCase:
    """Build a paged batch: pages of all sequences form one pool, randomly permuted.

    kv: "fp16" | "bf16" | "int8".  ``ctx`` lists the context length of each
    sequence.  Block table entries past a sequence's last page are 0, like the
    reference's zero-initialised tables (``model/paged_kv_cache.py:274-276``).
    """
    device = torch.device(device)
    B = len(ctx)
    cpu = torch.Generator().manual_seed(seed)
    n_pages = [int(math.ceil(c / page)) for c in ctx]
    P = max(1, sum(n_pages))
    perm = torch.randperm(P, generator=cpu)
    max_blocks = max(1, max(n_pages))
    bt = torch.zeros(B, max_blocks, dtype=torch.int32)
    off = 0
    for b, n in enumerate(n_pages):
        bt[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    dev_gen = torch.Generator(device=device).manual_seed(seed + 1000)
    shape = (P, Hkv, page, D)
    if kv == "int8":
        k_pool = torch.empty(shape, dtype=torch.int8, device=device)
        v_pool = torch.empty(shape, dtype=torch.int8, device=device)
        k_scale = torch.empty(shape[:3], dtype=scale_dtype, device=device)
        v_scale = torch.empty(shape[:3], dtype=scale_dtype, device=device)
        for pool, sc in ((k_pool, k_scale), (v_pool, v_scale)):
            for p0 in range(0, P, chunk_pages):
                p1 = min(P, p0 + chunk_pages)
                x = torch.randn((p1 - p0,) + shape[1:], generator=dev_gen, device=device, dtype=torch.float32)
                xi, s = quantize_per_vector(x, scale_dtype)
                pool[p0:p1] = xi
                sc[p0:p1] = s
    else:
        dt = {"fp16": torch.float16, "bf16": torch.bfloat16}[kv]
        k_pool = torch.randn(shape, generator=dev_gen, device=device, dtype=torch.float32).to(dt)
        v_pool = torch.randn(shape, generator=dev_gen, device=device, dtype=torch.float32).to(dt)
        k_scale = v_scale = None
    q = torch.randn((B, Hq, 1, D), generator=dev_gen, device=device, dtype=torch.float32).to(q_dtype)
    if per_seq_len:
        kv_len = torch.tensor(ctx, dtype=torch.int32, device=device)
    else:
        assert len(set(ctx)) == 1
        kv_len = torch.tensor([ctx[0]], dtype=torch.int32, device=device)
    return PagedCase(q=q, k_pool=k_pool, v_pool=v_pool, block_table=bt.to(device), kv_len=kv_len,
                     page_size=page, ctx=list(ctx), k_scale=k_scale, v_scale=v_scale)


# ------------------------------------------------------------------ configs


def cfg2_lengths(seed: int = 1, B: int = 16):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(256, 4097, (B,), generator=g).tolist()


def cfg5_lengths(seed: int = 4, B: int = 256, sigma: float = 1.0):
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(B, generator=g, dtype=torch.float64)
    ctx = torch.exp(math.log(2048.0) + sigma * z).round().clamp(128, 32768)
    return [int(c) for c in ctx.tolist()]


def cfg2(device) -> PagedCase:
    return paged_case(cfg2_lengths(), Hq=32, Hkv=8, D=128, page=16, seed=1, device=device, kv="fp16",
                      q_dtype=torch.float16)


def cfg3(device) -> PagedCase:
    return paged_case([8192] * 64, Hq=32, Hkv=8, D=128, page=16, seed=2, device=device, kv="int8",
                      q_dtype=torch.bfloat16, per_seq_len=False)


def cfg5(device) -> PagedCase:
    return paged_case(cfg5_lengths(), Hq=64, Hkv=8, D=128, page=16, seed=4, device=device, kv="int8",
                      q_dtype=torch.bfloat16)


def config_variant(name: str, device, i: int) -> PagedCase:
    """Input set i (>= 1) of decode config `name`: the config's lengths and shapes with
    other K/V data and another page permutation (seed + 1000 i), so that timing can
    rotate through sets whose total exceeds the MALL."""
    ctx = {"cfg2": cfg2_lengths(), "cfg3": [8192] * 64, "cfg5": cfg5_lengths()}[name]
    kw = {"cfg2": dict(Hq=32, Hkv=8, D=128, page=16, seed=1, kv="fp16", q_dtype=torch.float16),
          "cfg3": dict(Hq=32, Hkv=8, D=128, page=16, seed=2, kv="int8", q_dtype=torch.bfloat16, per_seq_len=False),
          "cfg5": dict(Hq=64, Hkv=8, D=128, page=16, seed=4, kv="int8", q_dtype=torch.bfloat16)}[name]
    kw["seed"] += 1000 * i
    return paged_case(ctx, device=device, **kw)


def cfg1():
    g = torch.Generator().manual_seed(0)
    q = torch.randn((1, 32, 1, 64), generator=g)
    k = torch.randn((1, 8, 512, 64), generator=g)
    v = torch.randn((1, 8, 512, 64), generator=g)
    return q, k, v


def cfg4(device, B=4, T=2048, Hq=32, Hkv=8, D=128):
    g = torch.Generator().manual_seed(3)
    q = (torch.randn((B, Hq, T, D), generator=g) * 0.5).to(torch.bfloat16)
    k = (torch.randn((B, Hkv, T, D), generator=g) * 0.5).to(torch.bfloat16)
    v = (torch.randn((B, Hkv, T, D), generator=g) * 0.5).to(torch.bfloat16)
    return q.to(device), k.to(device), v.to(device)


# ---------------------------------------------------------- algorithmic work


def decode_bytes(case: PagedCase) -> int:
    """Algorithmic HBM bytes of one paged decode call: every live K/V element,
    its scales, q and out once, one int32 table entry per live page and the
    kv_len entries.  Split-K partials and padding are overhead, not counted."""
    B, Hq, _, D = case.q.shape
    Hkv = case.k_pool.shape[1]
    tokens = sum(case.ctx)
    pages = sum(int(math.ceil(c / case.page_size)) for c in case.ctx)
    kv = tokens * Hkv * D * case.k_pool.element_size() * 2
    sc = tokens * Hkv * case.k_scale.element_size() * 2 if case.k_scale is not None else 0
    qo = 2 * B * Hq * D * case.q.element_size()
    lens = 4 * case.kv_len.numel() if case.kv_len.numel() > 1 else 0
    return kv + sc + qo + 4 * pages + lens


def prefill_flops(B: int, Hq: int, T: int, D: int) -> int:
    """Causal prefill FLOPs with the T^2/2 convention (benchmarks/benchmark_kernel/bench_attention_compare.py:51-54)."""
    return 4 * B * Hq * T * T * D // 2
