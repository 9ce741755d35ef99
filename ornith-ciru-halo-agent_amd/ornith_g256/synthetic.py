"""Seeded synthetic layer weights generated directly on the GPU.

Distributions follow the benchmark definition: 4-bit codes uniform in
[0, 15] (signed int4 uniform in [-8, 7] stored as code = q + 8), fp16 scales
uniform in [0.005, 0.02] with offset = fp16(-8 * scale) (exact), router
weights and the shared-expert gate ~ N(0, 0.02) in bf16.  Banks use the
reference N32 layouts (routed_storage_n32_consumer.cpp:1-2).
"""
from __future__ import annotations

import torch

E, H, I = 256, 2048, 512


def _codes(gen, shape, device):
    # full-range int32 words: every nibble uniform in [0, 15]
    return torch.randint(-2 ** 31, 2 ** 31, shape, generator=gen, dtype=torch.int64, device=device).to(torch.int32)


def _meta(gen, shape, device, lo=0.005, hi=0.02):
    scale = torch.empty(shape, dtype=torch.float32, device=device).uniform_(lo, hi, generator=gen).half()
    offset = (scale.float() * -8.0).half()
    return (scale.view(torch.int16).to(torch.int32) & 0xFFFF) | (offset.view(torch.int16).to(torch.int32) << 16)


def bank(gen, n, k, device, experts=None):
    """codes int32 [(E,) N/32, K/256, 32, 32] and meta int32 [(E,) N/32, K/256, 32]."""
    lead = (experts,) if experts else ()
    codes = _codes(gen, lead + (n // 32, k // 256, 32, 32), device)
    meta = _meta(gen, lead + (n // 32, k // 256, 32), device)
    return codes, meta


def moe_layer(seed, device, router_bias=None):
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    w13 = bank(gen, 2 * I, H, device, E)
    w2 = bank(gen, H, I, device, E)
    s13 = bank(gen, 2 * I, H, device)
    s2 = bank(gen, H, I, device)
    router = (torch.randn((E, H), generator=gen, device=device) * 0.02).to(torch.bfloat16)
    gate = (torch.randn((H,), generator=gen, device=device) * 0.02).to(torch.bfloat16)
    return dict(w13=w13, w2=w2, s13=s13, s2=s2, router=router, gate=gate, bias=router_bias)


def zipf_bias(s, seed, device):
    """Additive fp32 router-logit bias b_e = -s * ln(rank_e) with a seeded
    random rank permutation, so expert popularity follows a Zipf(s) profile."""
    gen = torch.Generator(device='cpu')
    gen.manual_seed(seed)
    rank = torch.randperm(E, generator=gen).to(torch.float32) + 1.0
    return (-s * torch.log(rank)).to(device)
