"""PyTorch CPU eager restatement of the reference's dequant + matmul semantics
for the quantized MoE layer and the dense G256 linear.

TEST INFRASTRUCTURE ONLY: the reported CPU baseline of bench.py (its
``cpu_baseline`` leg), timed on the host cores.  It is not bit-exact with
anything (fp32 BLAS order); the exact A8 oracle is ornith_oracle.py.  The
product path never imports it.

Semantics (the reference's bf16 prefill path, dense_g256_consumer.cpp:192-229,
applied to every projection, with the MoE structure of method.py:165-183 and
shared_kernel.py:33-62):
  * W = fp32(scale) * code + fp32(offset) per (row, 256-group), from packed
    4-bit codes (eight per uint32 word, low nibble first) and fp16
    (scale | offset << 16) words, dequantised on every call;
  * x' = H128(x) in fp32 (Sylvester Hadamard of each 128 block / sqrt(128));
  * y = x' @ W^T in fp32;
  * MoE: router logits fp32, softmax, top-8, renormalise; per expert
    silu(gate) * up then the down projection, weighted by the routing
    weight; the shared expert gated by sigmoid(x . w_gate); bf16 output.
Weights are kept row-major ([N, K/8] words, [N, K/256] meta): the storage
tile order is a layout choice, not part of the arithmetic.
"""
from __future__ import annotations

import math

import torch

E, TOP, H, I = 256, 8, 2048, 512
_SHIFTS = torch.arange(0, 32, 4, dtype=torch.int32)


def _hadamard128():
    h = torch.ones(1, 1)
    while h.shape[0] < 128:
        h = torch.cat([torch.cat([h, h], 1), torch.cat([h, -h], 1)], 0)
    return (h / math.sqrt(128)).float()


_H128 = _hadamard128()


def h128(x: torch.Tensor) -> torch.Tensor:
    """fp32 H128 of each 128 block of the last axis."""
    shape = x.shape
    return (x.reshape(-1, 128) @ _H128).reshape(shape)


def dequantize(words: torch.Tensor, meta: torch.Tensor) -> torch.Tensor:
    """words int32 [N, K/8], meta int32 [N, K/256] -> fp32 [N, K]."""
    n, kw = words.shape
    codes = ((words.unsqueeze(-1) >> _SHIFTS) & 15).reshape(n, kw * 8).float()
    scale = (meta & 0xFFFF).to(torch.int16).view(torch.float16).float()
    offset = ((meta >> 16) & 0xFFFF).to(torch.int16).view(torch.float16).float()
    g = codes.reshape(n, -1, 256)
    return (g * scale.unsqueeze(-1) + offset.unsqueeze(-1)).reshape(n, kw * 8)


def dense(x_bf16: torch.Tensor, words, meta) -> torch.Tensor:
    return (h128(x_bf16.float()) @ dequantize(words, meta).T).to(torch.bfloat16)


def random_bank(gen, experts, n, k):
    """Packed words [E?, N, K/8] and meta [E?, N, K/256] with the benchmark's
    distributions: codes uniform in [0, 15], scale ~ U(0.005, 0.02), offset = -8 scale."""
    lead = (experts,) if experts else ()
    words = torch.randint(-2 ** 31, 2 ** 31, lead + (n, k // 8), generator=gen, dtype=torch.int64).to(torch.int32)
    scale = (torch.rand(lead + (n, k // 256), generator=gen) * 0.015 + 0.005).half()
    offset = (scale.float() * -8.0).half()
    meta = (scale.view(torch.int16).to(torch.int32) & 0xFFFF) | (offset.view(torch.int16).to(torch.int32) << 16)
    return words, meta


def random_layer(seed):
    gen = torch.Generator().manual_seed(seed)
    return dict(w13=random_bank(gen, E, 2 * I, H), w2=random_bank(gen, E, H, I),
                s13=random_bank(gen, 0, 2 * I, H), s2=random_bank(gen, 0, H, I),
                router=(torch.randn((E, H), generator=gen) * 0.02).to(torch.bfloat16),
                gate=(torch.randn((H,), generator=gen) * 0.02).to(torch.bfloat16))


def route(x_bf16, router, bias=None):
    logits = x_bf16.float() @ router.float().T
    if bias is not None:
        logits = logits + bias
    p = torch.softmax(logits, dim=-1)
    w, ids = torch.topk(p, TOP, dim=-1)
    return w / w.sum(-1, keepdim=True), ids


def _expert(xt, w13, m13, w2, m2):
    gy = xt @ dequantize(w13, m13).T
    mid = torch.nn.functional.silu(gy[:, :I]) * gy[:, I:]
    return h128(mid) @ dequantize(w2, m2).T


def moe_layer(x_bf16, layer, bias=None):
    """One MoE layer: routed top-8 + shared expert, bf16 out; returns (out, distinct experts)."""
    w, ids = route(x_bf16, layer['router'], bias)
    xt = h128(x_bf16.float())
    out = torch.zeros(x_bf16.shape[0], H)
    (w13, m13), (w2, m2) = layer['w13'], layer['w2']
    experts = torch.unique(ids)
    for e in experts.tolist():
        tok, slot = (ids == e).nonzero(as_tuple=True)
        out.index_add_(0, tok, _expert(xt[tok], w13[e], m13[e], w2[e], m2[e]) * w[tok, slot].unsqueeze(-1))
    gate = torch.sigmoid(x_bf16.float() @ layer['gate'].float())
    out += _expert(xt, *layer['s13'], *layer['s2']) * gate.unsqueeze(-1)
    return out.to(torch.bfloat16), int(experts.numel())
