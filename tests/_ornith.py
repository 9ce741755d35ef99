"""Shared helpers for the tests: seeded synthetic inputs in the reference
storage layouts, the golden shared-math table, and GPU upload helpers."""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np

from oracle import ornith_oracle as O

GOLDEN = Path(__file__).resolve().parent / 'golden'
SHARED_TABLE = GOLDEN / 'shared_math_reference.safetensors'
# sha256 recorded by the reference (native/shared_math_reference.json:2)
SHARED_TABLE_SHA256 = '11552ec53b62b229d0ab42b4e865d0175724cd51c4eef01c05e66e930f27d2eb'


def read_safetensors(path):
    """Minimal safetensors reader (header JSON + raw little-endian data)."""
    raw = Path(path).read_bytes()
    n = int.from_bytes(raw[:8], 'little')
    header = json.loads(raw[8:8 + n])
    base = 8 + n
    out = {}
    dt = {'F32': np.float32, 'BF16': np.uint16, 'F16': np.float16, 'I32': np.int32, 'U32': np.uint32}
    for name, info in header.items():
        if name == '__metadata__':
            continue
        lo, hi = info['data_offsets']
        out[name] = np.frombuffer(raw[base + lo:base + hi], dtype=dt[info['dtype']]).reshape(info['shape'])
    return out


def load_shared_tables():
    data = SHARED_TABLE.read_bytes()
    assert hashlib.sha256(data).hexdigest() == SHARED_TABLE_SHA256
    t = read_safetensors(SHARED_TABLE)
    return t['silu_fp32'].copy(), t['sigmoid_bf16'].copy()


class Bank:
    """G256 4-bit bank: codes uint32 in tile layout, meta uint32 (scale|offset<<16)."""

    def __init__(self, rng, E, N, K, tile=32, lo=0.005, hi=0.02):
        shape = (E, N // tile, K // 256, 32, tile) if E else (N // tile, K // 256, 32, tile)
        self.E, self.N, self.K, self.tile = E, N, K, tile
        self.codes = rng.integers(0, 2 ** 32, size=shape, dtype=np.uint32)
        scale = rng.uniform(lo, hi, size=((E,) if E else ()) + (N, K // 256)).astype(np.float32)
        self.sbits = O.f32_to_f16_bits(scale)
        self.obits = O.f32_to_f16_bits(np.float32(-8) * O.f16_bits_to_f32(self.sbits))
        if E:
            self.meta = np.stack([O.pack_meta(self.sbits[e], self.obits[e], tile) for e in range(E)])
        else:
            self.meta = O.pack_meta(self.sbits, self.obits, tile)

    def expert(self, e=None):
        """(codes uint8 [N,K], scale bits, offset bits) of one expert."""
        if e is None:
            return O.from_tile_layout(self.codes), self.sbits, self.obits
        return O.from_tile_layout(self.codes[e]), self.sbits[e], self.obits[e]

    def unpack_all(self, experts):
        codes = {}
        for e in experts:
            codes[int(e)] = O.from_tile_layout(self.codes[int(e)])
        return codes


class LazyExperts:
    """Dict-like view that unpacks expert codes on first use (oracle input)."""

    def __init__(self, bank):
        self.bank = bank
        self.cache = {}

    def __getitem__(self, e):
        e = int(e)
        if e not in self.cache:
            self.cache[e] = O.from_tile_layout(self.bank.codes[e])
        return self.cache[e]


def bf16_normal(rng, shape, std=1.0):
    return O.f32_to_bf16((rng.standard_normal(shape) * std).astype(np.float32))


def random_routing(rng, T, E=256, top=8):
    """Distinct expert ids per token and positive weights summing to ~1."""
    ids = np.stack([rng.choice(E, size=top, replace=False) for _ in range(T)]).astype(np.int32)
    w = rng.uniform(0.01, 1.0, size=(T, top)).astype(np.float32)
    w = (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
    return w, ids


def moe_weights(seed, E=256):
    rng = np.random.default_rng(seed)
    w13 = Bank(rng, E, 1024, 2048)
    w2 = Bank(rng, E, 2048, 512)
    s13 = Bank(rng, 0, 1024, 2048)
    s2 = Bank(rng, 0, 2048, 512)
    router = bf16_normal(rng, (256, 2048), 0.02)
    gate = bf16_normal(rng, (1, 2048), 0.02)
    return dict(w13=w13, w2=w2, s13=s13, s2=s2, router=router, gate=gate)


def oracle_routed(x, w, ids, w13, w2, qmax=127):
    return O.routed_layer(x, w, ids, LazyExperts(w13), w13.sbits, w13.obits,
                          LazyExperts(w2), w2.sbits, w2.obits, qmax=qmax)


# ---- torch side ---------------------------------------------------------------
def to_dev(a, device):
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        return torch.from_numpy(a.view(np.int32)).to(device)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).to(device).view(torch.bfloat16)
    return torch.from_numpy(a).to(device)


def from_dev(t, dtype=None):
    import torch
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    a = t.numpy()
    return a.view(dtype) if dtype is not None else a
