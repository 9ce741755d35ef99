"""Checkpoint admission and the one-time N16 -> N32 repack of G256 banks.

Admission restates the reference's strict packed-bank loader
(plugin-site/ornith_g256/loader.py:17-54, method.py:12-32): every field is
loaded exactly once, with exactly the registered shape and dtype, from a
materialised tensor; metadata arrives on the CPU as uint32 words whose fp16
(scale, offset) halves must be finite with scale >= 2^-14.  Nothing is
padded, sliced or converted.

The repack (method.py:124-158, dense_n32.py:32-33) runs once per bank on the
GPU through the library's ``ornith_repack_n16_to_n32`` kernel.
"""
from __future__ import annotations

import torch

from . import native

MIN_SCALE = 2.0 ** -14
ROUTED_FIELDS = ('w13_tilebank_codes', 'w13_tilebank_metadata', 'w2_tilebank_codes', 'w2_tilebank_metadata')
ROUTED_PREFIX = 'routed_experts.'


class AdmissionError(ValueError):
    """A checkpoint tensor does not match the bank it is loaded into."""


def routed_shapes(experts=256, hidden=2048, inter=512, tile=16):
    """Registered shapes of the four routed bank fields (method.py:113-117)."""
    out = {}
    for proj, n, k in (('w13', 2 * inter, hidden), ('w2', hidden, inter)):
        out[f'{proj}_tilebank_codes'] = (experts, n // tile, k // 256, 32, tile)
        out[f'{proj}_tilebank_metadata'] = (experts, n // tile, k // 256, tile)
    return out


def dense_shapes(n, k, tile=16):
    """Shapes of a dense G256 linear's codes and metadata (method.py:44-45)."""
    if not 0 < n <= 12288 or n % 16 or not 0 < k <= 8192 or k % 256:
        raise AdmissionError(f'unsupported G256 linear geometry N{n}/K{k}')
    return {'g256_codes': (n // tile, k // 256, 32, tile), 'g256_metadata': (n // tile, k // 256, tile)}


def check_metadata(name, meta: torch.Tensor):
    """loader.py:31-36: CPU uint32 words of (fp16 scale, fp16 offset), finite,
    scale >= 2^-14."""
    if meta.device.type != 'cpu' or meta.dtype != torch.uint32:
        raise AdmissionError(f'{name}: metadata is admitted as CPU uint32 words')
    pairs = meta.contiguous().view(torch.float16).reshape(*meta.shape, 2)
    if not bool(torch.isfinite(pairs).all()):
        raise AdmissionError(f'{name}: non-finite scale or offset')
    if not bool((pairs[..., 0] >= MIN_SCALE).all()):
        raise AdmissionError(f'{name}: scale below 2^-14')


class BankLoader:
    """Strict one-shot loader of a fixed set of named bank fields."""

    def __init__(self, shapes: dict, dtypes: dict | None = None):
        self.shapes = dict(shapes)
        self.dtypes = dtypes or {k: torch.uint32 for k in shapes}
        self.loaded: dict[str, torch.Tensor] = {}
        self.sealed = False

    def load(self, name, value: torch.Tensor):
        if self.sealed:
            raise AdmissionError(f'{name}: banks already sealed')
        if name not in self.shapes:
            raise AdmissionError(f'unsupported bank field {name}')
        if name in self.loaded:
            raise AdmissionError(f'duplicate bank field {name}')
        if value.device.type == 'meta':
            raise AdmissionError(f'{name}: tensor is not materialised')
        if tuple(value.shape) != tuple(self.shapes[name]) or value.dtype != self.dtypes[name]:
            raise AdmissionError(f'{name}: got {tuple(value.shape)} {value.dtype}, '
                                 f'expected {tuple(self.shapes[name])} {self.dtypes[name]}')
        if name.endswith('metadata'):
            check_metadata(name, value)
        self.loaded[name] = value.contiguous()

    def load_prefixed(self, items, prefix=ROUTED_PREFIX):
        """Checkpoint (key, tensor) pairs with keys `prefix + field` (loader.py:21-24);
        yields the keys consumed."""
        for key, value in items:
            if not key.startswith(prefix):
                raise AdmissionError(f'unsupported checkpoint key {key}')
            self.load(key[len(prefix):], value)
            yield key

    def seal(self):
        missing = set(self.shapes) - set(self.loaded)
        if missing:
            raise AdmissionError(f'incomplete bank load, missing {sorted(missing)}')
        self.sealed = True
        return self.loaded


def repack_n32(codes16: torch.Tensor, meta16: torch.Tensor, n: int, k: int):
    """N16 banks (on the GPU) -> new N32 tensors [..., N/32, K/256, 32, 32] and
    [..., N/32, K/256, 32], through the library's repack kernel."""
    if codes16.device.type != 'cuda' or meta16.device != codes16.device:
        raise ValueError('the repack runs on GPU-resident banks')
    if codes16.element_size() != 4 or meta16.element_size() != 4:
        raise ValueError('banks are 32-bit words')
    if not codes16.is_contiguous() or not meta16.is_contiguous():
        raise ValueError('banks must be contiguous')
    lead = tuple(codes16.shape[:-4])
    banks = int(torch.Size(lead).numel())
    if tuple(codes16.shape[-4:]) != (n // 16, k // 256, 32, 16) or tuple(meta16.shape) != lead + (n // 16, k // 256, 16):
        raise ValueError(f'not N16 banks of N{n}/K{k}: {tuple(codes16.shape)}, {tuple(meta16.shape)}')
    if n % 32:
        raise ValueError(f'N{n} is not a multiple of 32')
    codes32 = torch.empty(lead + (n // 32, k // 256, 32, 32), dtype=codes16.dtype, device=codes16.device)
    meta32 = torch.empty(lead + (n // 32, k // 256, 32), dtype=meta16.dtype, device=meta16.device)
    native.check(native.lib().ornith_repack_n16_to_n32(native.ptr(codes16), native.ptr(meta16), native.ptr(codes32),
                                                       native.ptr(meta32), banks, n, k,
                                                       native.stream(codes16)), 'N16 -> N32 repack')
    return codes32, meta32
