"""Shared-expert SiLU / sigmoid tables.

The reference ships native/shared_math_reference.safetensors (silu_fp32 and
sigmoid_bf16, one entry per raw bf16 bit pattern) and refuses to run the
fused shared slot unless its sha256 matches the receipt
(plugin-site/ornith_g256/moe_shared.py:45-61).  The same file ships in this
package's data/ directory and is checked the same way.
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np

TABLE = Path(__file__).resolve().parent / 'data' / 'shared_math_reference.safetensors'
SHA256 = '11552ec53b62b229d0ab42b4e865d0175724cd51c4eef01c05e66e930f27d2eb'


def load_numpy():
    raw = TABLE.read_bytes()
    if hashlib.sha256(raw).hexdigest() != SHA256:
        raise RuntimeError(f'{TABLE.name}: sha256 is not {SHA256}; the SiLU/sigmoid tables cannot be trusted')
    n = int.from_bytes(raw[:8], 'little')
    header = json.loads(raw[8:8 + n])
    out = {}
    for name, dtype, np_dtype in (('silu_fp32', 'F32', np.float32), ('sigmoid_bf16', 'BF16', np.uint16)):
        info = header[name]
        if info['dtype'] != dtype or info['shape'] != [65536]:
            raise RuntimeError(f'{TABLE.name}: {name} must be {dtype} with 65536 entries, found '
                               f"{info['dtype']} {info['shape']}")
        lo, hi = info['data_offsets']
        out[name] = np.frombuffer(raw[8 + n + lo:8 + n + hi], dtype=np_dtype).copy()
    return out['silu_fp32'], out['sigmoid_bf16']


def load(device):
    """(silu f32 [65536], sigmoid bf16 [65536]) on `device`."""
    import torch
    silu, sigmoid = load_numpy()
    return (torch.from_numpy(silu).to(device),
            torch.from_numpy(sigmoid.view(np.int16)).to(device).view(torch.bfloat16))
