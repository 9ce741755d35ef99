"""CPU restatement of the Ornith G256 quantized-MoE arithmetic (numpy).

TEST INFRASTRUCTURE ONLY.  This module is the correctness oracle: it may be
imported by ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py``, and only to check results.  The product path (the HIP
library behind ``ornith_g256``) never calls it and fails loudly when the HIP
extension is missing.

Every function cites the reference file:line whose arithmetic it restates.
All floating-point steps are float32 numpy element-wise operations (IEEE
round-to-nearest-even, no fused multiply-add), evaluated in the exact order
the reference kernels use, so the results are bit-exact by construction.
Integer dot products are computed with float64 matrix products of small
integers: every partial sum is an integer below 2**53, so the result is
exact whatever order BLAS chooses.

Pinning (what checks each function, tests/test_oracle.py):
  * bf16/fp16 helpers      - exhaustive over all 65536 bit patterns against
                             torch's own conversions.
  * h128                   - closed form H @ v with the Sylvester matrix in
                             float64, H @ H = 128 I, brute force on unit vectors.
  * quantize               - brute-force per-element recomputation in Python
                             floats with explicit rounding, special cases
                             (zero group, non-finite, huge values).
  * group dots / tree      - brute force with Python ints on tiny shapes;
                             planted-mistake checks (wrong sign, transposed
                             operand, dropped offset) fail.
  * portable_exp           - known answers, |rel err| vs math.exp < 4 ulp,
                             special cases from the reference comments.
  * shared silu / sigmoid  - golden table shipped in the reference
                             (native/shared_math_reference.safetensors).
  * router / top-k         - the reduction order is this library's own
                             declared order (the reference's Triton row-dot
                             and vLLM topk_softmax orders are compiler- or
                             library-chosen and not importable here): the
                             declared order is pinned by brute force and
                             float64 agreement, top-k by brute force on
                             small inputs.  Against the reference itself:
                             parity unpinned.
  * permute                - counts against numpy bincount, stable order
                             against argsort(kind='stable').
  * head_w8_tile_layout     - every byte against the reference's scalar
                             tile_word index, low-K byte first, with a
                             planted transposed layout that must fail.
  * h128 order, quantize, routed_layer_shared, reduce_slots, head_w8,
    portable_exp, shared_fixed8
                           - bit for bit against scalar statement-by-statement
                             restatements of the reference kernels
                             (tests/_transcribe.py), each with planted
                             mistakes that must fail (tests/test_oracle_pins.py).
  * add_bf16               - against torch's CPU bf16 addition on 2M pairs.
"""
from __future__ import annotations

import math
import numpy as np

E, TOP, H, I, G = 256, 8, 2048, 512, 256
WORDS = G // 8
INV_SQRT128 = np.uint32(0x3DB504F3).view(np.float32)   # routed_storage_n32_consumer.cpp:12
F32 = np.float32

# Sticky flag bits, routed_storage_n32_consumer.cpp:33,51,58,86-87,115,174,183
FLAG_NONFINITE_INPUT = 1
FLAG_INVALID_ACTIVATION = 2
FLAG_INVALID_EXPERT = 4
FLAG_NONFINITE_PROJECTION = 8
FLAG_NONFINITE_MIDDLE = 16
FLAG_NONFINITE_OUTPUT = 32
# dense_g256_api.h:14-19
DENSE_NONFINITE_INPUT = 1
DENSE_INVALID_ACTIVATION = 2
DENSE_NONFINITE_PROJECTION = 4
DENSE_NONFINITE_BF16 = 8


# ----------------------------------------------------------------------------
# bf16 / fp16 helpers (routed_storage_n32_consumer.cpp:17-21)
# ----------------------------------------------------------------------------
def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(value: np.ndarray) -> np.ndarray:
    """bf16 round-to-nearest-even with the reference's NaN rule (:17-21)."""
    b = np.asarray(value, dtype=np.float32).view(np.uint32)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    rne = ((b.astype(np.uint64) + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((b >> 16) | 0x40).astype(np.uint16), rne)


def bf16_round(value: np.ndarray) -> np.ndarray:
    return bf16_to_f32(f32_to_bf16(value))


def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def f32_to_f16_bits(value: np.ndarray) -> np.ndarray:
    # numpy float32 -> float16 conversion is IEEE round-to-nearest-even,
    # the same as __float2half_rn.
    return np.asarray(value, dtype=np.float32).astype(np.float16).view(np.uint16)


# ----------------------------------------------------------------------------
# 128-point Hadamard transform (routed_storage_n32_consumer.cpp:22-43,
# dense_g256_consumer.cpp:27-40): seven ascending butterflies in fp32,
# then multiply by 0x3db504f3.
# ----------------------------------------------------------------------------
def h128(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    shape = x.shape
    assert shape[-1] % 128 == 0
    v = x.reshape(-1, 128).copy()
    step = 1
    while step < 128:
        w = v.reshape(v.shape[0], 128 // (2 * step), 2, step)
        a = w[:, :, 0, :]
        b = w[:, :, 1, :]
        # dst[l] = src[lo] + src[lo+step] (bit clear), src[lo] - src[lo+step] (bit set)
        v = np.stack([a + b, a - b], axis=2).reshape(v.shape[0], 128)
        step *= 2
    return (v * INV_SQRT128).astype(np.float32).reshape(shape)


# ----------------------------------------------------------------------------
# Group activation quantisation (routed_storage_n32_consumer.cpp:44-76,
# dense_g256_api.h:32-35).  Returns q (int32), fp16 scale bits, int32 sums
# and the sticky flag bits raised.
# ----------------------------------------------------------------------------
def quantize(x: np.ndarray, qmax: int = 127, group: int = G, invalid_flag: int = FLAG_INVALID_ACTIVATION):
    x = np.asarray(x, dtype=np.float32)
    rows, k = x.shape
    assert k % group == 0
    v = x.reshape(rows, k // group, group)
    finite = np.isfinite(v)
    flags = 0 if finite.all() else invalid_flag
    v = np.where(finite, v, F32(0))
    absmax = np.max(np.abs(v), axis=2)
    with np.errstate(over='ignore', invalid='ignore'):
        raw = (absmax / F32(qmax)).astype(np.float32)
    valid = np.isfinite(raw) & (raw <= F32(65504))
    if not valid.all():
        flags |= invalid_flag
    zero = (absmax == 0) | ~valid
    scale_f32 = np.where(zero, F32(1), np.maximum(raw, F32(2.0 ** -14))).astype(np.float32)
    scale_bits = f32_to_f16_bits(scale_f32)
    scale = f16_bits_to_f32(scale_bits)
    with np.errstate(over='ignore', invalid='ignore', divide='ignore'):
        ratio = (v / scale[:, :, None]).astype(np.float32)
    q = np.rint(ratio)
    q = np.where(zero[:, :, None], 0, q)
    q = np.clip(q, -qmax, qmax).astype(np.int32)
    sums = q.sum(axis=2).astype(np.int32)
    return q.reshape(rows, k), scale_bits, sums, flags


def pack_planes(q: np.ndarray):
    """Low (unsigned) / high (signed) nibble planes, 8 values per word, low K
    nibble first (routed_storage_n32_consumer.cpp:65-71).  Kept for format
    comparison; the MI355X kernels use int8 activations instead."""
    q = np.asarray(q, dtype=np.int64)
    lo = q & 15
    hi = (q - lo) // 16
    rows, k = q.shape
    shifts = (4 * np.arange(8, dtype=np.uint64))
    low = ((lo.reshape(rows, k // 8, 8).astype(np.uint64) & 15) << shifts).sum(axis=2).astype(np.uint32)
    high = ((hi.reshape(rows, k // 8, 8).astype(np.uint64) & 15) << shifts).sum(axis=2).astype(np.uint32)
    return low, high


# ----------------------------------------------------------------------------
# Weight storage (dense_g256_api.h:25-27, routed_storage_n32_consumer.cpp:2,
# method.py:44-45,113-117, method.py:143-147).
# codes: unsigned 4-bit, [N, K] uint8 logical.  meta: fp16 scale | offset<<16.
# ----------------------------------------------------------------------------
def pack_codes_words(codes: np.ndarray) -> np.ndarray:
    """[N, K] 4-bit codes -> [N, K/8] uint32, low K nibble first."""
    codes = np.asarray(codes, dtype=np.uint32)
    n, k = codes.shape
    shifts = (4 * np.arange(8, dtype=np.uint32))
    return (codes.reshape(n, k // 8, 8) << shifts).sum(axis=2, dtype=np.uint64).astype(np.uint32)


def unpack_codes_words(words: np.ndarray) -> np.ndarray:
    words = np.asarray(words, dtype=np.uint32)
    n, kw = words.shape
    shifts = (4 * np.arange(8, dtype=np.uint32))
    return ((words[:, :, None] >> shifts) & 15).reshape(n, kw * 8).astype(np.uint8)


def to_tile_layout(codes: np.ndarray, tile: int) -> np.ndarray:
    """[N, K] codes -> tile-bank uint32 [N/tile, K/256, 32, tile]; element
    ((n/tile*K/256 + g)*32 + j)*tile + n%tile holds K values 256g+8j..+7."""
    words = pack_codes_words(codes)                      # [N, K/8]
    n, kw = words.shape
    return np.ascontiguousarray(
        words.reshape(n // tile, tile, kw // WORDS, WORDS).transpose(0, 2, 3, 1))


def from_tile_layout(bank: np.ndarray) -> np.ndarray:
    nt, groups, words, tile = bank.shape
    w = bank.transpose(0, 3, 1, 2).reshape(nt * tile, groups * words)
    return unpack_codes_words(w)


def pack_meta(scale_bits: np.ndarray, offset_bits: np.ndarray, tile: int) -> np.ndarray:
    """fp16 (scale, offset) [N, K/256] -> uint32 [N/tile, K/256, tile]."""
    m = (np.asarray(scale_bits, np.uint32) | (np.asarray(offset_bits, np.uint32) << 16))
    n, groups = m.shape
    return np.ascontiguousarray(m.reshape(n // tile, tile, groups).transpose(0, 2, 1))


def n16_to_n32(codes16: np.ndarray, meta16: np.ndarray):
    """N16 -> N32 bank repack (method.py:143-147, dense_n32.py:113-114)."""
    e = codes16.shape[:-4]
    nt, groups = codes16.shape[-4], codes16.shape[-3]
    c = codes16.reshape(*e, nt // 2, 2, groups, 32, 16)
    c = np.moveaxis(c, -4, -2).reshape(*e, nt // 2, groups, 32, 32)
    m = meta16.reshape(*e, nt // 2, 2, groups, 16)
    m = np.moveaxis(m, -3, -2).reshape(*e, nt // 2, groups, 32)
    return np.ascontiguousarray(c), np.ascontiguousarray(m)


def signed_to_affine(q4: np.ndarray, scale_f32: np.ndarray):
    """Signed int4 in [-8,7] with an fp16 scale -> the reference's affine
    storage: code = q+8, offset = fp16(-8 * scale).  Exact: x8 is a power of
    two and stays in fp16 normal range for scales >= 2^-14."""
    code = (np.asarray(q4, np.int32) + 8).astype(np.uint8)
    scale_bits = f32_to_f16_bits(scale_f32)
    offset_bits = f32_to_f16_bits(F32(-8) * f16_bits_to_f32(scale_bits))
    return code, scale_bits, offset_bits


# ----------------------------------------------------------------------------
# Exact integer group dots and the fp32 group tree
# (routed_storage_n32_consumer.cpp:138-158, dense_g256_api.h:35-38).
# ----------------------------------------------------------------------------
def group_dots(q: np.ndarray, codes: np.ndarray) -> np.ndarray:
    """q int [M, K], codes uint8 [N, K] -> exact int64 dots [M, N, K/256]."""
    m, k = q.shape
    n = codes.shape[0]
    groups = k // G
    qf = np.asarray(q, np.float64).reshape(m, groups, G)
    cf = np.asarray(codes, np.float64).reshape(n, groups, G)
    out = np.empty((m, n, groups), dtype=np.int64)
    for g in range(groups):
        out[:, :, g] = (qf[:, g, :] @ cf[:, g, :].T).astype(np.int64)
    return out


def tree(dots, act_scale_bits, act_sums, w_scale_bits, w_offset_bits):
    """acc = acc + (RN(sw*RN(sa*dot)) + RN(off*RN(sa*sum))), ascending groups.
    dots [M,N,Gs]; act_* [M,Gs]; w_* [N,Gs] -> fp32 [M,N]."""
    m, n, groups = dots.shape
    sa = f16_bits_to_f32(act_scale_bits)
    sw = f16_bits_to_f32(w_scale_bits)
    off = f16_bits_to_f32(w_offset_bits)
    acc = np.zeros((m, n), dtype=np.float32)
    with np.errstate(over='ignore', invalid='ignore'):
        for g in range(groups):
            scaled_dot = (sa[:, g][:, None] * dots[:, :, g].astype(np.float32)).astype(np.float32)
            scaled_sum = (sa[:, g] * np.asarray(act_sums[:, g], np.float32)).astype(np.float32)
            product = (sw[:, g][None, :] * scaled_dot).astype(np.float32)
            correction = (off[:, g][None, :] * scaled_sum[:, None]).astype(np.float32)
            acc = (acc + (product + correction).astype(np.float32)).astype(np.float32)
    return acc


def quant_linear(act_f32, codes, w_scale_bits, w_offset_bits, qmax=127):
    """Transformed fp32 activations -> fp32 projection (A8/A4 path) + flags."""
    q, sbits, sums, flags = quantize(act_f32, qmax)
    dots = group_dots(q, codes)
    return tree(dots, sbits, sums, w_scale_bits, w_offset_bits), flags


# ----------------------------------------------------------------------------
# Dense G256 linear (dense_g256_consumer.cpp:172-189 launch;
# dense_n32 dense_g256_consumer.cpp:360-378) and the bf16 prefill operands
# (dense_g256_consumer.cpp:192-246).
# ----------------------------------------------------------------------------
def dense_a8(x_bf16, codes, w_scale_bits, w_offset_bits):
    """x bf16 bits [M,K]; codes [N,K] -> (out bf16 bits [M,N], diag f32, flags)."""
    x = bf16_to_f32(x_bf16)
    flags = 0 if np.isfinite(x).all() else DENSE_NONFINITE_INPUT
    tx = h128(x)
    if not np.isfinite(tx).all():
        flags |= DENSE_NONFINITE_INPUT
    y, f = quant_linear(tx, codes, w_scale_bits, w_offset_bits)
    flags |= f
    if not np.isfinite(y).all():
        flags |= DENSE_NONFINITE_PROJECTION
    out = f32_to_bf16(y)
    if ((out & 0x7F80) == 0x7F80).any():
        flags |= DENSE_NONFINITE_BF16
    return out, y, flags


def dequantize_bf16(codes, w_scale_bits, w_offset_bits):
    """bf16(RN(RN(s*code) + off)) [N,K] (dense_g256_consumer.cpp:209-229)."""
    n, k = codes.shape
    s = np.repeat(f16_bits_to_f32(w_scale_bits), G, axis=1)
    o = np.repeat(f16_bits_to_f32(w_offset_bits), G, axis=1)
    v = ((s * codes.astype(np.float32)).astype(np.float32) + o).astype(np.float32)
    return f32_to_bf16(v)


def transform_bf16(x_bf16):
    """bf16(H128(x)) (dense_g256_consumer.cpp:192-206)."""
    return f32_to_bf16(h128(bf16_to_f32(x_bf16)))


# ----------------------------------------------------------------------------
# Deterministic exp (kernels/routed_storage/portable_exp.h:6-26).
# ----------------------------------------------------------------------------
_EXP_C = [np.uint32(v).view(np.float32) for v in (
    0x3FB8AA3B,  # log2(e)             0x1.715476p+0
    0x3F317200,  # ln2 high             0x1.62e400p-1
    0x35BFBE8E,  # ln2 low              0x1.7f7d1cp-20
)]
_EXP_P = [np.float32(float.fromhex(h)) for h in (
    '0x1.a01a02p-16', '0x1.a01a02p-13', '0x1.6c16c2p-10', '0x1.111112p-7',
    '0x1.555556p-5', '0x1.555556p-3', '0x1p-1', '0x1p+0', '0x1p+0')]


def portable_exp(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    n_float = np.rint((x * _EXP_C[0]).astype(np.float32)).astype(np.float32)
    n_float = np.where(np.isfinite(n_float), n_float, F32(0))
    high = (n_float * _EXP_C[1]).astype(np.float32)
    low = (n_float * _EXP_C[2]).astype(np.float32)
    r = ((x - high).astype(np.float32) - low).astype(np.float32)
    p = np.full_like(x, _EXP_P[0])
    for c in _EXP_P[1:]:
        p = ((p * r).astype(np.float32) + c).astype(np.float32)
    n = np.clip(n_float, -300, 300).astype(np.int32)
    with np.errstate(over='ignore', invalid='ignore'):
        out = np.ldexp(p, n).astype(np.float32)
    out = np.where(x <= F32(-104), F32(0), out)
    out = np.where(x >= F32(89), F32(np.inf), out)
    out = np.where(np.isnan(x), x, out)
    return out.astype(np.float32)


def silu_portable(g: np.ndarray) -> np.ndarray:
    """g / RN(1 + pexp(-g)) with a correctly rounded division (:173)."""
    g = np.asarray(g, np.float32)
    den = (F32(1) + portable_exp(-g)).astype(np.float32)
    with np.errstate(over='ignore', invalid='ignore', divide='ignore'):
        return (g / den).astype(np.float32)


# ----------------------------------------------------------------------------
# Routed MoE layer, A8 or A4 (routed_storage_n32_consumer.cpp:319-351 and the
# kernels it launches; prefill.h grouped jobs use the same per-route math).
# ----------------------------------------------------------------------------
def _valid(ids):
    return (ids >= 0) & (ids < E)


def routed_layer(x_bf16, route_w, ids, w13_codes, w13_sbits, w13_obits,
                 w2_codes, w2_sbits, w2_obits, qmax=127):
    """x_bf16 [T,H] bits; route_w f32 [T,8]; ids i32 [T,8];
    w13_codes [E,1024,2048] uint8; w13_sbits/obits [E,1024,8];
    w2_codes [E,2048,512]; w2_sbits/obits [E,2048,2].
    Returns dict(out bf16 bits [T,H], final f32 [T,H], gate_y [R,1024],
    middle [R,512], route_out [R,H], flags)."""
    T = x_bf16.shape[0]
    R = T * TOP
    ids = np.asarray(ids, np.int32).reshape(R)
    rw = np.asarray(route_w, np.float32).reshape(R)
    valid = _valid(ids)
    flags = 0
    if (~valid & (ids != -1)).any():
        flags |= FLAG_INVALID_EXPERT
    live_tok = valid.reshape(T, TOP).any(axis=1)
    x = bf16_to_f32(x_bf16)
    if (~np.isfinite(x[live_tok])).any():
        flags |= FLAG_NONFINITE_INPUT
    tx = h128(x)
    tx[~live_tok] = 0
    if (~np.isfinite(tx)).any():
        flags |= FLAG_NONFINITE_INPUT
    q, sbits, sums, f = quantize(tx, qmax)
    flags |= f
    gate_y = np.zeros((R, 2 * I), np.float32)
    for e in np.unique(ids[valid]):
        rs = np.nonzero(ids == e)[0]
        toks = rs // TOP
        dots = group_dots(q[toks], w13_codes[e])
        gate_y[rs] = tree(dots, sbits[toks], sums[toks], w13_sbits[e], w13_obits[e])
    if (~np.isfinite(gate_y)).any():
        flags |= FLAG_NONFINITE_PROJECTION
    g, up = gate_y[:, :I], gate_y[:, I:]
    with np.errstate(over='ignore', invalid='ignore'):
        middle = (silu_portable(g) * up).astype(np.float32)
    middle[~valid] = 0
    if (~np.isfinite(middle)).any():
        flags |= FLAG_NONFINITE_MIDDLE
    dx = h128(middle)
    if (~np.isfinite(middle)).any() or (~np.isfinite(dx)).any():
        flags |= FLAG_NONFINITE_INPUT
    q2, sbits2, sums2, f = quantize(dx, qmax)
    flags |= f
    route_out = np.zeros((R, H), np.float32)
    for e in np.unique(ids[valid]):
        rs = np.nonzero(ids == e)[0]
        dots = group_dots(q2[rs], w2_codes[e])
        route_out[rs] = tree(dots, sbits2[rs], sums2[rs], w2_sbits[e], w2_obits[e])
    if (~np.isfinite(route_out)).any():
        flags |= FLAG_NONFINITE_PROJECTION
    final, out, f = reduce_slots(route_out, rw, ids, T)
    flags |= f
    return dict(out=out, final=final, gate_y=gate_y, middle=middle, route_out=route_out,
                act_q=q, act_scale=sbits, act_sum=sums, flags=flags)


def reduce_slots(route_out, rw, ids, T):
    """Slot-order fp32 sum of route_out * weight, bf16 RNE
    (routed_storage_n32_consumer.cpp:176-184)."""
    ids = ids.reshape(T, TOP)
    rw = rw.reshape(T, TOP)
    ro = route_out.reshape(T, TOP, -1)
    acc = np.zeros((T, ro.shape[2]), np.float32)
    with np.errstate(over='ignore', invalid='ignore'):
        for s in range(TOP):
            v = _valid(ids[:, s])
            prod = (ro[:, s, :] * rw[:, s][:, None]).astype(np.float32)
            acc = np.where(v[:, None], (acc + prod).astype(np.float32), acc)
    out = f32_to_bf16(acc)
    flags = 0
    if (~np.isfinite(acc)).any() or ((out & 0x7F80) == 0x7F80).any():
        flags |= FLAG_NONFINITE_OUTPUT
    return acc, out, flags


def routed_layer_shared(x_bf16, route_w, ids, w13_codes, w13_sbits, w13_obits,
                        w2_codes, w2_sbits, w2_obits,
                        s13_codes, s13_sbits, s13_obits, s2_codes, s2_sbits, s2_obits,
                        shared_logit_bf16, silu_table_f32, sigmoid_table_bf16):
    """Fused shared-expert-as-ninth-slot decode
    (routed_storage_n32_consumer.cpp:187-307, 385-401).  Shared rows round
    their linear outputs to bf16, use the tabulated SiLU and sigmoid.
    Returns dict(out, shared_out (bf16 bits), final, gate_y, route_out, flags)."""
    T = x_bf16.shape[0]
    R = T * TOP
    RS = R + T
    ids = np.asarray(ids, np.int32).reshape(R)
    rw = np.asarray(route_w, np.float32).reshape(R)
    valid = _valid(ids)
    flags = 0
    if (~valid & (ids != -1)).any():
        flags |= FLAG_INVALID_EXPERT
    x = bf16_to_f32(x_bf16)
    if (~np.isfinite(x)).any():
        flags |= FLAG_NONFINITE_INPUT
    tx = h128(x)          # fused_transform_quantize<0>: no liveness zeroing (:237-239)
    if (~np.isfinite(tx)).any():
        flags |= FLAG_NONFINITE_INPUT
    q, sbits, sums, f = quantize(tx)
    flags |= f
    gate_y = np.zeros((RS, 2 * I), np.float32)
    for e in np.unique(ids[valid]):
        rs = np.nonzero(ids == e)[0]
        toks = rs // TOP
        gate_y[rs] = tree(group_dots(q[toks], w13_codes[e]), sbits[toks], sums[toks],
                          w13_sbits[e], w13_obits[e])
    toks = np.arange(T)
    gate_y[R:] = bf16_round(tree(group_dots(q, s13_codes), sbits, sums, s13_sbits, s13_obits))
    if (~np.isfinite(gate_y)).any():
        flags |= FLAG_NONFINITE_PROJECTION
    g, up = gate_y[:, :I], gate_y[:, I:]
    with np.errstate(over='ignore', invalid='ignore'):
        mid_routed = (silu_portable(g[:R]) * up[:R]).astype(np.float32)
        silu_sh = silu_table_f32[g[R:].view(np.uint32) >> 16]
        mid_shared = bf16_round((silu_sh * up[R:]).astype(np.float32))
    mid_routed[~valid] = 0
    middle = np.concatenate([mid_routed, mid_shared])
    if (~np.isfinite(middle)).any():
        flags |= FLAG_NONFINITE_MIDDLE | FLAG_NONFINITE_INPUT
    dx = h128(middle)
    if (~np.isfinite(dx)).any():
        flags |= FLAG_NONFINITE_INPUT
    q2, sbits2, sums2, f = quantize(dx)
    flags |= f
    route_out = np.zeros((RS, H), np.float32)
    for e in np.unique(ids[valid]):
        rs = np.nonzero(ids == e)[0]
        route_out[rs] = tree(group_dots(q2[rs], w2_codes[e]), sbits2[rs], sums2[rs],
                             w2_sbits[e], w2_obits[e])
    route_out[R:] = bf16_round(tree(group_dots(q2[R:], s2_codes), sbits2[R:], sums2[R:],
                                    s2_sbits, s2_obits))
    if (~np.isfinite(route_out)).any():
        flags |= FLAG_NONFINITE_PROJECTION
    final, out, f = reduce_slots(route_out[:R], rw, ids, T)
    flags |= f
    gate = bf16_to_f32(sigmoid_table_bf16[np.asarray(shared_logit_bf16, np.uint16)])
    with np.errstate(over='ignore', invalid='ignore'):
        shared = (route_out[R:] * gate[:, None]).astype(np.float32)
    shared_out = f32_to_bf16(shared)
    if (~np.isfinite(shared)).any():
        flags |= FLAG_NONFINITE_OUTPUT
    return dict(out=out, shared_out=shared_out, final=final, gate_y=gate_y,
                middle=middle, route_out=route_out, flags=flags)


def shared_fixed8(x_bf16, s13_codes, s13_sbits, s13_obits, s2_codes, s2_sbits, s2_obits, gate_w_bf16,
                  silu_table_f32, sigmoid_table_bf16):
    """Production shared expert of decode rows
    (iu4_correctness/shared_kernel.py:33-62): two dense A8 projections with
    bf16 outputs (dense_n32 dense_g256_consumer.cpp:360-378), vLLM
    silu_and_mul in bf16 (SiLU rounded to bf16, then a bf16 product; SiLU
    taken from the reference's SiLU table), the scalar gate rounded to bf16
    (declared row-dot order) and torch.sigmoid in bf16 times down, rounded to
    bf16.  Returns (out bf16 bits [M,2048], flags)."""
    gu, _, f1 = dense_a8(x_bf16, s13_codes, s13_sbits, s13_obits)
    g, up = gu[:, :I], gu[:, I:]
    silu = bf16_round(np.asarray(silu_table_f32, np.float32)[g])
    act = f32_to_bf16((silu * bf16_to_f32(up)).astype(np.float32))
    down, _, f2 = dense_a8(act, s2_codes, s2_sbits, s2_obits)
    logit = f32_to_bf16(router_logits(x_bf16, np.asarray(gate_w_bf16).reshape(1, -1))[:, 0])
    gate = bf16_to_f32(np.asarray(sigmoid_table_bf16, np.uint16)[logit])
    out = f32_to_bf16((gate[:, None] * bf16_to_f32(down)).astype(np.float32))
    flags = f1 | f2
    if ((out & 0x7F80) == 0x7F80).any():
        flags |= DENSE_NONFINITE_BF16
    return out, flags


def add_bf16(a_bits, b_bits):
    """bf16 + bf16 -> bf16 as torch computes it (fp32 sum, one RNE rounding);
    the routed + shared combination done by the MoE runner."""
    return f32_to_bf16((bf16_to_f32(a_bits) + bf16_to_f32(b_bits)).astype(np.float32))


# ----------------------------------------------------------------------------
# Router: fp32 logits, softmax, top-8, renormalise.  The reference computes
# the logits with a Triton row-dot (iu4_correctness/gates_projection.py:18-26,
# 36-42) and selects experts in vLLM's topk_softmax (contract: moe_base.py:
# 57-64, dtypes :53-54).  Both reduction orders are compiler/library-chosen,
# so this library declares its own fixed order, restated here:
#   logit[t,e] = bias[e] + butterfly64( lane partial sums ), lane l
#   accumulating fma(x[k], w[k], acc) sequentially over k = 8c..8c+7 for
#   c = l, l+64, l+128, l+192.
# ----------------------------------------------------------------------------
def _butterfly64(acc):
    """xor-butterfly over the last axis (64 lanes): acc[l] + acc[l^off] for
    off = 1,2,4,8,16,32.  Returns lane 0 (all lanes agree)."""
    lanes = np.arange(64)
    for off in (1, 2, 4, 8, 16, 32):
        acc = (acc + acc[..., lanes ^ off]).astype(np.float32)
    return acc[..., 0]


def router_logits(x_bf16, w_bf16, bias=None, chunk=16):
    """x bits [T,2048], w bits [Nr,2048] -> fp32 [T,Nr] in the declared order."""
    T = x_bf16.shape[0]
    nr = w_bf16.shape[0]
    x = bf16_to_f32(x_bf16).reshape(T, 4, 64, 8)     # [t, i, lane, j]: k = (64i+lane)*8+j
    w = bf16_to_f32(w_bf16).reshape(nr, 4, 64, 8)
    out = np.empty((T, nr), np.float32)
    for t0 in range(0, T, chunk):
        xs = x[t0:t0 + chunk]
        acc = np.zeros((xs.shape[0], nr, 64), np.float32)
        with np.errstate(over='ignore', invalid='ignore'):
            for i in range(4):
                for j in range(8):
                    # fma(x, w, acc): exact product (float64 holds it), one
                    # rounding of the sum to fp32.  Rounding the float64 sum
                    # first cannot change the fp32 result here: the product
                    # has <= 16 significant bits, acc <= 24.
                    prod = xs[:, None, i, :, j].astype(np.float64) * w[None, :, i, :, j].astype(np.float64)
                    acc = (acc.astype(np.float64) + prod).astype(np.float32)
        out[t0:t0 + chunk] = _butterfly64(acc)
    if bias is not None:
        out = (out + np.asarray(bias, np.float32)[None, :]).astype(np.float32)
    return out


def softmax_topk(logits, k=TOP):
    """Declared order: m = max; e = pexp(l - m); s = butterfly64 over lanes of
    ((e[l] + e[l+64]) + e[l+128]) + e[l+192]; p = e / s; select the k largest
    p (ties -> lower expert id), descending; w_j = p_j / (sequential slot-order
    sum of the selected p).  Returns (weights f32 [T,k], ids i32 [T,k], p)."""
    logits = np.asarray(logits, np.float32)
    T, n = logits.shape
    assert n == E
    m = logits.max(axis=1)
    ex = portable_exp((logits - m[:, None]).astype(np.float32))
    v = ex.reshape(T, 4, 64)
    part = v[:, 0, :]
    for i in range(1, 4):
        part = (part + v[:, i, :]).astype(np.float32)
    s = _butterfly64(part)
    p = (ex / s[:, None]).astype(np.float32)
    # stable descending selection: sort by (-p, id)
    order = np.lexsort((np.broadcast_to(np.arange(n), (T, n)), -p.astype(np.float64)), axis=1)
    ids = order[:, :k].astype(np.int32)
    sel = np.take_along_axis(p, ids, axis=1)
    tot = np.zeros(T, np.float32)
    for j in range(k):
        tot = (tot + sel[:, j]).astype(np.float32)
    w = (sel / tot[:, None]).astype(np.float32)
    return w, ids, p


# ----------------------------------------------------------------------------
# Token permute (routed_storage_n32_prefill.h:19-42): counts, exclusive
# offsets and per-expert route lists.  The reference fills each list with
# atomic cursors (any order); this library's order is stable (ascending route
# index), so the oracle returns that order.
# ----------------------------------------------------------------------------
def permute(ids, n_experts=E):
    ids = np.asarray(ids, np.int32).reshape(-1)
    v = (ids >= 0) & (ids < n_experts)
    counts = np.bincount(ids[v], minlength=n_experts).astype(np.int32)
    offsets = np.zeros(n_experts + 1, np.int32)
    offsets[1:] = np.cumsum(counts)
    routes = np.nonzero(v)[0][np.argsort(ids[v], kind='stable')].astype(np.int32)
    return counts, offsets, routes


# ----------------------------------------------------------------------------
# W8 G128 LM head (head_i8_tile_consumer.cpp:30-106, api :22-36).
# ----------------------------------------------------------------------------
def head_w8(x_bf16, w_i8, w_scale_bits):
    """x bits [M,2048]; w int8 [N,2048]; scales fp16 bits [N,16]."""
    x = bf16_to_f32(x_bf16)
    tx = h128(x)
    q, sbits, _, flags = quantize(tx, 127, group=128)
    M, K = q.shape
    N = w_i8.shape[0]
    qf = q.reshape(M, 16, 128).astype(np.float64)
    wf = np.asarray(w_i8, np.float64).reshape(N, 16, 128)
    sa = f16_bits_to_f32(sbits)
    sw = f16_bits_to_f32(w_scale_bits)
    acc = np.zeros((M, N), np.float32)
    for g in range(16):
        dot = (qf[:, g, :] @ wf[:, g, :].T).astype(np.float32)
        scaled = (sa[:, g][:, None] * dot).astype(np.float32)
        term = (sw[:, g][None, :] * scaled).astype(np.float32)
        acc = (acc + term).astype(np.float32)
    return f32_to_bf16(acc), acc, flags


def head_w8_tile_layout(w_i8):
    """int8 [N,2048] -> uint32 [N/16, 128, 4, 16] (head_i8_tile_api.h:1-2,
    consumer :19-21): word (n, kword) packs K bytes 4kword..+3, low first."""
    w = np.asarray(w_i8, np.int8).view(np.uint8).astype(np.uint32)
    N = w.shape[0]
    words = (w.reshape(N, 512, 4) << (8 * np.arange(4, dtype=np.uint32))).sum(axis=2, dtype=np.uint64).astype(np.uint32)
    return np.ascontiguousarray(words.reshape(N // 16, 16, 128, 4).transpose(0, 2, 3, 1))


def argmax_first(values):
    """Top-1 with ties resolved to the lowest index (numpy argmax rule)."""
    return np.argmax(values, axis=-1).astype(np.int64)
