"""Scalar, statement-by-statement restatements of the reference kernels, used
only to pin the vectorised oracle (oracle/ornith_oracle.py) on small inputs.

Each function follows one reference kernel literally: one lane's arithmetic
at a time, numpy float32 scalars for every fp32 operation (each rounds to
nearest even, no fused multiply-add), Python ints for the integer dots.  The
oracle is written in vectorised form over whole arrays; the two are written
independently, so a dropped rounding, a swapped operand or a changed order in
either shows up as a bit difference.  Optional `mistake` arguments plant one
specific error, for the tests that check a pin can fail.

Sources (reference files):
  routed_storage_n32_consumer.cpp:17-21 (bf16 RNE), :34-41 (H128 lanes),
  :44-76 (A8 quantise + nibble planes), :138-157 (projection dot and tree),
  :168-175 (middle), :176-184 (slot reduce), :187-230 (shared-slot
  projection), :231-295 (fused transform/quantise, both modes),
  :296-307 (shared reduce); portable_exp.h:6-26;
  head_i8_tile_consumer.cpp:30-106 (W8 head).
"""
from __future__ import annotations

import numpy as np

F = np.float32
INV_SQRT128 = np.uint32(0x3DB504F3).view(np.float32)
E, TOP, H, I = 256, 8, 2048, 512


def bf16_rne(v) -> int:
    """routed_storage_n32_consumer.cpp:17-21."""
    b = int(np.float32(v).view(np.uint32))
    if (b & 0x7FFFFFFF) > 0x7F800000:
        return ((b >> 16) | 0x40) & 0xFFFF
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) & 0xFFFF


def bf16_f32(bits) -> np.float32:
    return np.uint32(int(bits) << 16).view(np.float32)


def f16_f32(bits) -> np.float32:
    return F(np.uint16(bits).view(np.float16))


def portable_exp(x) -> np.float32:
    """portable_exp.h:6-26, one scalar."""
    x = F(x)
    if np.isnan(x):
        return x
    if x <= F(-104):
        return F(0)
    if x >= F(89):
        return F(np.inf)
    n_float = F(np.rint(F(x * F(float.fromhex('0x1.715476p+0')))))
    n = int(n_float)
    high = F(n_float * F(float.fromhex('0x1.62e400p-1')))
    low = F(n_float * F(float.fromhex('0x1.7f7d1cp-20')))
    r = F(F(x - high) - low)
    p = F(float.fromhex('0x1.a01a02p-16'))
    for c in ('0x1.a01a02p-13', '0x1.6c16c2p-10', '0x1.111112p-7', '0x1.555556p-5', '0x1.555556p-3',
              '0x1p-1', '0x1p+0', '0x1p+0'):
        p = F(F(p * r) + F(float.fromhex(c)))
    return F(np.ldexp(p, n))


def h128_block(values, mistake=None):
    """One 128-value block, lane by lane (routed_storage_n32_consumer.cpp:34-41):
    dst[lane] = lane&step ? src[lo]-src[lo+step] : src[lo]+src[lo+step],
    steps 1, 2, ..., 64, then src[lane] * InvSqrt128.
    mistake='descending': steps 64, 32, ..., 1."""
    src = [F(v) for v in values]
    steps = [1, 2, 4, 8, 16, 32, 64]
    if mistake == 'descending':
        steps = steps[::-1]
    for step in steps:
        dst = [None] * 128
        for lane in range(128):
            lo = lane & ~step
            dst[lane] = F(src[lo] - src[lo + step]) if lane & step else F(src[lo] + src[lo + step])
        src = dst
    return [F(v * INV_SQRT128) for v in src]


def quantize_group(values, qmax=127):
    """One 256-group (routed_storage_n32_consumer.cpp:44-76): returns q, fp16
    scale bits, sum, the low (unsigned) and high (signed) nibble of each q,
    and the flag bits raised."""
    flags = 0
    vals, absmax = [], F(0)
    for v in values:
        v = F(v)
        if not np.isfinite(v):
            flags |= 2
            v = F(0)
        vals.append(v)
        absmax = max(absmax, F(abs(v)))
    raw = F(absmax / F(qmax))
    valid = bool(np.isfinite(raw)) and raw <= F(65504)
    if not valid:
        flags |= 2
    zero = absmax == F(0) or not valid
    scale = np.float16(F(1) if zero else max(raw, F(2.0 ** -14)))
    sf = F(scale)
    q, lo, hi, total = [], [], [], 0
    for v in vals:
        t = 0 if zero else int(np.rint(F(v / sf)))
        t = -qmax if t < -qmax else (qmax if t > qmax else t)
        total += t
        q.append(t)
        lo.append(t & 15)
        hi.append((t - (t & 15)) // 16)
    return q, int(scale.view(np.uint16)), total, lo, hi, flags


def transform_quantize(row, qmax=127):
    """fused_transform_quantize<0> over one activation row: H128 per 128
    block, then quantize per 256 group (routed_storage_n32_consumer.cpp:231-295)."""
    tx = []
    for b in range(len(row) // 128):
        tx += h128_block(row[128 * b:128 * (b + 1)])
    groups = [quantize_group(tx[256 * g:256 * (g + 1)], qmax) for g in range(len(tx) // 256)]
    return tx, groups


def projection_columns(codes, sbits, obits, groups, columns):
    """Output columns `columns` of one route: ascending groups, value = value +
    (product + correction) with scaled_dot = sa*dot, scaled_sum = sa*sum,
    product = sw*scaled_dot, correction = off*scaled_sum (:152-157).  The
    group dot is sudot8(code, lo unsigned) + 16 * sudot8(code, hi signed)
    (:146-149), formed for all columns at once in int64 (exact)."""
    cols = list(columns)
    dots = []
    for g, (_, _, _, lo, hi, _) in enumerate(groups):
        c = np.asarray(codes[cols, 256 * g:256 * (g + 1)], np.int64)
        dots.append(c @ np.asarray(lo, np.int64) + 16 * (c @ np.asarray(hi, np.int64)))
    out = []
    for i, n in enumerate(cols):
        value = F(0)
        for g, (_, sa_bits, total, _, _, _) in enumerate(groups):
            sa = f16_f32(sa_bits)
            scaled_dot = F(sa * F(int(dots[g][i])))
            scaled_sum = F(sa * F(total))
            product = F(f16_f32(sbits[n][g]) * scaled_dot)
            correction = F(f16_f32(obits[n][g]) * scaled_sum)
            value = F(value + F(product + correction))
        out.append(value)
    return out


def shared_slot_token(x_bits, ids, weights, experts, down_experts, shared_up, shared_down, shared_logit_bits,
                      silu_table, sigmoid_table, columns, mistake=None):
    """One token of the shared-expert-as-ninth-slot decode
    (routed_storage_n32_consumer.cpp:187-307): returns, for the requested
    output columns, (routed bf16 bits, routed fp32 sum, shared bf16 bits).
    experts[e] / down_experts[e] / shared_*: (codes uint8 [N,K], scale bits
    [N,G], offset bits [N,G]).
    mistake: 'no_gate_round' (shared gate/up outputs not rounded to bf16),
    'silu_unrounded_index' (SiLU table indexed by the unrounded gate bits),
    'no_down_round' (shared down output gated before its bf16 rounding),
    'reverse_slots' (slot sum in descending slot order)."""
    row = [bf16_f32(b) for b in x_bits]
    _, xg = transform_quantize(row)
    slots = [(s, int(ids[s])) for s in range(TOP)] + [(TOP, -2)]         # -2: the shared slot
    middles = []
    for s, e in slots:
        shared = s == TOP
        if not shared and not 0 <= e < E:
            middles.append([F(0)] * I)       # invalid route: Mode 1 writes zeros
            continue
        codes, sb, ob = shared_up if shared else experts[e]
        gate_y = []
        for v in projection_columns(codes, sb, ob, xg, range(2 * I)):
            raw = v
            if shared and mistake != 'no_gate_round':
                v = bf16_f32(bf16_rne(v))
            gate_y.append((v, raw))
        mid = []
        for c in range(I):
            (g, g_raw), (up, _) = gate_y[c], gate_y[I + c]
            if shared:
                index_of = g_raw if mistake == 'silu_unrounded_index' else g
                silu = F(silu_table[int(np.float32(index_of).view(np.uint32)) >> 16])
                value = F(silu * up)
                value = bf16_f32(bf16_rne(value))
            else:
                silu = F(g / F(F(1) + portable_exp(F(-g))))
                value = F(silu * up)
            mid.append(value)
        middles.append(mid)
    route_out = {}
    for (s, e), mid in zip(slots, middles):
        shared = s == TOP
        if not shared and not 0 <= e < E:
            continue
        _, mg = transform_quantize(mid)
        codes, sb, ob = shared_down if shared else down_experts[e]
        out = {}
        for n, v in zip(columns, projection_columns(codes, sb, ob, mg, columns)):
            if shared and mistake != 'no_down_round':
                v = bf16_f32(bf16_rne(v))
            out[n] = v
        route_out[s] = out
    order = range(TOP - 1, -1, -1) if mistake == 'reverse_slots' else range(TOP)
    gate = bf16_f32(sigmoid_table[int(shared_logit_bits)])
    result = []
    for n in columns:
        total = F(0)
        for s in order:
            if 0 <= int(ids[s]) < E:
                total = F(total + F(route_out[s][n] * F(weights[s])))
        shared_value = F(route_out[TOP][n] * gate)
        result.append((bf16_rne(total), total, bf16_rne(shared_value)))
    return result


def reduce_slots(route_out, weights, ids, T, mistake=None):
    """routed_storage_n32_consumer.cpp:176-184: per (token, column) a
    sequential fp32 sum over valid slots 0..7 of route_out * weight."""
    Hc = route_out.shape[1]
    out = np.zeros((T, Hc), np.float32)
    order = range(TOP - 1, -1, -1) if mistake == 'reverse_slots' else range(TOP)
    for t in range(T):
        for c in range(Hc):
            total = F(0)
            for s in order:
                r = t * TOP + s
                if 0 <= int(ids[r]) < E:
                    total = F(total + F(route_out[r, c] * F(weights[r])))
            out[t, c] = total
    return out


def head_w8_row(x_bits, w_i8, w_scale_bits, mistake=None):
    """W8 G128 head for one row (head_i8_tile_consumer.cpp:30-106): H128,
    encode_a8 per 128 group (32 lanes x 4 values), then per column
    scaled = sa*dot, term = sw*scaled, value = value + term, groups 0..15.
    mistake: 'swap_scales' (sw multiplied first), 'descending' (groups 15..0).
    Returns (fp32 values, bf16 bits)."""
    row = [bf16_f32(b) for b in x_bits]
    tx = []
    for b in range(16):
        tx += h128_block(row[128 * b:128 * (b + 1)])
    enc = []
    for g in range(16):
        vals = tx[128 * g:128 * (g + 1)]
        maximum = F(0)
        clean = []
        for v in vals:
            v = v if np.isfinite(v) else F(0)
            clean.append(v)
            maximum = max(maximum, F(abs(v)))
        raw = F(maximum / F(127))
        valid = bool(np.isfinite(raw)) and raw <= F(65504)
        scale = np.float16(F(1) if maximum == F(0) or not valid else max(raw, F(2.0 ** -14)))
        sf = F(scale)
        q = []
        for v in clean:
            t = 0 if maximum == F(0) or not valid else int(np.rint(F(v / sf)))
            q.append(-127 if t < -127 else (127 if t > 127 else t))
        enc.append((q, sf))
    values, bits = [], []
    groups = range(15, -1, -1) if mistake == 'descending' else range(16)
    for n in range(w_i8.shape[0]):
        value = F(0)
        for g in groups:
            q, sa = enc[g]
            dot = int(np.asarray(w_i8[n, 128 * g:128 * (g + 1)], np.int64) @ np.asarray(q, np.int64))
            sw = f16_f32(w_scale_bits[n, g])
            if mistake == 'swap_scales':
                term = F(sa * F(sw * F(dot)))
            else:
                scaled = F(sa * F(dot))
                term = F(sw * scaled)
            value = F(value + term)
        values.append(value)
        bits.append(bf16_rne(value))
    return np.array(values, np.float32), np.array(bits, np.uint16)


def fixed8_row(x_bits, up_bank, down_bank, gate_w_bits, silu_table, sigmoid_table, columns, mistake=None):
    """Production shared expert of one row (iu4_correctness/shared_kernel.py:
    33-62) for the requested output columns: dense A8 gate/up with bf16
    outputs, act = bf16(bf16(silu) * up) (vLLM silu_and_mul), dense A8 down
    (bf16), scalar gate = bf16(fp32 row dot), out = bf16(sigmoid_bf16 * down).
    mistake: 'no_silu_round' (SiLU kept in fp32, as the fused ninth slot does),
    'fp32_gate' (sigmoid applied to the unrounded fp32 logit's bf16 truncation)."""
    row = [bf16_f32(b) for b in x_bits]
    _, xg = transform_quantize(row)
    codes, sb, ob = up_bank
    gu = [bf16_rne(v) for v in projection_columns(codes, sb, ob, xg, range(2 * I))]
    act = []
    for c in range(I):
        silu = F(silu_table[gu[c]])
        if mistake != 'no_silu_round':
            silu = bf16_f32(bf16_rne(silu))
        act.append(bf16_rne(F(silu * bf16_f32(gu[I + c]))))
    _, ag = transform_quantize([bf16_f32(a) for a in act])
    codes, sb, ob = down_bank
    down = [bf16_rne(v) for v in projection_columns(codes, sb, ob, ag, columns)]
    # scalar gate: lane partials over k = 8c..8c+7, c = lane + 64 i, then the xor butterfly
    lanes = []
    for lane in range(64):
        acc = F(0)
        for i in range(4):
            for j in range(8):
                k = (64 * i + lane) * 8 + j
                acc = F(np.float64(acc) + np.float64(row[k]) * np.float64(bf16_f32(gate_w_bits[k])))
        lanes.append(acc)
    lanes = np.array(lanes, np.float32)
    for off in (1, 2, 4, 8, 16, 32):
        lanes = (lanes + lanes[np.arange(64) ^ off]).astype(np.float32)
    logit_bits = bf16_rne(lanes[0])
    if mistake == 'fp32_gate':
        logit_bits = int(np.float32(lanes[0]).view(np.uint32)) >> 16
    gate = bf16_f32(sigmoid_table[logit_bits])
    return [bf16_rne(F(gate * bf16_f32(d))) for d in down]
