"""Pins the CPU oracle against the golden data the reference ships, closed
forms, brute force and planted mistakes.  CPU only."""
import math

import numpy as np
import pytest

from _ornith import Bank, SHARED_TABLE_SHA256, bf16_normal, load_shared_tables, random_routing
from oracle import ornith_oracle as O


# ---------------------------------------------------------------------------
# bf16 / fp16 conversions: exhaustive against torch
# ---------------------------------------------------------------------------
def test_bf16_round_trip_and_rne_against_torch():
    import torch
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = O.bf16_to_f32(bits)
    tf = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(f.view(np.uint32), tf.view(np.uint32))
    rng = np.random.default_rng(0)
    v = rng.standard_normal(200_000).astype(np.float32) * np.float32(10) ** rng.integers(-30, 30, 200_000).astype(np.float32)
    v = np.concatenate([v, f[np.isfinite(f)], (f[np.isfinite(f)] * np.float32(1.0000001)).astype(np.float32)])
    mine = O.f32_to_bf16(v)
    ref = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(mine, ref)
    # NaN rule of the reference (routed_storage_n32_consumer.cpp:19): quiet bit set, payload kept
    nan = np.array([0x7F800001, 0xFF812345], dtype=np.uint32).view(np.float32)
    assert list(O.f32_to_bf16(nan)) == [0x7FC0, 0xFFC1]


def test_fp16_conversion_against_torch():
    import torch
    rng = np.random.default_rng(1)
    v = np.concatenate([rng.uniform(0.005, 0.02, 100_000), rng.uniform(2 ** -16, 2 ** -13, 10_000),
                        rng.uniform(-70000, 70000, 10_000)]).astype(np.float32)
    np.testing.assert_array_equal(O.f32_to_f16_bits(v), torch.from_numpy(v).half().view(torch.int16).numpy().view(np.uint16))


# ---------------------------------------------------------------------------
# H128: closed form (Sylvester Hadamard) and invariants
# ---------------------------------------------------------------------------
def _sylvester(n):
    h = np.array([[1.0]])
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


def test_h128_matches_sylvester_closed_form():
    H = _sylvester(128)
    rng = np.random.default_rng(2)
    x = rng.standard_normal((64, 256)).astype(np.float32)
    got = O.h128(x).astype(np.float64)
    ref = (x.astype(np.float64).reshape(64, 2, 128) @ H.T / math.sqrt(128)).reshape(64, 256)
    assert np.max(np.abs(got - ref)) < 1e-5 * np.max(np.abs(ref))
    # unit vectors: exact +-1/sqrt(128) entries in natural (Sylvester) order
    e = np.eye(128, dtype=np.float32)
    np.testing.assert_array_equal(O.h128(e), (H.T * O.INV_SQRT128).astype(np.float32))
    # involution up to rounding: H H = 128 I
    back = O.h128(O.h128(x))
    assert np.max(np.abs(back - x)) < 1e-5 * np.max(np.abs(x))


def test_h128_planted_mistake_fails():
    """A butterfly with reversed subtraction order (src[hi]-src[lo]) is caught."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, 128)).astype(np.float32)
    v = x.copy()
    step = 1
    while step < 128:
        w = v.reshape(4, 128 // (2 * step), 2, step)
        v = np.stack([w[:, :, 0] + w[:, :, 1], w[:, :, 1] - w[:, :, 0]], axis=2).reshape(4, 128)
        step *= 2
    assert not np.array_equal((v * O.INV_SQRT128).astype(np.float32), O.h128(x))


# ---------------------------------------------------------------------------
# Group quantisation: brute force in Python floats, special cases
# ---------------------------------------------------------------------------
def _quant_brute(vals, qmax):
    vals = [float(np.float32(v)) if math.isfinite(v) else 0.0 for v in vals]
    absmax = max(abs(v) for v in vals)
    raw = float(np.float32(absmax) / np.float32(qmax))
    valid = math.isfinite(raw) and raw <= 65504
    zero = absmax == 0 or not valid
    scale = float(np.float16(np.float32(1.0 if zero else max(raw, 2.0 ** -14))))
    q = []
    for v in vals:
        t = 0 if zero else int(np.rint(np.float32(v) / np.float32(scale)))
        q.append(max(-qmax, min(qmax, t)))
    return q, scale


@pytest.mark.parametrize('qmax', [127, 7])
def test_quantize_brute_force(qmax):
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((6, 512)) * rng.uniform(1e-3, 100, (6, 1))).astype(np.float32)
    x[2, :256] = 0
    x[3, 5] = np.nan
    x[4, 300] = np.inf
    q, sb, sums, flags = O.quantize(x, qmax)
    for r in range(6):
        for g in range(2):
            bq, bs = _quant_brute(x[r, 256 * g:256 * (g + 1)], qmax)
            assert list(q[r, 256 * g:256 * (g + 1)]) == bq
            assert float(O.f16_bits_to_f32(sb[r, g])) == bs
            assert sums[r, g] == sum(bq)
    assert flags == O.FLAG_INVALID_ACTIVATION
    assert sb[2, 0] == 0x3C00 and not q[2, :256].any()       # zero group: scale 1, codes 0


def test_quantize_overflow_scale_is_invalid():
    x = np.full((1, 256), 3e38, dtype=np.float32)     # absmax/127 > 65504 -> invalid, scale 1, q 0
    q, sb, sums, flags = O.quantize(x, 127)
    assert flags == O.FLAG_INVALID_ACTIVATION and sb[0, 0] == 0x3C00 and not q.any()


def test_pack_planes_round_trip():
    rng = np.random.default_rng(5)
    q = rng.integers(-127, 128, size=(3, 256))
    low, high = O.pack_planes(q)
    lo = (low[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 15
    hi = (high[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 15
    hi = np.where(hi >= 8, hi.astype(np.int64) - 16, hi)
    np.testing.assert_array_equal((lo + 16 * hi).reshape(3, 256), q)


# ---------------------------------------------------------------------------
# Storage layouts (dense_g256_api.h:25-27, method.py:143-147)
# ---------------------------------------------------------------------------
def test_tile_layout_index_formula():
    rng = np.random.default_rng(6)
    N, K = 64, 512
    codes = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    for tile in (16, 32):
        bank = O.to_tile_layout(codes, tile).reshape(-1)
        for n, k in [(0, 0), (5, 9), (17, 255), (33, 256), (63, 511)]:
            g, j, d = k // 256, (k % 256) // 8, k % 8
            word = bank[((n // tile * (K // 256) + g) * 32 + j) * tile + n % tile]
            assert (word >> (4 * d)) & 15 == codes[n, k]
        np.testing.assert_array_equal(O.from_tile_layout(O.to_tile_layout(codes, tile)), codes)


def test_n16_to_n32_repack_equals_direct_n32():
    rng = np.random.default_rng(7)
    N, K = 96, 512
    codes = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    sb = rng.integers(0, 2 ** 16, size=(N, K // 256), dtype=np.uint16)
    ob = rng.integers(0, 2 ** 16, size=(N, K // 256), dtype=np.uint16)
    c32, m32 = O.n16_to_n32(O.to_tile_layout(codes, 16), O.pack_meta(sb, ob, 16))
    np.testing.assert_array_equal(c32, O.to_tile_layout(codes, 32))
    np.testing.assert_array_equal(m32, O.pack_meta(sb, ob, 32))


def _w8_tile_word(n, kword, K=2048):
    """The W8 head's physical word index, head_i8_tile_consumer.cpp:19-21:
    words [N/16, K/16, 4, 16]; word kword of column n packs K bytes
    4*kword..4*kword+3, the lowest K byte in the lowest byte
    (head_i8_tile_api.h:1)."""
    return ((n // 16 * (K // 16) + kword // 4) * 4 + (kword & 3)) * 16 + (n & 15)


def _w8_layout_transposed(w_i8):
    """Planted mistake: the two inner axes of the tile swapped
    ([N/16, K/16, 16, 4] instead of [N/16, K/16, 4, 16])."""
    good = O.head_w8_tile_layout(w_i8)
    return np.ascontiguousarray(good.reshape(-1, 128, 4, 16).transpose(0, 1, 3, 2))


def _w8_layout_high_first(w_i8):
    """Planted mistake: bytes packed with the highest K byte first."""
    good = O.head_w8_tile_layout(w_i8)
    return good.byteswap()


def _check_w8_layout(words, w_i8):
    N, K = w_i8.shape
    flat = words.reshape(-1)
    wb = w_i8.view(np.uint8)
    for n in range(N):
        for kword in range(K // 4):
            word = int(flat[_w8_tile_word(n, kword, K)])
            for b in range(4):
                if (word >> (8 * b)) & 0xFF != wb[n, 4 * kword + b]:
                    return False
    return True


def test_w8_head_tile_layout_matches_reference_index():
    rng = np.random.default_rng(61)
    N, K = 48, 2048
    w = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    words = O.head_w8_tile_layout(w)
    assert words.shape == (N // 16, K // 16, 4, 16) and words.dtype == np.uint32
    assert _check_w8_layout(words, w)
    # Every byte of the bank is covered exactly once by the reference index.
    idx = {_w8_tile_word(n, kw, K) for n in range(N) for kw in range(K // 4)}
    assert len(idx) == words.size and min(idx) == 0 and max(idx) == words.size - 1
    # Planted mistakes must fail the same check.
    assert not _check_w8_layout(_w8_layout_transposed(w), w)
    assert not _check_w8_layout(_w8_layout_high_first(w), w)


def test_signed_int4_maps_to_affine_exactly():
    rng = np.random.default_rng(8)
    q4 = rng.integers(-8, 8, size=(32, 256))
    scale = rng.uniform(0.005, 0.02, size=(32, 1)).astype(np.float32)
    code, sb, ob = O.signed_to_affine(q4, scale)
    s = O.f16_bits_to_f32(sb).astype(np.float64)
    o = O.f16_bits_to_f32(ob).astype(np.float64)
    np.testing.assert_array_equal(s * code + o, s * q4)      # offset = -8 * scale exactly


# ---------------------------------------------------------------------------
# Integer dots and the fp32 tree: brute force; planted mistakes fail
# ---------------------------------------------------------------------------
def _tree_brute(q, codes, sb, sums, wsb, wob):
    M, K = q.shape
    N = codes.shape[0]
    out = np.zeros((M, N), np.float32)
    for m in range(M):
        for n in range(N):
            acc = np.float32(0)
            for g in range(K // 256):
                dot = sum(int(q[m, k]) * int(codes[n, k]) for k in range(256 * g, 256 * (g + 1)))
                sa = O.f16_bits_to_f32(sb[m, g])
                sw, off = O.f16_bits_to_f32(wsb[n, g]), O.f16_bits_to_f32(wob[n, g])
                term = np.float32(sw * np.float32(sa * np.float32(dot))) + np.float32(off * np.float32(sa * np.float32(sums[m, g])))
                acc = np.float32(acc + np.float32(term))
            out[m, n] = acc
    return out


def test_group_dots_and_tree_brute_force():
    rng = np.random.default_rng(9)
    bank = Bank(rng, 0, 32, 512)
    codes, wsb, wob = bank.expert()
    x = rng.standard_normal((2, 512)).astype(np.float32)
    q, sb, sums, _ = O.quantize(x)
    got = O.tree(O.group_dots(q, codes[:5]), sb, sums, wsb[:5], wob[:5])
    np.testing.assert_array_equal(got.view(np.uint32), _tree_brute(q, codes[:5], sb, sums, wsb[:5], wob[:5]).view(np.uint32))


def test_tree_planted_mistakes_fail():
    rng = np.random.default_rng(10)
    bank = Bank(rng, 0, 32, 512)
    codes, wsb, wob = bank.expert()
    x = rng.standard_normal((3, 512)).astype(np.float32)
    q, sb, sums, _ = O.quantize(x)
    good = O.tree(O.group_dots(q, codes), sb, sums, wsb, wob)
    # dropped offset term
    assert not np.array_equal(good, O.tree(O.group_dots(q, codes), sb, sums, wsb, np.zeros_like(wob)))
    # transposed scale/offset roles
    assert not np.array_equal(good, O.tree(O.group_dots(q, codes), sb, sums, wob, wsb))
    # signed codes (q4 = code - 8) instead of unsigned
    assert not np.array_equal(good, O.tree(O.group_dots(q, codes.astype(np.int64) - 8), sb, sums, wsb, wob))
    # the tree against fp64 dequant-matmul: close (the quantized path is an approximation of it)
    w = O.f16_bits_to_f32(np.repeat(wsb, 256, 1)).astype(np.float64) * codes + O.f16_bits_to_f32(np.repeat(wob, 256, 1))
    exact = x.astype(np.float64) @ w.T       # the tree consumed quantized x itself
    assert np.corrcoef(good.ravel(), exact.ravel())[0, 1] > 0.999


def test_dense_a8_against_fp64_dequant():
    rng = np.random.default_rng(11)
    bank = Bank(rng, 0, 64, 2048, tile=16)
    codes, wsb, wob = bank.expert()
    x = bf16_normal(rng, (3, 2048))
    out, diag, flags = O.dense_a8(x, codes, wsb, wob)
    w = O.f16_bits_to_f32(np.repeat(wsb, 256, 1)).astype(np.float64) * codes + O.f16_bits_to_f32(np.repeat(wob, 256, 1))
    exact = O.h128(O.bf16_to_f32(x)).astype(np.float64) @ w.T
    rel = np.abs(diag - exact).max() / np.abs(exact).max()
    assert flags == 0 and rel < 2e-2
    np.testing.assert_array_equal(out, O.f32_to_bf16(diag))


def test_dequantize_bf16_closed_form():
    rng = np.random.default_rng(12)
    bank = Bank(rng, 0, 32, 256)
    codes, wsb, wob = bank.expert()
    got = O.bf16_to_f32(O.dequantize_bf16(codes, wsb, wob)).astype(np.float64)
    ref = O.f16_bits_to_f32(np.repeat(wsb, 256, 1)).astype(np.float64) * codes + O.f16_bits_to_f32(np.repeat(wob, 256, 1))
    assert np.max(np.abs(got - ref) / np.maximum(np.abs(ref), 1e-6)) <= 2 ** -8


# ---------------------------------------------------------------------------
# portable exp (portable_exp.h:6-26) and the shared golden tables
# ---------------------------------------------------------------------------
def test_portable_exp_known_answers_and_accuracy():
    assert O.portable_exp(np.float32(0)) == 1.0
    assert O.portable_exp(np.float32(-104)) == 0.0 and O.portable_exp(np.float32(-200)) == 0.0
    assert np.isinf(O.portable_exp(np.float32(89))) and np.isnan(O.portable_exp(np.float32(np.nan)))
    x = np.linspace(-80, 80, 100_001).astype(np.float32)
    got = O.portable_exp(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert np.max(np.abs(got - ref) / ulp) < 4


def test_shared_table_sha256_and_semantics(shared_tables):
    silu, sigmoid = shared_tables
    import hashlib
    from _ornith import SHARED_TABLE
    assert hashlib.sha256(SHARED_TABLE.read_bytes()).hexdigest() == SHARED_TABLE_SHA256
    g = O.bf16_to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16)).astype(np.float64)
    fin = np.isfinite(g)
    with np.errstate(over='ignore', invalid='ignore'):
        ref_silu = g / (1 + np.exp(-g))
        ref_sig = 1 / (1 + np.exp(-g))
    err = np.abs(silu[fin] - ref_silu[fin]) / np.maximum(np.abs(ref_silu[fin]), 1e-30)
    assert np.nanmax(np.where(np.abs(g[fin]) < 80, err, 0)) < 1e-5
    s = O.bf16_to_f32(sigmoid)[fin].astype(np.float64)
    assert np.max(np.abs(s - ref_sig[fin])) <= 2 ** -8
    # the portable SiLU of the routed path agrees with the table to a few ulp
    mid = fin & (np.abs(g) < 40)
    ps = O.silu_portable(g[mid].astype(np.float32)).astype(np.float64)
    assert np.max(np.abs(ps - silu[mid]) / np.maximum(np.abs(silu[mid]), 1e-30)) < 1e-5


# ---------------------------------------------------------------------------
# Router, top-k, permute
# ---------------------------------------------------------------------------
def test_router_logits_declared_order_vs_fp64():
    rng = np.random.default_rng(13)
    x = bf16_normal(rng, (5, 2048))
    w = bf16_normal(rng, (257, 2048), 0.02)
    got = O.router_logits(x, w).astype(np.float64)
    ref = O.bf16_to_f32(x).astype(np.float64) @ O.bf16_to_f32(w).astype(np.float64).T
    assert np.max(np.abs(got - ref)) < 1e-5
    # brute force of the declared order on one (t, e): 64 lane partials, xor butterfly
    xf, wf = O.bf16_to_f32(x[2]), O.bf16_to_f32(w[100])
    lanes = []
    for lane in range(64):
        acc = np.float32(0)
        for i in range(4):
            for j in range(8):
                k = (64 * i + lane) * 8 + j
                acc = np.float32(np.float64(acc) + np.float64(xf[k]) * np.float64(wf[k]))
        lanes.append(acc)
    lanes = np.array(lanes, np.float32)
    for off in (1, 2, 4, 8, 16, 32):
        lanes = (lanes + lanes[np.arange(64) ^ off]).astype(np.float32)
    assert lanes[0].view(np.uint32) == got.astype(np.float32)[2, 100].view(np.uint32)


def test_softmax_topk_brute_force():
    rng = np.random.default_rng(14)
    logits = rng.standard_normal((20, 256)).astype(np.float32)
    logits[3, 10] = logits[3, 200] = 9.0        # exact tie: lower id first
    w, ids, p = O.softmax_topk(logits)
    for t in range(20):
        order = sorted(range(256), key=lambda e: (-float(p[t, e]), e))[:8]
        assert list(ids[t]) == order
        tot = np.float32(0)
        for e in order:
            tot = np.float32(tot + p[t, e])
        np.testing.assert_array_equal(w[t], (p[t, order] / tot).astype(np.float32))
    assert list(ids[3, :2]) == [10, 200]
    # matches an fp64 softmax closely and selects the same set
    ref = np.exp(logits.astype(np.float64) - logits.max(1, keepdims=True))
    ref /= ref.sum(1, keepdims=True)
    assert np.max(np.abs(p - ref)) < 1e-6


def test_permute_counts_offsets_stable_order():
    rng = np.random.default_rng(15)
    _, ids = random_routing(rng, 50)
    ids[3, 2] = -1
    ids[7, 0] = 999
    counts, offsets, routes = O.permute(ids)
    flat = ids.reshape(-1)
    valid = (flat >= 0) & (flat < 256)
    np.testing.assert_array_equal(counts, np.bincount(flat[valid], minlength=256))
    assert offsets[-1] == valid.sum()
    for e in range(256):
        seg = routes[offsets[e]:offsets[e + 1]]
        assert (flat[seg] == e).all() and (np.diff(seg) > 0).all()


def test_routed_layer_a8_vs_fp64_reference():
    """The exact A8 layer stays close to fp64 dequant + matmul semantics."""
    from _ornith import moe_weights, oracle_routed
    w = moe_weights(21, E=256)
    rng = np.random.default_rng(16)
    x = bf16_normal(rng, (2, 2048))
    rw, ids = random_routing(rng, 2)
    r = oracle_routed(x, rw, ids, w['w13'], w['w2'])
    assert r['flags'] == 0
    # fp64 reference
    xt = O.h128(O.bf16_to_f32(x)).astype(np.float64)
    out = np.zeros((2, 2048))
    for t in range(2):
        for s in range(8):
            e = ids[t, s]
            c13, s13, o13 = w['w13'].expert(e)
            W = O.f16_bits_to_f32(np.repeat(s13, 256, 1)).astype(np.float64) * c13 + O.f16_bits_to_f32(np.repeat(o13, 256, 1))
            gy = W @ xt[t]
            g, up = gy[:512], gy[512:]
            mid = g / (1 + np.exp(-g)) * up
            c2, s2, o2 = w['w2'].expert(e)
            W2 = O.f16_bits_to_f32(np.repeat(s2, 256, 1)).astype(np.float64) * c2 + O.f16_bits_to_f32(np.repeat(o2, 256, 1))
            H = _sylvester(128) / math.sqrt(128)
            mt = (mid.reshape(4, 128) @ H.T).reshape(512)
            out[t] += rw[t, s] * (W2 @ mt)
    cos = (r['final'].ravel() @ out.ravel()) / np.linalg.norm(r['final']) / np.linalg.norm(out)
    assert cos > 0.999
