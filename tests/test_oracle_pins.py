"""Pins of the oracle functions that the reference's golden table and the
closed-form checks in test_oracle.py leave open: each is compared bit for
bit with a scalar, statement-by-statement restatement of the reference
kernel (tests/_transcribe.py), and each check comes with planted mistakes
that must fail it.  CPU only."""
import numpy as np
import pytest

import _transcribe as S
from _ornith import Bank, bf16_normal
from oracle import ornith_oracle as O


# ---------------------------------------------------------------------------
# H128: the exact butterfly order (routed_storage_n32_consumer.cpp:34-41)
# ---------------------------------------------------------------------------
def _wide_range_rows(rng, rows):
    """Values spanning many binades, so that rounding order shows in the bits."""
    mant = rng.standard_normal((rows, 128))
    return (mant * np.float64(2.0) ** rng.integers(-12, 12, (rows, 128))).astype(np.float32)


def test_h128_equals_lane_transcription_and_order_is_pinned():
    rng = np.random.default_rng(100)
    x = _wide_range_rows(rng, 24)
    got = O.h128(x)
    for r in range(x.shape[0]):
        ref = np.array(S.h128_block(x[r]), np.float32)
        np.testing.assert_array_equal(got[r].view(np.uint32), ref.view(np.uint32))
    # the same butterflies in descending step order give the same matrix but
    # other roundings: the oracle must not agree with it
    differs = sum(not np.array_equal(got[r].view(np.uint32),
                                     np.array(S.h128_block(x[r], 'descending'), np.float32).view(np.uint32))
                  for r in range(x.shape[0]))
    assert differs > 0


def test_h128_planted_descending_order_in_the_oracle_fails():
    rng = np.random.default_rng(101)
    x = _wide_range_rows(rng, 8)

    def h128_descending(v):
        v = v.copy()
        for step in (64, 32, 16, 8, 4, 2, 1):
            w = v.reshape(v.shape[0], 128 // (2 * step), 2, step)
            v = np.stack([w[:, :, 0] + w[:, :, 1], w[:, :, 0] - w[:, :, 1]], axis=2).reshape(v.shape[0], 128)
        return (v * O.INV_SQRT128).astype(np.float32)

    planted = h128_descending(x)
    ref = np.stack([np.array(S.h128_block(r), np.float32) for r in x])
    assert not np.array_equal(planted.view(np.uint32), ref.view(np.uint32))


# ---------------------------------------------------------------------------
# quantize: lane transcription incl. nibble planes (:44-76)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize('qmax', [127, 7])
def test_quantize_equals_transcription(qmax):
    rng = np.random.default_rng(102)
    x = (rng.standard_normal((4, 512)) * np.float64(2.0) ** rng.integers(-20, 20, (4, 1))).astype(np.float32)
    x[1, 7] = np.nan
    q, sb, sums, flags = O.quantize(x, qmax)
    for r in range(4):
        for g in range(2):
            tq, tsb, tsum, lo, hi, tf = S.quantize_group(x[r, 256 * g:256 * (g + 1)], qmax)
            assert list(q[r, 256 * g:256 * (g + 1)]) == tq and sb[r, g] == tsb and sums[r, g] == tsum
            assert all(l + 16 * h == v for l, h, v in zip(lo, hi, tq))
    assert flags == O.FLAG_INVALID_ACTIVATION


# ---------------------------------------------------------------------------
# routed_layer_shared: one token against the scalar transcription of
# routed_storage_n32_consumer.cpp:187-307
# ---------------------------------------------------------------------------
@pytest.fixture(scope='module')
def shared_case(shared_tables):
    silu, sigmoid = shared_tables
    rng = np.random.default_rng(103)
    E = 12                               # experts 0..11 are enough for one token
    w13, w2 = Bank(rng, E, 1024, 2048), Bank(rng, E, 2048, 512)
    s13, s2 = Bank(rng, 0, 1024, 2048), Bank(rng, 0, 2048, 512)
    x = bf16_normal(rng, (1, 2048))
    ids = np.array([[3, 11, 0, -1, 7, 3, 5, 9]], np.int32)       # a padding slot and a repeated expert
    rw = rng.uniform(0.05, 1.0, (1, 8)).astype(np.float32)
    rw = (rw / rw.sum()).astype(np.float32)
    logit = O.f32_to_bf16(np.array([0.37], np.float32))
    up = {e: w13.expert(e) for e in range(E)}
    down = {e: w2.expert(e) for e in range(E)}
    ref = O.routed_layer_shared(x, rw, ids, {e: up[e][0] for e in up}, w13.sbits, w13.obits,
                                {e: down[e][0] for e in down}, w2.sbits, w2.obits, *s13.expert(), *s2.expert(),
                                logit, silu, sigmoid)
    columns = list(range(0, 2048, 97))[:20] + [2047]
    args = (x[0], ids[0], rw[0], up, down, s13.expert(), s2.expert(), logit[0], silu, sigmoid, columns)
    return ref, args, columns


def _compare(ref, rows, columns):
    out = np.array([r[0] for r in rows], np.uint16)
    final = np.array([r[1] for r in rows], np.float32)
    shared = np.array([r[2] for r in rows], np.uint16)
    return (np.array_equal(out, ref['out'][0, columns]) and
            np.array_equal(final.view(np.uint32), ref['final'][0, columns].view(np.uint32)) and
            np.array_equal(shared, ref['shared_out'][0, columns]))


def test_routed_layer_shared_equals_transcription(shared_case):
    ref, args, columns = shared_case
    assert ref['flags'] == 0
    assert _compare(ref, S.shared_slot_token(*args), columns)


@pytest.mark.parametrize('mistake', ['no_gate_round', 'silu_unrounded_index', 'no_down_round', 'reverse_slots'])
def test_routed_layer_shared_planted_mistakes_fail(shared_case, mistake):
    ref, args, columns = shared_case
    assert not _compare(ref, S.shared_slot_token(*args, mistake=mistake), columns)


# ---------------------------------------------------------------------------
# reduce_slots: sequential slot order (:176-184)
# ---------------------------------------------------------------------------
def test_reduce_slots_equals_sequential_loop_and_order_is_pinned():
    rng = np.random.default_rng(104)
    T = 6
    ro = (rng.standard_normal((T * 8, 64)) * np.float64(2.0) ** rng.integers(-10, 10, (T * 8, 1))).astype(np.float32)
    w = rng.uniform(0.01, 1.0, T * 8).astype(np.float32)
    ids = rng.integers(0, 256, T * 8).astype(np.int32)
    ids[[3, 17, 30]] = [-1, 300, -7]                              # skipped (padding) and invalid slots
    final, out, _ = O.reduce_slots(ro, w, ids, T)
    seq = S.reduce_slots(ro, w, ids, T)
    np.testing.assert_array_equal(final.view(np.uint32), seq.view(np.uint32))
    np.testing.assert_array_equal(out, O.f32_to_bf16(seq))
    rev = S.reduce_slots(ro, w, ids, T, mistake='reverse_slots')
    assert not np.array_equal(final.view(np.uint32), rev.view(np.uint32))


# ---------------------------------------------------------------------------
# add_bf16 (the MoE runner's routed + shared sum) against torch CPU bf16
# ---------------------------------------------------------------------------
def test_add_bf16_equals_torch_cpu():
    import torch
    rng = np.random.default_rng(105)
    n = 1 << 20
    a = rng.integers(0, 1 << 16, n, dtype=np.uint32).astype(np.uint16)
    b = rng.integers(0, 1 << 16, n, dtype=np.uint32).astype(np.uint16)
    # plus pairs of similar magnitude (cancellation) and the special values
    c = O.f32_to_bf16(rng.standard_normal(n).astype(np.float32))
    d = O.f32_to_bf16((-O.bf16_to_f32(c) * np.float32(1.0078125)).astype(np.float32))
    special = np.array([0x0000, 0x8000, 0x7F80, 0xFF80, 0x7FC0, 0x0001, 0x7F7F, 0xFF7F], np.uint16)
    a = np.concatenate([a, c, np.repeat(special, 8)])
    b = np.concatenate([b, d, np.tile(special, 8)])
    mine = O.add_bf16(a, b)
    ta = torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)
    tb = torch.from_numpy(b.view(np.int16)).view(torch.bfloat16)
    ref = (ta + tb).view(torch.int16).numpy().view(np.uint16)
    nan = (O.bf16_to_f32(ref) != O.bf16_to_f32(ref))
    assert np.array_equal(np.isnan(O.bf16_to_f32(mine)), nan)
    np.testing.assert_array_equal(mine[~nan], ref[~nan])


# ---------------------------------------------------------------------------
# head_w8: one row against the transcription of head_i8_tile_consumer.cpp:30-106
# ---------------------------------------------------------------------------
def test_head_w8_equals_transcription_and_planted_mistakes_fail():
    rng = np.random.default_rng(106)
    N = 48
    x = bf16_normal(rng, (2, 2048))
    w = rng.integers(-127, 128, (N, 2048)).astype(np.int8)
    sbits = O.f32_to_f16_bits(rng.uniform(0.002, 0.02, (N, 16)).astype(np.float32))
    out, acc, flags = O.head_w8(x, w, sbits)
    assert flags == 0
    for r in range(2):
        vals, bits = S.head_w8_row(x[r], w, sbits)
        np.testing.assert_array_equal(acc[r].view(np.uint32), vals.view(np.uint32))
        np.testing.assert_array_equal(out[r], bits)
    for mistake in ('swap_scales', 'descending'):
        vals = np.concatenate([S.head_w8_row(x[r], w, sbits, mistake)[0] for r in range(2)])
        assert not np.array_equal(acc.reshape(-1).view(np.uint32), vals.view(np.uint32)), mistake


def test_portable_exp_equals_transcription():
    rng = np.random.default_rng(107)
    x = np.concatenate([rng.uniform(-110, 95, 4000), rng.uniform(-1, 1, 2000),
                        [0.0, -0.0, -104.0, -103.99, 88.99, 89.0, np.nan, np.inf, -np.inf]]).astype(np.float32)
    got = O.portable_exp(x)
    ref = np.array([S.portable_exp(v) for v in x], np.float32)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


# ---------------------------------------------------------------------------
# shared_fixed8: one row against the transcription of shared_kernel.py:33-62
# ---------------------------------------------------------------------------
def test_shared_fixed8_equals_transcription_and_planted_mistakes_fail(shared_tables):
    silu, sigmoid = shared_tables
    rng = np.random.default_rng(108)
    s13, s2 = Bank(rng, 0, 1024, 2048), Bank(rng, 0, 2048, 512)
    x = bf16_normal(rng, (2, 2048))
    gw = bf16_normal(rng, (2048,), 0.02)
    out, flags = O.shared_fixed8(x, *s13.expert(), *s2.expert(), gw, silu, sigmoid)
    assert flags == 0
    cols = list(range(0, 2048, 61))
    for r in range(2):
        ref = S.fixed8_row(x[r], s13.expert(), s2.expert(), gw, silu, sigmoid, cols)
        np.testing.assert_array_equal(out[r, cols], np.array(ref, np.uint16))
    for mistake in ('no_silu_round', 'fp32_gate'):
        bad = np.concatenate([S.fixed8_row(x[r], s13.expert(), s2.expert(), gw, silu, sigmoid, cols, mistake)
                              for r in range(2)]).astype(np.uint16)
        assert not np.array_equal(out[:, cols].reshape(-1), bad), mistake
