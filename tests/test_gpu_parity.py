"""GPU parity: every C-ABI entry against the CPU oracle, bit-exact.

All calls go through the C ABI (ctypes) of the built HIP library on torch's
current stream; the oracle only checks.  Shapes are the reference's real
shapes (E=256, H=2048, I=512, G=256) at token counts the oracle finishes in
seconds; larger token counts are covered by size-independent properties
(batch invariance below, and the skewed workloads in test_gpu_workloads.py).
"""
import ctypes as C

import numpy as np
import pytest

from _ornith import (Bank, LazyExperts, bf16_normal, from_dev, moe_weights, oracle_routed, random_routing,
                     to_dev)
from oracle import ornith_oracle as O

pytestmark = pytest.mark.gpu


def _native():
    from ornith_g256 import native
    return native


def _sync():
    import torch
    torch.cuda.synchronize()


def _flags(device):
    import torch
    return torch.zeros(1, dtype=torch.int32, device=device)


@pytest.fixture(scope='module')
def moe(device):
    w = moe_weights(1234)
    d = {k: (to_dev(v.codes, device), to_dev(v.meta, device)) for k, v in w.items() if isinstance(v, Bank)}
    return w, d


# ---------------------------------------------------------------------------
# Dense G256 (dense_g256_consumer.cpp:172-189; dense_n32 :360-378)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize('M,N,K,tile', [(1, 6144, 2048, 16), (1, 6144, 2048, 32), (5, 1024, 2048, 16),
                                        (16, 2048, 512, 32), (3, 48, 768, 16), (64, 1024, 4096, 16),
                                        (9, 2080, 2048, 32), (2, 128, 8192, 16), (65, 96, 512, 16),
                                        (8, 6144, 2048, 32), (8, 2080, 2048, 16), (7, 48, 768, 16),
                                        (6, 1024, 2048, 32), (33, 2080, 2048, 16)])
def test_dense_a8_bit_exact(device, M, N, K, tile):
    import torch
    native = _native()
    print(f'dense M={M} N={N} K={K} tile={tile}', flush=True)
    rng = np.random.default_rng(7 + M + N + K)
    bank = Bank(rng, 0, N, K, tile=tile)
    x = bf16_normal(rng, (M, K))
    ref_out, ref_diag, ref_flags = O.dense_a8(x, *bank.expert())
    layout = native.dense_layout(max(M, 16), N, K)
    ws = torch.empty(layout.workspace_bytes, dtype=torch.uint8, device=device)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=device)
    flags = _flags(device)
    xd, cd, md = to_dev(x, device), to_dev(bank.codes, device), to_dev(bank.meta, device)
    h = native.lib()
    fn = h.ornith_dense_g256_launch if tile == 16 else h.ornith_dense_g256_launch_n32
    st = fn(native.ptr(xd), native.ptr(cd), native.ptr(md), native.ptr(ws), ws.numel(), native.ptr(out),
            native.ptr(flags), M, max(M, 16), N, K, 8, 128, 2, native.stream(xd))
    assert st == 0
    _sync()
    np.testing.assert_array_equal(from_dev(out), ref_out)
    diag = from_dev(ws[layout.projection:layout.projection + M * N * 4].view(torch.float32)).reshape(M, N)
    np.testing.assert_array_equal(diag.view(np.uint32), ref_diag.view(np.uint32))
    assert int(flags.item()) == ref_flags


@pytest.mark.parametrize('M,N,K', [(7, 96, 512), (1120, 6144, 2048)])
def test_dense_prepare_bf16_bit_exact(device, M, N, K):
    """bf16 prefill operands; 1120 x 6144 x 2048 is the benchmark's dense
    prefill shape."""
    import torch
    native = _native()
    print(f'dense prepare M={M} N={N} K={K}', flush=True)
    rng = np.random.default_rng(99 + M)
    bank = Bank(rng, 0, N, K, tile=16)
    x = bf16_normal(rng, (M, K))
    codes, sb, ob = bank.expert()
    xd, cd, md = to_dev(x, device), to_dev(bank.codes, device), to_dev(bank.meta, device)
    tx = torch.empty((M, K), dtype=torch.bfloat16, device=device)
    wt = torch.empty((N, K), dtype=torch.bfloat16, device=device)
    flags = _flags(device)
    st = native.lib().ornith_dense_g256_prepare_bf16(native.ptr(xd), native.ptr(cd), native.ptr(md),
                                                     native.ptr(tx), native.ptr(wt), native.ptr(flags), M, N, K,
                                                     native.stream(xd))
    assert st == 0
    _sync()
    np.testing.assert_array_equal(from_dev(tx), O.transform_bf16(x))
    np.testing.assert_array_equal(from_dev(wt), O.dequantize_bf16(codes, sb, ob))
    assert int(flags.item()) == 0


@pytest.mark.parametrize('M', [2, 8, 16])
def test_dense_nonfinite_flags(device, M):
    import torch
    native = _native()
    print(f'dense nonfinite M={M}', flush=True)
    rng = np.random.default_rng(5)
    N, K = 64, 256
    bank = Bank(rng, 0, N, K, tile=32)
    x = bf16_normal(rng, (M, K))
    x[1, 17] = 0x7FC0   # NaN
    ref_out, ref_diag, ref_flags = O.dense_a8(x, *bank.expert())
    layout = native.dense_layout(16, N, K)
    ws = torch.empty(layout.workspace_bytes, dtype=torch.uint8, device=device)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=device)
    flags = _flags(device)
    xd, cd, md = to_dev(x, device), to_dev(bank.codes, device), to_dev(bank.meta, device)
    st = native.lib().ornith_dense_g256_launch_n32(native.ptr(xd), native.ptr(cd), native.ptr(md), native.ptr(ws),
                                                   ws.numel(), native.ptr(out), native.ptr(flags), M, 16, N, K, 8,
                                                   128, 2, native.stream(xd))
    assert st == 0
    _sync()
    assert ref_flags & 1 and int(flags.item()) == ref_flags
    np.testing.assert_array_equal(from_dev(out)[0], ref_out[0])


# ---------------------------------------------------------------------------
# Routed A8 / A4 (routed_storage_n32_consumer.cpp:319-370)
# ---------------------------------------------------------------------------
def _run_routed(native, device, d, x, w, ids, entry, Tcap=None):
    import torch
    T = x.shape[0]
    Tcap = Tcap or max(T, 1)
    layout = native.routed_layout(Tcap)
    ws = torch.empty(layout.workspace_bytes, dtype=torch.uint8, device=device)
    out = torch.empty((T, 2048), dtype=torch.bfloat16, device=device)
    flags = _flags(device)
    xd, wd, idd = to_dev(x, device), to_dev(w, device), to_dev(ids, device)
    fn = getattr(native.lib(), entry)
    st = fn(*[native.ptr(t) for t in (xd, wd, idd, d['w13'][0], d['w13'][1], d['w2'][0], d['w2'][1], ws)],
            ws.numel(), native.ptr(out), native.ptr(flags), T, Tcap, native.stream(xd))
    assert st == 0
    _sync()
    final = from_dev(ws[layout.final_f32:layout.final_f32 + T * 2048 * 4].view(torch.float32)).reshape(T, 2048)
    return from_dev(out), final, int(flags.item())


@pytest.mark.parametrize('T,entry,qmax', [(1, 'ornith_routed_direct_launch', 127),
                                          (4, 'ornith_routed_direct_launch', 127),
                                          (32, 'ornith_routed_direct_launch', 127),
                                          (3, 'ornith_routed_direct_launch_a4', 7),
                                          (70, 'ornith_routed_direct_launch_a4_prefill', 7),
                                          (20, 'ornith_routed_direct_launch_a4_prefill', 127),
                                          (150, 'ornith_routed_direct_launch', 127),
                                          (2, 'ornith_routed_direct_launch', 127),
                                          (33, 'ornith_routed_direct_launch', 127)])
def test_routed_bit_exact(device, moe, T, entry, qmax):
    native = _native()
    print(f'routed T={T} {entry}', flush=True)
    w, d = moe
    rng = np.random.default_rng(1000 + T)
    x = bf16_normal(rng, (T, 2048))
    rw, ids = random_routing(rng, T)
    ref = oracle_routed(x, rw, ids, w['w13'], w['w2'], qmax=qmax)
    out, final, flags = _run_routed(native, device, d, x, rw, ids, entry)
    np.testing.assert_array_equal(final.view(np.uint32), ref['final'].view(np.uint32))
    np.testing.assert_array_equal(out, ref['out'])
    assert flags == ref['flags']


@pytest.mark.parametrize('T', [5, 48])
def test_routed_padding_and_invalid_ids(device, moe, T):
    """-1 padding slots are skipped silently; out-of-range ids raise flag 4
    and contribute nothing; a token with no live slot outputs zeros.  T = 48
    runs the prefill path, whose permuted route list holds only live routes."""
    native = _native()
    print(f'routed padding/invalid T={T}', flush=True)
    w, d = moe
    rng = np.random.default_rng(77)
    x = bf16_normal(rng, (T, 2048))
    rw, ids = random_routing(rng, T)
    ids[0, 3] = -1
    ids[1, :] = -1
    ids[2, 7] = 300
    ids[4, 0] = -5
    ref = oracle_routed(x, rw, ids, w['w13'], w['w2'])
    out, final, flags = _run_routed(native, device, d, x, rw, ids, 'ornith_routed_direct_launch', Tcap=max(8, T))
    np.testing.assert_array_equal(final.view(np.uint32), ref['final'].view(np.uint32))
    np.testing.assert_array_equal(out, ref['out'])
    assert flags == ref['flags'] == 4
    assert not out[1].any()


@pytest.mark.parametrize('case', ['dup', 'pad', 'none'])
def test_routed_single_token_edge_ids(device, moe, case):
    """T == 1 runs the per-tile kernel: duplicate experts (two routes on one
    bank), -1 padding, and a token with no live slot."""
    native = _native()
    w, d = moe
    rng = np.random.default_rng(79)
    x = bf16_normal(rng, (1, 2048))
    rw, ids = random_routing(rng, 1)
    if case == 'dup':
        ids[0, 5] = ids[0, 2]
    elif case == 'pad':
        ids[0, [1, 6]] = -1
    else:
        ids[0, :] = -1
    ref = oracle_routed(x, rw, ids, w['w13'], w['w2'])
    out, final, flags = _run_routed(native, device, d, x, rw, ids, 'ornith_routed_direct_launch', Tcap=4)
    np.testing.assert_array_equal(final.view(np.uint32), ref['final'].view(np.uint32))
    np.testing.assert_array_equal(out, ref['out'])
    assert flags == ref['flags']


def test_routed_skewed_expert(device, moe):
    """Many routes on one expert (more than one route batch of a block)."""
    native = _native()
    w, d = moe
    rng = np.random.default_rng(78)
    T = 140                 # 140 routes on expert 17: three 64-route tiles
    x = bf16_normal(rng, (T, 2048))
    rw, ids = random_routing(rng, T)
    ids[:, 0] = 17          # duplicates inside a token are legal: two routes to one expert
    ref = oracle_routed(x, rw, ids, w['w13'], w['w2'])
    out, final, flags = _run_routed(native, device, d, x, rw, ids, 'ornith_routed_direct_launch')
    np.testing.assert_array_equal(final.view(np.uint32), ref['final'].view(np.uint32))
    np.testing.assert_array_equal(out, ref['out'])


# ---------------------------------------------------------------------------
# Shared expert as ninth slot (routed_storage_n32_consumer.cpp:385-401)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize('T', [1, 16])
def test_shared_tables_bit_exact(device, moe, shared_tables, T):
    import torch
    native = _native()
    w, d = moe
    silu, sigmoid = shared_tables
    rng = np.random.default_rng(2000 + T)
    x = bf16_normal(rng, (T, 2048))
    rw, ids = random_routing(rng, T)
    logit = bf16_normal(rng, (T,), 0.5)
    s13, s2 = w['s13'], w['s2']
    ref = O.routed_layer_shared(x, rw, ids, LazyExperts(w['w13']), w['w13'].sbits, w['w13'].obits,
                                LazyExperts(w['w2']), w['w2'].sbits, w['w2'].obits,
                                *s13.expert(), *s2.expert(), logit, silu, sigmoid)
    layout = native.routed_layout(16, 'shared')
    ws = torch.empty(layout.workspace_bytes, dtype=torch.uint8, device=device)
    out = torch.empty((T, 2048), dtype=torch.bfloat16, device=device)
    sh = torch.empty((T, 2048), dtype=torch.bfloat16, device=device)
    flags = _flags(device)
    xd = to_dev(x, device)
    native.routed_shared_tables(xd, to_dev(rw, device), to_dev(ids, device), d['w13'][0], d['w13'][1],
                                d['w2'][0], d['w2'][1], d['s13'][0], d['s13'][1], d['s2'][0], d['s2'][1],
                                to_dev(logit, device), to_dev(silu, device), to_dev(sigmoid, device), ws, out, sh,
                                flags, 16)
    _sync()
    np.testing.assert_array_equal(from_dev(out), ref['out'])
    np.testing.assert_array_equal(from_dev(sh), ref['shared_out'])
    assert int(flags.item()) == ref['flags']


# ---------------------------------------------------------------------------
# Router + softmax/top-8 and the whole layer
# ---------------------------------------------------------------------------
@pytest.mark.parametrize('T,biased', [(1, False), (33, False), (64, True), (256, False), (257, True), (300, True),
                                      (700, False)])
def test_router_topk_bit_exact(device, moe, T, biased):
    import torch
    native = _native()
    w, _ = moe
    rng = np.random.default_rng(3000 + T)
    x = bf16_normal(rng, (T, 2048))
    bias = (-1.1 * np.log(1 + rng.permutation(256))).astype(np.float32) if biased else None
    logits_ref = O.router_logits(x, np.concatenate([w['router'], w['gate']]), None)
    if biased:
        logits_ref[:, :256] = (logits_ref[:, :256] + bias[None, :]).astype(np.float32)
    wref, iref, _ = O.softmax_topk(logits_ref[:, :256])
    xd = to_dev(x, device)
    logits = torch.empty((T, 257), dtype=torch.float32, device=device)
    tw = torch.empty((T, 8), dtype=torch.float32, device=device)
    ti = torch.empty((T, 8), dtype=torch.int32, device=device)
    sl = torch.empty((T,), dtype=torch.bfloat16, device=device)
    native.router_topk(xd, to_dev(w['router'], device), to_dev(bias, device) if biased else None,
                       to_dev(w['gate'][0], device), logits, tw, ti, sl)
    _sync()
    np.testing.assert_array_equal(from_dev(logits).view(np.uint32), logits_ref.view(np.uint32))
    np.testing.assert_array_equal(from_dev(ti), iref)
    np.testing.assert_array_equal(from_dev(tw).view(np.uint32), wref.view(np.uint32))
    np.testing.assert_array_equal(from_dev(sl), O.f32_to_bf16(logits_ref[:, 256]))


@pytest.mark.parametrize('T', [1, 2, 32, 33, 96, 300])
def test_moe_layer_bit_exact(device, moe, shared_tables, T):
    import torch
    native = _native()
    w, d = moe
    silu, sigmoid = shared_tables
    rng = np.random.default_rng(4000 + T)
    x = bf16_normal(rng, (T, 2048))
    logits = O.router_logits(x, np.concatenate([w['router'], w['gate']]))
    rw, ids, _ = O.softmax_topk(logits[:, :256])
    logit_bf16 = O.f32_to_bf16(logits[:, 256])
    ref = O.routed_layer_shared(x, rw, ids, LazyExperts(w['w13']), w['w13'].sbits, w['w13'].obits,
                                LazyExperts(w['w2']), w['w2'].sbits, w['w2'].obits,
                                *w['s13'].expert(), *w['s2'].expert(), logit_bf16, silu, sigmoid)
    expected = O.add_bf16(ref['out'], ref['shared_out'])
    layout = native.routed_layout(T, 'layer')
    ws = torch.empty(layout.workspace_bytes, dtype=torch.uint8, device=device)
    out = torch.empty((T, 2048), dtype=torch.bfloat16, device=device)
    tw = torch.empty((T, 8), dtype=torch.float32, device=device)
    ti = torch.empty((T, 8), dtype=torch.int32, device=device)
    sl = torch.empty((T,), dtype=torch.bfloat16, device=device)
    flags = _flags(device)
    xd = to_dev(x, device)
    native.moe_layer(xd, to_dev(w['router'], device), None, to_dev(w['gate'][0], device), d['w13'][0], d['w13'][1],
                     d['w2'][0], d['w2'][1], d['s13'][0], d['s13'][1], d['s2'][0], d['s2'][1],
                     to_dev(silu, device), to_dev(sigmoid, device), ws, tw, ti, sl, out, flags, T)
    _sync()
    np.testing.assert_array_equal(from_dev(ti), ids)
    np.testing.assert_array_equal(from_dev(tw).view(np.uint32), rw.view(np.uint32))
    np.testing.assert_array_equal(from_dev(out), expected)
    assert int(flags.item()) == ref['flags']


@pytest.mark.parametrize('T', [1120, 8192])
def test_moe_layer_batch_invariance_full_size(device, moe, shared_tables, T):
    """At the benchmark sizes, where the oracle is too slow: every token's
    result is exact and depends on that token alone, so rows of a T-token
    layer equal the same rows run as a 300-token layer (prefill path, itself
    checked against the oracle), a 32-token layer (decode path) and single
    tokens (single-token path), bit for bit, ids and weights included."""
    import torch
    native = _native()
    w, d = moe
    silu, sigmoid = shared_tables
    print(f'layer batch invariance T={T}', flush=True)
    rng = np.random.default_rng(6000 + T)
    x = to_dev(bf16_normal(rng, (T, 2048)), device)
    weights = [to_dev(w['router'], device), None, to_dev(w['gate'][0], device), d['w13'][0], d['w13'][1],
               d['w2'][0], d['w2'][1], d['s13'][0], d['s13'][1], d['s2'][0], d['s2'][1], to_dev(silu, device),
               to_dev(sigmoid, device)]

    def layer(xs):
        n = xs.shape[0]
        ws = torch.empty(native.routed_layout(n, 'layer').workspace_bytes, dtype=torch.uint8, device=device)
        out = torch.empty((n, 2048), dtype=torch.bfloat16, device=device)
        tw = torch.empty((n, 8), dtype=torch.float32, device=device)
        ti = torch.empty((n, 8), dtype=torch.int32, device=device)
        sl = torch.empty((n,), dtype=torch.bfloat16, device=device)
        flags = _flags(device)
        native.moe_layer(xs.contiguous(), *weights, ws, tw, ti, sl, out, flags, n)
        _sync()
        assert int(flags.item()) == 0
        return out, ti, tw, sl

    full = layer(x)
    for lo, hi in [(0, 300), (T - 300, T), (T // 2, T // 2 + 32), (T - 1, T), (T // 3, T // 3 + 1)]:
        part = layer(x[lo:hi])
        for a, b in zip(part, full):
            assert torch.equal(a.view(torch.uint8), b[lo:hi].contiguous().view(torch.uint8)), (lo, hi)


@pytest.mark.parametrize('T', [1, 32, 300])
def test_moe_layer_graph_replays(device, moe, shared_tables, T):
    """The layer captured in a HIP graph (the bench's timed path): three
    replays on new inputs, with eager layer calls and synchronisations in
    between, each bit-identical to an eager call on the same input."""
    import torch
    native = _native()
    w, d = moe
    silu, sigmoid = shared_tables
    print(f'layer graph replays T={T}', flush=True)
    rng = np.random.default_rng(5000 + T)
    xs_host = [bf16_normal(rng, (T, 2048)) for _ in range(4)]
    layout = native.routed_layout(T, 'layer')
    ws = torch.empty(layout.workspace_bytes, dtype=torch.uint8, device=device)
    xs = torch.empty((T, 2048), dtype=torch.bfloat16, device=device)
    out = torch.empty((T, 2048), dtype=torch.bfloat16, device=device)
    tw = torch.empty((T, 8), dtype=torch.float32, device=device)
    ti = torch.empty((T, 8), dtype=torch.int32, device=device)
    sl = torch.empty((T,), dtype=torch.bfloat16, device=device)
    flags = _flags(device)
    args = [to_dev(w['router'], device), None, to_dev(w['gate'][0], device), d['w13'][0], d['w13'][1], d['w2'][0],
            d['w2'][1], d['s13'][0], d['s13'][1], d['s2'][0], d['s2'][1], to_dev(silu, device),
            to_dev(sigmoid, device), ws, tw, ti, sl, out, flags, T]
    layer = lambda: native.moe_layer(xs, *args)

    def eager(xh):
        xs.copy_(to_dev(xh, device))
        layer()
        _sync()
        return out.clone(), ti.clone(), tw.clone(), sl.clone()

    refs = [eager(xh) for xh in xs_host[:3]]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        layer()                                   # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    _sync()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        layer()
    for i, xh in enumerate(xs_host[:3]):
        eager(xs_host[3])                         # the program's own eager work in between
        xs.copy_(to_dev(xh, device))
        _sync()
        g.replay()
        _sync()
        for got, want in zip((out, ti, tw, sl), refs[i]):
            assert torch.equal(got.view(torch.uint8), want.view(torch.uint8)), f'replay {i}'
    assert int(flags.item()) == 0


def _tied_router(router, case):
    """Router rows repeated so that logits (and probabilities) tie exactly:
    'quads' -- experts 4j..4j+3 share a row (ties decided by the lower id);
    'three' -- three distinct rows (about 85 experts per value: more than 64
    candidates above any threshold, the selection's fallback);
    'flat' -- one row (all 256 probabilities equal: picks 0..7)."""
    r = router.copy()
    e = np.arange(256)
    if case == 'quads':
        r[:] = router[e - e % 4]
    elif case == 'three':
        r[:] = router[e % 3]
    else:
        r[:] = router[0]
    return r


@pytest.mark.parametrize('case', ['quads', 'three', 'flat'])
def test_router_topk_ties(device, moe, case):
    """Exact probability ties between experts, one wave per token (T = 40)."""
    import torch
    native = _native()
    w, _ = moe
    T = 40
    rng = np.random.default_rng(3500)
    x = bf16_normal(rng, (T, 2048))
    router = _tied_router(w['router'], case)
    logits_ref = O.router_logits(x, np.concatenate([router, w['gate']]), None)
    wref, iref, _ = O.softmax_topk(logits_ref[:, :256])
    logits = torch.empty((T, 257), dtype=torch.float32, device=device)
    tw = torch.empty((T, 8), dtype=torch.float32, device=device)
    ti = torch.empty((T, 8), dtype=torch.int32, device=device)
    sl = torch.empty((T,), dtype=torch.bfloat16, device=device)
    native.router_topk(to_dev(x, device), to_dev(router, device), None, to_dev(w['gate'][0], device),
                       logits, tw, ti, sl)
    _sync()
    np.testing.assert_array_equal(from_dev(logits).view(np.uint32), logits_ref.view(np.uint32))
    np.testing.assert_array_equal(from_dev(ti), iref)
    np.testing.assert_array_equal(from_dev(tw).view(np.uint32), wref.view(np.uint32))
    if case == 'flat':
        assert (iref == np.arange(8)[None, :]).all()


@pytest.mark.parametrize('case', ['quads', 'three', 'flat'])
def test_moe_layer_single_token_ties(device, moe, shared_tables, case):
    """The single-token layer selects its experts inside the gate-up kernel;
    exact probability ties must give the oracle's picks, weights and output."""
    import torch
    native = _native()
    w, d = moe
    silu, sigmoid = shared_tables
    rng = np.random.default_rng(3600)
    x = bf16_normal(rng, (1, 2048))
    router = _tied_router(w['router'], case)
    logits = O.router_logits(x, np.concatenate([router, w['gate']]))
    rw, ids, _ = O.softmax_topk(logits[:, :256])
    ref = O.routed_layer_shared(x, rw, ids, LazyExperts(w['w13']), w['w13'].sbits, w['w13'].obits,
                                LazyExperts(w['w2']), w['w2'].sbits, w['w2'].obits,
                                *w['s13'].expert(), *w['s2'].expert(), O.f32_to_bf16(logits[:, 256]), silu, sigmoid)
    expected = O.add_bf16(ref['out'], ref['shared_out'])
    layout = native.routed_layout(1, 'layer')
    ws = torch.empty(layout.workspace_bytes, dtype=torch.uint8, device=device)
    out = torch.empty((1, 2048), dtype=torch.bfloat16, device=device)
    tw = torch.empty((1, 8), dtype=torch.float32, device=device)
    ti = torch.empty((1, 8), dtype=torch.int32, device=device)
    sl = torch.empty((1,), dtype=torch.bfloat16, device=device)
    flags = _flags(device)
    native.moe_layer(to_dev(x, device), to_dev(router, device), None, to_dev(w['gate'][0], device), d['w13'][0],
                     d['w13'][1], d['w2'][0], d['w2'][1], d['s13'][0], d['s13'][1], d['s2'][0], d['s2'][1],
                     to_dev(silu, device), to_dev(sigmoid, device), ws, tw, ti, sl, out, flags, 1)
    _sync()
    np.testing.assert_array_equal(from_dev(ti), ids)
    np.testing.assert_array_equal(from_dev(tw).view(np.uint32), rw.view(np.uint32))
    np.testing.assert_array_equal(from_dev(out), expected)
    assert int(flags.item()) == ref['flags']


# ---------------------------------------------------------------------------
# Heads
# ---------------------------------------------------------------------------
# Rows run in tiles of 16 on the matrix cores: 1..64 rows cover one to four
# row tiles (40, 33, 24, 56, 13 and 30 leave partial tiles; 13 and 30 also
# partial 4-row store groups); 65536 and 248320 are the
# reference's full head widths (head_i8_tile_api.h:22), where every wave
# streams two (65536) or seven to eight (248320) column tiles.
@pytest.mark.parametrize('M,N,dots', [(1, 256, False), (3, 1024, True), (40, 4096, False), (64, 4096, True),
                                      (33, 1024, False), (17, 256, True), (1, 65536, False), (64, 248320, False),
                                      (24, 65536, False), (56, 65536, False), (13, 4096, False),
                                      (30, 1024, False)])
def test_head_w8_bit_exact(device, M, N, dots):
    import torch
    native = _native()
    print(f'W8 head M={M} N={N} dots={dots}', flush=True)
    rng = np.random.default_rng(500 + M)
    w8 = rng.integers(-127, 128, size=(N, 2048), dtype=np.int64).astype(np.int8)
    sbits = O.f32_to_f16_bits(rng.uniform(0.0005, 0.002, size=(N, 16)).astype(np.float32))
    x = bf16_normal(rng, (M, 2048))
    ref_out, ref_diag, ref_flags = O.head_w8(x, w8, sbits)
    layout = native.HeadLayout()
    h = native.lib()
    assert h.ornith_head_i8_tile_get_layout(64, N, C.byref(layout)) == 0
    ws = torch.empty(layout.workspace_bytes, dtype=torch.uint8, device=device)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=device)
    gd = torch.empty((M, N, 16), dtype=torch.int32, device=device) if dots else None
    flags = _flags(device)
    xd = to_dev(x, device)
    wd = to_dev(O.head_w8_tile_layout(w8), device)
    sd = torch.from_numpy(sbits.view(np.int16)).to(device)
    st = h.ornith_head_i8_tile_launch(native.ptr(xd), native.ptr(wd), native.ptr(sd), native.ptr(ws), ws.numel(),
                                      native.ptr(out), native.ptr(gd), gd.numel() * 4 if dots else 0,
                                      native.ptr(flags), M, 64, N, 2, native.stream(xd))
    assert st == 0
    _sync()
    np.testing.assert_array_equal(from_dev(out), ref_out)
    diag = from_dev(ws[layout.projection:layout.projection + M * N * 4].view(torch.float32)).reshape(M, N)
    np.testing.assert_array_equal(diag.view(np.uint32), ref_diag.view(np.uint32))
    # greedy hand-off on the bf16 logits
    am = torch.empty((M,), dtype=torch.int64, device=device)
    native.logits_argmax(out, am)
    _sync()
    np.testing.assert_array_equal(from_dev(am), O.argmax_first(O.bf16_to_f32(ref_out)))
    if dots:
        tx = O.h128(O.bf16_to_f32(x))
        q, _, _, _ = O.quantize(tx, 127, group=128)
        ref_dots = np.einsum('mgk,ngk->mng', q.reshape(M, 16, 128).astype(np.int64),
                             w8.reshape(N, 16, 128).astype(np.int64))
        np.testing.assert_array_equal(from_dev(gd), ref_dots)
    assert int(flags.item()) == ref_flags


@pytest.mark.parametrize('case', ['ties', 'nan', 'signed_zero', 'neg_inf'])
def test_logits_argmax_rules(device, case):
    """The greedy hand-off follows torch/numpy argmax: the first maximum, the
    first NaN if any, -0 equal to +0, all -inf gives column 0."""
    import torch
    native = _native()
    rng = np.random.default_rng(77)
    M, N = 6, 5000
    v = rng.standard_normal((M, N)).astype(np.float32)
    if case == 'ties':
        v[:, [17, 400, 4999]] = 9.0
        v[3, :] = 1.0
    elif case == 'nan':
        v[:, 2500] = np.nan
        v[:, 3000] = np.nan
        v[1, 0] = np.nan
    elif case == 'signed_zero':
        v[:] = -1.0
        v[:, 100] = -0.0
        v[:, 50] = 0.0
    else:
        v[:] = -np.inf
    bits = O.f32_to_bf16(v)
    am = torch.empty((M,), dtype=torch.int64, device=device)
    native.logits_argmax(to_dev(bits, device), am)
    _sync()
    np.testing.assert_array_equal(from_dev(am), O.argmax_first(O.bf16_to_f32(bits)))


# 1..32 rows take the 32x32x32 streaming head (2080 columns = 65 code tiles
# over 32 waves: ranges of 2 and 3 tiles), 48 rows the row-tile kernel; 32
# and 96 columns give a single wave with one and three tiles
@pytest.mark.parametrize('M,N', [(1, 4096), (32, 151936), (17, 2080), (48, 8192), (5, 32), (32, 96)])
def test_head_g256_logits_and_argmax(device, M, N):
    import torch
    native = _native()
    print(f'g256 head M={M} N={N}', flush=True)
    rng = np.random.default_rng(600 + M)
    bank = Bank(rng, 0, N, 2048, tile=32)
    x = bf16_normal(rng, (M, 2048))
    ref_out, ref_diag, ref_flags = O.dense_a8(x, *bank.expert())
    xd, cd, md = to_dev(x, device), to_dev(bank.codes, device), to_dev(bank.meta, device)
    ws = torch.empty(native.lib().ornith_dense_g256_head_workspace_bytes(64, N), dtype=torch.uint8, device=device)
    logits = torch.empty((M, N), dtype=torch.float32, device=device)
    lb = torch.empty((M, N), dtype=torch.bfloat16, device=device)
    am = torch.empty((M,), dtype=torch.int64, device=device)
    flags = _flags(device)
    native.dense_head(xd, cd, md, ws, logits, lb, am, flags, 64)
    _sync()
    np.testing.assert_array_equal(from_dev(logits).view(np.uint32), ref_diag.view(np.uint32))
    np.testing.assert_array_equal(from_dev(lb), ref_out)
    np.testing.assert_array_equal(from_dev(am), O.argmax_first(ref_diag))
    assert int(flags.item()) == ref_flags


@pytest.mark.parametrize('case', ['ties', 'nan'])
@pytest.mark.parametrize('M', [5, 20])
def test_head_g256_argmax_ties_and_nan(device, case, M):
    """Equal logits across every wave's range (argmax = lowest column) and NaN
    logits in two columns (argmax = the first NaN column, both flags)."""
    import torch
    native = _native()
    N = 2080
    print(f'g256 head {case} M={M} N={N}', flush=True)
    rng = np.random.default_rng(700 + M)
    bank = Bank(rng, 0, N, 2048, tile=32)
    if case == 'ties':
        bank.codes[...] = bank.codes[0:1, :, :, 0:1]
        bank.sbits[...] = bank.sbits[0:1]
        bank.obits[...] = bank.obits[0:1]
    else:
        bank.sbits[1501, 3] = 0x7e00
        bank.sbits[1003, 6] = 0x7e00
    bank.meta = O.pack_meta(bank.sbits, bank.obits, 32)
    x = bf16_normal(rng, (M, 2048))
    ref_out, ref_diag, ref_flags = O.dense_a8(x, *bank.expert())
    expect = O.argmax_first(ref_diag)
    assert (expect == (0 if case == 'ties' else 1003)).all()
    xd, cd, md = to_dev(x, device), to_dev(bank.codes, device), to_dev(bank.meta, device)
    ws = torch.empty(native.lib().ornith_dense_g256_head_workspace_bytes(64, N), dtype=torch.uint8, device=device)
    logits = torch.empty((M, N), dtype=torch.float32, device=device)
    lb = torch.empty((M, N), dtype=torch.bfloat16, device=device)
    am = torch.empty((M,), dtype=torch.int64, device=device)
    flags = _flags(device)
    native.dense_head(xd, cd, md, ws, logits, lb, am, flags, 64)
    _sync()
    np.testing.assert_array_equal(from_dev(logits).view(np.uint32), ref_diag.view(np.uint32))
    np.testing.assert_array_equal(from_dev(lb), ref_out)
    np.testing.assert_array_equal(from_dev(am), expect)
    assert int(flags.item()) == ref_flags


def test_silu_short_form_matches_full_form_everywhere(device):
    """The prefill gate/up epilogue's short SiLU form (2^-60 <= |g| <= 80)
    against the full form (portable exp special cases, IEEE division), bit
    for bit, for every fp32 value of that domain, on the device."""
    from ornith_g256 import native
    checked, mismatches = native.silu_selfcheck()
    assert checked == 1111490562          # 2 signs x (2^-60 .. 80] in fp32
    assert mismatches == 0
