"""GPU: the 2..32-token layer with router, top-8 and sort in one launch,
against the three-kernel path and the oracle.

The one-launch route kernel hands the router logits and the selected expert
ids between its blocks as tagged words (tag = hash of the call's sequence
number and the word index; the sequence number is shared with the
single-token kernel), so besides the results these tests cover many calls on
one workspace, single-token and multi-token calls interleaved on it, a
workspace of random bytes, one holding another call's words, and graph
replays.  Every case compares every output byte for byte.
"""
import numpy as np
import pytest

from _ornith import Bank, LazyExperts, bf16_normal, from_dev, moe_weights, to_dev
from oracle import ornith_oracle as O

pytestmark = pytest.mark.gpu

PATHS = (0, 1)      # 0: one launch, 1: three kernels


def _native():
    from ornith_g256 import native
    return native


@pytest.fixture(scope='module')
def moe(device):
    w = moe_weights(5151)
    d = {k: (to_dev(v.codes, device), to_dev(v.meta, device)) for k, v in w.items() if isinstance(v, Bank)}
    return w, d


class _Path:
    def __init__(self, path):
        self.path = path

    def __enter__(self):
        self.prev = _native().decode_route_path(self.path)

    def __exit__(self, *exc):
        _native().decode_route_path(self.prev)
        return False


def _args(device, w, d, tables, bias):
    silu, sigmoid = tables
    return (to_dev(w['router'], device), None if bias is None else to_dev(bias, device), to_dev(w['gate'][0], device),
            d['w13'][0], d['w13'][1], d['w2'][0], d['w2'][1], d['s13'][0], d['s13'][1], d['s2'][0], d['s2'][1],
            to_dev(silu, device), to_dev(sigmoid, device))


def _layer(device, w, d, tables, x, bias=None, ws=None, cap=32):
    import torch
    native = _native()
    T = x.shape[0]
    if ws is None:
        ws = torch.empty(native.routed_layout(cap, 'layer').workspace_bytes, dtype=torch.uint8, device=device)
    out = torch.empty((T, 2048), dtype=torch.bfloat16, device=device)
    tw = torch.empty((T, 8), dtype=torch.float32, device=device)
    ti = torch.empty((T, 8), dtype=torch.int32, device=device)
    sl = torch.empty((T,), dtype=torch.bfloat16, device=device)
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    native.moe_layer(to_dev(x, device), *_args(device, w, d, tables, bias), ws, tw, ti, sl, out, flags, cap)
    torch.cuda.synchronize()
    return {'out': from_dev(out), 'w': from_dev(tw).view(np.uint32), 'ids': from_dev(ti), 'logit': from_dev(sl),
            'flags': int(flags.item())}


def _same(a, b):
    assert a.keys() == b.keys()
    for k in a:
        np.testing.assert_array_equal(np.asarray(a[k]), np.asarray(b[k]), err_msg=k)


def _layer_oracle(w, tables, x, bias=None):
    silu, sigmoid = tables
    logits = O.router_logits(x, np.concatenate([w['router'], w['gate']]))
    if bias is not None:
        logits[:, :256] = (logits[:, :256] + bias[None, :]).astype(np.float32)
    rw, ids, _ = O.softmax_topk(logits[:, :256])
    ref = O.routed_layer_shared(x, rw, ids, LazyExperts(w['w13']), w['w13'].sbits, w['w13'].obits,
                                LazyExperts(w['w2']), w['w2'].sbits, w['w2'].obits, *w['s13'].expert(),
                                *w['s2'].expert(), O.f32_to_bf16(logits[:, 256]), silu, sigmoid)
    return O.add_bf16(ref['out'], ref['shared_out']), rw, ids, O.f32_to_bf16(logits[:, 256]), ref['flags']


@pytest.mark.parametrize('T,biased', [(2, False), (9, True), (17, False), (32, True)])
def test_route_paths_agree_with_oracle(device, moe, shared_tables, T, biased):
    w, d = moe
    rng = np.random.default_rng(100 + T)
    x = bf16_normal(rng, (T, 2048))
    bias = (-1.3 * np.log(1 + rng.permutation(256))).astype(np.float32) if biased else None
    print(f'decode route T={T} biased={biased}', flush=True)
    res = {}
    for path in PATHS:
        with _Path(path):
            res[path] = _layer(device, w, d, shared_tables, x, bias)
    _same(res[0], res[1])
    expected, rw, ids, logit, flags = _layer_oracle(w, shared_tables, x, bias)
    np.testing.assert_array_equal(res[0]['out'], expected)
    np.testing.assert_array_equal(res[0]['ids'], ids)
    np.testing.assert_array_equal(res[0]['w'], rw.view(np.uint32))
    np.testing.assert_array_equal(res[0]['logit'], logit)
    assert res[0]['flags'] == flags == 0


def test_route_ties_one_launch(device, moe, shared_tables):
    """Router rows repeated so that many probabilities tie exactly (the
    selection's fallback beyond 64 candidates included) on both paths."""
    w, d = moe
    w = dict(w)
    rng = np.random.default_rng(7)
    base = w['router'][:3].copy()
    w['router'] = np.concatenate([np.repeat(base[:1], 100, 0), np.repeat(base[1:2], 100, 0),
                                  np.repeat(base[2:3], 56, 0)])
    x = bf16_normal(rng, (12, 2048))
    print('decode route ties', flush=True)
    res = {}
    for path in PATHS:
        with _Path(path):
            res[path] = _layer(device, w, d, shared_tables, x)
    _same(res[0], res[1])
    expected, rw, ids, logit, flags = _layer_oracle(w, shared_tables, x)
    np.testing.assert_array_equal(res[0]['ids'], ids)
    np.testing.assert_array_equal(res[0]['out'], expected)


def test_route_workspace_reuse_garbage_stale_and_interleaved(device, moe, shared_tables):
    """Calls on one workspace advance its sequence number (single-token calls
    interleaved with 32-token ones share it); a workspace of random bytes and
    a byte copy of a used one give the same results."""
    import torch
    native = _native()
    w, d = moe
    rng = np.random.default_rng(43)
    xs = [bf16_normal(rng, (32, 2048)) for _ in range(3)]
    x1 = bf16_normal(rng, (1, 2048))
    with _Path(1):
        expected = [_layer(device, w, d, shared_tables, x) for x in xs]
        expected1 = _layer(device, w, d, shared_tables, x1)
    nbytes = native.routed_layout(32, 'layer').workspace_bytes
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    with _Path(0):
        print('decode route workspace reuse', flush=True)
        for i in range(9):
            _same(_layer(device, w, d, shared_tables, xs[i % 3], ws=ws), expected[i % 3])
            if i % 2:
                _same(_layer(device, w, d, shared_tables, x1, ws=ws), expected1)
        print('decode route garbage workspace', flush=True)
        g = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=device)
        _same(_layer(device, w, d, shared_tables, xs[1], ws=g), expected[1])
        print('decode route copied workspace', flush=True)
        stale = ws.clone()
        _same(_layer(device, w, d, shared_tables, xs[0], ws=stale), expected[0])
        _same(_layer(device, w, d, shared_tables, xs[2], ws=ws), expected[2])


def test_route_graph_replays_one_launch(device, moe, shared_tables):
    """The layer captured in a HIP graph: replays of one graph keep handing
    off (the sequence number lives in device memory), with eager calls on the
    same workspace in between."""
    import torch
    native = _native()
    w, d = moe
    rng = np.random.default_rng(47)
    xs = [bf16_normal(rng, (32, 2048)) for _ in range(3)]
    with _Path(1):
        expected = [_layer(device, w, d, shared_tables, x)['out'] for x in xs]
    ws = torch.empty(native.routed_layout(32, 'layer').workspace_bytes, dtype=torch.uint8, device=device)
    xd = to_dev(xs[0], device)
    out = torch.empty((32, 2048), dtype=torch.bfloat16, device=device)
    tw = torch.empty((32, 8), dtype=torch.float32, device=device)
    ti = torch.empty((32, 8), dtype=torch.int32, device=device)
    sl = torch.empty((32,), dtype=torch.bfloat16, device=device)
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    args = _args(device, w, d, shared_tables, None) + (ws, tw, ti, sl, out, flags, 32)
    with _Path(0):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            native.moe_layer(xd, *args)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            native.moe_layer(xd, *args)
        for i in range(6):
            xd.copy_(to_dev(xs[i % 3], device))
            g.replay()
            torch.cuda.synchronize()
            np.testing.assert_array_equal(from_dev(out), expected[i % 3])
            native.moe_layer(xd, *args)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(from_dev(out), expected[i % 3])
        assert int(flags.item()) == 0


def test_route_kernels_that_ran(device, moe, shared_tables):
    """Path 0 runs router, top-8 and sort as one launch on the MI355X; path 1
    as three kernels."""
    native = _native()
    w, d = moe
    x = bf16_normal(np.random.default_rng(53), (32, 2048))
    for path, first in ((0, {'route_select'}), (1, {'route', 'topk', 'sort'})):
        with _Path(path), native.KernelTimer('*') as t:
            _layer(device, w, d, shared_tables, x)
            ran = set(t.names())
        assert first <= ran and not (ran & ({'route', 'topk', 'sort', 'route_select'} - first)), (path, ran)
