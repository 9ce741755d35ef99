"""GPU: the single-token (T == 1) layer in one launch against the three-kernel
path and the oracle.

The one-launch kernel hands the router logits and the middle rows between
blocks as tagged words (tag = hash of the call's sequence number and the word index),
so these tests also cover what that protocol must survive: many calls on one
workspace, a workspace full of garbage, a workspace holding another call's
words, and graph replays.  Every case compares every output byte for byte.
"""
import numpy as np
import pytest

from _ornith import Bank, LazyExperts, bf16_normal, from_dev, moe_weights, oracle_routed, random_routing, to_dev
from oracle import ornith_oracle as O

pytestmark = pytest.mark.gpu

PATHS = (0, 1)      # 0: one launch, 1: three kernels


def _native():
    from ornith_g256 import native
    return native


@pytest.fixture(scope='module')
def moe(device):
    w = moe_weights(4321)
    d = {k: (to_dev(v.codes, device), to_dev(v.meta, device)) for k, v in w.items() if isinstance(v, Bank)}
    return w, d


class _Path:
    def __init__(self, path):
        self.path = path

    def __enter__(self):
        self.prev = _native().single_token_path(self.path)

    def __exit__(self, *exc):
        _native().single_token_path(self.prev)
        return False


def _layer(device, w, d, tables, x, bias=None, ws=None):
    import torch
    native = _native()
    silu, sigmoid = tables
    if ws is None:
        ws = torch.empty(native.routed_layout(1, 'layer').workspace_bytes, dtype=torch.uint8, device=device)
    out = torch.empty((1, 2048), dtype=torch.bfloat16, device=device)
    tw = torch.empty((1, 8), dtype=torch.float32, device=device)
    ti = torch.empty((1, 8), dtype=torch.int32, device=device)
    sl = torch.empty((1,), dtype=torch.bfloat16, device=device)
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    native.moe_layer(to_dev(x, device), to_dev(w['router'], device), None if bias is None else to_dev(bias, device),
                     to_dev(w['gate'][0], device), d['w13'][0], d['w13'][1], d['w2'][0], d['w2'][1], d['s13'][0],
                     d['s13'][1], d['s2'][0], d['s2'][1], to_dev(silu, device), to_dev(sigmoid, device), ws, tw, ti,
                     sl, out, flags, 1)
    torch.cuda.synchronize()
    return {'out': from_dev(out), 'w': from_dev(tw).view(np.uint32), 'ids': from_dev(ti), 'logit': from_dev(sl),
            'flags': int(flags.item())}


def _routed(device, d, x, rw, ids, entry):
    import torch
    native = _native()
    layout = native.routed_layout(1)
    ws = torch.empty(layout.workspace_bytes, dtype=torch.uint8, device=device)
    out = torch.empty((1, 2048), dtype=torch.bfloat16, device=device)
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    xd = to_dev(x, device)
    st = getattr(native.lib(), entry)(*[native.ptr(t) for t in (xd, to_dev(rw, device), to_dev(ids, device),
                                                                d['w13'][0], d['w13'][1], d['w2'][0], d['w2'][1],
                                                                ws)],
                                      ws.numel(), native.ptr(out), native.ptr(flags), 1, 1, native.stream(xd))
    assert st == 0
    torch.cuda.synchronize()
    final = from_dev(ws[layout.final_f32:layout.final_f32 + 2048 * 4].view(torch.float32))
    return {'out': from_dev(out), 'final': final.view(np.uint32).reshape(1, 2048), 'flags': int(flags.item())}


def _shared_tables(device, d, tables, x, rw, ids, logit):
    import torch
    native = _native()
    silu, sigmoid = tables
    ws = torch.empty(native.routed_layout(1, 'shared').workspace_bytes, dtype=torch.uint8, device=device)
    out = torch.empty((1, 2048), dtype=torch.bfloat16, device=device)
    sh = torch.empty((1, 2048), dtype=torch.bfloat16, device=device)
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    native.routed_shared_tables(to_dev(x, device), to_dev(rw, device), to_dev(ids, device), d['w13'][0], d['w13'][1],
                                d['w2'][0], d['w2'][1], d['s13'][0], d['s13'][1], d['s2'][0], d['s2'][1],
                                to_dev(logit, device), to_dev(silu, device), to_dev(sigmoid, device), ws, out, sh,
                                flags, 1)
    torch.cuda.synchronize()
    return {'out': from_dev(out), 'shared': from_dev(sh), 'flags': int(flags.item())}


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
    return O.add_bf16(ref['out'], ref['shared_out']), rw, ids, ref['flags']


@pytest.mark.parametrize('biased', [False, True])
def test_layer_paths_agree_with_oracle(device, moe, shared_tables, biased):
    w, d = moe
    rng = np.random.default_rng(11 + biased)
    x = bf16_normal(rng, (1, 2048))
    bias = (-1.3 * np.log(1 + rng.permutation(256))).astype(np.float32) if biased else None
    print(f'single-token layer biased={biased}', flush=True)
    res = {}
    for path in PATHS:
        with _Path(path):
            res[path] = _layer(device, w, d, shared_tables, x, bias)
    _same(res[0], res[1])
    expected, rw, ids, flags = _layer_oracle(w, shared_tables, x, bias)
    np.testing.assert_array_equal(res[0]['out'], expected)
    np.testing.assert_array_equal(res[0]['ids'], ids)
    np.testing.assert_array_equal(res[0]['w'], rw.view(np.uint32))
    assert res[0]['flags'] == flags == 0


@pytest.mark.parametrize('entry,qmax', [('ornith_routed_direct_launch', 127), ('ornith_routed_direct_launch_a4', 7)])
@pytest.mark.parametrize('case', ['plain', 'dup', 'pad', 'none', 'invalid'])
def test_routed_paths_agree_with_oracle(device, moe, entry, qmax, case):
    w, d = moe
    rng = np.random.default_rng(hash((entry, case)) % 1000)
    x = bf16_normal(rng, (1, 2048))
    rw, ids = random_routing(rng, 1)
    if case == 'dup':
        ids[0, 5] = ids[0, 2]
    elif case == 'pad':
        ids[0, [1, 6]] = -1
    elif case == 'none':
        ids[0, :] = -1
    elif case == 'invalid':
        ids[0, 3] = 300
        ids[0, 6] = -7
    print(f'single-token routed {entry} case={case}', flush=True)
    res = {}
    for path in PATHS:
        with _Path(path):
            res[path] = _routed(device, d, x, rw, ids, entry)
    _same(res[0], res[1])
    ref = oracle_routed(x, rw, ids, w['w13'], w['w2'], qmax=qmax)
    np.testing.assert_array_equal(res[0]['final'], ref['final'].view(np.uint32))
    np.testing.assert_array_equal(res[0]['out'], ref['out'])
    assert res[0]['flags'] == ref['flags']


@pytest.mark.parametrize('case', ['plain', 'pad'])
def test_shared_tables_paths_agree(device, moe, shared_tables, case):
    w, d = moe
    silu, sigmoid = shared_tables
    rng = np.random.default_rng(23)
    x = bf16_normal(rng, (1, 2048))
    rw, ids = random_routing(rng, 1)
    if case == 'pad':
        ids[0, [0, 7]] = -1
    logit = bf16_normal(rng, (1,), 0.5)
    print(f'single-token shared tables case={case}', flush=True)
    res = {}
    for path in PATHS:
        with _Path(path):
            res[path] = _shared_tables(device, d, shared_tables, x, rw, ids, logit)
    _same(res[0], res[1])
    ref = O.routed_layer_shared(x, rw, ids, LazyExperts(w['w13']), w['w13'].sbits, w['w13'].obits,
                                LazyExperts(w['w2']), w['w2'].sbits, w['w2'].obits, *w['s13'].expert(),
                                *w['s2'].expert(), logit, silu, sigmoid)
    np.testing.assert_array_equal(res[0]['out'], ref['out'])
    np.testing.assert_array_equal(res[0]['shared'], ref['shared_out'])
    assert res[0]['flags'] == ref['flags']


def test_layer_workspace_reuse_garbage_and_stale_words(device, moe, shared_tables):
    """Calls on one workspace advance its sequence number; a workspace of
    random bytes, and one holding a byte copy of a used workspace (the other
    call's tagged words and sequence number), give the same results."""
    import torch
    native = _native()
    w, d = moe
    rng = np.random.default_rng(31)
    xs = [bf16_normal(rng, (1, 2048)) for _ in range(3)]
    with _Path(1):
        expected = [_layer(device, w, d, shared_tables, x) for x in xs]
    nbytes = native.routed_layout(1, 'layer').workspace_bytes
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    with _Path(0):
        print('single-token workspace reuse', flush=True)
        for i in range(12):
            _same(_layer(device, w, d, shared_tables, xs[i % 3], ws=ws), expected[i % 3])
        print('single-token garbage workspace', flush=True)
        g = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=device)
        _same(_layer(device, w, d, shared_tables, xs[1], ws=g), expected[1])
        print('single-token copied workspace', flush=True)
        stale = ws.clone()                       # words of the last call on ws (input xs[2])
        _same(_layer(device, w, d, shared_tables, xs[0], ws=stale), expected[0])
        _same(_layer(device, w, d, shared_tables, xs[2], ws=ws), expected[2])


def test_layer_graph_replays_one_launch(device, moe, shared_tables):
    """The one-launch layer captured in a HIP graph: the sequence number lives
    in device memory, so replays of the same graph keep handing off."""
    import torch
    native = _native()
    w, d = moe
    silu, sigmoid = shared_tables
    rng = np.random.default_rng(37)
    xs = [bf16_normal(rng, (1, 2048)) for _ in range(4)]
    with _Path(1):
        expected = [_layer(device, w, d, shared_tables, x)['out'] for x in xs]
    ws = torch.empty(native.routed_layout(1, 'layer').workspace_bytes, dtype=torch.uint8, device=device)
    xd = to_dev(xs[0], device)
    out = torch.empty((1, 2048), dtype=torch.bfloat16, device=device)
    tw = torch.empty((1, 8), dtype=torch.float32, device=device)
    ti = torch.empty((1, 8), dtype=torch.int32, device=device)
    sl = torch.empty((1,), dtype=torch.bfloat16, device=device)
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    args = (to_dev(w['router'], device), None, to_dev(w['gate'][0], device), d['w13'][0], d['w13'][1], d['w2'][0],
            d['w2'][1], d['s13'][0], d['s13'][1], d['s2'][0], d['s2'][1], to_dev(silu, device),
            to_dev(sigmoid, device), ws, tw, ti, sl, out, flags, 1)
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
        for i in range(8):
            xd.copy_(to_dev(xs[i % 4], device))
            g.replay()
            torch.cuda.synchronize()
            np.testing.assert_array_equal(from_dev(out), expected[i % 4])
            # an eager call between replays advances the same sequence number
            native.moe_layer(xd, *args)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(from_dev(out), expected[i % 4])
        assert int(flags.item()) == 0


def test_single_token_kernels_that_ran(device, moe, shared_tables):
    """Path 0 runs the one-launch kernel on the MI355X (256 blocks
    resident); path 1 the three kernels."""
    native = _native()
    w, d = moe
    x = bf16_normal(np.random.default_rng(41), (1, 2048))
    for path, names in ((0, {'layer1'}), (1, {'route1', 'gateup1', 'down1'})):
        with _Path(path), native.KernelTimer('*') as t:
            _layer(device, w, d, shared_tables, x)
            ran = set(t.names())
        assert ran == names, (path, ran)
