"""GPU: the give-up path of the one-launch kernels' hand-off waits.

The single-token layer kernel and the 2..32-token route kernel pass values
between blocks through tagged words and wait for them with bounded polls.
With the poll limit set to 0 from the host every wait gives up at once, so
the time-out path runs deterministically while every kernel still exits
normally.  Checked here, for one token (layer1) and 17 tokens (route +
top-8 + sort in one launch), on a caller workspace and on the no-allocation
entry's static scratch:

  1. a call with the limit at 0 returns, raises sticky flag 64, and marks
     the workspace poisoned;
  2. with the limit back at its default, the next call on that workspace
     still raises flag 64 (a poisoned workspace gives every wait up);
  3. after ornith_mi355x_workspace_reset the next call is flag-free and
     byte-identical to a call on a fresh workspace.

On the give-up path the kernels compute on whatever the hand-off words
hold; every index they derive stays in range (expert ids come from the
selection's lane positions, never from word contents; ids that the route
kernel gathers from words are range-checked by its sort; a bf16 logit
indexes a 65536-entry table), so the stale values only change results,
which flag 64 marks as unusable.
"""
import numpy as np
import pytest

from _ornith import Bank, bf16_normal, from_dev, moe_weights, to_dev

pytestmark = pytest.mark.gpu

TIMEOUT = 64


def _native():
    from ornith_g256 import native
    return native


@pytest.fixture(scope='module')
def moe(device):
    w = moe_weights(7070)
    d = {k: (to_dev(v.codes, device), to_dev(v.meta, device)) for k, v in w.items() if isinstance(v, Bank)}
    return w, d


class _Setting:
    def __init__(self, **kw):
        self.kw = kw

    def __enter__(self):
        n = _native()
        self.prev = {}
        if 'spins' in self.kw:
            self.prev['spins'] = n.handoff_spin_limit(self.kw['spins'])
        if 'single' in self.kw:
            self.prev['single'] = n.single_token_path(self.kw['single'])
        if 'route' in self.kw:
            self.prev['route'] = n.decode_route_path(self.kw['route'])

    def __exit__(self, *exc):
        n = _native()
        if 'spins' in self.prev:
            n.handoff_spin_limit(self.prev['spins'])
        if 'single' in self.prev:
            n.single_token_path(self.prev['single'])
        if 'route' in self.prev:
            n.decode_route_path(self.prev['route'])
        return False


def _call(device, w, d, tables, x, ws, static=False):
    """One layer call; returns (outputs, flags, kernels that ran)."""
    import torch
    native = _native()
    silu, sigmoid = tables
    T = x.shape[0]
    out = torch.empty((T, 2048), dtype=torch.bfloat16, device=device)
    tw = torch.empty((T, 8), dtype=torch.float32, device=device)
    ti = torch.empty((T, 8), dtype=torch.int32, device=device)
    sl = torch.empty((T,), dtype=torch.bfloat16, device=device)
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    args = (to_dev(x, device), to_dev(w['router'], device), None, to_dev(w['gate'][0], device),
            d['w13'][0], d['w13'][1], d['w2'][0], d['w2'][1], d['s13'][0], d['s13'][1], d['s2'][0], d['s2'][1],
            to_dev(silu, device), to_dev(sigmoid, device))
    with native.KernelTimer('*') as t:
        if static:
            native.moe_layer_static(*args, tw, ti, sl, out, flags)
        else:
            native.moe_layer(*args, ws, tw, ti, sl, out, flags, 32)
        torch.cuda.synchronize()                   # every kernel exited normally
        ran = set(t.names())
    res = {'out': from_dev(out), 'w': from_dev(tw).view(np.uint32), 'ids': from_dev(ti), 'logit': from_dev(sl)}
    return res, int(flags.item()), ran


def _same(a, b):
    for k in a:
        np.testing.assert_array_equal(a[k], b[k], err_msg=k)


@pytest.mark.parametrize('static', [False, True])
@pytest.mark.parametrize('T,kernel', [(1, 'layer1'), (17, 'route_select')])
def test_handoff_timeout_poisons_until_reset(device, moe, shared_tables, T, kernel, static):
    import torch
    native = _native()
    w, d = moe
    print(f'hand-off give-up path: T={T} ({kernel}), static scratch={static}', flush=True)
    rng = np.random.default_rng(7100 + T)
    x = bf16_normal(rng, (T, 2048))
    cap_bytes = native.routed_layout(32, 'layer').workspace_bytes
    fresh = torch.zeros(cap_bytes, dtype=torch.uint8, device=device)
    ws = None if static else torch.zeros(cap_bytes, dtype=torch.uint8, device=device)
    with _Setting(single=0, route=0):
        ref, f0, ran = _call(device, w, d, shared_tables, x, fresh)
        assert f0 == 0 and kernel in ran, (f0, ran)
        if static:
            native.workspace_reset(None)
        with _Setting(spins=0):
            _, f1, ran = _call(device, w, d, shared_tables, x, ws, static)
        assert kernel in ran and f1 & TIMEOUT, (f1, ran)
        _, f2, _ = _call(device, w, d, shared_tables, x, ws, static)      # default limit, still poisoned
        assert f2 & TIMEOUT, f2
        native.workspace_reset(ws)
        got, f3, _ = _call(device, w, d, shared_tables, x, ws, static)
        assert f3 == 0, f3
        _same(got, ref)
        got2, f4, _ = _call(device, w, d, shared_tables, x, ws, static)   # and the sequence runs on
        assert f4 == 0
        _same(got2, ref)
