"""The no-allocation layer entry (ornith_moe_layer_launch_static) against the
workspace entry it wraps (ornith_moe_layer_launch), bit for bit, on two
calls in a row (the second with fewer tokens, so stale scratch contents from
the first would show), then a single-token call."""
import numpy as np
import pytest

from _ornith import bf16_normal, from_dev, moe_weights, to_dev

pytestmark = pytest.mark.gpu


def test_static_layer_entry_matches_workspace_entry(device, shared_tables):
    import torch
    from ornith_g256 import native
    silu, sigmoid = shared_tables
    w = moe_weights(4321)
    d = {k: (to_dev(w[k].codes, device), to_dev(w[k].meta, device)) for k in ('w13', 'w2', 's13', 's2')}
    weights = [to_dev(w['router'], device), None, to_dev(w['gate'][0], device), d['w13'][0], d['w13'][1],
               d['w2'][0], d['w2'][1], d['s13'][0], d['s13'][1], d['s2'][0], d['s2'][1], to_dev(silu, device),
               to_dev(sigmoid, device)]

    def outputs(T):
        return (torch.empty((T, 8), dtype=torch.float32, device=device),
                torch.empty((T, 8), dtype=torch.int32, device=device),
                torch.empty((T,), dtype=torch.bfloat16, device=device),
                torch.empty((T, 2048), dtype=torch.bfloat16, device=device),
                torch.zeros(1, dtype=torch.int32, device=device))

    rng = np.random.default_rng(91)
    for T in (32, 5, 1):
        print(f'static layer entry T={T}', flush=True)
        x = to_dev(bf16_normal(rng, (T, 2048)), device)
        tw, ti, sl, out, flags = outputs(T)
        native.moe_layer_static(x, *weights, tw, ti, sl, out, flags)
        torch.cuda.synchronize()
        ws = torch.empty(native.routed_layout(T, 'layer').workspace_bytes, dtype=torch.uint8, device=device)
        rtw, rti, rsl, rout, rflags = outputs(T)
        native.moe_layer(x, *weights, ws, rtw, rti, rsl, rout, rflags, T)
        torch.cuda.synchronize()
        for got, want in ((out, rout), (ti, rti), (tw, rtw), (sl, rsl)):
            assert torch.equal(got.view(torch.uint8), want.view(torch.uint8)), T
        assert int(flags.item()) == int(rflags.item()) == 0


def test_static_layer_entry_rejects_large_batches():
    import ctypes as C
    from ornith_g256 import native
    h = native.lib()
    p = C.c_void_p(0x10000)
    assert h.ornith_moe_layer_launch_static(*([p] * 19), 33, None) == 1       # hipErrorInvalidValue
    assert h.ornith_moe_layer_launch_static(*([None] * 19), 0, None) == 0     # T == 0: nothing touched
