"""GPU checks of the benchmark workloads as specified and of the host-side
dispatch, all through the C ABI or the ornith_g256 torch ops:

* the 1120-token layer under the Zipf(1.1) router bias and the 8192-token
  layer under Zipf(1.3) (batch invariance against smaller runs that are
  themselves oracle-checked), and a 300-token layer under Zipf(1.3) checked
  against the oracle (one expert holds nearly every token: many m-tiles);
* the dense linear at the benchmark's 1120 x 6144 x 2048 prefill shape
  through ``dense_out`` (bf16 operands + GEMM) against an fp64 dequant-matmul
  (tolerance: the GEMM's summation order is hipBLASLt's, as in the reference);
* the N16-bank build of the library (the reference's parent routed library
  role) against the oracle;
* ``routed_out`` with a mixed prefill/decode phase plan.
"""
import numpy as np
import pytest

from _ornith import LazyExperts, bf16_normal, from_dev, moe_weights, oracle_routed, random_routing, to_dev
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
    d = {k: (to_dev(w[k].codes, device), to_dev(w[k].meta, device)) for k in ('w13', 'w2', 's13', 's2')}
    return w, d


def _zipf_bias(s, seed):
    """b_e = -s * ln(rank_e), seeded rank permutation (the benchmark's router bias)."""
    rank = np.random.default_rng(seed).permutation(256).astype(np.float64) + 1.0
    return (-s * np.log(rank)).astype(np.float32)


def _layer_fn(native, device, w, d, silu, sigmoid, bias, tile=32, banks=None):
    import torch
    banks = banks or d
    weights = [to_dev(w['router'], device), None if bias is None else to_dev(bias, device),
               to_dev(w['gate'][0], device), banks['w13'][0], banks['w13'][1], banks['w2'][0], banks['w2'][1],
               d['s13'][0], d['s13'][1], d['s2'][0], d['s2'][1], to_dev(silu, device), to_dev(sigmoid, device)]

    def layer(xs):
        n = xs.shape[0]
        ws = torch.empty(native.routed_layout(n, 'layer', tile=tile).workspace_bytes, dtype=torch.uint8,
                         device=device)
        out = torch.empty((n, 2048), dtype=torch.bfloat16, device=device)
        tw = torch.empty((n, 8), dtype=torch.float32, device=device)
        ti = torch.empty((n, 8), dtype=torch.int32, device=device)
        sl = torch.empty((n,), dtype=torch.bfloat16, device=device)
        flags = _flags(device)
        native.moe_layer(xs.contiguous(), *weights, ws, tw, ti, sl, out, flags, n, tile=tile)
        _sync()
        return out, ti, tw, sl, int(flags.item())
    return layer


def _oracle_layer(w, x, bias, silu, sigmoid):
    logits = O.router_logits(x, np.concatenate([w['router'], w['gate']]))
    if bias is not None:
        logits[:, :256] = (logits[:, :256] + bias[None, :]).astype(np.float32)
    rw, ids, _ = O.softmax_topk(logits[:, :256])
    ref = O.routed_layer_shared(x, rw, ids, LazyExperts(w['w13']), w['w13'].sbits, w['w13'].obits,
                                LazyExperts(w['w2']), w['w2'].sbits, w['w2'].obits,
                                *w['s13'].expert(), *w['s2'].expert(), O.f32_to_bf16(logits[:, 256]), silu, sigmoid)
    return rw, ids, O.add_bf16(ref['out'], ref['shared_out']), ref['flags']


# ---------------------------------------------------------------------------
# Skewed routing
# ---------------------------------------------------------------------------
def test_moe_layer_zipf13_300_tokens_vs_oracle(device, moe, shared_tables):
    """300 tokens under the Zipf(1.3) bias: the most popular expert takes
    nearly every token (more than 128 routes, several 64-route m-tiles)."""
    native = _native()
    w, d = moe
    silu, sigmoid = shared_tables
    print('layer T=300 zipf 1.3 vs oracle', flush=True)
    rng = np.random.default_rng(7300)
    x = bf16_normal(rng, (300, 2048))
    bias = _zipf_bias(1.3, 11)
    rw, ids, expected, ref_flags = _oracle_layer(w, x, bias, silu, sigmoid)
    counts = np.bincount(ids.reshape(-1), minlength=256)
    assert counts.max() > 128, counts.max()
    out, ti, tw, sl, flags = _layer_fn(native, device, w, d, silu, sigmoid, bias)(to_dev(x, device))
    np.testing.assert_array_equal(from_dev(ti), ids)
    np.testing.assert_array_equal(from_dev(tw).view(np.uint32), rw.view(np.uint32))
    np.testing.assert_array_equal(from_dev(out), expected)
    assert flags == ref_flags == 0


@pytest.mark.parametrize('T,s', [(1120, 1.1), (8192, 1.3)])
def test_moe_layer_zipf_full_size_batch_invariance(device, moe, shared_tables, T, s):
    """The benchmark's skewed prefill workloads: every row of the T-token
    layer equals the same row run in a 300-token layer (prefill path, checked
    against the oracle above), a 32-token layer (decode path) and as a single
    token, ids and weights included; flags stay clear."""
    import torch
    native = _native()
    w, d = moe
    silu, sigmoid = shared_tables
    print(f'layer batch invariance T={T} zipf {s}', flush=True)
    rng = np.random.default_rng(8000 + T)
    x = to_dev(bf16_normal(rng, (T, 2048)), device)
    bias = _zipf_bias(s, 11)
    layer = _layer_fn(native, device, w, d, silu, sigmoid, bias)
    full = layer(x)
    assert full[4] == 0
    counts = np.bincount(from_dev(full[1]).reshape(-1), minlength=256)
    print(f'  top expert routes {counts.max()}, experts used {int((counts > 0).sum())}', flush=True)
    assert counts.max() > T // 2                  # a heavily skewed expert: many m-tiles on one bank
    for lo, hi in [(0, 300), (T - 300, T), (T // 2, T // 2 + 32), (T - 1, T), (T // 3, T // 3 + 1)]:
        part = layer(x[lo:hi])
        assert part[4] == 0
        for a, b in zip(part[:4], full[:4]):
            assert torch.equal(a.view(torch.uint8), b[lo:hi].contiguous().view(torch.uint8)), (lo, hi)


# ---------------------------------------------------------------------------
# Dense linear at the prefill shape through dense_out
# ---------------------------------------------------------------------------
@pytest.mark.parametrize('M,N,K', [(1120, 6144, 2048), (300, 512, 4096), (2100, 4096, 2048), (8192, 2048, 4096)])
def test_dense_out_prefill_tolerance(device, M, N, K):
    """dense_out with more rows than the A8 crossover: bf16(H128 x) @
    bf16(dequantised W)^T on this library's code-reading GEMM at every shape
    (the benchmark's 1120 x 6144 x 2048, K = 4096, and the large products
    the reference gives hipBLASLt).  The bf16 operands are bit-exact
    (test_gpu_parity); the reduction order is the kernel's own, so the
    product is checked by tolerance against fp64: cosine >= 0.9999 and max
    |err| <= 1e-2 * max |ref|."""
    import torch
    from _ornith import Bank
    native = _native()
    print(f'dense_out {M} x {N} x {K}', flush=True)
    rng = np.random.default_rng(M + N)
    bank = Bank(rng, 0, N, K, tile=16)
    x = bf16_normal(rng, (M, K))
    ws = torch.empty((M + 15) // 16 * 16 * K * 2, dtype=torch.uint8, device=device)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=device)
    flags = _flags(device)
    with native.KernelTimer('*') as kt:
        native.dense_out(to_dev(x, device), to_dev(bank.codes, device), to_dev(bank.meta, device), ws, out, flags,
                         M, N, K, 2, 64)
        _sync()
        assert set(kt.names()) == {'transform_bf16_frag', 'dense_gemm'}, kt.names()   # the library GEMM ran
    got = O.bf16_to_f32(from_dev(out)).astype(np.float64)
    xt = O.bf16_to_f32(O.transform_bf16(x)).astype(np.float64)
    wt = O.bf16_to_f32(O.dequantize_bf16(*bank.expert())).astype(np.float64)
    ref = xt @ wt.T
    cos = float((got.ravel() @ ref.ravel()) / (np.linalg.norm(got) * np.linalg.norm(ref)))
    err = float(np.abs(got - ref).max() / np.abs(ref).max())
    print(f'  cosine {cos:.7f}  max rel err {err:.2e}', flush=True)
    assert cos >= 0.9999 and err <= 1e-2
    assert int(flags.item()) == 0


# slices on the MI355X's 256 CUs: 8, 3, 4 and 8
@pytest.mark.parametrize('M,N,K,slices', [(300, 512, 4096, 8), (1120, 2048, 4096, 3), (1120, 1024, 2048, 4),
                                           (65, 96, 4096, 8)])
def test_dense_gemm_split_k(device, M, N, K, slices):
    """A GEMM grid that fills few of the chip's block slots splits K when the
    workspace holds the fp32 slice sums: the slices' sums are added in slice
    order (dense_slices ran), the result is deterministic, and it meets the
    same tolerance against fp64 as the unsplit GEMM (cosine >= 0.9999, max
    |err| <= 1e-2 * max |ref|)."""
    import torch
    from _ornith import Bank
    native = _native()
    print(f'dense gemm split K: {M} x {N} x {K}, {slices} slices', flush=True)
    rng = np.random.default_rng(4000 + M + N)
    bank = Bank(rng, 0, N, K, tile=16)
    x = bf16_normal(rng, (M, K))
    xt_bytes = (M + 15) // 16 * 16 * K * 2
    ws = torch.empty(xt_bytes + native.DENSE_SLICE_BYTES + 256, dtype=torch.uint8, device=device)
    xd, cd, md = to_dev(x, device), to_dev(bank.codes, device), to_dev(bank.meta, device)
    outs = []
    for bytes_ in (ws.numel(), ws.numel(), xt_bytes):      # split twice, then unsplit
        out = torch.empty((M, N), dtype=torch.bfloat16, device=device)
        flags = _flags(device)
        with native.KernelTimer('*') as kt:
            assert native.lib().ornith_dense_g256_gemm_bf16(native.ptr(xd), native.ptr(cd), native.ptr(md),
                                                            native.ptr(ws), bytes_, native.ptr(out), native.ptr(flags),
                                                            M, N, K, native.stream(xd)) == 0
            _sync()
            names = set(kt.names())
        assert ('dense_slices' in names) == (bytes_ != xt_bytes), names
        assert int(flags.item()) == 0
        outs.append(from_dev(out))
    np.testing.assert_array_equal(outs[0], outs[1])
    ref = (O.bf16_to_f32(O.transform_bf16(x)).astype(np.float64)
           @ O.bf16_to_f32(O.dequantize_bf16(*bank.expert())).astype(np.float64).T)
    for got in (outs[0], outs[2]):
        g = O.bf16_to_f32(got).astype(np.float64)
        cos = float((g.ravel() @ ref.ravel()) / (np.linalg.norm(g) * np.linalg.norm(ref)))
        err = float(np.abs(g - ref).max() / np.abs(ref).max())
        print(f'  cosine {cos:.8f}  max rel err {err:.2e}', flush=True)
        assert cos >= 0.9999 and err <= 1e-2


def test_dense_out_split_k_through_the_op(device):
    """dense_out with the workspace configure() sizes (bf16(H128 x) plus the
    split-K slice sums) at 300 x 512 x 4096, whose 16 tiles split K: the op
    runs the slices and their ordered sum, within the fp64 tolerance."""
    import torch
    from _ornith import Bank
    native = _native()
    M, N, K = 300, 512, 4096
    rng = np.random.default_rng(4321)
    bank = Bank(rng, 0, N, K, tile=16)
    x = bf16_normal(rng, (M, K))
    ws = torch.empty((M + 15) // 16 * 16 * K * 2 + native.DENSE_SLICE_BYTES, dtype=torch.uint8, device=device)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=device)
    flags = _flags(device)
    with native.KernelTimer('*') as kt:
        native.dense_out(to_dev(x, device), to_dev(bank.codes, device), to_dev(bank.meta, device), ws, out, flags,
                         M, N, K, 2, 64)
        _sync()
        assert set(kt.names()) == {'transform_bf16_frag', 'dense_gemm', 'dense_slices'}, kt.names()
    got = O.bf16_to_f32(from_dev(out)).astype(np.float64)
    ref = (O.bf16_to_f32(O.transform_bf16(x)).astype(np.float64)
           @ O.bf16_to_f32(O.dequantize_bf16(*bank.expert())).astype(np.float64).T)
    cos = float((got.ravel() @ ref.ravel()) / (np.linalg.norm(got) * np.linalg.norm(ref)))
    err = float(np.abs(got - ref).max() / np.abs(ref).max())
    assert cos >= 0.9999 and err <= 1e-2, (cos, err)
    assert int(flags.item()) == 0


# ---------------------------------------------------------------------------
# N16-bank build (the parent routed library role, routed_direct_api.h:7)
# ---------------------------------------------------------------------------
def _n32_to_n16(codes, meta):
    """N32 banks -> the same weights in N16 tiles (test-side data layout)."""
    E, nt, G = codes.shape[:3]
    c16 = codes.reshape(E, nt, G, 32, 2, 16).permute(0, 1, 4, 2, 3, 5).contiguous().reshape(E, 2 * nt, G, 32, 16)
    m16 = meta.reshape(E, nt, G, 2, 16).permute(0, 1, 3, 2, 4).contiguous().reshape(E, 2 * nt, G, 16)
    return c16, m16


@pytest.fixture(scope='module')
def n16_banks(moe):
    _, d = moe
    return {k: _n32_to_n16(*d[k]) for k in ('w13', 'w2')}


@pytest.mark.parametrize('T,entry,qmax', [(1, 'ornith_routed_direct_launch', 127),
                                          (5, 'ornith_routed_direct_launch', 127),
                                          (32, 'ornith_routed_direct_launch', 127),
                                          (70, 'ornith_routed_direct_launch_a4_prefill', 7),
                                          (100, 'ornith_routed_direct_launch', 127)])
def test_routed_n16_build_bit_exact(device, moe, n16_banks, T, entry, qmax):
    import torch
    native = _native()
    w, _ = moe
    print(f'routed N16 build T={T} {entry}', flush=True)
    rng = np.random.default_rng(1600 + T)
    x = bf16_normal(rng, (T, 2048))
    rw, ids = random_routing(rng, T)
    ref = oracle_routed(x, rw, ids, w['w13'], w['w2'], qmax=qmax)
    layout = native.routed_layout(T, tile=16)
    ws = torch.empty(layout.workspace_bytes, dtype=torch.uint8, device=device)
    out = torch.empty((T, 2048), dtype=torch.bfloat16, device=device)
    flags = _flags(device)
    xd, wd, idd = to_dev(x, device), to_dev(rw, device), to_dev(ids, device)
    b = n16_banks
    fn = getattr(native.lib(16), entry)
    st = fn(*[native.ptr(t) for t in (xd, wd, idd, b['w13'][0], b['w13'][1], b['w2'][0], b['w2'][1], ws)],
            ws.numel(), native.ptr(out), native.ptr(flags), T, T, native.stream(xd))
    assert st == 0
    _sync()
    np.testing.assert_array_equal(from_dev(out), ref['out'])
    assert int(flags.item()) == ref['flags']


@pytest.mark.parametrize('T', [1, 33])
def test_moe_layer_n16_build_bit_exact(device, moe, n16_banks, shared_tables, T):
    native = _native()
    w, d = moe
    silu, sigmoid = shared_tables
    print(f'layer N16 build T={T}', flush=True)
    rng = np.random.default_rng(1700 + T)
    x = bf16_normal(rng, (T, 2048))
    rw, ids, expected, ref_flags = _oracle_layer(w, x, None, silu, sigmoid)
    out, ti, tw, _, flags = _layer_fn(native, device, w, d, silu, sigmoid, None, tile=16,
                                      banks=n16_banks)(to_dev(x, device))
    np.testing.assert_array_equal(from_dev(ti), ids)
    np.testing.assert_array_equal(from_dev(out), expected)
    assert flags == ref_flags


# ---------------------------------------------------------------------------
# routed_out with a mixed prefill/decode phase plan
# ---------------------------------------------------------------------------
def test_routed_out_phase_segments(device, moe):
    """A 100-token batch of a decode segment (rows 0..39, A8) followed by a
    prefill segment (rows 40..99, A4, as the reference's phase dispatch runs
    them, native.py:161-168) equals the oracle run per segment."""
    import torch
    native = _native()
    w, d = moe
    print('routed_out phase segments', flush=True)
    native.reset_binding()
    try:
        ws_bytes = native.configure({'routed_storage_n32': True}, 128, [])
        rng = np.random.default_rng(1800)
        T = 100
        x = bf16_normal(rng, (T, 2048))
        rw, ids = random_routing(rng, T)
        ref_a8 = oracle_routed(x[:40], rw[:40], ids[:40], w['w13'], w['w2'], qmax=127)
        ref_a4 = oracle_routed(x[40:], rw[40:], ids[40:], w['w13'], w['w2'], qmax=7)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
        out = torch.empty((T, 2048), dtype=torch.bfloat16, device=device)
        flags = _flags(device)
        with native.phase_segments([(0, 40, False)]):
            native.routed_out(to_dev(x, device), to_dev(rw, device), to_dev(ids, device), d['w13'][0], d['w13'][1],
                              d['w2'][0], d['w2'][1], ws, out, flags, 128)
        _sync()
        got = from_dev(out)
        np.testing.assert_array_equal(got[:40], ref_a8['out'])
        np.testing.assert_array_equal(got[40:], ref_a4['out'])
        assert int(flags.item()) == 0
    finally:
        native.reset_binding()


# ---------------------------------------------------------------------------
# Storage conversion and the quantized-layer methods (method.py, runtime.py)
# ---------------------------------------------------------------------------
def test_repack_kernel_matches_oracle(device):
    """ornith_repack_n16_to_n32 against the oracle's N16 -> N32 permutation
    (method.py:143-147) on three banks, and on a dense head-width bank."""
    import torch
    from ornith_g256 import storage
    print('repack N16 -> N32', flush=True)
    rng = np.random.default_rng(1900)
    for banks, n, k in ((3, 96, 512), (1, 248320 // 8, 2048)):
        c16 = rng.integers(0, 2 ** 32, size=(banks, n // 16, k // 256, 32, 16), dtype=np.uint32)
        m16 = rng.integers(0, 2 ** 32, size=(banks, n // 16, k // 256, 16), dtype=np.uint32)
        c32, m32 = storage.repack_n32(to_dev(c16, device), to_dev(m16, device), n, k)
        _sync()
        rc, rm = O.n16_to_n32(c16, m16)
        np.testing.assert_array_equal(from_dev(c32).view(np.uint32), rc)
        np.testing.assert_array_equal(from_dev(m32).view(np.uint32), rm)


def _moe_module(device, d):
    """A layer holding the checkpoint (N16, CPU uint32) form of the test
    experts, loaded through the strict loader and moved to the GPU."""
    import torch
    from ornith_g256 import methods
    layer = torch.nn.Module()
    m = methods.G256MoEMethod('model.layers.0.mlp.experts')
    m.create_weights(layer)
    for proj in ('w13', 'w2'):
        c16, m16 = _n32_to_n16(*d[proj])
        layer.load_packed(f'{proj}_tilebank_codes', c16.cpu().view(torch.uint32))
        layer.load_packed(f'{proj}_tilebank_metadata', m16.cpu().view(torch.uint32))
    m.process_weights_after_loading(layer)
    layer.to(device)
    layer.quant_method = m
    return layer


@pytest.mark.parametrize('mode', ['storage_n32', 'n16', 'decode_n32'])
def test_moe_method_through_runtime(device, moe, mode):
    """Checkpoint banks -> loader -> Runtime (repack as configured) ->
    G256MoEMethod.apply, for the three routed storage configurations of the
    reference (runtime.py:35-46): sole N32 storage, N16 banks, N16 banks with
    N32 copies for batches of at most 8 tokens."""
    import torch
    from ornith_g256 import methods, native
    w, d = moe
    print(f'MoE method runtime mode={mode}', flush=True)
    native.reset_binding()
    try:
        model = torch.nn.Module()
        model.experts = _moe_module(device, d)
        settings = {'storage_n32': {'routed_storage_n32': True, 'routed_library': str(native.library_path(32))},
                    'n16': {'routed_library': str(native.library_path(16))},
                    'decode_n32': {'routed_decode_n32': True, 'routed_n32_library': str(native.library_path(32))}}[mode]
        rt = methods.Runtime(model, settings, 64, device)
        if mode != 'n16':
            assert rt.repacked_bytes == 256 * (1_081_344 + 540_672)
        rng = np.random.default_rng(1950)
        for T in (4, 40):
            x = bf16_normal(rng, (T, 2048))
            rw, ids = random_routing(rng, T)
            ref = oracle_routed(x, rw, ids, w['w13'], w['w2'])
            out = model.experts.quant_method.apply(model.experts, to_dev(x, device), to_dev(rw, device),
                                                   to_dev(ids, device))
            _sync()
            np.testing.assert_array_equal(from_dev(out), ref['out'])
        assert rt.check_error_flags() == [0]
    finally:
        native.reset_binding()


def test_router_gate_and_shared_expert_through_runtime(device, moe, shared_tables):
    """A MoE block bound to the Runtime the way the vLLM adapter binds it:
    the router gate (RouterGateMethod) gives the fp32 logits and, in the same
    launch, the shared expert's gate logit; the routed launch runs the shared
    expert as the fused ninth slot (N16 routed banks through the N16 build,
    the shared expert's dense banks repacked to N32 by the Runtime); the
    step's decode rows of the shared output are then recomputed by fixed8.
    Every output against the oracle, bit for bit."""
    import torch
    from ornith_g256 import methods, native
    w, d = moe
    silu, sigmoid = shared_tables
    print('router gate + shared expert through the runtime', flush=True)
    native.reset_binding()
    try:
        model = torch.nn.Module()
        model.layers = torch.nn.ModuleList([torch.nn.Module()])
        blk = model.layers[0].mlp = torch.nn.Module()
        blk.experts = _moe_module(device, d)
        blk.gate = torch.nn.Module()
        blk.gate.weight = torch.nn.Parameter(to_dev(w['router'], device), requires_grad=False)
        blk.gate.quant_method = methods.RouterGateMethod('layers.0.mlp.gate')
        blk.shared_expert = torch.nn.Module()
        for name, key, (n, k) in (('gate_up_proj', 's13', (1024, 2048)), ('down_proj', 's2', (2048, 512))):
            lin = torch.nn.Module()
            m = methods.G256LinearMethod(f'layers.0.mlp.shared_expert.{name}', n, k)
            m.create_weights(lin)
            c16, m16 = _n32_to_n16(d[key][0][None], d[key][1][None])
            lin.load_packed('g256_codes', c16[0].cpu().view(torch.uint32))
            lin.load_packed('g256_metadata', m16[0].cpu().view(torch.uint32))
            m.process_weights_after_loading(lin)
            lin.to(device)
            lin.quant_method = m
            setattr(blk.shared_expert, name, lin)
        blk.shared_expert.expert_gate = torch.nn.Module()
        blk.shared_expert.expert_gate.weight = torch.nn.Parameter(to_dev(w['gate'], device), requires_grad=False)
        rt = methods.Runtime(model, {'routed_library': str(native.library_path(16))}, 64, device)
        shared = rt.shared['layers.0.mlp.shared_expert']
        assert blk.gate.quant_method.shared is shared and blk.shared_expert._ornith_shared is shared
        rng = np.random.default_rng(2500)
        T = 5
        x = bf16_normal(rng, (T, 2048))
        xd = to_dev(x, device)
        logits = blk.gate.quant_method.apply(blk.gate, xd)
        ref_logits = O.router_logits(x, np.concatenate([w['router'], w['gate']]))
        np.testing.assert_array_equal(from_dev(logits).view(np.uint32), ref_logits[:, :256].view(np.uint32))
        rw, ids, _ = O.softmax_topk(ref_logits[:, :256])
        shared_out = torch.empty((T, 2048), dtype=torch.bfloat16, device=device)
        with native.step_phases(((0, 2, True), (2, T, False))):
            out = blk.experts.quant_method.apply(blk.experts, xd, to_dev(rw, device), to_dev(ids, device),
                                                 shared=shared, shared_out=shared_out)
        _sync()
        ref = O.routed_layer_shared(x, rw, ids, LazyExperts(w['w13']), w['w13'].sbits, w['w13'].obits,
                                    LazyExperts(w['w2']), w['w2'].sbits, w['w2'].obits, *w['s13'].expert(),
                                    *w['s2'].expert(), O.f32_to_bf16(ref_logits[:, 256]), silu, sigmoid)
        np.testing.assert_array_equal(from_dev(out), ref['out'])
        got = from_dev(shared_out)
        np.testing.assert_array_equal(got[:2], ref['shared_out'][:2])            # prefill rows: ninth slot
        fixed, _ = O.shared_fixed8(x[2:], *w['s13'].expert(), *w['s2'].expert(), w['gate'][0], silu, sigmoid)
        np.testing.assert_array_equal(got[2:], fixed)                            # decode rows: fixed8
        assert rt.check_error_flags() == [0] * len(rt.layer_names)
    finally:
        native.reset_binding()


def test_dense_method_and_flag_lifecycle(device):
    """G256LinearMethod through the runtime at one row (A8 path, bit-exact)
    and 70 rows (bf16 operands + GEMM, tolerance); then a non-finite input
    raises the layer's flag, which the step lifecycle turns into a fault."""
    import torch
    from _ornith import Bank
    from ornith_g256 import lifecycle, methods, native
    print('dense method + lifecycle', flush=True)
    native.reset_binding()
    try:
        rng = np.random.default_rng(1990)
        N, K = 1024, 2048
        bank = Bank(rng, 0, N, K, tile=16)
        model = torch.nn.Module()
        model.proj = torch.nn.Module()
        m = methods.G256LinearMethod('model.layers.0.self_attn.o_proj', N, K)
        m.create_weights(model.proj)
        model.proj.load_packed('g256_codes', torch.from_numpy(bank.codes.view(np.int32)).view(torch.uint32))
        model.proj.load_packed('g256_metadata', torch.from_numpy(bank.meta.view(np.int32)).view(torch.uint32))
        m.process_weights_after_loading(model.proj)
        model.to(device)
        model.proj.quant_method = m
        rt = methods.Runtime(model, {'routed_storage_n32': True, 'dense_a8_max_rows': 64}, 128, device)
        steps = rt.step_flags()
        tk = steps.open('decode')
        x1 = bf16_normal(rng, (1, K))
        y1 = m.apply(model.proj, to_dev(x1, device))
        x70 = bf16_normal(rng, (70, K))
        y70 = m.apply(model.proj, to_dev(x70, device))
        steps.capture(tk)
        assert steps.check_through(tk) == (0,)
        np.testing.assert_array_equal(from_dev(y1), O.dense_a8(x1, *bank.expert())[0])
        got = O.bf16_to_f32(from_dev(y70)).astype(np.float64)
        ref = (O.bf16_to_f32(O.transform_bf16(x70)).astype(np.float64)
               @ O.bf16_to_f32(O.dequantize_bf16(*bank.expert())).astype(np.float64).T)
        cos = float((got.ravel() @ ref.ravel()) / (np.linalg.norm(got) * np.linalg.norm(ref)))
        assert cos >= 0.9999 and np.abs(got - ref).max() <= 1e-2 * np.abs(ref).max()
        tk = steps.open('bad input')
        x1[0, 5] = 0x7FC0                          # NaN
        m.apply(model.proj, to_dev(x1, device))
        steps.capture(tk)
        with pytest.raises(lifecycle.OrnithWorkerFault, match="'proj': 3"):
            steps.check_through(tk)
    finally:
        native.reset_binding()


# ---------------------------------------------------------------------------
# Production shared expert (fixed8, shared_kernel.py:33-62)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize('M', [1, 8, 13, 70])
def test_shared_fixed8_bit_exact(device, moe, shared_tables, M):
    """The reference's fixed8 shared expert (dense A8 gate/up, bf16 SiLU * up,
    dense A8 down, bf16 sigmoid gate) against the oracle, bit for bit; M = 13
    and 70 span the reference's eight-row chunks and the dense kernels'
    fused / separate activation paths."""
    import torch
    native = _native()
    w, d = moe
    silu, sigmoid = shared_tables
    print(f'shared fixed8 M={M}', flush=True)
    rng = np.random.default_rng(2100 + M)
    x = bf16_normal(rng, (M, 2048))
    ref, ref_flags = O.shared_fixed8(x, *w['s13'].expert(), *w['s2'].expert(), w['gate'][0], silu, sigmoid)
    ws = torch.empty(native.shared_fixed8_bytes(max(M, 8)), dtype=torch.uint8, device=device)
    out = torch.empty((M, 2048), dtype=torch.bfloat16, device=device)
    flags = _flags(device)
    native.shared_fixed8(to_dev(x, device), d['s13'][0], d['s13'][1], d['s2'][0], d['s2'][1],
                         to_dev(w['gate'][0], device), to_dev(silu, device), to_dev(sigmoid, device), ws, out, flags,
                         max(M, 8))
    _sync()
    np.testing.assert_array_equal(from_dev(out), ref)
    assert int(flags.item()) == ref_flags == 0


# ---------------------------------------------------------------------------
# Dense linear on the bf16 matrix cores, reading the 4-bit codes
# ---------------------------------------------------------------------------
@pytest.mark.parametrize('M,N,K', [(1120, 6144, 2048), (65, 96, 512), (300, 1040, 768), (257, 128, 8192)])
def test_dense_gemm_bf16_tolerance(device, M, N, K):
    """ornith_dense_g256_gemm_bf16 against fp64 products of the exact bf16
    operands (bf16(H128 x), bf16 dequantised weights): cosine >= 0.9999 and
    max |err| <= 1e-2 * max |ref|; partial row and column blocks included."""
    import torch
    from _ornith import Bank
    native = _native()
    print(f'dense gemm bf16 M={M} N={N} K={K}', flush=True)
    rng = np.random.default_rng(3000 + M)
    bank = Bank(rng, 0, N, K, tile=16)
    x = bf16_normal(rng, (M, K))
    Mp = (M + 15) // 16 * 16                      # the transformed rows, padded with zero rows
    ws = torch.empty(Mp * K * 2, dtype=torch.uint8, device=device)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=device)
    flags = _flags(device)
    xd, cd, md = to_dev(x, device), to_dev(bank.codes, device), to_dev(bank.meta, device)   # alive until the sync
    assert native.lib().ornith_dense_g256_gemm_bf16(native.ptr(xd), native.ptr(cd), native.ptr(md), native.ptr(ws),
                                                    ws.numel() - 2, native.ptr(out), native.ptr(flags), M, N, K,
                                                    native.stream(xd)) != 0                     # workspace too small
    st = native.lib().ornith_dense_g256_gemm_bf16(native.ptr(xd), native.ptr(cd), native.ptr(md), native.ptr(ws),
                                                  ws.numel(), native.ptr(out), native.ptr(flags), M, N, K,
                                                  native.stream(xd))
    assert st == 0
    _sync()
    xt = O.transform_bf16(x)
    # fragment order: (r, k) at ((r // 16 * K // 32 + k // 32) * 64 + 16 * (k % 32 // 8) + r % 16) * 8 + k % 8
    frag = from_dev(ws.view(torch.bfloat16)).reshape(Mp // 16, K // 32, 4, 16, 8)
    rows = frag.transpose(0, 3, 1, 2, 4).reshape(Mp, K)
    np.testing.assert_array_equal(rows[:M], xt)
    assert not rows[M:].view(np.uint16).any()
    got = O.bf16_to_f32(from_dev(out)).astype(np.float64)
    ref = (O.bf16_to_f32(xt).astype(np.float64)
           @ O.bf16_to_f32(O.dequantize_bf16(*bank.expert())).astype(np.float64).T)
    cos = float((got.ravel() @ ref.ravel()) / (np.linalg.norm(got) * np.linalg.norm(ref)))
    err = float(np.abs(got - ref).max() / np.abs(ref).max())
    print(f'  cosine {cos:.8f}  max rel err {err:.2e}', flush=True)
    assert cos >= 0.9999 and err <= 1e-2
    assert int(flags.item()) == 0
