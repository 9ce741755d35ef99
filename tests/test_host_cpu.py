"""Host-side policy of the package, on the CPU: phase plans for mixed
batches, the per-step lifecycle of the sticky native flags (with a fake
device transport, as the reference tests its lifecycle through an injected
transport, lifecycle.py:76), strict checkpoint admission, the repack entry's
argument checks, the quantized-layer methods before binding and the vLLM
registration's contracts."""
import pytest

from ornith_g256 import lifecycle as L
from ornith_g256 import phases as P


# ---------------------------------------------------------------------------
# Phase plans (phase_dispatch.py:13-34)
# ---------------------------------------------------------------------------
def test_plan_merges_consecutive_same_phase_requests():
    plan = P.plan_segments([10, 20, 40, 5, 30], [False, False, True, True, False])
    assert plan == ((0, 30, False), (30, 75, True), (75, 105, False))


def test_plan_is_empty_for_small_or_single_phase_batches():
    assert P.plan_segments([30, 34], [False, True]) == ()            # 64 rows: not more than 64
    assert P.plan_segments([30, 35], [False, True]) == ((0, 30, False), (30, 65, True))
    assert P.plan_segments([100, 50], [True, True]) == ()
    assert P.plan_segments([100, 50], [False, False]) == ()
    assert P.plan_segments([], []) == ()


def test_plan_skips_empty_requests_and_rejects_bad_input():
    assert P.plan_segments([40, 0, 40], [False, True, True]) == ((0, 40, False), (40, 80, True))
    with pytest.raises(ValueError):
        P.plan_segments([1, 2], [True])
    with pytest.raises(ValueError):
        P.plan_segments([-1, 80], [True, False])


def test_request_phases():
    assert P.request_phases([0, 10, 12], [12, 10, 12]) == [True, False, False]


def test_phase_context_selects_segments_per_call():
    from ornith_g256 import native
    assert native._active_plan(200) == ()
    with native.phase_segments([(0, 40, False), (40, 100, True)]):
        assert native._active_plan(100) == ((0, 40, False), (40, 100, True))
        # rows past the plan run as prefill; batches shorter than the plan run unsplit
        assert native._active_plan(130) == ((0, 40, False), (40, 100, True), (100, 130, True))
        assert native._active_plan(99) == ()
    assert native._active_plan(100) == ()


# ---------------------------------------------------------------------------
# Flag lifecycle (lifecycle.py:69-193)
# ---------------------------------------------------------------------------
class FakeTransport:
    """Device flags as a Python list; snapshots copy it."""

    def __init__(self, n):
        self.flags = [0] * n
        self.log = []

    def width(self):
        return len(self.flags)

    def new_slot(self):
        return {'copy': None}

    def clear(self):
        self.log.append('clear')
        self.flags = [0] * len(self.flags)

    def queue(self, slot):
        self.log.append('queue')
        slot['copy'] = list(self.flags)

    def finish(self, slot):
        self.log.append('finish')
        return tuple(slot['copy'])


def _lifecycle(n=3, inflight=2):
    t = FakeTransport(n)
    return L.StepLifecycle([f'layers.{i}.mlp' for i in range(n)], inflight, transport=t), t


def test_healthy_steps_clear_snapshot_and_complete():
    lc, t = _lifecycle()
    for i in range(5):
        tk = lc.begin(f'step{i}')
        lc.snapshot(tk)
        assert lc.complete(tk) == (0, 0, 0)
    assert t.log[:3] == ['clear', 'queue', 'finish']
    assert lc.clears == lc.snapshots == lc.completed == 5


def test_a_raised_flag_poisons_the_worker():
    lc, t = _lifecycle()
    tk = lc.begin('decode')
    t.flags[1] = 4                                    # invalid expert id in layer 1
    lc.snapshot(tk)
    with pytest.raises(L.OrnithWorkerFault, match='layers.1.mlp'):
        lc.complete(tk)
    with pytest.raises(L.OrnithWorkerFault):
        lc.begin('next')                              # poisoned: no further steps


def test_a_later_healthy_step_cannot_hide_an_earlier_fault():
    lc, t = _lifecycle(inflight=3)
    first = lc.begin('a')
    t.flags[0] = 8
    lc.snapshot(first)
    second = lc.begin('b')                            # clears the device flags again
    lc.snapshot(second)
    with pytest.raises(L.OrnithWorkerFault, match="step 0 \\(a\\)"):
        lc.complete(second)


def test_completion_requires_a_snapshot_and_the_pool_is_bounded():
    lc, _ = _lifecycle(inflight=2)
    a = lc.begin('a')
    lc.begin('b')
    with pytest.raises(RuntimeError, match='in flight'):
        lc.begin('c')
    with pytest.raises(RuntimeError, match='snapshot'):
        lc.complete(a)


def test_abort_captures_flags_and_reraises():
    lc, t = _lifecycle()
    tk = lc.begin('prefill')
    with pytest.raises(ValueError, match='boom'):
        lc.abort(tk, ValueError('boom'))
    assert isinstance(lc.fault, L.OrnithWorkerFault)
    lc2, t2 = _lifecycle()
    tk2 = lc2.begin('prefill')
    t2.flags[2] = 1
    with pytest.raises(L.OrnithWorkerFault) as info:
        lc2.abort(tk2, ValueError('boom'))
    assert isinstance(info.value.__cause__, ValueError)


def test_drain_checks_every_pending_step():
    lc, t = _lifecycle(inflight=3)
    lc.begin('a')
    lc.begin('b')
    lc.drain()
    assert lc.completed == 2
    lc.begin('c')
    t.flags[0] = 32
    with pytest.raises(L.OrnithWorkerFault):
        lc.drain()


def test_bad_construction():
    with pytest.raises(ValueError):
        L.StepLifecycle(['a'], 0, transport=FakeTransport(1))
    with pytest.raises(ValueError):
        L.StepLifecycle(['a', 'b'], 1, transport=FakeTransport(1))


# ---------------------------------------------------------------------------
# Checkpoint admission (loader.py:17-54, method.py:12-32)
# ---------------------------------------------------------------------------
def _meta(shape, scale=0.01, offset=-0.08):
    import torch
    pair = torch.tensor([scale, offset], dtype=torch.float16).view(torch.int32)
    return pair.expand(shape).contiguous().view(torch.uint32)


def test_bank_loader_is_strict():
    import torch
    from ornith_g256 import storage as S
    shapes = S.dense_shapes(64, 512)
    ld = S.BankLoader(shapes)
    codes = torch.zeros(shapes['g256_codes'], dtype=torch.uint32)
    with pytest.raises(S.AdmissionError, match='expected'):
        ld.load('g256_codes', torch.zeros(shapes['g256_codes'], dtype=torch.int32))       # dtype
    with pytest.raises(S.AdmissionError, match='expected'):
        ld.load('g256_codes', torch.zeros((4, 2, 32, 32), dtype=torch.uint32))           # N32 instead of N16
    with pytest.raises(S.AdmissionError, match='unsupported'):
        ld.load('g256_extra', codes)
    ld.load('g256_codes', codes)
    with pytest.raises(S.AdmissionError, match='duplicate'):
        ld.load('g256_codes', codes)
    with pytest.raises(S.AdmissionError, match='incomplete'):
        ld.seal()
    ld.load('g256_metadata', _meta(shapes['g256_metadata']))
    ld.seal()
    with pytest.raises(S.AdmissionError, match='sealed'):
        ld.load('g256_metadata', _meta(shapes['g256_metadata']))


@pytest.mark.parametrize('scale,offset,match', [(2 ** -15, 0.0, '2\\^-14'), (float('nan'), 0.0, 'non-finite'),
                                                (0.01, float('inf'), 'non-finite')])
def test_metadata_admission(scale, offset, match):
    from ornith_g256 import storage as S
    shapes = S.dense_shapes(32, 256)
    with pytest.raises(S.AdmissionError, match=match):
        S.BankLoader(shapes).load('g256_metadata', _meta(shapes['g256_metadata'], scale, offset))


def test_routed_shapes_and_prefixed_keys():
    import torch
    from ornith_g256 import storage as S
    shapes = S.routed_shapes(experts=2)
    assert shapes['w13_tilebank_codes'] == (2, 64, 8, 32, 16) and shapes['w2_tilebank_metadata'] == (2, 128, 2, 16)
    ld = S.BankLoader(shapes)
    with pytest.raises(S.AdmissionError, match='key'):
        list(ld.load_prefixed([('experts.w13_tilebank_codes', torch.zeros(1))]))
    items = [(S.ROUTED_PREFIX + k, torch.zeros(v, dtype=torch.uint32) if k.endswith('codes') else _meta(v))
             for k, v in shapes.items()]
    assert list(ld.load_prefixed(items)) == [k for k, _ in items]
    ld.seal()
    with pytest.raises(S.AdmissionError):
        S.dense_shapes(12304, 2048)


def test_repack_abi_validation():
    import ctypes as C
    from ornith_g256 import native
    h = native.lib()
    p = C.c_void_p
    assert h.ornith_repack_n16_to_n32(None, None, None, None, 0, 1024, 2048, None) == 0
    assert h.ornith_repack_n16_to_n32(p(0x1000), p(0x2000), p(0x3000), p(0x4000), 1, 1040, 2048, None) == 1  # N % 32
    assert h.ornith_repack_n16_to_n32(p(0x1000), p(0x2000), p(0x3000), p(0x4000), 1, 1024, 2000, None) == 1  # K % 256
    assert h.ornith_repack_n16_to_n32(None, p(0x2000), p(0x3000), p(0x4000), 1, 1024, 2048, None) == 1
    big = 1 << 32
    assert h.ornith_repack_n16_to_n32(p(big), p(2 * big), p(big + 64), p(4 * big), 1, 1024, 2048, None) == 1   # overlap


# ---------------------------------------------------------------------------
# Methods and the vLLM registration (method.py, config.py, moe_base.py)
# ---------------------------------------------------------------------------
def test_methods_register_n16_banks_and_refuse_unbound_use():
    import torch
    from ornith_g256 import methods as M
    layer = torch.nn.Module()
    m = M.G256MoEMethod('model.layers.0.mlp.experts')
    m.create_weights(layer)
    assert layer.w13_tilebank_codes.shape == (256, 64, 8, 32, 16) and layer.w13_tilebank_codes.dtype == torch.uint32
    with pytest.raises(RuntimeError):
        m.apply(layer, torch.zeros(1, 2048), torch.zeros(1, 8), torch.zeros(1, 8, dtype=torch.int32))
    dense = torch.nn.Module()
    d = M.G256LinearMethod('model.layers.0.self_attn.o_proj', 2048, 4096)
    d.create_weights(dense)
    assert dense.g256_codes.shape == (128, 16, 32, 16)
    with pytest.raises(ValueError):
        M.W8HeadMethod('lm_head', 151936, 2048)


def test_vllm_plugin_contracts():
    from types import SimpleNamespace as NS
    from ornith_g256 import vllm_plugin as V
    V.check_quant_config(dict(quant_method='ornith_g256', group_size=256, transform_block=128, activation_bits=8))
    with pytest.raises(ValueError):
        V.check_quant_config(dict(quant_method='ornith_g256', group_size=128, transform_block=128, activation_bits=8))
    V.check_routing_contract(NS(scoring_func='softmax', renormalize=True))
    with pytest.raises(ValueError):
        V.check_routing_contract(NS(scoring_func='sigmoid', renormalize=True))
    with pytest.raises(ValueError):
        V.check_routing_contract(NS(e_score_correction_bias=object()))
    assert V.ROUTED_PREFIX.search('model.language_model.layers.12.mlp.experts')
    try:
        import vllm  # noqa: F401
    except ImportError:
        with pytest.raises(ImportError):
            V.register()
