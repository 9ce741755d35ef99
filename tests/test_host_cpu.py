"""Host-side policy of the package, on the CPU: phase plans for mixed
batches, the per-step checks of the sticky native flags (with a list-backed
ring standing in for the device and its pinned snapshots), strict checkpoint admission, the repack entry's
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
# Per-step flag checks (policy of lifecycle.py:69-193)
# ---------------------------------------------------------------------------
class ListRing:
    """Device flags as a Python list; ring rows are list copies."""

    def __init__(self, n, depth):
        self.flags = [0] * n
        self.slots = n
        self.rows = [None] * depth
        self.log = []

    def zero(self):
        self.log.append('zero')
        self.flags = [0] * self.slots

    def capture(self, row):
        self.log.append(f'capture{row}')
        self.rows[row] = list(self.flags)

    def read(self, row):
        self.log.append(f'read{row}')
        return tuple(self.rows[row])


def _steps(n=3, depth=2):
    ring = ListRing(n, depth)
    return L.StepFlags([f'layers.{i}.mlp' for i in range(n)], depth, ring=ring), ring


def test_healthy_steps_zero_capture_and_check():
    sf, ring = _steps()
    for i in range(5):
        s = sf.open(f'step{i}')
        assert s == i
        sf.capture(s)
        assert sf.check_through(s) == (0, 0, 0)
    assert ring.log[:3] == ['zero', 'capture0', 'read0']
    assert ring.log[3:6] == ['zero', 'capture1', 'read1']      # step 1 uses ring row 1
    assert sf.zeroed == sf.captured == sf.read_rows == 5


def test_a_raised_flag_poisons_the_worker():
    sf, ring = _steps()
    s = sf.open('decode')
    ring.flags[1] = 4                                 # invalid expert id in layer 1
    sf.capture(s)
    with pytest.raises(L.OrnithWorkerFault, match='layers.1.mlp'):
        sf.check_through(s)
    with pytest.raises(L.OrnithWorkerFault):
        sf.open('next')                               # poisoned: no further steps


def test_a_later_healthy_step_cannot_hide_an_earlier_fault():
    sf, ring = _steps(depth=3)
    first = sf.open('a')
    ring.flags[0] = 8
    sf.capture(first)
    second = sf.open('b')                             # zeroes the device flags again
    sf.capture(second)
    with pytest.raises(L.OrnithWorkerFault, match="step 0 \\(a\\)"):
        sf.check_through(second)


def test_checking_a_later_step_keeps_the_earlier_flags():
    sf, ring = _steps(depth=3)
    a, b = sf.open('a'), sf.open('b')
    sf.capture(a)
    sf.capture(b)
    assert sf.check_through(b) == (0, 0, 0)
    assert sf.checked == 2
    assert sf.check_through(a) == (0, 0, 0)           # kept for its own caller
    with pytest.raises(RuntimeError, match='not open'):
        sf.check_through(a)                           # taken once


def test_check_requires_a_capture_and_the_ring_is_bounded():
    sf, _ = _steps(depth=2)
    a = sf.open('a')
    sf.open('b')
    with pytest.raises(RuntimeError, match='steps are open'):
        sf.open('c')
    with pytest.raises(RuntimeError, match='captured'):
        sf.check_through(a)
    with pytest.raises(RuntimeError, match='not open'):
        sf.capture(7)


def test_ring_rows_are_reused_in_order():
    sf, ring = _steps(depth=2)
    for i in range(6):
        s = sf.open(str(i))
        sf.capture(s)
        if i % 2:
            sf.check_through(s)
    assert [e for e in ring.log if e.startswith('capture')] == ['capture0', 'capture1'] * 3


def test_fail_captures_flags_and_reraises():
    sf, ring = _steps()
    s = sf.open('prefill')
    with pytest.raises(ValueError, match='boom'):
        sf.fail(s, ValueError('boom'))
    assert isinstance(sf.fault, L.OrnithWorkerFault)
    sf2, ring2 = _steps()
    s2 = sf2.open('prefill')
    ring2.flags[2] = 1
    with pytest.raises(L.OrnithWorkerFault) as info:
        sf2.fail(s2, ValueError('boom'))
    assert isinstance(info.value.__cause__, ValueError)


def test_a_failing_device_copy_poisons():
    sf, ring = _steps()

    def broken(row):
        raise OSError('copy engine gone')
    ring.capture = broken
    s = sf.open('x')
    with pytest.raises(L.OrnithWorkerFault, match='copying'):
        sf.capture(s)
    with pytest.raises(L.OrnithWorkerFault):
        sf.open('y')


def test_flush_checks_every_open_step():
    sf, ring = _steps(depth=3)
    sf.open('a')
    sf.open('b')
    sf.flush()
    assert sf.read_rows == 2 and sf.checked == 2
    sf.open('c')
    ring.flags[0] = 32
    with pytest.raises(L.OrnithWorkerFault):
        sf.flush()


def test_bad_construction():
    with pytest.raises(ValueError):
        L.StepFlags(['a'], 0, ring=ListRing(1, 1))
    with pytest.raises(ValueError):
        L.StepFlags(['a', 'b'], 1, ring=ListRing(1, 1))


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
