"""Host-side policy of the package, on the CPU: phase plans for mixed
batches and the per-step lifecycle of the sticky native flags (with a fake
device transport, as the reference tests its lifecycle through an injected
transport, lifecycle.py:76)."""
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
