"""The vLLM wiring on the CPU, against stub vLLM modules (vLLM is not
installed here): registration routes the block's router gate, the quantized
linears and the routed experts to this package's methods and bridges vLLM's
SharedExperts; the bridge defers a small batch's shared forward to the routed
launch and repairs the step's decode rows of a large one; the methods drive
the right native entries (the native calls are recorded, not run).

Reference hook points: the router gate (iu4_correctness/gates.py:113-139),
the fused shared slot (moe_shared.py:19-77), the fixed8 decode repair
(iu4_correctness/shared_live.py:110-147)."""
import sys
import types
from types import SimpleNamespace as NS

import pytest
import torch

from ornith_g256 import methods, native, vllm_plugin as V


# ---------------------------------------------------------------------------
# stub vLLM
# ---------------------------------------------------------------------------
class _LinearBase(torch.nn.Module):
    pass


class _LinearMethodBase:
    pass


class _Unquantized(_LinearMethodBase):
    def create_weights(self, layer, input_size_per_partition, output_partition_sizes, input_size, output_size,
                       params_dtype, **extra):
        layer.register_parameter('weight', torch.nn.Parameter(
            torch.empty((sum(output_partition_sizes), input_size_per_partition), dtype=params_dtype),
            requires_grad=False))

    def apply(self, layer, x, bias=None):
        return x @ layer.weight.t()


class _FusedMoEMethodBase:
    def __init__(self, moe):
        self.moe = moe


class _RoutedExperts(torch.nn.Module):
    pass


class _ParallelLMHead(torch.nn.Module):
    pass


class _QuantizationConfig:
    pass


class _SharedExperts:
    """vLLM's shared-expert runner: computes the shared MLP into its output
    slot when called with its own order."""

    def __init__(self, layer, order=0):
        self._layer, self._order, self._output, self._output_idx = layer, order, [None], 0

    def _determine_shared_experts_order(self, x):
        return self._order

    def forward(self, shared_experts_input, order):
        if order != self._determine_shared_experts_order(shared_experts_input):
            return None
        self._output[self._output_idx] = self._layer(shared_experts_input)


@pytest.fixture
def vllm_stub(monkeypatch):
    registered = {}

    def register_quantization_config(name):
        def deco(cls):
            registered[name] = cls
            return cls
        return deco

    mods = {
        'vllm': {}, 'vllm.model_executor': {}, 'vllm.model_executor.layers': {},
        'vllm.model_executor.layers.fused_moe': {},
        'vllm.model_executor.layers.fused_moe.fused_moe_method_base': {'FusedMoEMethodBase': _FusedMoEMethodBase},
        'vllm.model_executor.layers.fused_moe.routed_experts': {'RoutedExperts': _RoutedExperts},
        'vllm.model_executor.layers.fused_moe.runner': {},
        'vllm.model_executor.layers.fused_moe.runner.shared_experts': {'SharedExperts': _SharedExperts},
        'vllm.model_executor.layers.linear': {'LinearBase': _LinearBase, 'LinearMethodBase': _LinearMethodBase,
                                              'UnquantizedLinearMethod': _Unquantized},
        'vllm.model_executor.layers.quantization': {'register_quantization_config': register_quantization_config},
        'vllm.model_executor.layers.quantization.base_config': {'QuantizationConfig': _QuantizationConfig},
        'vllm.model_executor.layers.vocab_parallel_embedding': {'ParallelLMHead': _ParallelLMHead},
    }
    for name, attrs in mods.items():
        m = types.ModuleType(name)
        m.__dict__.update(attrs)
        monkeypatch.setitem(sys.modules, name, m)
    forward = _SharedExperts.forward
    yield registered
    _SharedExperts.forward = forward
    if hasattr(_SharedExperts, '_ornith_bridge'):
        del _SharedExperts._ornith_bridge


def _config(registered):
    cls = V.register()
    assert registered['ornith_g256'] is cls
    return cls(dict(quant_method='ornith_g256', group_size=256, transform_block=128, activation_bits=8))


# ---------------------------------------------------------------------------
# registration
# ---------------------------------------------------------------------------
def test_register_routes_gate_linears_and_experts(vllm_stub):
    cfg = _config(vllm_stub)
    gate = _LinearBase()
    m = cfg.get_quant_method(gate, 'model.layers.3.mlp.gate')
    assert type(m).__name__ == 'RouterGateAdapter'
    m.create_weights(gate, 2048, [256], 2048, 256, torch.bfloat16)
    assert isinstance(gate.quant_method, methods.RouterGateMethod) and gate.weight.shape == (256, 2048)
    lin = _LinearBase()
    assert type(cfg.get_quant_method(lin, 'model.layers.3.mlp.shared_expert.gate_up_proj')).__name__ == 'LinearAdapter'
    assert type(cfg.get_quant_method(lin, 'model.layers.3.linear_attn.in_proj_ba')) is _Unquantized
    assert type(cfg.get_quant_method(lin, 'model.layers.3.mlp.shared_expert_gate')) is _Unquantized
    experts = _RoutedExperts()
    experts.moe_config = NS(moe_parallel_config=NS(tp_size=1, ep_size=1, dp_size=1, use_ep=False), num_experts=256,
                            experts_per_token=8, hidden_dim=2048, intermediate_size=512)
    moe = cfg.get_quant_method(experts, 'model.layers.3.mlp.experts')
    assert type(moe).__name__ == 'MoEAdapter' and moe.topk_indices_dtype == torch.int32
    assert getattr(_SharedExperts, '_ornith_bridge', False)


# ---------------------------------------------------------------------------
# the shared-expert bridge
# ---------------------------------------------------------------------------
class _FakeShared:
    def __init__(self):
        self.pending, self.runtime, self.repaired = None, object(), []

    def decode_rows(self, rt, x, out):
        self.repaired.append((rt, x.shape[0], out))


class _MLP(torch.nn.Module):
    def forward(self, x):
        return x * 2


def test_bridge_defers_small_batches_to_the_routed_launch(vllm_stub):
    cfg = _config(vllm_stub)
    experts = _RoutedExperts()
    experts.moe_config = NS(moe_parallel_config=NS(tp_size=1, ep_size=1, dp_size=1, use_ep=False), num_experts=256,
                            experts_per_token=8, hidden_dim=2048, intermediate_size=512)
    adapter = cfg.get_quant_method(experts, 'model.layers.0.mlp.experts')
    calls = []
    adapter.impl.apply = lambda *a, **k: calls.append((a, k)) or 'routed'
    mlp = _MLP()
    mlp._ornith_shared = shared = _FakeShared()
    runner = _SharedExperts(mlp)
    x = torch.ones((5, 8))
    assert runner.forward(x, order=1) is None and shared.pending is None      # not its turn
    assert runner.forward(x, order=0) is None
    assert runner._output[0] is shared.pending and shared.pending.shape == x.shape
    pending = shared.pending
    assert adapter.apply(experts, x, 'w', 'ids', shared_experts=runner, shared_experts_input=x) == 'routed'
    (args, kw), = calls
    assert kw['shared'] is shared and kw['shared_out'] is pending and kw['shared_input'] is x
    assert shared.pending is None                                             # consumed
    adapter.apply(experts, x, 'w', 'ids', shared_experts=runner, shared_experts_input=x)
    assert 'shared' not in calls[-1][1]                                       # nothing pending: routed only


def test_bridge_repairs_decode_rows_of_large_batches(vllm_stub):
    _config(vllm_stub)
    mlp = _MLP()
    mlp._ornith_shared = shared = _FakeShared()
    runner = _SharedExperts(mlp)
    x = torch.ones((40, 8))
    runner.forward(x, order=0)
    assert torch.equal(runner._output[0], x * 2) and not shared.repaired     # no step phases: no decode rows
    with native.step_phases(((0, 30, True), (30, 40, False))):
        runner.forward(x, order=0)
        runner.forward(x, order=1)                                            # not its turn: no second repair
    (rt, rows, out), = shared.repaired
    assert rt is shared.runtime and rows == 40 and out is runner._output[0]
    plain = _SharedExperts(_MLP())                                            # a shared MLP the library does not serve
    plain.forward(x, order=0)
    assert torch.equal(plain._output[0], x * 2)


# ---------------------------------------------------------------------------
# the methods against recorded native calls
# ---------------------------------------------------------------------------
def _recorder(monkeypatch, name, effect=None):
    calls = []

    def fn(*a, **k):
        calls.append((a, k))
        if effect:
            effect(*a, **k)
    monkeypatch.setattr(native, name, fn)
    return calls


def _shared_expert():
    mlp = torch.nn.Module()
    mlp.gate_up_proj, mlp.down_proj, mlp.expert_gate = torch.nn.Module(), torch.nn.Module(), torch.nn.Module()
    mlp.gate_up_proj.quant_method = methods.G256LinearMethod('b.gate_up_proj', 1024, 2048)
    mlp.down_proj.quant_method = methods.G256LinearMethod('b.down_proj', 2048, 512)
    mlp.gate_up_proj.quant_method.slot = 3
    mlp.expert_gate.weight = torch.nn.Parameter(torch.zeros((1, 2048), dtype=torch.bfloat16), requires_grad=False)
    sh = methods.SharedExpert('model.layers.0.mlp.shared_expert', mlp)
    sh.banks = tuple(torch.full((2,), i) for i in range(4))
    return sh


def _runtime(**kw):
    rt = NS(routed_storage_n32=False, routed_decode_n32=False, routed_n32_max_rows=8, workspace=torch.zeros(4),
            slots=tuple(torch.zeros(1, dtype=torch.int32) for _ in range(4)), capacity=64,
            shared_tables=('silu', 'sigmoid'))
    rt.__dict__.update(kw)
    return rt


def test_router_gate_forms_logits_and_the_shared_gate_logit(monkeypatch):
    sh = _shared_expert()
    gate = methods.RouterGateMethod('model.layers.0.mlp.gate')
    gate.shared = sh

    def fill(x, w, bias, shared_w, logits, weights, ids, shared_logit):
        assert bias is None and shared_w.shape == (2048,)
        logits.copy_(torch.arange(logits.numel(), dtype=torch.float32).view_as(logits))
        shared_logit.fill_(1.5)
    calls = _recorder(monkeypatch, 'router_topk', fill)
    layer = NS(weight=torch.zeros((256, 2048), dtype=torch.bfloat16))
    x = torch.zeros((2, 3, 2048), dtype=torch.bfloat16)
    out = gate.apply(layer, x)
    assert out.shape == (2, 3, 256) and out.dtype == torch.float32
    assert torch.equal(out.reshape(6, 256)[1], torch.arange(257, 257 + 256, dtype=torch.float32))
    assert len(calls) == 1 and torch.equal(sh.gate_logit, torch.full((6,), 1.5, dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        gate.apply(layer, x, bias=torch.zeros(256))


@pytest.mark.parametrize('mode,tile', [('n16', 16), ('storage_n32', 32), ('decode_n32', 32)])
def test_moe_apply_with_shared_runs_fused_slot_then_fixed8_on_decode_rows(monkeypatch, mode, tile):
    sh = _shared_expert()
    m = methods.G256MoEMethod('model.layers.0.mlp.experts')
    m.runtime = rt = _runtime(routed_storage_n32=mode == 'storage_n32', routed_decode_n32=mode == 'decode_n32')
    m.slot = 1
    layer = NS(_ornith_loader=NS(sealed=True), w13_tilebank_codes='c13', w13_tilebank_metadata='m13',
               w2_tilebank_codes='c2', w2_tilebank_metadata='m2', w13_n32_codes='n13', w13_n32_metadata='nm13',
               w2_n32_codes='n2', w2_n32_metadata='nm2')
    fused = _recorder(monkeypatch, 'routed_shared_tables', lambda *a, **k: a[16].fill_(7))
    fixed = _recorder(monkeypatch, 'shared_fixed8', lambda *a, **k: a[9].fill_(9))
    T = 5
    x = torch.zeros((T, 2048), dtype=torch.bfloat16)
    shared_out = torch.zeros_like(x)
    sh.gate_logit = torch.zeros((T,), dtype=torch.bfloat16)
    with native.step_phases(((0, 2, True), (2, 5, False))):
        m.apply(layer, x, 'w', 'ids', shared=sh, shared_out=shared_out)
    (a, k), = fused
    routed = ('n13', 'nm13', 'n2', 'nm2') if mode == 'decode_n32' else ('c13', 'm13', 'c2', 'm2')
    assert a[3:7] == routed and k['tile'] == tile
    assert all(a[7 + i] is sh.banks[i] for i in range(4)) and a[17] is rt.slots[1] and a[18] == 16
    assert sh.gate_logit is None                                              # one launch per router launch
    (a, k), = fixed                                                           # decode rows 2..5 only
    assert a[0].shape == (3, 2048) and a[10] is rt.slots[3]
    assert torch.all(shared_out[:2] == 7) and torch.all(shared_out[2:] == 9)
    with pytest.raises(RuntimeError, match='gate logit'):
        m.apply(layer, x, 'w', 'ids', shared=sh, shared_out=shared_out)       # no router launch this step
    with pytest.raises(ValueError):
        m.apply(layer, torch.zeros((17, 2048)), 'w', 'ids', shared=sh, shared_out=torch.zeros((17, 2048)))


def test_step_runs_cover_every_row():
    from ornith_g256 import phases
    assert phases.step_runs([3, 0, 2, 4], [True, False, False, True]) == ((0, 3, True), (3, 5, False), (5, 9, True))
    assert phases.step_runs([1, 1], [False, False]) == ((0, 2, False),)
    with native.step_phases(((0, 3, True), (3, 5, False), (5, 9, True))):
        assert native.decode_runs(9) == ((3, 5),)
        assert native.decode_runs(4) == ((3, 4),)
        assert native.decode_runs(3) == ()
    assert native.decode_runs(9) == ()
