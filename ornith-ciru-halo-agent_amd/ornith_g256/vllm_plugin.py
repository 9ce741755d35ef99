"""vLLM registration of the ``ornith_g256`` quantization method.

Imports vLLM only inside ``register()``; nothing else in the package needs
it.  The mapping follows the reference's OrnithG256Config
(plugin-site/ornith_g256/config.py:7-58): the checkpoint's
quantize_config.json must be exactly {quant_method: ornith_g256,
group_size: 256, transform_block: 128, activation_bits: 8}; RoutedExperts of
``layers.N.mlp.experts`` get the routed G256 method, the dense suffixes below
the dense G256 linear, ``ParallelLMHead`` the W8 head, everything else stays
unquantized.  The routing contract is the one the routed kernels implement:
E256/top-8/H2048/I512, plain renormalised softmax top-8, one rank, no
EP/TP/SP, int32 top-k ids (moe_base.py:12-67).

Besides the quantized layers, the block's router gate (``layers.N.mlp.gate``,
an unquantized bf16 [256, 2048] linear) runs on this library's router kernel
(the reference routes it to its own row-dot, iu4_correctness/gates.py:113-139),
and the block's shared expert (``layers.N.mlp.shared_expert``) is served by
this library: for batches of at most 16 rows vLLM's shared-expert forward is
deferred to the block's routed launch, which runs it as the fused ninth slot
(moe_shared.py:19-77); the step's decode rows are then recomputed by fixed8
(shared_live.py:110-147), for larger batches after vLLM's own shared forward.

The methods themselves (weights, repack, apply) are those of methods.py; the
vLLM classes here only adapt vLLM's call signatures to them.
"""
from __future__ import annotations

import re

QUANT_CONFIG = dict(quant_method='ornith_g256', group_size=256, transform_block=128, activation_bits=8)
DENSE_SUFFIXES = ('.linear_attn.in_proj_qkvz', '.linear_attn.out_proj', '.self_attn.qkv_proj',
                  '.self_attn.o_proj', '.mlp.shared_expert.gate_up_proj', '.mlp.shared_expert.down_proj')
ROUTED_PREFIX = re.compile(r'layers\.[0-9]+\.mlp\.experts$')
ROUTER_GATE = re.compile(r'layers\.[0-9]+\.mlp\.gate$')


def check_quant_config(config: dict):
    """config.py:15-20: the checkpoint's quantization settings, exactly."""
    bad = {k: config.get(k) for k, v in QUANT_CONFIG.items() if config.get(k) != v}
    if bad:
        raise ValueError(f'ornith_g256 needs {QUANT_CONFIG}; got {bad}')


def check_routing_contract(layer):
    """moe_base.py:54-67: ordinary renormalised softmax top-8, nothing else."""
    if (getattr(layer, 'apply_router_weight_on_input', False) or getattr(layer, 'use_grouped_topk', False)
            or getattr(layer, 'custom_routing_function', None) is not None
            or getattr(layer, 'num_expert_group', None) is not None or getattr(layer, 'topk_group', None) is not None
            or getattr(layer, 'e_score_correction_bias', None) is not None
            or getattr(layer, 'scoring_func', 'softmax') != 'softmax' or not getattr(layer, 'renormalize', True)
            or getattr(layer, 'routed_scaling_factor', 1.0) != 1.0):
        raise ValueError('ornith_g256 routed experts need plain renormalised softmax top-8 routing')


def bridge_shared_experts(SharedExperts):
    """Wrap vLLM's SharedExperts.forward (once) so a shared expert this
    library serves (its MLP carries ``_ornith_shared``, set by
    methods.Runtime) is computed by the library:
      * at most 16 rows: no forward here; the output slot gets an empty
        buffer that the block's routed launch fills (fused ninth slot);
      * more rows: vLLM's forward, then the step's decode rows recomputed."""
    if getattr(SharedExperts, '_ornith_bridge', False):
        return
    from . import methods, native
    forward = SharedExperts.forward

    def bridged(self, shared_experts_input, order):
        shared = getattr(self._layer, '_ornith_shared', None)
        if shared is None:
            return forward(self, shared_experts_input, order)
        rows = shared_experts_input.shape[0]
        computes = order == self._determine_shared_experts_order(shared_experts_input)
        if rows <= methods.SharedExpert.fused_max_rows:
            if computes:
                shared.pending = shared_experts_input.new_empty(shared_experts_input.shape)
                self._output[self._output_idx] = shared.pending
            return None
        result = forward(self, shared_experts_input, order)
        if computes and native.decode_runs(rows):
            shared.decode_rows(shared.runtime, shared_experts_input, self._output[self._output_idx])
        return result

    SharedExperts.forward = bridged
    SharedExperts._ornith_bridge = True


def register():
    """Register OrnithG256Config with vLLM (raises ImportError without vLLM)."""
    import torch
    from vllm.model_executor.layers.fused_moe.fused_moe_method_base import FusedMoEMethodBase
    from vllm.model_executor.layers.linear import LinearBase, LinearMethodBase, UnquantizedLinearMethod
    from vllm.model_executor.layers.quantization import register_quantization_config
    from vllm.model_executor.layers.quantization.base_config import QuantizationConfig
    from vllm.model_executor.layers.vocab_parallel_embedding import ParallelLMHead
    from vllm.model_executor.layers.fused_moe.runner.shared_experts import SharedExperts

    from . import methods

    class LinearAdapter(LinearMethodBase):
        def __init__(self, prefix, head=False):
            self.prefix, self.head, self.impl = prefix, head, None

        def create_weights(self, layer, input_size_per_partition, output_partition_sizes, input_size, output_size,
                           params_dtype, **extra):
            if (input_size_per_partition != input_size or sum(output_partition_sizes) != output_size
                    or params_dtype != torch.bfloat16 or getattr(layer, 'tp_size', 1) != 1):
                raise ValueError(f'{self.prefix}: ornith_g256 linears are unsharded bf16')
            cls = methods.W8HeadMethod if self.head else methods.G256LinearMethod
            self.impl = cls(self.prefix, output_size, input_size)
            self.impl.create_weights(layer)
            layer.quant_method = self.impl

        def process_weights_after_loading(self, layer):
            self.impl.process_weights_after_loading(layer)

        def apply(self, layer, x, bias=None):
            return self.impl.apply(layer, x, bias)

    class RouterGateAdapter(UnquantizedLinearMethod):
        """vLLM's unquantized weights; the product through the router kernel."""

        def __init__(self, prefix):
            super().__init__()
            self.impl = methods.RouterGateMethod(prefix)

        def create_weights(self, layer, *args, **kwargs):
            super().create_weights(layer, *args, **kwargs)
            layer.quant_method = self.impl

        def apply(self, layer, x, bias=None):
            return self.impl.apply(layer, x, bias)

    class MoEAdapter(FusedMoEMethodBase):
        def __init__(self, moe, prefix):
            super().__init__(moe)
            parallel = moe.moe_parallel_config
            if any(getattr(parallel, k) != 1 for k in ('tp_size', 'ep_size', 'dp_size')) or parallel.use_ep:
                raise ValueError('ornith_g256 routed experts run on one rank without expert parallelism')
            if (moe.num_experts, moe.experts_per_token, moe.hidden_dim, moe.intermediate_size) != (256, 8, 2048, 512):
                raise ValueError('ornith_g256 routed experts are E256/top-8/H2048/I512')
            self.impl = methods.G256MoEMethod(prefix)

        @property
        def topk_indices_dtype(self):
            return torch.int32

        def create_weights(self, layer, num_experts, hidden_size, intermediate_size_per_partition, params_dtype,
                           **extra):
            self.impl.create_weights(layer)
            layer.quant_method = self.impl

        def process_weights_after_loading(self, layer):
            self.impl.process_weights_after_loading(layer)

        def apply(self, layer, x, topk_weights, topk_ids, shared_experts=None, shared_experts_input=None):
            shared = getattr(getattr(shared_experts, '_layer', None), '_ornith_shared', None)
            if shared is None or shared.pending is None:
                return self.impl.apply(layer, x, topk_weights, topk_ids)
            pending, shared.pending = shared.pending, None
            return self.impl.apply(layer, x, topk_weights, topk_ids, shared=shared, shared_out=pending,
                                   shared_input=shared_experts_input)

    @register_quantization_config('ornith_g256')
    class OrnithG256Config(QuantizationConfig):
        def __init__(self, config):
            super().__init__()
            check_quant_config(config)
            self.checkpoint_config = dict(config)

        @classmethod
        def get_name(cls):
            return 'ornith_g256'

        def get_supported_act_dtypes(self):
            return [torch.bfloat16]

        @classmethod
        def get_min_capability(cls):
            return 0

        @staticmethod
        def get_config_filenames():
            return ['quantize_config.json']

        @classmethod
        def from_config(cls, config):
            return cls(config)

        def get_quant_method(self, layer, prefix):
            from vllm.model_executor.layers.fused_moe.routed_experts import RoutedExperts
            if isinstance(layer, RoutedExperts):
                if not ROUTED_PREFIX.search(prefix):
                    raise ValueError(f'unsupported routed module {prefix}')
                check_routing_contract(layer)
                return MoEAdapter(layer.moe_config, prefix)
            if isinstance(layer, ParallelLMHead):
                return LinearAdapter(prefix, head=True)
            if isinstance(layer, LinearBase) and ROUTER_GATE.search(prefix):
                return RouterGateAdapter(prefix)
            if isinstance(layer, LinearBase):
                return LinearAdapter(prefix) if prefix.endswith(DENSE_SUFFIXES) else UnquantizedLinearMethod()
            return None

    bridge_shared_experts(SharedExperts)
    return OrnithG256Config
