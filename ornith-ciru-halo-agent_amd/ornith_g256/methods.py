"""Quantized-layer methods and the worker runtime, without vLLM.

These are the parts of the reference plugin that own weights and call the
native ops (plugin-site/ornith_g256/method.py, runtime.py), written against
plain ``torch.nn.Module`` layers so they run with or without vLLM; the vLLM
registration that routes vLLM's layers to them is in vllm_plugin.py.

* ``G256LinearMethod`` - a dense G256 linear: N16 banks
  [N/16, K/256, 32, 16] / [N/16, K/256, 16] (method.py:35-62).
* ``W8HeadMethod`` - the W8 G128 LM head: [15520, 128, 4, 16] words and
  fp16 scales [248320, 16], applied in chunks of 64 rows (method.py:65-88).
* ``G256MoEMethod`` - the routed experts: four N16 banks
  (method.py:100-122), optionally repacked to N32 once on the GPU
  (method.py:124-158), and ``apply`` (method.py:165-183).
* ``RouterGateMethod`` - a MoE block's router gate: fp32 logits from this
  library's router kernel (the reference routes the gate to its own row-dot,
  iu4_correctness/gates.py:113-139), and in the same launch the block's
  shared-expert gate logit.
* ``SharedExpert`` - a MoE block's always-on shared expert: the fused ninth
  routed slot for batches of at most 16 rows (moe_shared.py:19-77) and the
  ``fixed8`` recompute of the step's decode rows (shared_live.py:110-147).
* ``Runtime`` - binds every method to one workspace arena and one sticky
  flag slot per layer (runtime.py:13-97).
"""
from __future__ import annotations

import torch

from . import native, storage


def _register(layer, shapes, dtypes=None):
    dtypes = dtypes or {k: torch.uint32 for k in shapes}
    for name, shape in shapes.items():
        layer.register_parameter(name, torch.nn.Parameter(torch.empty(shape, dtype=dtypes[name]), requires_grad=False))
    loader = storage.BankLoader(shapes, dtypes)
    layer._ornith_loader = loader

    def load(name, value):
        with torch.no_grad():
            loader.load(name, value)
            getattr(layer, name).data = loader.loaded[name].to(getattr(layer, name).device)
    layer.load_packed = load
    return loader


class G256LinearMethod:
    fields = ('g256_codes', 'g256_metadata')

    def __init__(self, prefix, n, k):
        self.prefix, self.n, self.k = prefix, int(n), int(k)
        self.runtime, self.slot = None, None

    def create_weights(self, layer):
        _register(layer, storage.dense_shapes(self.n, self.k))

    def process_weights_after_loading(self, layer):
        layer._ornith_loader.seal()

    def apply(self, layer, x, bias=None):
        if self.runtime is None or not layer._ornith_loader.sealed or bias is not None:
            raise RuntimeError(f'{self.prefix}: needs sealed weights, no bias and a bound runtime')
        shape = x.shape[:-1]
        x = x.reshape(-1, self.k).contiguous()
        out = torch.empty((x.shape[0], self.n), dtype=x.dtype, device=x.device)
        rt = self.runtime
        native.dense_out(x, layer.g256_codes, layer.g256_metadata, rt.workspace, out, rt.slots[self.slot],
                         rt.capacity, self.n, self.k, rt.dense_geometry, rt.dense_a8_max_rows)
        return out.view(*shape, self.n)


class W8HeadMethod(G256LinearMethod):
    fields = ('head_tilebank_codes', 'head_scales')

    def __init__(self, prefix, n=native.HEAD_VOCAB, k=native.HIDDEN):
        if (n, k) != (native.HEAD_VOCAB, native.HIDDEN):
            raise ValueError('the W8 head is the full 248320 x 2048 vocabulary projection')
        super().__init__(prefix, n, k)

    def create_weights(self, layer):
        _register(layer, {'head_tilebank_codes': (self.n // 16, self.k // 16, 4, 16), 'head_scales': (self.n, 16)},
                  {'head_tilebank_codes': torch.uint32, 'head_scales': torch.float16})

    def apply(self, layer, x, bias=None):
        if self.runtime is None or not layer._ornith_loader.sealed or bias is not None:
            raise RuntimeError(f'{self.prefix}: needs sealed weights, no bias and a bound runtime')
        x = x.reshape(-1, self.k).contiguous()
        out = torch.empty((x.shape[0], self.n), dtype=x.dtype, device=x.device)
        rt = self.runtime
        for start in range(0, x.shape[0], native.HEAD_MAX_ROWS):
            end = start + native.HEAD_MAX_ROWS
            native.head_out(x[start:end], layer.head_tilebank_codes, layer.head_scales, rt.workspace,
                            out[start:end], rt.slots[self.slot], rt.head_geometry)
        return out


class G256MoEMethod:
    experts, hidden, inter, top = 256, 2048, 512, 8

    def __init__(self, prefix):
        self.prefix = prefix
        self.runtime, self.slot = None, None

    def create_weights(self, layer):
        _register(layer, storage.routed_shapes(self.experts, self.hidden, self.inter))
        layer._ornith_storage_n32 = False

    def process_weights_after_loading(self, layer):
        layer._ornith_loader.seal()

    def prepare_n32(self, layer, replace=False):
        """Repack the loaded N16 banks to N32 on the GPU once: replacing them
        (sole N32 storage) or as extra copies for small decode batches.
        Returns the bytes written."""
        if not layer._ornith_loader.sealed or self.runtime is not None:
            raise RuntimeError(f'{self.prefix}: N32 banks are prepared after loading and before binding')
        if layer._ornith_storage_n32 or hasattr(layer, 'w13_n32_codes'):
            raise RuntimeError(f'{self.prefix}: N32 banks are prepared once')
        total = 0
        with torch.no_grad():
            for proj, n, k in (('w13', 2 * self.inter, self.hidden), ('w2', self.hidden, self.inter)):
                codes, meta = getattr(layer, f'{proj}_tilebank_codes'), getattr(layer, f'{proj}_tilebank_metadata')
                c32, m32 = storage.repack_n32(codes, meta, n, k)
                if replace:
                    getattr(layer, f'{proj}_tilebank_codes').data = c32
                    getattr(layer, f'{proj}_tilebank_metadata').data = m32
                else:
                    layer.register_buffer(f'{proj}_n32_codes', c32, persistent=False)
                    layer.register_buffer(f'{proj}_n32_metadata', m32, persistent=False)
                total += c32.numel() * 4 + m32.numel() * 4
        layer._ornith_storage_n32 = bool(replace)
        return total

    def apply(self, layer, x, topk_weights, topk_ids, shared=None, shared_out=None, shared_input=None):
        """Routed experts of x (bf16 [T, 2048]) with vLLM's top-8 weights and
        ids; returns the routed output.  With `shared` (the block's
        SharedExpert) and `shared_out` (bf16 [T, 2048]), the shared expert's
        output is written to `shared_out` too: by the fused ninth slot in the
        same launch (T <= 16; the slot reads x), then the step's decode rows
        by fixed8 from `shared_input` (default x)."""
        rt = self.runtime
        if rt is None or not layer._ornith_loader.sealed:
            raise RuntimeError(f'{self.prefix}: needs sealed weights and a bound runtime')
        out = torch.empty_like(x)
        banks = (layer.w13_tilebank_codes, layer.w13_tilebank_metadata, layer.w2_tilebank_codes,
                 layer.w2_tilebank_metadata)
        if shared is not None:
            if shared_out is None or shared_out.shape != x.shape or x.shape[0] > SharedExpert.fused_max_rows:
                raise ValueError(f'{self.prefix}: the fused shared slot takes at most '
                                 f'{SharedExpert.fused_max_rows} rows and a [T, 2048] shared output')
            if rt.routed_storage_n32:
                routed, tile = banks, 32
            elif rt.routed_decode_n32:
                routed, tile = (layer.w13_n32_codes, layer.w13_n32_metadata, layer.w2_n32_codes,
                                layer.w2_n32_metadata), 32
            else:
                routed, tile = banks, 16
            shared.fused(rt, x, topk_weights, topk_ids, routed, tile, out, shared_out, rt.slots[self.slot])
            shared.decode_rows(rt, x if shared_input is None else shared_input, shared_out)
            return out
        if rt.routed_decode_n32:
            native.routed_out_n32(x, topk_weights, topk_ids, *banks, layer.w13_n32_codes, layer.w13_n32_metadata,
                                  layer.w2_n32_codes, layer.w2_n32_metadata, rt.workspace, out,
                                  rt.slots[self.slot], rt.capacity, rt.routed_n32_max_rows)
        else:
            native.routed_out(x, topk_weights, topk_ids, *banks, rt.workspace, out, rt.slots[self.slot],
                              rt.capacity)
        return out


class RouterGateMethod:
    """The router gate of a MoE block (an unquantized bf16 [256, 2048]
    linear): fp32 logits [T, 256] in this library's declared reduction order
    (ornith_router_topk).  When the block's shared expert is bound, the same
    launch also forms its bf16 gate logit and hands it to the SharedExpert
    for the block's routed launch that follows in the same step."""

    def __init__(self, prefix):
        self.prefix = prefix
        self.runtime, self.slot, self.shared = None, None, None

    def process_weights_after_loading(self, layer):
        pass

    def apply(self, layer, x, bias=None):
        w = layer.weight
        if bias is not None or w.dtype != torch.bfloat16 or tuple(w.shape) != (native.EXPERTS, native.HIDDEN):
            raise ValueError(f'{self.prefix}: the router gate is a bias-free bf16 [256, 2048] linear')
        shape = x.shape[:-1]
        x2 = x.reshape(-1, native.HIDDEN)
        if x2.stride(1) != 1:
            x2 = x2.contiguous()
        T = x2.shape[0]
        logits = torch.empty((T, native.EXPERTS + 1), dtype=torch.float32, device=x.device)
        weights = torch.empty((T, native.TOP), dtype=torch.float32, device=x.device)
        ids = torch.empty((T, native.TOP), dtype=torch.int32, device=x.device)
        gate_logit = torch.empty((T,), dtype=torch.bfloat16, device=x.device)
        native.router_topk(x2, w.contiguous(), None, None if self.shared is None else self.shared.gate_weight,
                           logits, weights, ids, gate_logit)
        if self.shared is not None:
            self.shared.gate_logit = gate_logit
        return logits[:, :native.EXPERTS].contiguous().view(*shape, native.EXPERTS)


class SharedExpert:
    """The always-on shared expert of one MoE block: `mlp` holds the dense
    G256 linears gate_up_proj [1024, 2048] and down_proj [2048, 512] (bound
    to G256LinearMethod) and the bf16 gate row expert_gate.weight [1, 2048].

    * ``prepare`` makes N32 copies of the two dense banks once, on the GPU
      (the layout the fused slot and fixed8 read; the N16 banks stay for the
      dense linears).
    * ``fused`` runs the routed experts and this expert as a ninth slot in
      one launch (at most 16 rows; SiLU and sigmoid from the reference's
      tables), with the gate logit the block's router launch formed.
    * ``decode_rows`` recomputes the step's decode rows with fixed8 (the
      reference's decode arithmetic: A8 dense gate/up and down, bf16 SiLU·up,
      bf16 sigmoid gate), overwriting those rows of the shared output.
    """
    fused_max_rows = 16

    def __init__(self, prefix, mlp):
        gu, dn = mlp.gate_up_proj, mlp.down_proj
        for lin, nk in ((gu, (2 * native.INTER, native.HIDDEN)), (dn, (native.HIDDEN, native.INTER))):
            m = getattr(lin, 'quant_method', None)
            if type(m) is not G256LinearMethod or (m.n, m.k) != nk:
                raise ValueError(f'{prefix}: shared expert projections must be G256 linears {nk}')
        g = mlp.expert_gate.weight
        if g.dtype != torch.bfloat16 or tuple(g.shape) != (1, native.HIDDEN):
            raise ValueError(f'{prefix}: expert_gate must be a bf16 [1, 2048] row')
        self.prefix, self.mlp = prefix, mlp
        self.banks = None              # N32 gate_up codes, meta, down codes, meta
        self.gate_logit = None         # bf16 [T] from this step's router launch
        self.pending = None            # shared output buffer a deferred vLLM forward left
        self.runtime = None

    @property
    def gate_weight(self):
        return self.mlp.expert_gate.weight.reshape(-1)

    def prepare(self):
        gu, dn = self.mlp.gate_up_proj, self.mlp.down_proj
        with torch.no_grad():
            self.banks = (*storage.repack_n32(gu.g256_codes, gu.g256_metadata, 2 * native.INTER, native.HIDDEN),
                          *storage.repack_n32(dn.g256_codes, dn.g256_metadata, native.HIDDEN, native.INTER))
        return sum(t.numel() * 4 for t in self.banks)

    def _ready(self, rt):
        if self.banks is None or rt is None or rt.shared_tables is None:
            raise RuntimeError(f'{self.prefix}: the shared expert is not prepared and bound')

    def fused(self, rt, x, topk_weights, topk_ids, routed, tile, out, shared_out, flags):
        self._ready(rt)
        T = x.shape[0]
        if self.gate_logit is None or self.gate_logit.shape[0] != T:
            raise RuntimeError(f'{self.prefix}: no gate logit of this step (the block router forms it)')
        x = x.contiguous()
        native.routed_shared_tables(x, topk_weights, topk_ids, *routed, *self.banks, self.gate_logit,
                                    *rt.shared_tables, rt.workspace, out, shared_out, flags,
                                    min(self.fused_max_rows, rt.capacity), tile=tile)
        self.gate_logit = None

    def decode_rows(self, rt, x, shared_out):
        """fixed8 on the current step's decode rows of x into shared_out."""
        self._ready(rt)
        runs = native.decode_runs(x.shape[0])
        if not runs:
            return
        flags = rt.slots[self.mlp.gate_up_proj.quant_method.slot]
        scratch = torch.empty_like(shared_out)
        for a, b in runs:
            native.shared_fixed8(x[a:b].contiguous(), *self.banks, self.gate_weight, *rt.shared_tables,
                                 rt.workspace, scratch[a:b], flags, rt.capacity)
            shared_out[a:b].copy_(scratch[a:b])


class Runtime:
    """One workspace arena and one int32 flag slot per quantized layer of
    `model` (modules whose ``quant_method`` is one of the methods above)."""

    def __init__(self, model: torch.nn.Module, settings: dict, capacity: int, device):
        self.device = torch.device(device)
        self.capacity = int(capacity)
        self.routed_decode_n32 = bool(settings.get('routed_decode_n32', False))
        self.routed_storage_n32 = bool(settings.get('routed_storage_n32', False))
        self.routed_n32_max_rows = int(settings.get('routed_n32_max_rows', 8))
        self.dense_geometry = int(settings.get('dense_geometry', 2))
        self.head_geometry = int(settings.get('head_geometry', 2))
        self.dense_a8_max_rows = int(settings.get('dense_a8_max_rows', 32))
        if self.dense_a8_max_rows not in (32, 64):
            raise ValueError('dense_a8_max_rows must be 32 or 64')
        if self.dense_geometry not in (0, 1, 2) or self.head_geometry not in (0, 1, 2):
            raise ValueError('geometry settings must be 0, 1 or 2')
        kinds = (G256LinearMethod, G256MoEMethod, RouterGateMethod)
        self.layers = [(name, m) for name, m in model.named_modules() if isinstance(getattr(m, 'quant_method', None), kinds)]
        modules = dict(model.named_modules())
        # shared experts: '<block>.shared_expert' MLPs whose projections are G256
        # linears; each is linked to its block's router gate '<block>.gate'
        self.shared = {}
        for name, mod in modules.items():
            if name.endswith('.mlp.shared_expert') and hasattr(mod, 'expert_gate') and all(
                    type(getattr(getattr(mod, p, None), 'quant_method', None)) is G256LinearMethod
                    for p in ('gate_up_proj', 'down_proj')):
                self.shared[name] = SharedExpert(name, mod)
        routed = [m for _, m in self.layers if isinstance(m.quant_method, G256MoEMethod)]
        dense = [m for _, m in self.layers if type(m.quant_method) is G256LinearMethod]
        for _, m in self.layers:
            if m.quant_method.runtime is not None:
                raise RuntimeError('a layer is already bound to a runtime')
        shapes = sorted({(m.quant_method.n, m.quant_method.k) for m in dense})
        size = native.configure(settings, self.capacity, shapes, shared_expert=bool(self.shared))
        self.repacked_bytes = 0
        for m in routed:
            if self.routed_storage_n32 or self.routed_decode_n32:
                self.repacked_bytes += m.quant_method.prepare_n32(m, replace=self.routed_storage_n32)
        for sh in self.shared.values():
            self.repacked_bytes += sh.prepare()
            sh.runtime = self
            sh.mlp._ornith_shared = sh
        self.shared_tables = None
        if self.shared:
            from . import tables
            self.shared_tables = tables.load(self.device)
        for name, m in self.layers:
            if isinstance(m.quant_method, RouterGateMethod):
                m.quant_method.shared = self.shared.get(name[:-len('gate')] + 'shared_expert')
        self.workspace = torch.empty(size, dtype=torch.uint8, device=self.device)
        self.error_flags = torch.zeros(len(self.layers), dtype=torch.int32, device=self.device)
        self.slots = tuple(self.error_flags[i:i + 1] for i in range(len(self.layers)))
        self.layer_names = tuple(name for name, _ in self.layers)
        for slot, (_, m) in enumerate(self.layers):
            m.quant_method.runtime, m.quant_method.slot = self, slot

    def reset_error_flags(self):
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError('reset the native flags outside graph capture')
        self.error_flags.zero_()

    def check_error_flags(self):
        flags = self.error_flags.cpu().tolist()
        raised = {n: v for n, v in zip(self.layer_names, flags) if v}
        if raised:
            raise RuntimeError(f'native error flags: {raised}')
        return flags

    def step_flags(self, depth=2):
        """A StepFlags checker over this runtime's flag slots."""
        from .lifecycle import StepFlags
        return StepFlags(self.layer_names, depth, flags=self.error_flags)
