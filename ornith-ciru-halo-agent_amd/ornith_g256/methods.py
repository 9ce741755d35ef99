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

    def apply(self, layer, x, topk_weights, topk_ids, shared_experts=None, shared_experts_input=None):
        rt = self.runtime
        if rt is None or not layer._ornith_loader.sealed:
            raise RuntimeError(f'{self.prefix}: needs sealed weights and a bound runtime')
        out = torch.empty_like(x)
        banks = (layer.w13_tilebank_codes, layer.w13_tilebank_metadata, layer.w2_tilebank_codes,
                 layer.w2_tilebank_metadata)
        if rt.routed_decode_n32:
            native.routed_out_n32(x, topk_weights, topk_ids, *banks, layer.w13_n32_codes, layer.w13_n32_metadata,
                                  layer.w2_n32_codes, layer.w2_n32_metadata, rt.workspace, out,
                                  rt.slots[self.slot], rt.capacity, rt.routed_n32_max_rows)
        else:
            native.routed_out(x, topk_weights, topk_ids, *banks, rt.workspace, out, rt.slots[self.slot],
                              rt.capacity)
        return out


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
        kinds = (G256LinearMethod, G256MoEMethod)
        self.layers = [(name, m) for name, m in model.named_modules() if isinstance(getattr(m, 'quant_method', None), kinds)]
        routed = [m for _, m in self.layers if isinstance(m.quant_method, G256MoEMethod)]
        dense = [m for _, m in self.layers if type(m.quant_method) is G256LinearMethod]
        for _, m in self.layers:
            if m.quant_method.runtime is not None:
                raise RuntimeError('a layer is already bound to a runtime')
        shapes = sorted({(m.quant_method.n, m.quant_method.k) for m in dense})
        size = native.configure(settings, self.capacity, shapes)
        self.repacked_bytes = 0
        for m in routed:
            if self.routed_storage_n32 or self.routed_decode_n32:
                self.repacked_bytes += m.quant_method.prepare_n32(m, replace=self.routed_storage_n32)
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
