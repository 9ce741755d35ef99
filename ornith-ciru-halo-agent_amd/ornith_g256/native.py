"""ctypes bindings of the MI355X HIP library and the ornith_g256 torch ops.

Mirrors the reference's plugin-site/ornith_g256/native.py: the same custom-op
names and signatures (ornith_g256::dense_out, routed_out, routed_out_n32,
head_out; native.py:121-224), the same validation (native.py:113-118,
176-180), the same error behaviour (RuntimeError on a non-zero native status,
native.py:109-110) and the same configure() that sizes one workspace arena
(native.py:28-104).  All launches go to torch's current stream with no host
synchronisation.  New ops: router_topk and moe_layer (router + routed +
shared expert in one launch sequence).

The library is loaded from this package's lib/ directory; if it is missing
every entry raises - there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import torch

_LIB = None
_libs = {}
_PHASE_SEGMENTS = ()

_ROUTED_FIELDS = ('workspace_bytes', 'gate_x', 'gate_low', 'gate_high', 'gate_scales', 'gate_sums', 'gate_y',
                  'middle', 'down_x', 'down_low', 'down_high', 'down_scales', 'down_sums', 'route_out', 'final_f32')


class DenseLayout(C.Structure):
    _fields_ = [(n, C.c_size_t) for n in
                ('workspace_bytes', 'transformed', 'low', 'high', 'scales', 'sums', 'projection')]


class RoutedLayout(C.Structure):
    _fields_ = [(n, C.c_size_t) for n in _ROUTED_FIELDS]


class HeadLayout(C.Structure):
    _fields_ = [(n, C.c_size_t) for n in
                ('workspace_bytes', 'transformed', 'activation_words', 'activation_scales', 'projection')]


P, I, S, L = C.c_void_p, C.c_int, C.c_size_t, C.c_int64
_SIGNATURES = {
    'ornith_routed_direct_get_layout': ([I, C.POINTER(RoutedLayout)], I),
    'ornith_routed_shared_get_layout': ([I, C.POINTER(RoutedLayout)], I),
    'ornith_moe_layer_get_layout': ([I, C.POINTER(RoutedLayout)], I),
    'ornith_routed_direct_launch': ([P] * 8 + [S] + [P] * 2 + [I] * 2 + [P], I),
    'ornith_routed_direct_launch_a4': ([P] * 8 + [S] + [P] * 2 + [I] * 2 + [P], I),
    'ornith_routed_direct_launch_a4_prefill': ([P] * 8 + [S] + [P] * 2 + [I] * 2 + [P], I),
    'ornith_routed_direct_launch_shared_tables': ([P] * 15 + [S] + [P] * 3 + [I] * 2 + [P], I),
    'ornith_routed_storage_n32': ([], I),
    'ornith_routed_prefill_output_tile': ([], I),
    'ornith_router_topk_launch': ([P, L] + [P] * 7 + [I, P], I),
    'ornith_moe_layer_launch': ([P] * 15 + [S] + [P] * 5 + [I] * 2 + [P], I),
    'ornith_mi355x_abi_version': ([], I),
    'ornith_dense_g256_abi_version': ([], C.c_uint32),
    'ornith_dense_g256_get_layout': ([I] * 4 + [C.POINTER(DenseLayout)], I),
    'ornith_dense_g256_launch': ([P] * 4 + [S] + [P] * 2 + [I] * 7 + [P], I),
    'ornith_dense_g256_prepare_bf16': ([P] * 6 + [I] * 3 + [P], I),
    'ornith_dense_g256_launch_n32': ([P] * 4 + [S] + [P] * 2 + [I] * 7 + [P], I),
    'ornith_dense_g256_n32_rows': ([], I),
    'ornith_dense_g256_head_workspace_bytes': ([I, I], S),
    'ornith_dense_g256_head_launch': ([P] * 4 + [S] + [P] * 4 + [I] * 3 + [P], I),
    'ornith_head_i8_tile_abi_version': ([], C.c_uint32),
    'ornith_head_i8_tile_get_layout': ([I, I, C.POINTER(HeadLayout)], I),
    'ornith_head_i8_tile_launch': ([P] * 4 + [S] + [P] * 2 + [S] + [P] + [I] * 4 + [P], I),
    'ornith_mi355x_timing_arm': ([C.c_char_p, I], I),
    'ornith_mi355x_timing_read': ([C.c_char_p, C.POINTER(I), C.POINTER(C.c_double)], I),
    'ornith_mi355x_timing_names': ([C.c_char_p, I], I),
}


def library_path() -> Path:
    return Path(__file__).resolve().parent / 'lib' / 'libornith_g256_mi355x.so'


def lib():
    """The loaded HIP library; raises if it has not been built."""
    global _LIB
    if _LIB is None:
        path = library_path()
        if not path.exists():
            raise RuntimeError(f'ornith_g256 HIP library missing: {path} (run __graft_entry__.build())')
        handle = C.CDLL(str(path))
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes, fn.restype = args, res
        _LIB = handle
    return _LIB


def configure(settings, capacity, shapes):
    """Size the shared workspace arena (reference native.py:28-104).  The
    library paths in settings must name this library (one .so serves the
    dense, routed and head roles)."""
    routed_activation_bits = settings.get('routed_activation_bits', 8)
    routed_prefill_activation_bits = settings.get('routed_prefill_activation_bits', 8)
    if settings.get('routed_storage_n32', False) and settings.get('routed_decode_n32', False):
        raise ValueError('Choose sole N32 storage or N32 decode shadows')
    if settings.get('routed_n32_max_rows', 8) not in (8, 16):
        raise ValueError('N32 routed decode crossover must be 8 or 16 rows')
    if routed_activation_bits not in (4, 8) or routed_prefill_activation_bits not in (4, 8):
        raise ValueError('G256 routed activation bits must be 4 or 8')
    if routed_activation_bits == routed_prefill_activation_bits == 4:
        raise ValueError('Choose either global routed A4 or prefill-only routed A4')
    if settings.get('routed_decode_n32', False) and routed_activation_bits != 8:
        raise ValueError('N32 routed decode requires A8 verification')
    suffix = ('_a4' if routed_activation_bits == 4 else
              '_a4_prefill' if routed_prefill_activation_bits == 4 else '')
    h = lib()
    for kind in ('dense', 'routed', 'head'):
        path = settings.get(kind + '_library')
        if path is not None and Path(path).resolve() != library_path():
            raise ValueError(f'{kind}_library must be {library_path()}')
    if settings.get('routed_storage_n32', False) and h.ornith_routed_storage_n32() != 32:
        raise ValueError('Sole N32 storage requires the full N32 consumer')
    _libs['routed'] = getattr(h, 'ornith_routed_direct_launch' + suffix)
    _libs['routed_verify'] = h.ornith_routed_direct_launch
    _libs['routed_prefill'] = h.ornith_routed_direct_launch_a4
    _libs['routed_n32'] = h.ornith_routed_direct_launch
    sizes = []
    for n, k in shapes:
        layout = DenseLayout()
        check(h.ornith_dense_g256_get_layout(capacity, n, k, 8, C.byref(layout)), 'dense layout')
        sizes.append(layout.workspace_bytes)
        sizes.append((capacity * k + n * k) * 2)
    layout = RoutedLayout()
    check(h.ornith_routed_direct_get_layout(capacity, C.byref(layout)), 'routed layout')
    sizes.append(layout.workspace_bytes)
    if not sizes or min(sizes) <= 0:
        raise RuntimeError('Native workspace query failed')
    return max(sizes)


def ptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


def stream(x):
    return C.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)


def check(status, operation):
    if status:
        raise RuntimeError(f'{operation} failed with native status {status}')


def validate(x, out, capacity, k):
    if (x.ndim != 2 or x.shape[1] != k or not 0 <= x.shape[0] <= capacity
            or x.dtype != torch.bfloat16 or x.device.type != 'cuda'
            or out.dtype != x.dtype or out.device != x.device
            or not x.is_contiguous() or not out.is_contiguous()):
        raise ValueError('Native G256 requires contiguous BF16 input/output within capacity')


def routed_layout(capacity, kind='routed'):
    layout = RoutedLayout()
    fn = {'routed': lib().ornith_routed_direct_get_layout,
          'shared': lib().ornith_routed_shared_get_layout,
          'layer': lib().ornith_moe_layer_get_layout}[kind]
    check(fn(capacity, C.byref(layout)), f'{kind} layout')
    return layout


def dense_layout(capacity, n, k):
    layout = DenseLayout()
    check(lib().ornith_dense_g256_get_layout(capacity, n, k, 8, C.byref(layout)), 'dense layout')
    return layout


# ----------------------------------------------------------------------------
# torch custom ops (reference native.py:121-224)
# ----------------------------------------------------------------------------
@torch.library.custom_op('ornith_g256::dense_out', mutates_args={'workspace', 'out', 'flags'}, device_types='cuda')
def dense_out(x: torch.Tensor, codes: torch.Tensor, metadata: torch.Tensor,
              workspace: torch.Tensor, out: torch.Tensor, flags: torch.Tensor,
              capacity: int, n: int, k: int, geometry: int, a8_max_rows: int) -> None:
    if _PHASE_SEGMENTS and x.shape[0] >= _PHASE_SEGMENTS[-1][1]:
        for start, end, prefill in _PHASE_SEGMENTS:
            _dense_impl(x[start:end], codes, metadata, workspace, out[start:end], flags,
                        capacity, n, k, geometry, 0 if prefill else capacity)
        end = _PHASE_SEGMENTS[-1][1]
        if end < x.shape[0]:
            _dense_impl(x[end:], codes, metadata, workspace, out[end:], flags, capacity, n, k, geometry, 0)
        return
    _dense_impl(x, codes, metadata, workspace, out, flags, capacity, n, k, geometry, a8_max_rows)


def _dense_impl(x, codes, metadata, workspace, out, flags, capacity, n, k, geometry, a8_max_rows):
    validate(x, out, capacity, k)
    h = lib()
    if x.shape[0] > a8_max_rows:
        # bf16 prefill semantics (dense_g256_consumer.cpp:192-246 + native.py:140-150):
        # bf16(H128 x) @ bf16(dequant W).T in the arena.
        weight_offset = capacity * k * 2
        transformed = workspace[:x.shape[0] * k * 2].view(torch.bfloat16).view(x.shape[0], k)
        weight = workspace[weight_offset:weight_offset + n * k * 2].view(torch.bfloat16).view(n, k)
        check(h.ornith_dense_g256_prepare_bf16(ptr(x), ptr(codes), ptr(metadata), ptr(transformed), ptr(weight),
                                               ptr(flags), x.shape[0], n, k, stream(x)),
              'G256 BF16 prefill preparation')
        torch.mm(transformed, weight.t(), out=out)
        return
    check(h.ornith_dense_g256_launch(ptr(x), ptr(codes), ptr(metadata), ptr(workspace), workspace.numel(),
                                     ptr(out), ptr(flags), x.shape[0], capacity, n, k, 8, 128, geometry,
                                     stream(x)), 'G256 dense')


@torch.library.custom_op('ornith_g256::routed_out', mutates_args={'workspace', 'out', 'flags'}, device_types='cuda')
def routed_out(x: torch.Tensor, routes: torch.Tensor, ids: torch.Tensor,
               gate: torch.Tensor, gate_meta: torch.Tensor, down: torch.Tensor, down_meta: torch.Tensor,
               workspace: torch.Tensor, out: torch.Tensor, flags: torch.Tensor, capacity: int) -> None:
    if _PHASE_SEGMENTS and x.shape[0] >= _PHASE_SEGMENTS[-1][1]:
        segments = list(_PHASE_SEGMENTS)
        if segments[-1][1] < x.shape[0]:
            segments.append((segments[-1][1], x.shape[0], True))
        for start, end, prefill in segments:
            _routed_out('routed_prefill' if prefill else 'routed_verify',
                        x[start:end], routes[start:end], ids[start:end],
                        gate, gate_meta, down, down_meta, workspace, out[start:end], flags, capacity)
        return
    _routed_out('routed', x, routes, ids, gate, gate_meta, down, down_meta, workspace, out, flags, capacity)


def _routed_out(kind, x, routes, ids, gate, gate_meta, down, down_meta, workspace, out, flags, capacity):
    validate(x, out, capacity, 2048)
    if (routes.dtype != torch.float32 or ids.dtype != torch.int32
            or routes.shape != (x.shape[0], 8) or ids.shape != routes.shape
            or routes.device != x.device or ids.device != x.device
            or not routes.is_contiguous() or not ids.is_contiguous()):
        raise ValueError('G256 routed input requires FP32 weights and INT32 IDs [T,8]')
    fn = _libs.get(kind) or lib().ornith_routed_direct_launch
    check(fn(*[ptr(t) for t in (x, routes, ids, gate, gate_meta, down, down_meta, workspace)],
             workspace.numel(), ptr(out), ptr(flags), x.shape[0], capacity, stream(x)), 'G256 ' + kind)


@torch.library.custom_op('ornith_g256::routed_out_n32', mutates_args={'workspace', 'out', 'flags'},
                         device_types='cuda')
def routed_out_n32(x: torch.Tensor, routes: torch.Tensor, ids: torch.Tensor,
                   gate: torch.Tensor, gate_meta: torch.Tensor,
                   down: torch.Tensor, down_meta: torch.Tensor,
                   gate_n32: torch.Tensor, gate_meta_n32: torch.Tensor,
                   down_n32: torch.Tensor, down_meta_n32: torch.Tensor,
                   workspace: torch.Tensor, out: torch.Tensor,
                   flags: torch.Tensor, capacity: int, n32_max_rows: int = 8) -> None:
    # This library stores routed banks in N32 only; both banks arguments must
    # be N32 (the reference kept an N16 parent for large T, native.py:187-202).
    if x.shape[0] <= n32_max_rows:
        bank = (gate_n32, gate_meta_n32, down_n32, down_meta_n32)
    else:
        bank = (gate, gate_meta, down, down_meta)
    _routed_out('routed_n32' if x.shape[0] <= n32_max_rows else 'routed', x, routes, ids, *bank,
                workspace, out, flags, capacity)


@torch.library.custom_op('ornith_g256::head_out', mutates_args={'workspace', 'out', 'flags'}, device_types='cuda')
def head_out(x: torch.Tensor, codes: torch.Tensor, scales: torch.Tensor,
             workspace: torch.Tensor, out: torch.Tensor, flags: torch.Tensor, geometry: int) -> None:
    validate(x, out, 64, 2048)
    check(lib().ornith_head_i8_tile_launch(ptr(x), ptr(codes), ptr(scales), ptr(workspace), workspace.numel(),
                                           ptr(out), None, 0, ptr(flags), x.shape[0], 64, 248320, geometry,
                                           stream(x)), 'W8 head')


@torch.library.custom_op('ornith_g256::router_topk', mutates_args={'logits', 'weights', 'ids', 'shared_logit'},
                         device_types='cuda')
def router_topk(x: torch.Tensor, router_weight: torch.Tensor, bias: torch.Tensor | None,
                shared_gate_weight: torch.Tensor | None, logits: torch.Tensor, weights: torch.Tensor,
                ids: torch.Tensor, shared_logit: torch.Tensor) -> None:
    T = x.shape[0]
    if (x.ndim != 2 or x.shape[1] != 2048 or x.stride(1) != 1 or x.dtype != torch.bfloat16
            or router_weight.shape != (256, 2048) or not router_weight.is_contiguous()
            or logits.shape != (T, 257) or logits.dtype != torch.float32 or not logits.is_contiguous()
            or weights.shape != (T, 8) or ids.shape != (T, 8) or ids.dtype != torch.int32):
        raise ValueError('router_topk requires x bf16 [T,2048], W [256,2048], logits f32 [T,257], outputs [T,8]')
    check(lib().ornith_router_topk_launch(ptr(x), x.stride(0), ptr(router_weight), ptr(bias),
                                          ptr(shared_gate_weight), ptr(logits), ptr(weights), ptr(ids),
                                          ptr(shared_logit), T, stream(x)), 'router top-k')


@dense_out.register_fake
def _dense_fake(x, codes, metadata, workspace, out, flags, capacity, n, k, geometry, a8_max_rows):
    return None


@routed_out.register_fake
def _routed_fake(x, routes, ids, gate, gate_meta, down, down_meta, workspace, out, flags, capacity):
    return None


@routed_out_n32.register_fake
def _routed_n32_fake(x, routes, ids, gate, gate_meta, down, down_meta, gate_n32, gate_meta_n32, down_n32,
                     down_meta_n32, workspace, out, flags, capacity, n32_max_rows=8):
    return None


@head_out.register_fake
def _head_fake(x, codes, scales, workspace, out, flags, geometry):
    return None


@router_topk.register_fake
def _router_fake(x, router_weight, bias, shared_gate_weight, logits, weights, ids, shared_logit):
    return None


# ----------------------------------------------------------------------------
# Direct (non-op) helpers used by the layer driver, tests and bench.
# ----------------------------------------------------------------------------
def routed_shared_tables(x, routes, ids, gate, gate_meta, down, down_meta, s_gate, s_gate_meta, s_down,
                         s_down_meta, shared_logit, silu, sigmoid, workspace, out, shared_out, flags, capacity):
    check(lib().ornith_routed_direct_launch_shared_tables(
        *[ptr(t) for t in (x, routes, ids, gate, gate_meta, down, down_meta, s_gate, s_gate_meta, s_down,
                           s_down_meta, shared_logit, silu, sigmoid, workspace)],
        workspace.numel(), ptr(out), ptr(shared_out), ptr(flags), x.shape[0], capacity, stream(x)),
        'G256 routed shared')


def moe_layer(x, router_weight, bias, shared_gate_weight, gate, gate_meta, down, down_meta, s_gate, s_gate_meta,
              s_down, s_down_meta, silu, sigmoid, workspace, topk_weights, topk_ids, shared_logit, out, flags,
              capacity):
    check(lib().ornith_moe_layer_launch(
        *[ptr(t) for t in (x, router_weight, bias, shared_gate_weight, gate, gate_meta, down, down_meta, s_gate,
                           s_gate_meta, s_down, s_down_meta, silu, sigmoid, workspace)],
        workspace.numel(), *[ptr(t) for t in (topk_weights, topk_ids, shared_logit, out, flags)],
        x.shape[0], capacity, stream(x)), 'G256 MoE layer')


def dense_head(x, codes, meta, workspace, logits, logits_bf16, argmax, flags, capacity):
    check(lib().ornith_dense_g256_head_launch(ptr(x), ptr(codes), ptr(meta), ptr(workspace), workspace.numel(),
                                              ptr(logits), ptr(logits_bf16), ptr(argmax), ptr(flags), x.shape[0],
                                              capacity, codes.shape[0] * 32, stream(x)), 'G256 head')


class KernelTimer:
    """Times launches of one library kernel ("*" = all) with HIP event pairs
    recorded on each launch's own stream (include/ornith_timing.h).  The
    launches themselves are unchanged."""

    def __init__(self, kernel: str = '*', capacity: int = 100_000):
        self.kernel, self.capacity = kernel, capacity

    def __enter__(self):
        check(lib().ornith_mi355x_timing_arm(self.kernel.encode(), self.capacity), "timing_arm")
        return self

    def __exit__(self, *exc):
        lib().ornith_mi355x_timing_arm(None, 0)
        return False

    def names(self):
        n = lib().ornith_mi355x_timing_names(None, 0)
        buf = C.create_string_buffer(n + 1)
        lib().ornith_mi355x_timing_names(buf, n + 1)
        return [v for v in buf.value.decode().split(',') if v]

    def read(self, kernel: str):
        """(launches, average milliseconds per launch) for `kernel`."""
        count, total = C.c_int(0), C.c_double(0.0)
        check(lib().ornith_mi355x_timing_read(kernel.encode(), C.byref(count), C.byref(total)), "timing_read")
        return count.value, (total.value / count.value if count.value else 0.0)
