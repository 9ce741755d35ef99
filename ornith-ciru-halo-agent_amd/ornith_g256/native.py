"""Host side of the MI355X Ornith G256 library: ctypes bindings and the
``ornith_g256::*`` torch ops.

Interface kept from the reference plugin (plugin-site/ornith_g256/native.py):
the op names and signatures ``dense_out``, ``routed_out``, ``routed_out_n32``
and ``head_out`` (native.py:121-212), the three layout Structures
(native.py:11-24), ``configure(settings, capacity, shapes)`` returning the
arena size (native.py:28-104), and the error behaviour - ``ValueError`` for a
bad setting or tensor, ``RuntimeError`` for a non-zero native status.

Design of this module:
  * Two builds of one source tree serve every reference library role.  The
    N32 build (``libornith_g256_mi355x.so``, storage marker 32) takes routed
    banks in N32 tiles; the N16 build (``libornith_g256_mi355x_n16.so``,
    marker 16) takes them in the checkpoint's N16 tiles.  Dense, head and
    router entries are identical in both.
  * ``configure`` resolves every library role to one of these builds and
    records a ``Binding`` (the launch function per dispatch kind, with the
    bank tile it expects).  Routed ops check that the banks they are handed
    have that tile width, so a mismatched layout fails before any launch.
  * Mixed prefill/decode batches are split by an explicit phase plan set with
    ``phase_segments(...)`` (see phases.py), not by a module global.
  * Launches go to torch's current stream and never synchronise.  There is
    no CPU fallback: a missing library raises on first use.
"""
from __future__ import annotations

import contextvars
import ctypes as C
from contextlib import contextmanager
from dataclasses import dataclass, field
from pathlib import Path

import torch

LIB_DIR = Path(__file__).resolve().parent / 'lib'
BUILDS = {32: 'libornith_g256_mi355x.so', 16: 'libornith_g256_mi355x_n16.so'}

HIDDEN, EXPERTS, TOP, INTER = 2048, 256, 8, 512
HEAD_VOCAB, HEAD_MAX_ROWS = 248320, 64
# fp32 slice sums of the dense GEMM's split K: slices x tiles stay within the
# chip's 2 x 256 block slots and a tile has 256 x 64 outputs
DENSE_SLICE_BYTES = 2 * 256 * 256 * 64 * 4
A8_ONLY_PREFILL_ROWS = 64      # _a4_prefill entries switch to A4 above this many tokens

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


# ---------------------------------------------------------------------------
# Library loading
# ---------------------------------------------------------------------------
_VP, _INT, _SZ, _I64 = C.c_void_p, C.c_int, C.c_size_t, C.c_int64
_ROUTED_LAUNCH = [_VP] * 8 + [_SZ] + [_VP] * 2 + [_INT] * 2 + [_VP]
_DENSE_LAUNCH = [_VP] * 4 + [_SZ] + [_VP] * 2 + [_INT] * 7 + [_VP]
_PROTOTYPES = {
    # routed (include/ornith_routed.h)
    'ornith_routed_direct_get_layout': ([_INT, C.POINTER(RoutedLayout)], _INT),
    'ornith_routed_direct_launch': (_ROUTED_LAUNCH, _INT),
    'ornith_routed_direct_launch_a4': (_ROUTED_LAUNCH, _INT),
    'ornith_routed_direct_launch_a4_prefill': (_ROUTED_LAUNCH, _INT),
    'ornith_routed_shared_get_layout': ([_INT, C.POINTER(RoutedLayout)], _INT),
    'ornith_routed_direct_launch_shared_tables': ([_VP] * 15 + [_SZ] + [_VP] * 3 + [_INT] * 2 + [_VP], _INT),
    'ornith_routed_storage_n32': ([], _INT),
    'ornith_routed_prefill_output_tile': ([], _INT),
    # router + whole layer (include/ornith_moe.h)
    'ornith_router_topk_launch': ([_VP, _I64] + [_VP] * 7 + [_INT, _VP], _INT),
    'ornith_moe_layer_get_layout': ([_INT, C.POINTER(RoutedLayout)], _INT),
    'ornith_moe_layer_launch': ([_VP] * 15 + [_SZ] + [_VP] * 5 + [_INT] * 2 + [_VP], _INT),
    'ornith_moe_layer_launch_static': ([_VP] * 19 + [_INT, _VP], _INT),
    'ornith_shared_fixed8_get_layout': ([_INT, C.POINTER(_SZ)], _INT),
    'ornith_shared_fixed8_launch': ([_VP] * 9 + [_SZ] + [_VP] * 2 + [_INT] * 2 + [_VP], _INT),
    'ornith_mi355x_abi_version': ([], _INT),
    'ornith_mi355x_single_token_path': ([_INT], _INT),
    'ornith_mi355x_decode_route_path': ([_INT], _INT),
    'ornith_mi355x_silu_selfcheck': ([_VP, _VP, _VP], _INT),
    'ornith_mi355x_handoff_spin_limit': ([_INT], _INT),
    'ornith_mi355x_workspace_reset': ([_VP, _SZ, _VP], _INT),
    # dense (include/ornith_dense.h)
    'ornith_dense_g256_abi_version': ([], C.c_uint32),
    'ornith_dense_g256_get_layout': ([_INT] * 4 + [C.POINTER(DenseLayout)], _INT),
    'ornith_dense_g256_launch': (_DENSE_LAUNCH, _INT),
    'ornith_dense_g256_prepare_bf16': ([_VP] * 6 + [_INT] * 3 + [_VP], _INT),
    'ornith_dense_g256_launch_n32': (_DENSE_LAUNCH, _INT),
    'ornith_dense_g256_gemm_bf16': ([_VP] * 4 + [_SZ] + [_VP] * 2 + [_INT] * 3 + [_VP], _INT),
    'ornith_dense_g256_n32_rows': ([], _INT),
    'ornith_dense_g256_head_workspace_bytes': ([_INT, _INT], _SZ),
    'ornith_dense_g256_head_launch': ([_VP] * 4 + [_SZ] + [_VP] * 4 + [_INT] * 3 + [_VP], _INT),
    # W8 head (include/ornith_head.h)
    'ornith_head_i8_tile_abi_version': ([], C.c_uint32),
    'ornith_head_i8_tile_shortlist': ([], C.c_int),
    'ornith_head_i8_tile_get_layout': ([_INT, _INT, C.POINTER(HeadLayout)], _INT),
    'ornith_head_i8_tile_launch': ([_VP] * 4 + [_SZ] + [_VP] * 2 + [_SZ] + [_VP] + [_INT] * 4 + [_VP], _INT),
    # storage conversion (include/ornith_storage.h)
    'ornith_repack_n16_to_n32': ([_VP] * 4 + [_INT] * 3 + [_VP], _INT),
    'ornith_logits_argmax_launch': ([_VP, _INT, _INT, _I64, _VP, _VP], _INT),
    # measurement (include/ornith_timing.h)
    'ornith_mi355x_timing_arm': ([C.c_char_p, _INT], _INT),
    'ornith_mi355x_timing_read': ([C.c_char_p, C.POINTER(_INT), C.POINTER(C.c_double)], _INT),
    'ornith_mi355x_timing_names': ([C.c_char_p, _INT], _INT),
    'ornith_mi355x_stage_trace_read': ([_VP, _SZ, _VP], _INT),
}
# entries that only some builds of the library export (bound when present)
_OPTIONAL: dict = {}

_handles: dict[int, C.CDLL] = {}


def library_path(tile: int = 32) -> Path:
    """Path of the build whose routed banks use `tile`-wide tiles (32 or 16)."""
    return LIB_DIR / BUILDS[tile]


def lib(tile: int = 32) -> C.CDLL:
    """The loaded HIP library (prototypes set); raises if it was not built."""
    handle = _handles.get(tile)
    if handle is None:
        path = library_path(tile)
        if not path.exists():
            raise RuntimeError(f'ornith_g256 HIP library missing: {path} (run __graft_entry__.build())')
        handle = C.CDLL(str(path))
        for name, (args, res) in _PROTOTYPES.items():
            fn = getattr(handle, name)
            fn.argtypes, fn.restype = args, res
        for name, (args, res) in _OPTIONAL.items():
            fn = getattr(handle, name, None)
            if fn is not None:
                fn.argtypes, fn.restype = args, res
        if handle.ornith_routed_storage_n32() != tile:
            raise RuntimeError(f'{path} reports routed tile {handle.ornith_routed_storage_n32()}, expected {tile}')
        _handles[tile] = handle
    return handle


def _build_of(path) -> int:
    """Which of this package's builds a configured library path names."""
    resolved = Path(path).expanduser().resolve()
    for tile, name in BUILDS.items():
        if resolved == (LIB_DIR / name).resolve():
            return tile
    raise ValueError(f'{path} is not one of this package\'s libraries ({", ".join(BUILDS.values())} in {LIB_DIR})')


def ptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


def stream(x):
    return C.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)


def check(status, operation):
    if status:
        raise RuntimeError(f'{operation}: native status {status}')


# ---------------------------------------------------------------------------
# configure(): settings -> binding + arena size
# ---------------------------------------------------------------------------
@dataclass
class Binding:
    """Launch function per dispatch kind, with the routed bank tile it reads."""
    routed: dict = field(default_factory=dict)      # kind -> (ctypes fn, tile)
    routed_suffix: str = ''
    libraries: dict = field(default_factory=dict)   # role -> tile of the build serving it
    settings_key: tuple = ()


_binding: Binding | None = None


def _settings_key(settings):
    keys = ('routed_activation_bits', 'routed_prefill_activation_bits', 'routed_storage_n32', 'routed_decode_n32',
            'routed_n32_max_rows', 'dense_library', 'routed_library', 'head_library', 'routed_n32_library')
    return tuple((k, str(settings.get(k))) for k in keys)


def configure(settings, capacity, shapes, shared_expert=False):
    """Resolve the library roles, bind the launch entries and return the
    workspace size the caller allocates once (the max over the routed
    layout, the dense layouts plus the GEMM's transformed rows, the W8 head
    layout and, with `shared_expert`, the fused shared slot and fixed8)."""
    global _binding
    a8 = settings.get('routed_activation_bits', 8)
    a8_prefill = settings.get('routed_prefill_activation_bits', 8)
    sole_n32 = bool(settings.get('routed_storage_n32', False))
    n32_decode = bool(settings.get('routed_decode_n32', False))
    if a8 not in (4, 8) or a8_prefill not in (4, 8):
        raise ValueError(f'routed activation bits must be 4 or 8, got {a8}/{a8_prefill}')
    if a8 == 4 and a8_prefill == 4:
        raise ValueError('set either routed_activation_bits=4 (all tokens) or '
                         'routed_prefill_activation_bits=4 (prefill only), not both')
    if sole_n32 and n32_decode:
        raise ValueError('routed_storage_n32 (N32 banks only) excludes routed_decode_n32 (N32 decode copies)')
    if settings.get('routed_n32_max_rows', 8) not in (8, 16):
        raise ValueError('routed_n32_max_rows must be 8 or 16')
    if n32_decode and a8 != 8:
        raise ValueError('routed_decode_n32 needs A8 routed activations')
    if n32_decode and not settings.get('routed_n32_library'):
        raise ValueError('routed_decode_n32 needs routed_n32_library')
    if not 0 <= int(capacity) <= 8192:
        raise ValueError(f'capacity {capacity} outside 0..8192')

    roles = {}
    for role in ('dense', 'routed', 'head'):
        path = settings.get(role + '_library')
        roles[role] = _build_of(path) if path is not None else (32 if role != 'routed' or sole_n32 else 16)
    if roles['routed'] != (32 if sole_n32 else 16):
        want = 'N32 (routed_storage_n32=True)' if sole_n32 else 'N16 (the checkpoint layout)'
        raise ValueError(f'routed_library must be the build that reads {want} banks: {library_path(32 if sole_n32 else 16)}')
    if n32_decode:
        roles['routed_n32'] = _build_of(settings['routed_n32_library'])
        if roles['routed_n32'] != 32:
            raise ValueError(f'routed_n32_library must be {library_path(32)}')

    key = _settings_key(settings)
    if _binding is not None and _binding.settings_key != key:
        raise RuntimeError('the native libraries are already configured with other settings in this process')
    suffix = '_a4' if a8 == 4 else '_a4_prefill' if a8_prefill == 4 else ''
    routed_lib = lib(roles['routed'])
    binding = Binding(routed_suffix=suffix, libraries=dict(roles), settings_key=key)
    binding.routed['routed'] = (getattr(routed_lib, 'ornith_routed_direct_launch' + suffix), roles['routed'])
    binding.routed['routed_verify'] = (routed_lib.ornith_routed_direct_launch, roles['routed'])
    binding.routed['routed_prefill'] = (routed_lib.ornith_routed_direct_launch_a4, roles['routed'])
    if n32_decode:
        binding.routed['routed_n32'] = (lib(32).ornith_routed_direct_launch, 32)

    sizes = [routed_layout(capacity, tile=roles['routed']).workspace_bytes]
    if n32_decode:
        parent, shadow = routed_layout(capacity, tile=roles['routed']), routed_layout(capacity, tile=32)
        if bytes(parent) != bytes(shadow):
            raise ValueError('the N32 decode library must keep its parent\'s workspace layout')
    for n, k in shapes:
        sizes.append(dense_layout(capacity, n, k, tile=roles['dense']).workspace_bytes)
        # the GEMM's bf16(H128 x), rows padded to 16, then its split-K slice sums
        sizes.append((int(capacity) + 15) // 16 * 16 * k * 2 + DENSE_SLICE_BYTES)
    sizes.append(head_layout(HEAD_MAX_ROWS, HEAD_VOCAB, tile=roles['head']).workspace_bytes)
    if shared_expert:
        # the fused ninth slot (at most 16 rows, any routed build) and fixed8
        for tile in {roles['routed'], 32}:
            sizes.append(routed_layout(min(16, int(capacity)), 'shared', tile=tile).workspace_bytes)
        sizes.append(shared_fixed8_bytes(capacity))
    if min(sizes) <= 0:
        raise RuntimeError('native workspace query returned an empty layout')
    _binding = binding
    return max(sizes)


def reset_binding():
    """Forget the configured binding (tests and tools that reconfigure)."""
    global _binding
    _binding = None


def routed_layout(capacity, kind='routed', tile=32):
    layout = RoutedLayout()
    query = {'routed': 'ornith_routed_direct_get_layout', 'shared': 'ornith_routed_shared_get_layout',
             'layer': 'ornith_moe_layer_get_layout'}[kind]
    check(getattr(lib(tile), query)(capacity, C.byref(layout)), f'{kind} layout for {capacity} tokens')
    return layout


def dense_layout(capacity, n, k, tile=32):
    layout = DenseLayout()
    check(lib(tile).ornith_dense_g256_get_layout(capacity, n, k, 8, C.byref(layout)), f'dense layout N{n} K{k}')
    return layout


def head_layout(capacity, n, tile=32):
    layout = HeadLayout()
    check(lib(tile).ornith_head_i8_tile_get_layout(capacity, n, C.byref(layout)), f'W8 head layout N{n}')
    return layout


# ---------------------------------------------------------------------------
# Mixed prefill/decode batches
# ---------------------------------------------------------------------------
_phase_plan: contextvars.ContextVar[tuple] = contextvars.ContextVar('ornith_phase_plan', default=())


@contextmanager
def phase_segments(segments):
    """Within this context, ops over a batch of at least `segments[-1][1]` rows
    run each (start, end, is_prefill) segment with its own precision: prefill
    segments on the A4 routed entry and the bf16 dense GEMM, decode segments
    on the A8 entries; rows past the last segment are prefill."""
    token = _phase_plan.set(tuple((int(a), int(b), bool(p)) for a, b, p in segments))
    try:
        yield
    finally:
        _phase_plan.reset(token)


# The phases of every row of the current model step, (start, end, is_prefill)
# runs covering the batch, also for single-phase and small batches (the
# plans above are only for the routed split).  The shared expert reads it to
# know its decode rows; unset means no decode rows.
_step_phases: contextvars.ContextVar[tuple] = contextvars.ContextVar('ornith_step_phases', default=())


@contextmanager
def step_phases(segments):
    """Within this context, the rows of a model step are in the phases
    `segments` ((start, end, is_prefill) runs from row 0); rows past the
    last run are prefill."""
    token = _step_phases.set(tuple((int(a), int(b), bool(p)) for a, b, p in segments))
    try:
        yield
    finally:
        _step_phases.reset(token)


def decode_runs(rows):
    """(start, end) runs of decode rows among the first `rows` rows of the
    current step (empty when no step phases are set)."""
    return tuple((a, min(b, rows)) for a, b, p in _step_phases.get() if not p and a < rows)


def _active_plan(rows):
    plan = _phase_plan.get()
    if not plan or rows < plan[-1][1]:
        return ()
    if plan[-1][1] < rows:
        plan = plan + ((plan[-1][1], rows, True),)
    return plan


# ---------------------------------------------------------------------------
# Tensor checks
# ---------------------------------------------------------------------------
def _check_rows(x, out, capacity, k):
    if x.ndim != 2 or x.shape[1] != k or x.dtype != torch.bfloat16 or x.device.type != 'cuda':
        raise ValueError(f'input must be a CUDA bf16 [rows, {k}] tensor, got {tuple(x.shape)} {x.dtype}')
    if not 0 <= x.shape[0] <= capacity:
        raise ValueError(f'{x.shape[0]} rows exceed the configured capacity {capacity}')
    if not x.is_contiguous() or not out.is_contiguous() or out.dtype != x.dtype or out.device != x.device:
        raise ValueError('input and output must be contiguous bf16 tensors on one device')


def _check_routing(x, weights, ids):
    T = x.shape[0]
    if (weights.dtype != torch.float32 or ids.dtype != torch.int32 or tuple(weights.shape) != (T, TOP)
            or tuple(ids.shape) != (T, TOP) or weights.device != x.device or ids.device != x.device
            or not weights.is_contiguous() or not ids.is_contiguous()):
        raise ValueError(f'routing must be contiguous fp32 weights and int32 ids of shape [{T}, {TOP}]')


def _check_banks(tile, gate, gate_meta, down, down_meta):
    """Routed banks [256, N/tile, K/256, 32, tile] codes and [256, N/tile, K/256, tile]
    meta (uint32 words; int32 views accepted)."""
    for name, t, n, k, meta in (('gate', gate, 1024, 2048, False), ('gate_meta', gate_meta, 1024, 2048, True),
                                ('down', down, 2048, 512, False), ('down_meta', down_meta, 2048, 512, True)):
        want = (EXPERTS, n // tile, k // 256) + (() if meta else (32,)) + (tile,)
        if t.element_size() != 4 or not t.is_contiguous():
            raise ValueError(f'{name} must be a contiguous 32-bit tensor')
        if t.ndim > 1 and tuple(t.shape) != want:
            raise ValueError(f'{name} has shape {tuple(t.shape)}; this library reads N{tile} banks {want}')
        if t.numel() != int(torch.Size(want).numel()):
            raise ValueError(f'{name} holds {t.numel()} words, N{tile} banks need {torch.Size(want).numel()}')


# ---------------------------------------------------------------------------
# torch ops (reference native.py:121-212)
# ---------------------------------------------------------------------------
def _dense_one(x, codes, metadata, workspace, out, flags, capacity, n, k, geometry, a8_max_rows):
    h = lib(_binding.libraries['dense'] if _binding else 32)
    _check_rows(x, out, capacity, k)
    rows = x.shape[0]
    if rows > a8_max_rows:
        # bf16 prefill semantics (dense_g256_consumer.cpp:192-246 and the
        # reference's torch.mm) on this library's GEMM, which reads the 4-bit
        # codes: bf16(H128 x) (rows padded to 16) takes the arena's front
        check(h.ornith_dense_g256_gemm_bf16(ptr(x), ptr(codes), ptr(metadata), ptr(workspace), workspace.numel(),
                                            ptr(out), ptr(flags), rows, n, k, stream(x)), 'dense bf16 GEMM')
        return
    check(h.ornith_dense_g256_launch(ptr(x), ptr(codes), ptr(metadata), ptr(workspace), workspace.numel(), ptr(out),
                                     ptr(flags), rows, capacity, n, k, 8, 128, geometry, stream(x)), 'dense A8')


@torch.library.custom_op('ornith_g256::dense_out', mutates_args={'workspace', 'out', 'flags'}, device_types='cuda')
def dense_out(x: torch.Tensor, codes: torch.Tensor, metadata: torch.Tensor,
              workspace: torch.Tensor, out: torch.Tensor, flags: torch.Tensor,
              capacity: int, n: int, k: int, geometry: int, a8_max_rows: int) -> None:
    plan = _active_plan(x.shape[0])
    if not plan:
        _dense_one(x, codes, metadata, workspace, out, flags, capacity, n, k, geometry, a8_max_rows)
        return
    for start, end, prefill in plan:
        _dense_one(x[start:end], codes, metadata, workspace, out[start:end], flags, capacity, n, k, geometry,
                   0 if prefill else capacity)


def _routed_one(kind, x, weights, ids, gate, gate_meta, down, down_meta, workspace, out, flags, capacity):
    _check_rows(x, out, capacity, HIDDEN)
    _check_routing(x, weights, ids)
    if _binding is None:
        raise RuntimeError('call native.configure(settings, capacity, shapes) before the routed ops')
    fn, tile = _binding.routed[kind]
    _check_banks(tile, gate, gate_meta, down, down_meta)
    args = [ptr(t) for t in (x, weights, ids, gate, gate_meta, down, down_meta, workspace)]
    check(fn(*args, workspace.numel(), ptr(out), ptr(flags), x.shape[0], capacity, stream(x)), f'routed ({kind})')


@torch.library.custom_op('ornith_g256::routed_out', mutates_args={'workspace', 'out', 'flags'}, device_types='cuda')
def routed_out(x: torch.Tensor, routes: torch.Tensor, ids: torch.Tensor,
               gate: torch.Tensor, gate_meta: torch.Tensor, down: torch.Tensor, down_meta: torch.Tensor,
               workspace: torch.Tensor, out: torch.Tensor, flags: torch.Tensor, capacity: int) -> None:
    plan = _active_plan(x.shape[0])
    if not plan:
        _routed_one('routed', x, routes, ids, gate, gate_meta, down, down_meta, workspace, out, flags, capacity)
        return
    for start, end, prefill in plan:
        _routed_one('routed_prefill' if prefill else 'routed_verify', x[start:end], routes[start:end],
                    ids[start:end], gate, gate_meta, down, down_meta, workspace, out[start:end], flags, capacity)


@torch.library.custom_op('ornith_g256::routed_out_n32', mutates_args={'workspace', 'out', 'flags'},
                         device_types='cuda')
def routed_out_n32(x: torch.Tensor, routes: torch.Tensor, ids: torch.Tensor,
                   gate: torch.Tensor, gate_meta: torch.Tensor,
                   down: torch.Tensor, down_meta: torch.Tensor,
                   gate_n32: torch.Tensor, gate_meta_n32: torch.Tensor,
                   down_n32: torch.Tensor, down_meta_n32: torch.Tensor,
                   workspace: torch.Tensor, out: torch.Tensor,
                   flags: torch.Tensor, capacity: int, n32_max_rows: int = 8) -> None:
    # small batches read the N32 copies through the N32 build, larger ones the
    # checkpoint's N16 banks through the N16 build (reference native.py:187-202)
    if x.shape[0] <= n32_max_rows:
        _routed_one('routed_n32', x, routes, ids, gate_n32, gate_meta_n32, down_n32, down_meta_n32, workspace, out,
                    flags, capacity)
    else:
        _routed_one('routed', x, routes, ids, gate, gate_meta, down, down_meta, workspace, out, flags, capacity)


@torch.library.custom_op('ornith_g256::head_out', mutates_args={'workspace', 'out', 'flags'}, device_types='cuda')
def head_out(x: torch.Tensor, codes: torch.Tensor, scales: torch.Tensor,
             workspace: torch.Tensor, out: torch.Tensor, flags: torch.Tensor, geometry: int) -> None:
    _check_rows(x, out, HEAD_MAX_ROWS, HIDDEN)
    h = lib(_binding.libraries['head'] if _binding else 32)
    check(h.ornith_head_i8_tile_launch(ptr(x), ptr(codes), ptr(scales), ptr(workspace), workspace.numel(), ptr(out),
                                       None, 0, ptr(flags), x.shape[0], HEAD_MAX_ROWS, HEAD_VOCAB, geometry,
                                       stream(x)), 'W8 head')


@torch.library.custom_op('ornith_g256::router_topk', mutates_args={'logits', 'weights', 'ids', 'shared_logit'},
                         device_types='cuda')
def router_topk(x: torch.Tensor, router_weight: torch.Tensor, bias: torch.Tensor | None,
                shared_gate_weight: torch.Tensor | None, logits: torch.Tensor, weights: torch.Tensor,
                ids: torch.Tensor, shared_logit: torch.Tensor) -> None:
    """Router logits, softmax/top-8/renormalise and (optionally) the shared
    expert's bf16 gate logit, in the library's declared reduction order."""
    T = x.shape[0]
    if x.ndim != 2 or x.shape[1] != HIDDEN or x.stride(1) != 1 or x.dtype != torch.bfloat16:
        raise ValueError('router input must be bf16 [T, 2048] with unit column stride')
    if tuple(router_weight.shape) != (EXPERTS, HIDDEN) or not router_weight.is_contiguous():
        raise ValueError('router weight must be a contiguous bf16 [256, 2048] tensor')
    if (tuple(logits.shape) != (T, EXPERTS + 1) or logits.dtype != torch.float32 or not logits.is_contiguous()
            or tuple(weights.shape) != (T, TOP) or tuple(ids.shape) != (T, TOP) or ids.dtype != torch.int32):
        raise ValueError(f'router outputs must be logits fp32 [{T}, 257], weights/ids [{T}, 8]')
    check(lib().ornith_router_topk_launch(ptr(x), x.stride(0), ptr(router_weight), ptr(bias),
                                          ptr(shared_gate_weight), ptr(logits), ptr(weights), ptr(ids),
                                          ptr(shared_logit), T, stream(x)), 'router top-8')


@dense_out.register_fake
def _(x, codes, metadata, workspace, out, flags, capacity, n, k, geometry, a8_max_rows):
    return None


@routed_out.register_fake
def _(x, routes, ids, gate, gate_meta, down, down_meta, workspace, out, flags, capacity):
    return None


@routed_out_n32.register_fake
def _(x, routes, ids, gate, gate_meta, down, down_meta, gate_n32, gate_meta_n32, down_n32, down_meta_n32,
      workspace, out, flags, capacity, n32_max_rows=8):
    return None


@head_out.register_fake
def _(x, codes, scales, workspace, out, flags, geometry):
    return None


@router_topk.register_fake
def _(x, router_weight, bias, shared_gate_weight, logits, weights, ids, shared_logit):
    return None


# ---------------------------------------------------------------------------
# Direct entry helpers (whole layer, shared-expert slot, G256 head)
# ---------------------------------------------------------------------------
def routed_shared_tables(x, routes, ids, gate, gate_meta, down, down_meta, s_gate, s_gate_meta, s_down,
                         s_down_meta, shared_logit, silu, sigmoid, workspace, out, shared_out, flags, capacity,
                         tile=32):
    """Routed experts plus the shared expert as a ninth slot
    (routed_storage_n32_consumer.cpp:385-401); shared banks are N32 dense."""
    args = [ptr(t) for t in (x, routes, ids, gate, gate_meta, down, down_meta, s_gate, s_gate_meta, s_down,
                             s_down_meta, shared_logit, silu, sigmoid, workspace)]
    check(lib(tile).ornith_routed_direct_launch_shared_tables(
        *args, workspace.numel(), ptr(out), ptr(shared_out), ptr(flags), x.shape[0], capacity, stream(x)),
        'routed + shared slot')


def moe_layer(x, router_weight, bias, shared_gate_weight, gate, gate_meta, down, down_meta, s_gate, s_gate_meta,
              s_down, s_down_meta, silu, sigmoid, workspace, topk_weights, topk_ids, shared_logit, out, flags,
              capacity, tile=32):
    """The whole MoE layer: router, top-8, routed experts, shared expert and
    the routed + shared sum, in one launch sequence."""
    args = [ptr(t) for t in (x, router_weight, bias, shared_gate_weight, gate, gate_meta, down, down_meta, s_gate,
                             s_gate_meta, s_down, s_down_meta, silu, sigmoid, workspace)]
    check(lib(tile).ornith_moe_layer_launch(*args, workspace.numel(),
                                            *[ptr(t) for t in (topk_weights, topk_ids, shared_logit, out, flags)],
                                            x.shape[0], capacity, stream(x)), 'MoE layer')


def moe_layer_static(x, router_weight, bias, shared_gate_weight, gate, gate_meta, down, down_meta, s_gate,
                     s_gate_meta, s_down, s_down_meta, silu, sigmoid, topk_weights, topk_ids, shared_logit, out, flags,
                     tile=32):
    """moe_layer for at most 32 tokens without a workspace: the library's own
    static device scratch is used (one per GPU; overlapping calls on one GPU race)."""
    args = [ptr(t) for t in (x, router_weight, bias, shared_gate_weight, gate, gate_meta, down, down_meta, s_gate,
                             s_gate_meta, s_down, s_down_meta, silu, sigmoid, topk_weights, topk_ids, shared_logit,
                             out, flags)]
    check(lib(tile).ornith_moe_layer_launch_static(*args, x.shape[0], stream(x)), 'MoE layer (static scratch)')


def shared_fixed8_bytes(capacity):
    size = _SZ(0)
    check(lib().ornith_shared_fixed8_get_layout(capacity, C.byref(size)), 'fixed8 layout')
    return size.value


def shared_fixed8(x, gate_up, gate_up_meta, down, down_meta, gate_weight, silu, sigmoid, workspace, out, flags,
                  capacity):
    """The production shared expert of decode rows (shared_kernel.py:33-62):
    dense A8 gate/up, bf16 SiLU * up, dense A8 down, bf16 sigmoid gate."""
    check(lib().ornith_shared_fixed8_launch(*[ptr(t) for t in (x, gate_up, gate_up_meta, down, down_meta,
                                                               gate_weight, silu, sigmoid, workspace)],
                                            workspace.numel(), ptr(out), ptr(flags), x.shape[0], capacity,
                                            stream(x)), 'shared expert (fixed8)')


def logits_argmax(logits, out):
    """Greedy hand-off: out int64 [M] = argmax of each row of bf16 logits [M, N]
    (first NaN, else first maximum)."""
    if logits.dtype != torch.bfloat16 or logits.ndim != 2 or logits.stride(1) != 1 or out.dtype != torch.int64:
        raise ValueError('logits must be bf16 [M, N] with unit column stride; out int64 [M]')
    check(lib().ornith_logits_argmax_launch(ptr(logits), logits.shape[0], logits.shape[1], logits.stride(0),
                                            ptr(out), stream(logits)), 'logits argmax')


def dense_head(x, codes, meta, workspace, logits, logits_bf16, argmax, flags, capacity):
    """G256 4-bit LM head: fp32 (and optional bf16) logits and the argmax."""
    check(lib().ornith_dense_g256_head_launch(ptr(x), ptr(codes), ptr(meta), ptr(workspace), workspace.numel(),
                                              ptr(logits), ptr(logits_bf16), ptr(argmax), ptr(flags), x.shape[0],
                                              capacity, codes.shape[0] * 32, stream(x)), 'G256 head')


def single_token_path(path=None, tile=32):
    """Which kernels run single-token (T == 1) routed and layer calls, for
    the process: 0 the one-launch kernel wherever its grid is resident at
    once, 1 the three kernels; None only queries.  Returns the previous
    setting.  Results are identical either way."""
    prev = lib(tile).ornith_mi355x_single_token_path(-1 if path is None else int(path))
    if prev < 0:
        raise ValueError(f'single-token path must be 0 or 1, got {path}')
    return prev


def silu_selfcheck(tile=32):
    """Both SiLU forms of the prefill gate/up epilogue over every fp32 value
    of the short form's domain (2^-60 <= |g| <= 80): (values compared,
    mismatching bit patterns) -- 0 mismatches expected."""
    dev = torch.device('cuda', torch.cuda.current_device())
    out = torch.zeros(3, dtype=torch.int32, device=dev)          # u64 count | u32 mismatches
    check(lib(tile).ornith_mi355x_silu_selfcheck(ptr(out), ptr(out[2:]), stream(out)), 'silu self-check')
    torch.cuda.synchronize()
    v = out.cpu().numpy().view('uint32')
    return int(v[0]) | (int(v[1]) << 32), int(v[2])


def decode_route_path(path=None, tile=32):
    """Which kernels run the router, top-8 and sort of 2..32-token layer
    calls, for the process: 0 one launch wherever its grid is resident at
    once, 1 three kernels; None only queries.  Returns the previous setting.
    Results are identical either way."""
    prev = lib(tile).ornith_mi355x_decode_route_path(-1 if path is None else int(path))
    if prev < 0:
        raise ValueError(f'decode route path must be 0 or 1, got {path}')
    return prev


def handoff_spin_limit(spins=None, tile=32):
    """Poll rounds of the one-launch kernels' hand-off waits, for the
    process (default 32768; 0 gives every wait up at once, for tests of the
    time-out path); None only queries.  Returns the previous setting."""
    prev = lib(tile).ornith_mi355x_handoff_spin_limit(-1 if spins is None else int(spins))
    if prev < 0:
        raise ValueError(f'hand-off spin limit must be 0..16777216, got {spins}')
    return prev


def workspace_reset(workspace=None, tile=32):
    """Zero a workspace on the current stream (clears the poisoned mark a
    hand-off time-out leaves); None resets the static scratch of
    moe_layer_static on the current device."""
    if workspace is None:
        dev = torch.device('cuda', torch.cuda.current_device())
        check(lib(tile).ornith_mi355x_workspace_reset(None, 0, stream(torch.empty(0, device=dev))),
              'static scratch reset')
    else:
        check(lib(tile).ornith_mi355x_workspace_reset(ptr(workspace), workspace.numel(), stream(workspace)),
              'workspace reset')


class KernelTimer:
    """Times launches of one library kernel ("*" = all) with HIP event pairs
    recorded on each launch's own stream (include/ornith_timing.h).  The
    launches themselves are unchanged."""

    def __init__(self, kernel: str = '*', capacity: int = 100_000, tile: int = 32):
        self.kernel, self.capacity, self.h = kernel, capacity, lib(tile)

    def __enter__(self):
        check(self.h.ornith_mi355x_timing_arm(self.kernel.encode(), self.capacity), 'timing arm')
        return self

    def __exit__(self, *exc):
        self.h.ornith_mi355x_timing_arm(None, 0)
        return False

    def names(self):
        n = self.h.ornith_mi355x_timing_names(None, 0)
        buf = C.create_string_buffer(n + 1)
        self.h.ornith_mi355x_timing_names(buf, n + 1)
        return [v for v in buf.value.decode().split(',') if v]

    def read(self, kernel: str):
        """(launches, average milliseconds per launch) for `kernel`."""
        count, total = _INT(0), C.c_double(0.0)
        check(self.h.ornith_mi355x_timing_read(kernel.encode(), C.byref(count), C.byref(total)), 'timing read')
        return count.value, (total.value / count.value if count.value else 0.0)
