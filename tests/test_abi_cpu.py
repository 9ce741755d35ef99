"""The C ABI library: loads, exports every symbol include/*.h declares, and
validates arguments on the host exactly like the reference (no GPU calls:
every case here returns before any launch)."""
import ctypes as C
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
INVALID = 1   # hipErrorInvalidValue


def _declared_symbols():
    names = set()
    for h in sorted((ROOT / 'include').glob('*.h')):
        text = h.read_text()
        names |= set(re.findall(r'ORNITH_EXPORT\s+[\w\s\*]+?\b(ornith_\w+)\s*\(', text))
    return names


@pytest.fixture(scope='module')
def lib():
    from ornith_g256 import native
    return native.lib()


@pytest.mark.parametrize('tile', [32, 16])
def test_every_declared_symbol_is_exported(tile):
    from ornith_g256 import native
    handle = native.lib(tile)
    names = _declared_symbols()
    assert len(names) >= 23
    for n in sorted(names):
        assert hasattr(handle, n), n
    # and nothing undeclared is exported
    import subprocess
    nm = subprocess.run(['nm', '-D', '--defined-only', str(native.library_path(tile))], capture_output=True, text=True)
    if nm.returncode == 0:
        exported = {l.split()[-1] for l in nm.stdout.splitlines() if ' T ' in l and 'ornith_' in l}
        assert exported == names


def test_markers(lib):
    from ornith_g256 import native
    assert lib.ornith_routed_storage_n32() == 32
    assert native.lib(16).ornith_routed_storage_n32() == 16     # the N16-bank build
    assert lib.ornith_routed_prefill_output_tile() == 32
    assert lib.ornith_dense_g256_abi_version() == 1
    assert lib.ornith_dense_g256_n32_rows() == 16
    assert lib.ornith_head_i8_tile_abi_version() == 1
    assert lib.ornith_head_i8_tile_shortlist() == 1
    assert lib.ornith_mi355x_abi_version() == 1


def test_both_builds_share_every_layout():
    """The N16 and N32 builds differ only in routed bank addressing: every
    workspace layout is byte-identical (the reference's pairing rule for an
    N32 decode library and its N16 parent, native.py:95-99)."""
    from ornith_g256 import native
    for tcap in (1, 16, 64, 1120, 8192):
        for kind in ('routed', 'layer'):
            assert bytes(native.routed_layout(tcap, kind, tile=16)) == bytes(native.routed_layout(tcap, kind, tile=32))
    assert bytes(native.routed_layout(16, 'shared', tile=16)) == bytes(native.routed_layout(16, 'shared', tile=32))


def test_routed_layout_contract(lib):
    from ornith_g256 import native
    for tcap in (0, 1, 16, 1120, 8192):
        l = native.routed_layout(tcap)
        offs = [getattr(l, f) for f in native._ROUTED_FIELDS[1:]]
        assert all(o % 256 == 0 for o in offs) and offs == sorted(offs)
        assert l.workspace_bytes >= offs[-1] + tcap * 2048 * 4
    layout = native.RoutedLayout()
    assert lib.ornith_routed_direct_get_layout(8193, C.byref(layout)) == INVALID
    assert lib.ornith_routed_direct_get_layout(-1, C.byref(layout)) == INVALID
    assert lib.ornith_routed_direct_get_layout(4, None) == INVALID
    assert lib.ornith_routed_shared_get_layout(17, C.byref(layout)) == INVALID
    assert lib.ornith_routed_shared_get_layout(16, C.byref(layout)) == 0


def _routed_args(T, Tcap, ws_bytes, ptrs=1):
    p = C.c_void_p(0x1000) if ptrs else None
    return [p] * 8 + [ws_bytes, p, p, T, Tcap, None]


def test_routed_launch_validation(lib):
    from ornith_g256 import native
    need = native.routed_layout(8).workspace_bytes
    for name in ('ornith_routed_direct_launch', 'ornith_routed_direct_launch_a4',
                 'ornith_routed_direct_launch_a4_prefill'):
        fn = getattr(lib, name)
        assert fn(*_routed_args(0, 8, need)) == 0                 # T == 0: success, no pointer touched
        assert fn(*_routed_args(0, 8, need, ptrs=0)) == 0
        assert fn(*_routed_args(9, 8, need)) == INVALID           # T > Tcap
        assert fn(*_routed_args(-1, 8, need)) == INVALID
        assert fn(*_routed_args(1, 8, need - 1)) == INVALID       # short workspace
        assert fn(*_routed_args(1, 8193, 1 << 40)) == INVALID     # Tcap > 8192
        assert fn(*_routed_args(1, 8, need, ptrs=0)) == INVALID   # null pointers
        args = _routed_args(1, 8, need)
        args[0] = C.c_void_p(0x1001)                              # misaligned input
        assert fn(*args) == INVALID
        args[0] = C.c_void_p(0x1008)                              # 8- but not 16-byte aligned input
        assert fn(*args) == INVALID


def test_dense_validation(lib):
    from ornith_g256 import native
    l = native.DenseLayout()
    assert lib.ornith_dense_g256_get_layout(16, 6144, 2048, 8, C.byref(l)) == 0
    assert lib.ornith_dense_g256_get_layout(16, 6144, 2048, 4, C.byref(l)) == INVALID
    assert lib.ornith_dense_g256_get_layout(16, 6152, 2048, 8, C.byref(l)) == INVALID   # N > 12288? no: N%16
    assert lib.ornith_dense_g256_get_layout(16, 12304, 2048, 8, C.byref(l)) == INVALID
    assert lib.ornith_dense_g256_get_layout(16, 248320, 2048, 8, C.byref(l)) == 0
    assert lib.ornith_dense_g256_get_layout(16, 1024, 2000, 8, C.byref(l)) == INVALID
    assert lib.ornith_dense_g256_get_layout(8193, 1024, 2048, 8, C.byref(l)) == INVALID
    assert lib.ornith_dense_g256_get_layout(16, 1024, 2048, 8, C.byref(l)) == 0
    ws = l.workspace_bytes
    p = C.c_void_p
    base = [p(0x10000), p(0x20000), p(0x30000), p(0x100000), ws, p(0x4000000), p(0x5000000)]
    # M == 0 succeeds without touching pointers, even null ones
    assert lib.ornith_dense_g256_launch(*([None] * 4 + [0] + [None] * 2), 0, 16, 1024, 2048, 8, 128, 2, None) == 0
    assert lib.ornith_dense_g256_launch(*base, 1, 16, 1024, 2048, 8, 64, 2, None) == INVALID   # transform
    assert lib.ornith_dense_g256_launch(*base, 1, 16, 1024, 2048, 8, 128, 3, None) == INVALID  # geometry
    assert lib.ornith_dense_g256_launch(*base, 17, 16, 1024, 2048, 8, 128, 2, None) == INVALID  # M > Mcap
    bad = list(base)
    bad[5] = p(0x100000 + 64)          # output overlaps the workspace
    assert lib.ornith_dense_g256_launch(*bad, 1, 16, 1024, 2048, 8, 128, 2, None) == INVALID
    bad = list(base)
    bad[0] = p(0x10008)                # input 8- but not 16-byte aligned (loaded as 16-byte words)
    assert lib.ornith_dense_g256_launch(*bad, 1, 16, 1024, 2048, 8, 128, 2, None) == INVALID
    assert lib.ornith_dense_g256_launch_n32(*bad, 1, 16, 1024, 2048, 8, 128, 2, None) == INVALID
    bad = list(base)
    bad[4] = ws - 1
    assert lib.ornith_dense_g256_launch(*bad, 1, 16, 1024, 2048, 8, 128, 2, None) == INVALID
    # N32 entry: M in 1..16, N % 32, geometry 2
    assert lib.ornith_dense_g256_launch_n32(*base, 0, 16, 1024, 2048, 8, 128, 2, None) == INVALID
    assert lib.ornith_dense_g256_launch_n32(*base, 17, 32, 1024, 2048, 8, 128, 2, None) == INVALID
    assert lib.ornith_dense_g256_launch_n32(*base, 1, 16, 1040, 2048, 8, 128, 2, None) == INVALID
    assert lib.ornith_dense_g256_launch_n32(*base, 1, 16, 1024, 2048, 8, 128, 1, None) == INVALID
    # prepare_bf16
    assert lib.ornith_dense_g256_prepare_bf16(*([None] * 6), 0, 1024, 2048, None) == 0
    assert lib.ornith_dense_g256_prepare_bf16(*([None] * 6), 1, 1024, 2048, None) == INVALID
    # gemm_bf16: workspace round_up(M, 16) * K * 2 bytes, 256-aligned; output 16-aligned
    p = C.c_void_p
    need = 32 * 2048 * 2
    args = lambda ws_bytes, out: (p(0x100000), p(0x2000000), p(0x3000000), p(0x4000000), ws_bytes, p(out),
                                  p(0x6000000))
    assert lib.ornith_dense_g256_gemm_bf16(*args(need, 0x5000000), 0, 1024, 2048, None) == 0
    assert lib.ornith_dense_g256_gemm_bf16(*args(need - 1, 0x5000000), 17, 1024, 2048, None) == INVALID
    assert lib.ornith_dense_g256_gemm_bf16(*args(need, 0x5000008), 17, 1024, 2048, None) == INVALID
    assert lib.ornith_dense_g256_gemm_bf16(*args(need, 0x5000000), 17, 1000, 2048, None) == INVALID   # N % 16
    assert lib.ornith_dense_g256_gemm_bf16(*args(need, 0x5000000), -1, 1024, 2048, None) == INVALID


def test_head_validation(lib):
    from ornith_g256 import native
    l = native.HeadLayout()
    assert lib.ornith_head_i8_tile_get_layout(64, 248320, C.byref(l)) == 0
    assert lib.ornith_head_i8_tile_get_layout(65, 248320, C.byref(l)) == INVALID
    assert lib.ornith_head_i8_tile_get_layout(64, 151936, C.byref(l)) == INVALID
    ws = l.workspace_bytes
    p = C.c_void_p
    args = [p(0x10000), p(0x200000), p(0x30000), p(0x10000000), ws, p(0x80000000)]
    # group_dots null iff bytes == 0
    assert lib.ornith_head_i8_tile_launch(*args, None, 4, p(0x90000000), 1, 64, 248320, 2, None) == INVALID
    assert lib.ornith_head_i8_tile_launch(*args, p(0xA0000000), 0, p(0x90000000), 1, 64, 248320, 2, None) == INVALID
    assert lib.ornith_head_i8_tile_launch(*args, None, 0, p(0x90000000), 0, 64, 248320, 2, None) == 0
    assert lib.ornith_head_i8_tile_launch(*args, None, 0, p(0x90000000), 65, 64, 248320, 2, None) == INVALID
    # G256 head: M <= 64, N % 32
    assert lib.ornith_dense_g256_head_workspace_bytes(65, 151936) == 0
    need = lib.ornith_dense_g256_head_workspace_bytes(64, 151936)
    hp = [p(0x10000), p(0x200000), p(0x30000), p(0x10000000), need, p(0x20000000), None, p(0x30000000),
          p(0x40000000)]
    assert lib.ornith_dense_g256_head_launch(*hp, 0, 64, 151936, None) == 0
    assert lib.ornith_dense_g256_head_launch(*hp, 1, 64, 151920, None) == INVALID


def test_router_and_layer_validation(lib):
    from ornith_g256 import native
    p = C.c_void_p(0x10000)
    assert lib.ornith_router_topk_launch(p, 2048, p, None, None, p, p, p, None, 0, None) == 0
    assert lib.ornith_router_topk_launch(p, 2047, p, None, None, p, p, p, None, 1, None) == INVALID
    assert lib.ornith_router_topk_launch(p, 2048, p, None, p, p, p, p, None, 1, None) == INVALID  # no shared out
    need = native.routed_layout(4, 'layer').workspace_bytes
    args = [p] * 15 + [need] + [p] * 5
    assert lib.ornith_moe_layer_launch(*args, 0, 4, None) == 0
    assert lib.ornith_moe_layer_launch(*args, 5, 4, None) == INVALID
    args[15] = need - 256
    assert lib.ornith_moe_layer_launch(*args, 1, 4, None) == INVALID


@pytest.fixture()
def fresh_binding():
    from ornith_g256 import native
    native.reset_binding()
    yield native
    native.reset_binding()


def test_logits_argmax_validation(lib):
    p = C.c_void_p(0x10000)
    fn = lib.ornith_logits_argmax_launch
    assert fn(None, 0, 100, 100, None, None) == 0          # M == 0
    assert fn(p, 2, 100, 99, p, None) == INVALID            # ld < N
    assert fn(None, 2, 100, 100, p, None) == INVALID        # null logits
    assert fn(p, 2, 100, 100, C.c_void_p(0x10004), None) == INVALID   # misaligned / overlapping output


def test_fixed8_validation(lib):
    from ornith_g256 import native
    size = native.shared_fixed8_bytes(8)
    assert size > 0 and native.shared_fixed8_bytes(16) > size
    with pytest.raises(RuntimeError):
        native.shared_fixed8_bytes(8193)
    p = C.c_void_p(0x10000)
    fn = lib.ornith_shared_fixed8_launch
    assert fn(*([p] * 9), size, p, p, 0, 8, None) == 0                    # M == 0: nothing touched
    assert fn(*([p] * 9), size - 1, p, p, 1, 8, None) == INVALID          # short workspace
    assert fn(*([p] * 9), size, p, p, 9, 8, None) == INVALID              # M > Mcap
    assert fn(*([p] * 9), size, p, p, 1, 8, None) == INVALID              # overlapping buffers


def test_configure_sizes_arena(fresh_binding):
    native = fresh_binding
    size = native.configure({'routed_storage_n32': True}, 64, [(12288, 2048), (1024, 2048)])
    assert size >= native.routed_layout(64).workspace_bytes
    assert size >= (64 * 2048 + 12288 * 2048) * 2
    assert size >= native.head_layout(64, 248320).workspace_bytes
    # the same settings again are accepted; other settings in a live process are not
    assert native.configure({'routed_storage_n32': True}, 64, [(12288, 2048), (1024, 2048)]) == size
    with pytest.raises(RuntimeError):
        native.configure({'routed_storage_n32': True, 'routed_prefill_activation_bits': 4}, 64, [])


@pytest.mark.parametrize('settings', [
    {'routed_activation_bits': 4, 'routed_prefill_activation_bits': 4},
    {'routed_activation_bits': 5},
    {'routed_storage_n32': True, 'routed_decode_n32': True},
    {'routed_n32_max_rows': 12},
    {'routed_decode_n32': True},                                        # no routed_n32_library
    {'routed_decode_n32': True, 'routed_activation_bits': 4, 'routed_n32_library': 'x'},
])
def test_configure_rejects_bad_settings(fresh_binding, settings):
    with pytest.raises(ValueError):
        fresh_binding.configure(settings, 64, [])


def test_configure_matches_bank_layout_to_library(fresh_binding):
    """Sole N32 storage needs the N32 build as routed library, the default
    (checkpoint N16 banks) the N16 build; a mismatch is refused before any
    launch could misread a bank."""
    native = fresh_binding
    with pytest.raises(ValueError, match='N32'):
        native.configure({'routed_storage_n32': True, 'routed_library': str(native.library_path(16))}, 8, [])
    with pytest.raises(ValueError, match='N16'):
        native.configure({'routed_library': str(native.library_path(32))}, 8, [])
    with pytest.raises(ValueError):
        native.configure({'routed_library': '/nonexistent/libornith_routed_direct.so'}, 8, [])
    native.configure({'routed_library': str(native.library_path(16))}, 8, [])
    fn, tile = native._binding.routed['routed']
    assert tile == 16
    native.reset_binding()
    native.configure({'routed_decode_n32': True, 'routed_n32_library': str(native.library_path(32))}, 8, [])
    assert native._binding.routed['routed_n32'][1] == 32 and native._binding.routed['routed'][1] == 16


def test_routed_op_refuses_banks_of_the_other_tile(fresh_binding):
    import torch
    native = fresh_binding
    native.configure({'routed_storage_n32': True}, 8, [])
    n16 = torch.empty((256, 64, 8, 32, 16), dtype=torch.int32)
    meta = torch.empty((256, 64, 8, 16), dtype=torch.int32)
    with pytest.raises(ValueError, match='N32'):
        native._check_banks(32, n16, meta, n16, meta)
    ok = (torch.empty((256, 32, 8, 32, 32), dtype=torch.int32), torch.empty((256, 32, 8, 32), dtype=torch.int32),
          torch.empty((256, 64, 2, 32, 32), dtype=torch.int32), torch.empty((256, 64, 2, 32), dtype=torch.int32))
    native._check_banks(32, *ok)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from ornith_g256 import native
    monkeypatch.setattr(native, '_handles', {})
    monkeypatch.setattr(native, 'LIB_DIR', tmp_path)
    with pytest.raises(RuntimeError, match='missing'):
        native.lib()


def test_handoff_spin_limit_and_workspace_reset_arguments(lib):
    """The hand-off poll limit is a process-wide setting (-1 queries); the
    workspace reset checks its arguments before any launch."""
    prev = lib.ornith_mi355x_handoff_spin_limit(-1)
    assert prev == 1 << 15
    assert lib.ornith_mi355x_handoff_spin_limit(0) == prev
    assert lib.ornith_mi355x_handoff_spin_limit(prev) == 0
    assert lib.ornith_mi355x_handoff_spin_limit(-2) == -1
    assert lib.ornith_mi355x_handoff_spin_limit((1 << 24) + 1) == -1
    assert lib.ornith_mi355x_handoff_spin_limit(-1) == prev
    assert lib.ornith_mi355x_workspace_reset(None, 256, None) == INVALID       # static scratch takes bytes 0
    assert lib.ornith_mi355x_workspace_reset(C.c_void_p(0x1008), 256, None) == INVALID   # not 256-aligned
    assert lib.ornith_mi355x_workspace_reset(C.c_void_p(0x1000), 258, None) == INVALID   # not whole words
