"""Compile the gfx950 HIP library in-tree.

hipcc cross-compiles without a GPU.  Flags: -ffp-contract=off keeps every
fp32 multiply and add separately rounded (the reference builds with the same
flag, scripts/build-native.sh:45-47); packed-fp32 instruction selection is
disabled; symbols are hidden except the extern "C" ABI.

Two builds come from the same sources: routed expert banks in N32 tiles
(libornith_g256_mi355x.so, the N32 storage library role) and in the
checkpoint's N16 tiles (libornith_g256_mi355x_n16.so, the parent routed
library role).  Everything but the routed bank addressing is identical.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG.parent / 'csrc'
LIBDIR = PKG / 'lib'
VARIANTS = {32: 'libornith_g256_mi355x.so', 16: 'libornith_g256_mi355x_n16.so'}
LIBNAME = VARIANTS[32]
SOURCES = ['act.hip', 'routing.hip', 'proj_gemv.hip', 'proj_mfma.hip', 'decode.hip', 'decode1.hip', 'head.hip',
           'timing.hip', 'storage.hip', 'shared.hip', 'gemm.hip', 'api.hip']
HIPCC = os.environ.get('HIPCC', '/opt/rocm/bin/hipcc')
FLAGS = ['--offload-arch=gfx950', '-O3', '-std=c++20', '-fPIC', '-ffp-contract=off',
         '-fhip-fp32-correctly-rounded-divide-sqrt', '-fvisibility=hidden',
         '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
         '-Wno-unused-result', '-Wno-unused-command-line-argument']


def library_path(tile: int = 32) -> Path:
    return LIBDIR / VARIANTS[tile]


TRACE_DIR = LIBDIR / 'trace'


def _compile(name, tile, objdir, extra=()):
    src = CSRC / name
    obj = objdir / (name + '.o')
    cmd = [HIPCC, *FLAGS, *extra, f'-DORNITH_ROUTED_TILE={tile}', '-c', str(src), '-o', str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode:
        raise RuntimeError(f'hipcc failed for {name} (tile {tile}):\n{res.stderr}')
    return obj, res.stderr


def _link(objs, out):
    tmp = out.with_suffix('.so.tmp')
    cmd = [HIPCC, '--offload-arch=gfx950', '-shared', '-fPIC', '-o', str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode:
        raise RuntimeError(f'link failed for {out.name}:\n{res.stderr}')
    os.replace(tmp, out)


def build(verbose: bool = False, jobs: int = 8) -> list[Path]:
    LIBDIR.mkdir(exist_ok=True)
    sources = [s for s in SOURCES if (CSRC / s).exists()]
    jobs_list = []
    for tile in VARIANTS:
        objdir = LIBDIR / f'obj{tile}'
        objdir.mkdir(exist_ok=True)
        jobs_list += [(name, tile, objdir) for name in sources]
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        results = list(pool.map(lambda j: _compile(*j), jobs_list))
    outs = []
    for tile, name in VARIANTS.items():
        objs = [obj for (obj, err), (_, t, _) in zip(results, jobs_list) if t == tile]
        if verbose:
            for (obj, err), (_, t, _) in zip(results, jobs_list):
                if t == tile and err.strip():
                    print(err)
        out = library_path(tile)
        _link(objs, out)
        outs.append(out)
    return outs


def build_stage_trace(jobs: int = 8) -> Path:
    """The N32 build with the single-token kernel's stage trace compiled in
    (-DORNITH_STAGE_TRACE), as lib/trace/libornith_g256_mi355x.so.  For
    measurement only (stage_trace.py); the product builds record nothing."""
    objdir = TRACE_DIR / 'obj'
    objdir.mkdir(parents=True, exist_ok=True)
    sources = [s for s in SOURCES if (CSRC / s).exists()]
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        results = list(pool.map(lambda n: _compile(n, 32, objdir, ('-DORNITH_STAGE_TRACE',)), sources))
    out = TRACE_DIR / VARIANTS[32]
    _link([obj for obj, _ in results], out)
    return out


if __name__ == '__main__':
    import sys
    print(build_stage_trace() if '--stage-trace' in sys.argv[1:] else build(verbose=True))
