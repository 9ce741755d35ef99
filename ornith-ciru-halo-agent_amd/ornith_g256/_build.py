"""Compile the gfx950 HIP library in-tree.

hipcc cross-compiles without a GPU.  Flags: -ffp-contract=off keeps every
fp32 multiply and add separately rounded (the reference builds with the same
flag, scripts/build-native.sh:45-47); packed-fp32 instruction selection is
disabled; symbols are hidden except the extern "C" ABI.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG.parent / 'csrc'
LIBDIR = PKG / 'lib'
LIBNAME = 'libornith_g256_mi355x.so'
SOURCES = ['act.hip', 'routing.hip', 'proj_gemv.hip', 'proj_mfma.hip', 'decode.hip', 'decode1.hip', 'head.hip', 'timing.hip',
           'api.hip']
HIPCC = os.environ.get('HIPCC', '/opt/rocm/bin/hipcc')
FLAGS = ['--offload-arch=gfx950', '-O3', '-std=c++20', '-fPIC', '-ffp-contract=off',
         '-fhip-fp32-correctly-rounded-divide-sqrt', '-fvisibility=hidden',
         '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
         '-Wno-unused-result', '-Wno-unused-command-line-argument']


def library_path() -> Path:
    return LIBDIR / LIBNAME


def build(verbose: bool = False, jobs: int = 8) -> Path:
    LIBDIR.mkdir(exist_ok=True)
    objdir = LIBDIR / 'obj'
    objdir.mkdir(exist_ok=True)
    sources = [s for s in SOURCES if (CSRC / s).exists()]

    def compile_one(name):
        src = CSRC / name
        obj = objdir / (name + '.o')
        cmd = [HIPCC, *FLAGS, '-c', str(src), '-o', str(obj)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode:
            raise RuntimeError(f'hipcc failed for {name}:\n{res.stderr}')
        if verbose and res.stderr.strip():
            print(res.stderr)
        return obj

    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(compile_one, sources))
    out = library_path()
    tmp = out.with_suffix('.so.tmp')
    cmd = [HIPCC, '--offload-arch=gfx950', '-shared', '-fPIC', '-o', str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode:
        raise RuntimeError(f'link failed:\n{res.stderr}')
    os.replace(tmp, out)
    return out


if __name__ == '__main__':
    print(build(verbose=True))
