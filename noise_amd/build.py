"""Build libnoise_hip.so in-tree with hipcc for gfx950 (no torch extension machinery).

    python -m noise_amd.build [--jobs N]

Each csrc/*.hip compiles to an object under noise_amd/_build/, then one shared library is linked next to
this file. The library depends only on the HIP runtime; it is loaded with ctypes after `import torch`, so
the process shares torch's libamdhip64 (same SONAME).
"""
import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / 'csrc'
BUILD = PKG / '_build'
LIB = PKG / 'libnoise_hip.so'
ARCH = 'gfx950'

HIPCC_FLAGS = [
    '-O3', '-std=c++17', f'--offload-arch={ARCH}', '-fPIC', '-mcode-object-version=5',
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
    '-Wno-unused-command-line-argument', '-munsafe-fp-atomics',
]


def hipcc():
    for cand in (os.environ.get('HIPCC'), shutil.which('hipcc'), '/opt/rocm/bin/hipcc'):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError('hipcc not found; the HIP library cannot be built')


def _compile(src, extra):
    obj = BUILD / (src.stem + '.o')
    cmd = [hipcc(), *HIPCC_FLAGS, *extra, '-c', str(src), '-o', str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f'hipcc failed for {src.name}:\n{res.stderr}')
    return obj


def build(jobs=8, extra=()):
    """Compile every csrc/*.hip and link libnoise_hip.so; returns the library path."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob('*.hip'))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, list(extra)), sources))
    tmp = LIB.with_suffix('.so.tmp')
    cmd = [hipcc(), f'--offload-arch={ARCH}', '-shared', '-fPIC', *map(str, objs), '-o', str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f'link failed:\n{res.stderr}')
    os.replace(tmp, LIB)
    return LIB


if __name__ == '__main__':
    ap = argparse.ArgumentParser()
    ap.add_argument('--jobs', type=int, default=8)
    args = ap.parse_args()
    print(build(args.jobs))
    sys.exit(0)
