"""ctypes binding of libnoise_hip.so (the C ABI of include/noise_hip.h).

The library is loaded after `import torch` so that it binds to torch's HIP runtime. There is no CPU
fallback: a missing or stale library raises.
"""
import ctypes
from pathlib import Path

import torch  # noqa: F401  (must precede the HIP library load: one libamdhip64 per process)

LIB_PATH = Path(__file__).resolve().parent / 'libnoise_hip.so'

_c_int, _c_long, _c_float, _c_size, _vp = ctypes.c_int, ctypes.c_long, ctypes.c_float, ctypes.c_size_t, ctypes.c_void_p
_fp = ctypes.POINTER(ctypes.c_float)

ERRORS = {-1: 'NOISE_EINVAL (rejected argument)', -2: 'NOISE_ENOSPC (workspace too small)',
          -3: 'NOISE_ENOTSUP (shape outside the kernel tiling)'}

# name -> argtypes; every entry point returns int.
SIGNATURES = {
    'noise_version': [],
    'noise_lowrank_linear_workspace_size': [_c_int, _c_int, ctypes.POINTER(_c_size)],
    'noise_lowrank_linear': [_vp, _c_long, _c_long, _vp, _c_int, _c_int, _vp, _vp, _vp, _c_int, _c_int, _c_int,
                             _vp, _vp, _c_int, _vp, _c_size, _vp],
    'noise_lowrank_mlp_workspace_size': [_c_int, _c_int, _c_int, _c_int, ctypes.POINTER(_c_size)],
    'noise_lowrank_mlp': [_vp, _c_long, _c_long, _vp, _vp, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _c_int,
                          _c_int, _c_int, _vp, _vp, _c_int, _vp, _c_size, _vp],
}

_lib = None


class NoiseHipError(RuntimeError):
    pass


def load(path=None):
    """Load the library and declare every entry point; raises if it is missing."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise NoiseHipError(f'{p} is missing: build it with `python -m noise_amd.build` (no CPU fallback)')
    lib = ctypes.CDLL(str(p))
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _c_int
    if path is None:
        _lib = lib
    return lib


def check(rc, what):
    if rc != 0:
        msg = ERRORS.get(rc, f'hipError_t {rc}')
        raise NoiseHipError(f'{what} failed: {msg}')


def call(name, *args):
    """Call an entry point and raise on a non-zero status."""
    check(getattr(load(), name)(*args), name)


def size_query(name, *args):
    out = _c_size(0)
    call(name, *args, ctypes.byref(out))
    return out.value
