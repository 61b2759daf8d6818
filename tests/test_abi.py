"""The C-ABI library loads and exports every symbol include/*.h declares; the host wrappers reject bad
arguments before any GPU call. CPU only (no compute calls)."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

from noise_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
_lib_EINVAL, _lib_ENOSPC = -1, -2


def declared_symbols():
    names = set()
    for h in (ROOT / 'include').glob('*.h'):
        text = re.sub(r'/\*.*?\*/', '', h.read_text(), flags=re.S)
        names |= set(re.findall(r'^\s*int\s+(noise_\w+)\s*\(', text, flags=re.M))
    return names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = declared_symbols()
    assert declared, 'no declarations parsed'
    for name in declared:
        assert hasattr(lib, name), name
    assert declared == set(_lib.SIGNATURES), declared ^ set(_lib.SIGNATURES)


def test_version_and_size_queries_run_on_cpu():
    assert _lib.load().noise_version() >= 100
    n = _lib.size_query('noise_lowrank_mlp_workspace_size', 4, 256, 512, 2048)
    assert n >= 4 * 256 * 2048 * 2
    with pytest.raises(_lib.NoiseHipError):
        _lib.size_query('noise_lowrank_mlp_workspace_size', 0, 256, 512, 2048)


def test_null_workspace_is_rejected_without_touching_the_gpu():
    rc = _lib.load().noise_lowrank_linear(None, 512, 0, None, 512, 512, None, None, None, 1, 16, 0, None, None, 0,
                                          None, 0, None)
    assert rc in (_lib_EINVAL, _lib_ENOSPC)


def test_ops_refuse_cpu_tensors():
    from noise_amd import ops
    x = torch.zeros(16, 512, dtype=torch.bfloat16)
    w = torch.zeros(512, 512, dtype=torch.bfloat16)
    a = torch.zeros(2, 512)
    with pytest.raises(ValueError, match='CUDA'):
        ops.lowrank_linear(x, w, a, a, torch.zeros(2))
