"""The C-ABI library loads and exports every symbol include/*.h declares, the ctypes signatures match
the header's prototypes argument by argument, and the entry points reject bad arguments before any
GPU work. CPU only (no compute calls)."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

from noise_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
EINVAL, ENOSPC = -1, -2

C_TYPES = {
    'int': ctypes.c_int, 'long': ctypes.c_long, 'float': ctypes.c_float, 'size_t': ctypes.c_size_t,
    'size_t*': ctypes.POINTER(ctypes.c_size_t), 'noise_stream_t': ctypes.c_void_p,
}


def declarations():
    """name -> list of ctypes types parsed from the prototypes in include/*.h."""
    out = {}
    for h in (ROOT / 'include').glob('*.h'):
        text = re.sub(r'/\*.*?\*/', '', h.read_text(), flags=re.S)
        for m in re.finditer(r'^\s*int\s+(noise_\w+)\s*\(([^)]*)\)\s*;', text, flags=re.M):
            name, params = m.group(1), ' '.join(m.group(2).split())
            types = []
            if params and params != 'void':
                for prm in params.split(','):
                    prm = prm.strip()
                    decl = re.sub(r'\s*\b\w+$', '', prm).replace('const ', '').replace(' ', '')
                    types.append(ctypes.c_void_p if decl.endswith('*') and decl != 'size_t*' else C_TYPES[decl])
            out[name] = types
    return out


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = declarations()
    assert len(declared) >= 20, sorted(declared)
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_lib.SIGNATURES), set(declared) ^ set(_lib.SIGNATURES)


def test_ctypes_signatures_match_header():
    for name, types in declarations().items():
        bound = _lib.SIGNATURES[name]
        assert len(bound) == len(types), (name, len(bound), len(types))
        for i, (b, t) in enumerate(zip(bound, types)):
            assert b == t, (name, i, b, t)


def test_version_and_size_queries_run_on_cpu():
    assert _lib.load().noise_version() >= 200
    n = _lib.size_query('noise_lowrank_mlp_workspace_size', 4, 256, 512, 2048)
    assert n >= 4 * 256 * 2048 * 2
    with pytest.raises(_lib.NoiseHipError):
        _lib.size_query('noise_lowrank_mlp_workspace_size', 0, 256, 512, 2048)
    head_ws = [_lib.size_query('noise_head_ce_workspace_size', 2, 256, 4096, f) for f in range(3)]
    # the split fp32 head holds [hi | lo] rows and a 3-part weight; the fp16 one h rows and a 2-part weight
    assert head_ws[_lib.HEAD_FP32_SPLIT] > head_ws[_lib.HEAD_FP32] > head_ws[_lib.HEAD_BF16]
    with pytest.raises(_lib.NoiseHipError):
        _lib.size_query('noise_head_ce_workspace_size', 2, 256, 4096, 3)
    assert _lib.value('noise_mlp_fc_parts', 2048) == 8
    assert _lib.value('noise_mlp_fc_parts', 100) == 0


def test_bad_arguments_are_rejected_without_touching_the_gpu():
    lib = _lib.load()
    rc = lib.noise_lowrank_linear(None, 512, 0, None, 512, 512, None, None, None, 1, 16, 0, None, None, 0, None, 0,
                                  None)
    assert rc in (EINVAL, ENOSPC)
    assert lib.noise_fitness(None, 8, 4, 0, None, None, None) == EINVAL
    assert lib.noise_fitness(1, 7, 4, 0, 1, 1, None) == EINVAL        # odd number of losses
    assert lib.noise_fitness(1, 8, 4, 5, 1, 1, None) == EINVAL        # unknown mode
    assert lib.noise_adam(None, None, None, None, 10, 1e-3, .5, .95, 1e-8, 1.0, None) == EINVAL
    # a bad tensor in the second 64-tensor chunk refuses the whole batch before the first chunk's launch (the
    # earlier tensors' addresses are never dereferenced: nothing is launched)
    good = (16, 16, 16, 16, 256, 1e-3, 1.0)
    ptr, count, _keep = _lib.adam_tensors([good] * 64 + [(None, 16, 16, 16, 256, 1e-3, 1.0)])
    assert lib.noise_adam_batch(ptr, count, .5, .95, 1e-8, None) == EINVAL
    ptr, count, _keep = _lib.adam_tensors([good] * 70 + [(16, 16, 16, 16, 256, 1e-3, 0.0)])  # bc2_sqrt must be > 0
    assert lib.noise_adam_batch(ptr, count, .5, .95, 1e-8, None) == EINVAL
    assert lib.noise_attention(1, 1, 100, 50, 0, 1, None, 0, 1, None, None, None, 0, None) == EINVAL  # T % 128
    # bf16 q, k, v with bf16 probabilities exists only for RMS-normalised q, k (the bounded-score softmax)
    assert lib.noise_attention(16, 1, 128, 50, 0, 3, None, 0, 16, None, None, None, 0, None) == EINVAL
    # the autocast row kernels: rows a multiple of T, something to write, lambdas in pairs, 16-byte alignment, the
    # embedding table and ids whenever x0 is needed
    ac = lambda x_in, wte, idx, lr, l0, x_out, h, rows=256, T=128, gate_w=None, gate=None: lib.noise_ac_stream(  # noqa
        x_in, wte, 4096, idx, 128, None, None, lr, l0, x_out, h, gate_w, gate, rows, T, None)
    assert ac(16, None, None, None, None, 16, 16, rows=200) == EINVAL
    assert ac(16, None, None, None, None, None, None) == EINVAL
    assert ac(16, 16, 16, 16, None, 16, 16) == EINVAL
    assert ac(None, None, None, None, None, 16, 16) == EINVAL           # x0 from the table, but no table
    assert ac(8, None, None, None, None, 16, 16) == EINVAL              # misaligned stream
    assert ac(16, None, None, None, None, 16, None, gate_w=16, gate=16) == EINVAL  # the gate needs h
    assert lib.noise_ac_qkv(None, 16, 16, None, None, 0, None, 0, 256, 128, None) == EINVAL
    assert lib.noise_ac_qkv(16, 16, 16, 16, None, 4096, 16, 128, 256, 128, None) == EINVAL  # gate without table
    # the allocation-free attention refuses moments beyond its fixed array (1024 x 2048 needs 16 Mi partials)
    assert lib.noise_attention_noalloc(1, 1024, 2048, 2048, 1, 1, None, 0, 1, None, 1, None) == ENOSPC
    assert lib.noise_attention_noalloc(1, 0, 2048, 2048, 1, 1, None, 0, 1, None, 1, None) == EINVAL
    head = lambda tgt, stride, red, loss, logits: lib.noise_head_ce(  # noqa: E731
        1, 0, None, 1, 4096, 1, 1, 1, 1, tgt, stride, 1, 256, 0, red, loss, logits, None, 0, None, 0, None)
    assert head(1, 0, 0, 1, None) == ENOSPC
    assert head(1, 0, 4, 1, None) == EINVAL          # unknown reduction
    assert head(1, -1, 1, 1, None) == EINVAL         # negative token stride
    assert head(None, 0, 0, 1, None) == EINVAL       # a loss needs targets
    assert head(None, 0, 0, None, None) == EINVAL    # nothing to produce
    assert head(None, 256, 0, None, 1) == ENOSPC     # logits only
    # the CE partials are read four at a time: vocab / 64 must be a multiple of 4
    assert lib.noise_head_ce_workspace_size(2, 256, 640, 1, ctypes.byref(ctypes.c_size_t(0))) == EINVAL
    assert lib.noise_head_ce(1, 0, None, 1, 640, 1, 1, 1, 1, 1, 0, 1, 256, 0, 0, 1, None, 1, 1 << 40, None, 0,
                             None) == EINVAL
    # the fp32 weight of NOISE_HEAD_FP32 (and its gain) must be 16-byte aligned; an unknown format is refused
    fmt = lambda w, gain, f: lib.noise_head_ce(  # noqa: E731
        16, 0, gain, w, 4096, f, 16, 16, 16, 16, 0, 1, 256, 0, 0, 16, None, 16, 1 << 40, None, 0, None)
    assert fmt(8, None, _lib.HEAD_FP32) == EINVAL
    assert fmt(16, 8, _lib.HEAD_FP32) == EINVAL
    assert fmt(16, None, 3) == EINVAL
    # WTILE copies need rows % 64 == 0, cols % 32 == 0 and 16-byte aligned pointers; the dense product knows the
    # ROWS and WTILE weight layouts only
    assert lib.noise_weight_tiles(16, 96, 512, 16, None) == EINVAL
    assert lib.noise_weight_tiles(16, 128, 48, 16, None) == EINVAL
    assert lib.noise_weight_tiles(8, 128, 512, 16, None) == EINVAL
    assert lib.noise_weight_tiles(None, 128, 512, 16, None) == EINVAL
    assert lib.noise_dense_bf16(16, 0, 2048, 512, 16, 3, 1, 256, 16, None) == EINVAL
    assert lib.noise_dense_bf16(16, 2, 2048, 512, 16, 0, 1, 256, 16, None) == EINVAL  # WTILE is not an x layout
    # a partial-sum row stride beyond the kernels' 32-bit field
    assert lib.noise_lowrank_resid(16, 16, 512, 512, 16, 16, 1, 1 << 33, 1, 16, 2, 256, 1, 16, None) == EINVAL
    assert lib.noise_embed_norm(None, 4096, None, None, None, None, 1, 16, 0, None, None) == EINVAL
    assert lib.noise_outer_update(None, 8, 1, 8, 1, 4, 2, 8, 1.0, 1, None) == EINVAL  # a null needs out == 1
    ptr, count, _keep = _lib.gather_params([(1, 1, None, 8, 4)])   # b null with in > 0
    assert lib.noise_gather_rows(1, 1 << 20, ptr, count, 1, 4, 2, None) == EINVAL
    ptr, count, _keep = _lib.gather_params([(1, 1, 1, 8, 4)])
    assert lib.noise_gather_rows(1, 1 << 20, ptr, count, 1, 4, 0, None) == EINVAL  # no pairs
    probe = lambda rows, K, vocab, P: lib.noise_readout_probes(  # noqa: E731
        16, vocab, 16, vocab, rows, K, 1, 1, 1, 1, K, 1, 0, 4, vocab, P, 512, 1, None)
    assert probe(None, 8, 4096, 16) == EINVAL      # every direction needs K == P
    assert probe(None, 16, 4000, 16) == EINVAL     # vocab % 256
    assert probe(None, 16, 8192, 16) == EINVAL     # vocab above 4096
    assert lib.noise_moved_heads(1, 1, 0.1, 1, 1, 2, 1, 128, 8, 1, 256, None) == EINVAL  # out_ld < heads * 64
    assert lib.noise_moved_heads(None, 1, 0.1, 1, 1, 2, 1, 128, 8, 1, 512, None) == EINVAL
    assert lib.noise_head_scores(1, 512, 1, 1, 0, 1, 128, 8, 1, None) == EINVAL          # no draws
    assert lib.noise_code_estimate(1, None, 2, 1, 128, 8, 1, None) == EINVAL


def test_ops_refuse_cpu_tensors():
    from noise_amd import ops
    x = torch.zeros(16, 512, dtype=torch.bfloat16)
    w = torch.zeros(512, 512, dtype=torch.bfloat16)
    a = torch.zeros(2, 512)
    with pytest.raises(ValueError, match='CUDA'):
        ops.lowrank_linear(x, w, a, a, torch.zeros(2))
    from noise_amd import credit
    with pytest.raises(ValueError, match='CUDA'):
        credit.code_estimate(torch.zeros(1, 8, 128, 2), torch.zeros(2, 1, 128, 8, 64, dtype=torch.bfloat16))


def test_tile16_layout_is_a_permutation_of_whole_tiles():
    """The TILE16 offsets are a bijection onto [0, rows * cols) and every 16 x 32 tile fills one contiguous
    KiB, so a producer's tile store and the GEMM's tile load are each eight whole 128-byte lines."""
    import torch
    from tests._util import tile16_index
    rows, cols = 64, 128
    idx = tile16_index(rows, cols)
    assert torch.equal(idx.flatten().sort().values, torch.arange(rows * cols))
    for g in range(rows // 16):
        for c in range(cols // 32):
            t = idx[16 * g:16 * g + 16, 32 * c:32 * c + 32].flatten()
            assert int(t.min()) % 512 == 0 and int(t.max() - t.min()) == 511
    # a tile's unit p holds row p // 4 and logical 8-column chunk (p % 4) ^ ((p // 8) % 4): the order of the
    # GEMM's XOR-swizzled 32-deep LDS stage
    for p in range(64):
        r, ch = p // 4, (p % 4) ^ ((p // 8) % 4)
        assert int(idx[r, 8 * ch]) == 8 * p
