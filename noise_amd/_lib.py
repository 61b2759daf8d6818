"""ctypes binding of libnoise_hip.so (the C ABI of include/noise_hip.h).

The library is loaded after `import torch` so that it binds to torch's HIP runtime. There is no CPU
fallback: a missing or stale library raises.
"""
import ctypes
from pathlib import Path

import torch  # noqa: F401  (must precede the HIP library load: one libamdhip64 per process)

LIB_PATH = Path(__file__).resolve().parent / 'libnoise_hip.so'

I, L, F, S, P = ctypes.c_int, ctypes.c_long, ctypes.c_float, ctypes.c_size_t, ctypes.c_void_p
SP = ctypes.POINTER(ctypes.c_size_t)

ERRORS = {-1: 'NOISE_EINVAL (rejected argument)', -2: 'NOISE_ENOSPC (workspace too small)',
          -3: 'NOISE_ENOTSUP (shape outside the kernel tiling)'}

FITNESS_ZSCORE, FITNESS_RANK = 0, 1
QK_BF16, QK_F16, QK_F16_Q_LOG2, QK_BF16_V_BF16 = 0, 1, 2, 3
LAYOUT_ROWS, LAYOUT_TILE16, LAYOUT_WTILE = 0, 1, 2
CE_MEMBER_MEAN, CE_NONE, CE_SUM, CE_MEAN = 0, 1, 2, 3
HEAD_BF16, HEAD_FP32_SPLIT, HEAD_FP32 = 0, 1, 2  # noise_head_ce's weight formats (NOISE_HEAD_*)

# name -> argtypes in declaration order; every entry point returns int. Pointers (device buffers,
# the stream) are c_void_p.
SIGNATURES = {
    'noise_version': [],
    'noise_lowrank_linear_workspace_size': [I, I, SP],
    'noise_lowrank_linear': [P, L, L, P, I, I, P, P, P, I, I, I, P, P, I, P, S, P],
    'noise_lowrank_mlp_workspace_size': [I, I, I, I, SP],
    'noise_lowrank_mlp': [P, L, L, P, P, I, I, P, P, P, P, P, I, I, I, P, P, I, P, S, P],
    'noise_cast_bf16': [P, P, L, I, P],
    'noise_embed_norm': [P, L, P, P, P, P, I, I, I, P, P],
    'noise_block_entry': [P, P, P, P, P, P, P, P, P, P, P, P, L, P, P, P, P, P, I, I, I, P, I, P, P],
    'noise_qkv': [P, P, P, P, P, P, P, I, I, I, P, P, P, P, L, P, P, P, L, P, P],
    'noise_attention_workspace_size': [I, I, SP],
    'noise_attention': [P, I, I, I, I, I, P, I, P, P, P, P, S, P],
    'noise_attention_noalloc': [P, I, I, I, I, I, P, I, P, P, P, P],
    'noise_lowrank_resid': [P, P, I, I, P, P, I, L, L, P, I, I, I, P, P],
    'noise_norm_dot': [P, P, P, P, P, I, I, I, P, I, P],
    'noise_ac_stream': [P, P, L, P, L, P, P, P, P, P, P, P, P, I, I, P],
    'noise_ac_qkv': [P, P, P, P, P, L, P, L, I, I, P],
    'noise_weight_tiles': [P, I, I, P, P],
    'noise_dense_bf16': [P, I, I, I, P, I, I, I, P, P],
    'noise_mlp_fc_parts': [I],
    'noise_mlp_fc': [P, P, I, I, P, P, P, P, I, I, I, P, I, P, P],
    'noise_head_ce_workspace_size': [I, I, I, I, SP],
    'noise_head_ce': [P, I, P, P, I, I, P, P, P, P, L, I, I, I, I, P, P, P, S, P, I, P],
    'noise_fitness': [P, I, I, I, P, P, P],
    'noise_outer_update': [P, L, P, L, P, I, I, I, F, P, P],
    'noise_outer_update_batch': [P, I, P, I, F, P],
    'noise_gather_rows': [P, L, P, I, P, I, I, P],
    'noise_readout_probes': [P, L, P, L, P, I, P, P, P, P, L, P, I, I, I, I, I, P, P],
    'noise_moved_heads': [P, P, F, P, P, I, I, I, I, P, L, P],
    'noise_head_scores': [P, L, P, P, I, I, I, I, P, P],
    'noise_code_estimate': [P, P, I, I, I, I, P, P],
    'noise_key_filter': [P, P, I, I, I, I, P, P],
    'noise_adam': [P, P, P, P, L, F, F, F, F, F, P],
    'noise_adam_batch': [P, I, F, F, F, P],
    'noise_hbm_stream': [P, I, P, I, L, P],
}



class OuterMat(ctypes.Structure):
    """noise_outer_mat_t of include/noise_hip.h (one matrix of a batched EGGROLL update)."""
    _fields_ = [('a', P), ('a_ld', L), ('b', P), ('b_ld', L), ('out', I), ('in_', I), ('grad', P)]


def outer_mats(items):
    """(a ptr or 0, a_ld, b ptr, b_ld, out, in, grad ptr) tuples -> (pointer to a host array, count)."""
    arr = (OuterMat * len(items))(*[OuterMat(*it) for it in items])
    return ctypes.cast(arr, P), len(items), arr


class GatherParam(ctypes.Structure):
    """noise_gather_param_t of include/noise_hip.h."""
    _fields_ = [('offsets', P), ('a', P), ('b', P), ('out', ctypes.c_int), ('in', ctypes.c_int)]


def gather_params(items):
    """A host array of noise_gather_param_t from (offsets, a, b, out, in) tuples of device pointers: returns
    (pointer, count, array) -- keep the array alive until the call is enqueued."""
    arr = (GatherParam * len(items))(*[GatherParam(*it) for it in items])
    return ctypes.cast(arr, P), len(items), arr


class AdamTensor(ctypes.Structure):
    """noise_adam_tensor_t of include/noise_hip.h."""
    _fields_ = [('param', P), ('grad', P), ('exp_avg', P), ('exp_avg_sq', P), ('n', L), ('step_size', F),
                ('bc2_sqrt', F)]


def adam_tensors(items):
    """A host array of noise_adam_tensor_t from (param, grad, exp_avg, exp_avg_sq, n, step_size, bc2_sqrt) tuples:
    returns (pointer, count, array) -- keep the array alive until the call is enqueued."""
    arr = (AdamTensor * len(items))(*[AdamTensor(*it) for it in items])
    return ctypes.cast(arr, P), len(items), arr


class Embed(ctypes.Structure):
    """noise_embed_t of include/noise_hip.h (the table a block entry recomputes x0 from)."""
    _fields_ = [('w', P), ('vocab', L), ('a', P), ('b', P), ('idx', P), ('idx_mstride', L)]


def embed(w, vocab, a, b, idx, idx_mstride=0):
    """A noise_embed_t (keep the returned object alive until the call is enqueued) and its pointer."""
    e = Embed(w, vocab, a, b, idx, idx_mstride)
    return e, ctypes.cast(ctypes.pointer(e), P)


class Pending(ctypes.Structure):
    """noise_pending_t: a c_proj output not yet added to the residual stream (see include/noise_hip.h)."""
    _fields_ = [('y', ctypes.c_void_p), ('u', ctypes.c_void_p), ('u_parts', ctypes.c_int),
                ('u_row_stride', ctypes.c_long), ('u_part_stride', ctypes.c_long), ('a', ctypes.c_void_p)]


def pending(*items):
    """ctypes array of Pending from (y_ptr, u_ptr, u_parts, u_row_stride, u_part_stride, a_ptr) tuples, and
    its length; (None, 0) when empty. Keep the returned array alive until the call is enqueued."""
    if not items:
        return None, 0
    arr = (Pending * len(items))(*[Pending(*it) for it in items])
    return ctypes.cast(arr, ctypes.c_void_p), len(items)


# Entry points whose int result is a value, not a status.
VALUE_RESULT = {'noise_version', 'noise_mlp_fc_parts'}

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
        fn.restype = I
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


def value(name, *args):
    return getattr(load(), name)(*args)


def size_query(name, *args):
    out = S(0)
    call(name, *args, ctypes.byref(out))
    return out.value
