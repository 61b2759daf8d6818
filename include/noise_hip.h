/* C ABI of libnoise_hip.so: the MI355X (gfx950) population-perturbed forward of the Noise 37.7M GPT.
 *
 * Conventions for every entry point:
 *  - pointers are device pointers (hipMalloc / torch CUDA tensors); bf16 buffers are passed as void*;
 *  - "members" are the population rows; member p uses perturbation row dir = p >> pair_shift
 *    (pair_shift = 1 when antithetic pairs 2j, 2j+1 share a_j, b_j, as train/val/eggroll.py:140-141
 *    builds them; 0 when a, b are given per member) and sign[p] = +-sigma;
 *  - rank-1 vectors follow the reference orientation (train/val/eggroll.py:56-58): for a weight
 *    W [out, in], `a` is [dirs, out] (output side) and `b` is [dirs, in] (input side);
 *  - activations are row-major [members * T, width]; member p owns rows p*T .. p*T+T-1;
 *  - work is enqueued on `stream` (a hipStream_t); nothing is synchronised, nothing allocated: any
 *    scratch comes from the caller's workspace, sized by the matching *_workspace_size query;
 *  - return 0 on success, a negative NOISE_E* code for a rejected argument, or a positive hipError_t.
 */
#ifndef NOISE_HIP_H
#define NOISE_HIP_H
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NOISE_OK 0
#define NOISE_EINVAL (-1)
#define NOISE_ENOSPC (-2)
#define NOISE_ENOTSUP (-3)

typedef void* noise_stream_t; /* hipStream_t */

/* Library version (major * 10000 + minor * 100 + patch). */
int noise_version(void);

/* y = x W^T + s_p (x . b_p) a_p^T per member, autocast rounding points: bf16 GEMM output, the GEMV
 * x.b rounded to bf16, the correction added in fp32.
 * Replaces `lowrank` (train/val/eggroll.py:56-58).
 *   x       bf16 [members, T, in], row r of member p at x + p*x_mstride + t*x_ld (x_mstride 0: one
 *           activation shared by every member)
 *   w       bf16 [out, in]
 *   y_f32   fp32 [members*T, out] (nullable); accumulate != 0 adds into it (residual update)
 *   y_bf16  bf16 [members*T, out] (nullable)
 * Workspace: noise_lowrank_linear_workspace_size(). */
int noise_lowrank_linear_workspace_size(int members, int T, size_t* bytes);
int noise_lowrank_linear(const void* x, long x_ld, long x_mstride, const void* w, int in, int out,
                         const float* a, const float* b, const float* sign, int members, int T, int pair_shift,
                         float* y_f32, void* y_bf16, int accumulate, void* workspace, size_t workspace_bytes,
                         noise_stream_t stream);

/* The relu^2 MLP sublayer with rank-1 perturbations on both matrices, per member:
 *   h = relu(lowrank(x, w_fc, a_fc, b_fc))^2 ;  y = lowrank(h, w_proj, a_proj, b_proj)
 * Replaces `F.relu(linear('mlp.c_fc.weight', .)).square()` -> `linear('mlp.c_proj.weight', .)`
 * (train/val/eggroll.py:93; model form utils/model.py:106-107).
 *   x       bf16 [members, T, d] (x_mstride as above)
 *   w_fc    bf16 [f, d];  a_fc [dirs, f], b_fc [dirs, d]
 *   w_proj  bf16 [d, f];  a_proj [dirs, d], b_proj [dirs, f]
 *   y_f32 / y_bf16 / accumulate as in noise_lowrank_linear; d % 128 == 0, f % 128 == 0.
 * Workspace: noise_lowrank_mlp_workspace_size(). */
int noise_lowrank_mlp_workspace_size(int members, int T, int d, int f, size_t* bytes);
int noise_lowrank_mlp(const void* x, long x_ld, long x_mstride, const void* w_fc, const void* w_proj, int d, int f,
                      const float* a_fc, const float* b_fc, const float* a_proj, const float* b_proj,
                      const float* sign, int members, int T, int pair_shift, float* y_f32, void* y_bf16,
                      int accumulate, void* workspace, size_t workspace_bytes, noise_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* NOISE_HIP_H */
