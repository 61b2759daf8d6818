// Readout-probe forward differences: the soft-capped cross-entropy of the head on the stream moved along each
// direction, minus the clean one, over the step (`cycle_derivatives` / `row_derivatives`,
// train/val/run.py:154-185; train/speedrun/run.py:90-103).
//
// Token i (clean stream x, |x|^2 = sq_i, logits base_i = W x, target t_i, step s_i) and direction j
// (W D_j = C_j, x . D_j = dots_ij, |D_j|^2 = dir_sq_j):
//   inv_ij = rsqrt((sq_i + 2 s_i dots_ij + s_i^2 dir_sq_j) / width + eps)     (the moved stream's exact RMS)
//   L_ij   = log sum_v exp(15 tanh((base_iv + s_i C_jv) inv_ij / 15)) - 15 tanh((base_it + s_i C_jt) inv_ij / 15)
//   out_ij = (L_ij - L_i0) / s_i  (0 for a target of -1; L_i0 at s = 0 with the clean RMS).
// The reference materialises z[n, P, V]; here one wave owns a token: its V logits stay in registers (V / 64
// per lane) while the C rows of its directions stream through (1 KiB coalesced loads), and each (token,
// direction) sum of V exponentials ends in one wave reduction. The cap and exp run in log2 units with the
// hardware exp2 and reciprocal, as the head's cross-entropy epilogue does.
#include "common.h"
#include "probes.h"

namespace {

constexpr int MAXC = 16;  // float4 chunks per lane: V <= 64 lanes x 4 x 16 = 4096
constexpr float L2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;
constexpr float EPS = 1.1920928955078125e-07f;  // finfo(float32).eps (train/val/run.py:58)

// 15 tanh(z / 15) in log2 units: z' log2(e) = 15 log2(e) - 30 log2(e) / (exp(2 z / 15) + 1)
__device__ __forceinline__ float cap_log2(float z) {
  const float ez = __builtin_amdgcn_exp2f(z * (2.f * L2E / 15.f));
  return fmaf(__builtin_amdgcn_rcpf(ez + 1.f), -30.f * L2E, 15.f * L2E);
}

__global__ void __launch_bounds__(256) probe_kernel(const ProbeArgs g) {
  const int lane = threadIdx.x & 63;
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= g.n) return;
  const int nc = g.V >> 8;
  const long yi = g.y[i];
  const bool valid = yi >= 0;
  const long t = valid ? yi : 0;
  const float s = g.steps[i], sq = g.sq[i];
  const float* bi = g.base + (long)i * g.base_ld;
  float4 b[MAXC];
#pragma unroll
  for (int c = 0; c < MAXC; ++c)
    if (c < nc) b[c] = *reinterpret_cast<const float4*>(bi + 256 * c + 4 * lane);
  const float base_t = t < g.V ? bi[t] : __builtin_nanf("");
  // clean loss
  const float inv0 = rsqrtf(sq / (float)g.width + EPS);
  float se = 0.f;
#pragma unroll
  for (int c = 0; c < MAXC; ++c)
    if (c < nc) {
      se += __builtin_amdgcn_exp2f(cap_log2(b[c].x * inv0)) + __builtin_amdgcn_exp2f(cap_log2(b[c].y * inv0));
      se += __builtin_amdgcn_exp2f(cap_log2(b[c].z * inv0)) + __builtin_amdgcn_exp2f(cap_log2(b[c].w * inv0));
    }
  se = group_sum<64>(se);
  const float clean = logf(se) - cap_log2(base_t * inv0) * LN2;
  for (int k = 0; k < g.K; ++k) {
    const long j = g.rows ? g.rows[(long)i * g.K + k] : k;
    const bool jok = j >= 0 && j < g.P;
    const float dj = g.dots[(long)i * g.dots_ld + k];
    const float ds = g.dir_sq_tok ? g.dir_sq[(long)i * g.K + k] : (jok ? g.dir_sq[j] : 0.f);
    const float inv = rsqrtf((sq + 2.f * s * dj + s * s * ds) / (float)g.width + EPS);
    const float* cj = g.C + (jok ? j : 0) * g.c_ld;
    float sm = 0.f;
#pragma unroll
    for (int c = 0; c < MAXC; ++c)
      if (c < nc) {
        const float4 cv = *reinterpret_cast<const float4*>(cj + 256 * c + 4 * lane);
        sm += __builtin_amdgcn_exp2f(cap_log2(fmaf(s, cv.x, b[c].x) * inv)) +
              __builtin_amdgcn_exp2f(cap_log2(fmaf(s, cv.y, b[c].y) * inv));
        sm += __builtin_amdgcn_exp2f(cap_log2(fmaf(s, cv.z, b[c].z) * inv)) +
              __builtin_amdgcn_exp2f(cap_log2(fmaf(s, cv.w, b[c].w) * inv));
      }
    sm = group_sum<64>(sm);
    const float moved = logf(sm) - cap_log2(fmaf(s, t < g.V ? cj[t] : 0.f, base_t) * inv) * LN2;
    if (lane == 0) g.out[(long)i * g.K + k] = jok ? (moved - clean) / s * (valid ? 1.f : 0.f) : __builtin_nanf("");
  }
}

}  // namespace

int probe_launch(const ProbeArgs& g, hipStream_t stream) {
  if (!g.base || !g.C || !g.y || !g.steps || !g.sq || !g.dots || !g.dir_sq || !g.out || g.n <= 0 || g.K <= 0 ||
      g.P <= 0 || g.width <= 0 || g.V <= 0 || g.V % 256 || g.V > 256 * MAXC || g.base_ld < g.V || g.c_ld < g.V ||
      g.base_ld % 4 || g.c_ld % 4 || g.dots_ld < g.K || (!g.rows && g.K != g.P) ||
      (((uintptr_t)g.base | (uintptr_t)g.C) & 15))
    return NOISE_EINVAL;
  const long grid = ((long)g.n + 3) / 4;
  if (grid > 0x7fffffffL) return NOISE_ENOTSUP;
  hipLaunchKernelGGL(probe_kernel, dim3((unsigned)grid), dim3(256), 0, stream, g);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}
