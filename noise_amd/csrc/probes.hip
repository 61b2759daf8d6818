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
// direction) sum of V exponentials ends in one wave reduction. The C row of the next direction is loaded while the
// current one is summed (two rows in registers: 2 waves per SIMD instead of 5, and 3.21 -> 1.43 ms on 1024 tokens x
// 512 directions x 4096 vocabulary: the row's load latency, not the arithmetic, had set the time). The cap and exp
// run in log2 units with the hardware exp2 and reciprocal, as the head's cross-entropy epilogue does; the moved
// RMS's reciprocal and the cap's 2 log2(e) / 15 are one multiplier.
#include "common.h"
#include "probes.h"

namespace {

constexpr int MAXC = 16;  // float4 chunks per lane: V <= 64 lanes x 4 x 16 = 4096
constexpr float L2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;
constexpr float EPS = 1.1920928955078125e-07f;  // finfo(float32).eps (train/val/run.py:58)

constexpr float K2 = 2.f * L2E / 15.f;
// 15 tanh(z / 15) in log2 units from y = z 2 log2(e) / 15: z' log2(e) = 15 log2(e) - 30 log2(e) / (2^y + 1)
__device__ __forceinline__ float cap_log2_y(float y) {
  return fmaf(__builtin_amdgcn_rcpf(__builtin_amdgcn_exp2f(y) + 1.f), -30.f * L2E, 15.f * L2E);
}
__device__ __forceinline__ float cap_log2(float z) { return cap_log2_y(z * K2); }

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
  const float inv0 = rsqrtf(sq / (float)g.width + EPS), m0 = inv0 * K2;
  float se = 0.f;
#pragma unroll
  for (int c = 0; c < MAXC; ++c)
    if (c < nc) {
      se += __builtin_amdgcn_exp2f(cap_log2_y(b[c].x * m0)) + __builtin_amdgcn_exp2f(cap_log2_y(b[c].y * m0));
      se += __builtin_amdgcn_exp2f(cap_log2_y(b[c].z * m0)) + __builtin_amdgcn_exp2f(cap_log2_y(b[c].w * m0));
    }
  se = group_sum<64>(se);
  const float clean = logf(se) - cap_log2(base_t * inv0) * LN2;
  // the C row of direction k + 1 is loaded while direction k is summed
  auto row_of = [&](int k) -> long {
    const long j = g.rows ? g.rows[(long)i * g.K + k] : k;
    return j >= 0 && j < g.P ? j : -1;
  };
  float4 cn[MAXC];
  long jn = row_of(0);
#pragma unroll
  for (int c = 0; c < MAXC; ++c)
    if (c < nc) cn[c] = *reinterpret_cast<const float4*>(g.C + (jn >= 0 ? jn : 0) * g.c_ld + 256 * c + 4 * lane);
  for (int k = 0; k < g.K; ++k) {
    const long j = jn;
    const bool jok = j >= 0;
    float4 cv[MAXC];
#pragma unroll
    for (int c = 0; c < MAXC; ++c) cv[c] = cn[c];
    if (k + 1 < g.K) {
      jn = row_of(k + 1);
#pragma unroll
      for (int c = 0; c < MAXC; ++c)
        if (c < nc) cn[c] = *reinterpret_cast<const float4*>(g.C + (jn >= 0 ? jn : 0) * g.c_ld + 256 * c + 4 * lane);
    }
    const float dj = g.dots[(long)i * g.dots_ld + k];
    const float ds = g.dir_sq_tok ? g.dir_sq[(long)i * g.K + k] : (jok ? g.dir_sq[j] : 0.f);
    const float inv = rsqrtf((sq + 2.f * s * dj + s * s * ds) / (float)g.width + EPS), mv = inv * K2;
    const float* cj = g.C + (jok ? j : 0) * g.c_ld;
    float sm = 0.f;
#pragma unroll
    for (int c = 0; c < MAXC; ++c)
      if (c < nc) {
        sm += __builtin_amdgcn_exp2f(cap_log2_y(fmaf(s, cv[c].x, b[c].x) * mv)) +
              __builtin_amdgcn_exp2f(cap_log2_y(fmaf(s, cv[c].y, b[c].y) * mv));
        sm += __builtin_amdgcn_exp2f(cap_log2_y(fmaf(s, cv[c].z, b[c].z) * mv)) +
              __builtin_amdgcn_exp2f(cap_log2_y(fmaf(s, cv[c].w, b[c].w) * mv));
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
