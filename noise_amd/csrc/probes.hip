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
// current one is summed, into the other of two register sets (2 waves per SIMD instead of 5: 3.21 -> 1.43 ms on 1024
// tokens x 512 directions x 4096 vocabulary, the row's load latency, not the arithmetic, had set the time). The
// per-token scalars come through the scalar data cache, and nothing the sum needs is loaded after that row, so the
// sum does not wait for it (vector loads complete in issue order): 1.43 -> 0.92 ms; with each direction's wait
// stated (the previous output store may stay in flight) and the last direction outside the loop: 0.84 ms. The cap and exp
// run in log2 units with the hardware exp2 and reciprocal, as the head's cross-entropy epilogue does; the moved
// RMS's reciprocal and the cap's 2 log2(e) / 15 are one multiplier.
#include <type_traits>

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

// ROWS: the directions' rows come from g.rows (per token); otherwise direction k is row k.
// A wave-uniform load through the scalar data cache (s_load), for inputs the kernel never writes: it waits on its own
// counter, not behind the vector loads of the C rows.
template <typename T>
__device__ __forceinline__ T ld_uniform(const T* p) {
  return *(const __attribute__((address_space(4))) T*)p;
}

// NCT: the vocabulary's 256-entry chunks when fixed at compile time (16: the model's 4096), 0 when read from g.V;
// a fixed count leaves the loop without branches, so the next row's loads stay where they are issued.
template <bool ROWS, int NCT>
__global__ void __launch_bounds__(256) probe_kernel(const ProbeArgs g) {
  const int lane = threadIdx.x & 63;
  const int i = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));  // this wave's token
  if (i >= g.n) return;
  const int nc = NCT ? NCT : g.V >> 8;
  const long yi = ld_uniform(g.y + i);
  const bool valid = yi >= 0;
  const long t = valid ? yi : 0;
  const float s = ld_uniform(g.steps + i), sq = ld_uniform(g.sq + i);
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
  // Everything direction k + 1 needs (its C row, into the other of two register sets; its dot, |D|^2 and target C
  // entry; the row index of direction k + 2) is loaded before direction k is summed, so that those loads land during
  // the sum and the sum waits for none of them: vector memory operations complete in issue order, so a load the sum
  // needed, issued after them, would wait for all of them.
  // Every load below is unconditional, from an address kept in bounds, and no value is computed from a loaded one
  // before it is used: hipcc places such a computation next to the load, where its wait would also wait for the loads
  // issued since. A row index is checked where the next direction's loads need it; an invalid row or target leaves
  // NaN in the output whatever |D|^2 and the target's C entry hold, so those are used as loaded.
  auto row_raw = [&](int k) -> long {
    if constexpr (ROWS) return ld_uniform(g.rows + (long)i * g.K + k);
    else return k;
  };
  auto row_ok = [&](long j) -> long { return j >= 0 && j < g.P ? j : -1; };
  auto load_row = [&](long j, float4 (&dst)[MAXC]) {
    const float* cr = g.C + (j >= 0 ? j : 0) * g.c_ld + 4 * lane;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) dst[c] = *reinterpret_cast<const float4*>(cr + 256 * min(c, nc - 1));
  };
  const long tc = t < g.V ? t : 0;
  float dj, ds, ct;  // the scalars of the direction summed next
  auto load_scalars = [&](int k, long j) {
    const long jc = j >= 0 ? j : 0;
    dj = ld_uniform(g.dots + (long)i * g.dots_ld + k);
    ds = ld_uniform(g.dir_sq + (g.dir_sq_tok ? (long)i * g.K + k : jc));
    ct = ld_uniform(g.C + jc * g.c_ld + tc);
  };
  long jn = row_ok(row_raw(0)), jn2 = g.K > 1 ? row_raw(1) : -1;  // the rows of the next two directions (jn2 raw)
  float4 ca[MAXC], cb[MAXC];
  load_row(jn, ca);
  load_scalars(0, jn);
  // Direction k (row in cv): with PF, first the loads of direction k + 1 (its row into cn), then the wait for
  // direction k's own loads, stated here: VW vector operations may stay in flight, the 16 of that row and, after the
  // first direction, the previous direction's output store (vector memory operations complete in issue order). With
  // the waits stated and no direction without prefetch inside the loop, the compiler keeps them instead of the
  // stricter ones its tracking would place across the loop's joins.
  auto direction = [&](int k, const float4 (&cv)[MAXC], float4 (&cn)[MAXC], auto pf, auto vw) {
    constexpr bool PF = decltype(pf)::value;
    constexpr int VW = decltype(vw)::value;
    const long j = jn;
    const bool jok = j >= 0;
    const float djk = dj, dsk = ds, ctk = ct;
    if constexpr (PF) {
      jn = row_ok(jn2);
      load_row(jn, cn);
      load_scalars(k + 1, jn);
      if (k + 2 < g.K) jn2 = row_raw(k + 2);
    }
    __builtin_amdgcn_s_waitcnt((VW & 15) | (7 << 4) | (15 << 8) | ((VW >> 4) << 14));
    const float inv = rsqrtf((sq + 2.f * s * djk + s * s * dsk) / (float)g.width + EPS), mv = inv * K2;
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
    const float moved = logf(sm) - cap_log2(fmaf(s, ctk, base_t) * inv) * LN2;
    if (lane == 0) g.out[(long)i * g.K + k] = jok ? (moved - clean) / s * (valid ? 1.f : 0.f) : __builtin_nanf("");
  };
  using pf_t = std::true_type;
  using last_t = std::false_type;
  using first_w = std::integral_constant<int, MAXC>;   // nothing but the prefetched row after direction 0's
  using next_w = std::integral_constant<int, MAXC + 1>; // and the previous direction's output store
  using none_w = std::integral_constant<int, 0>;
  if (g.K == 1) {
    direction(0, ca, cb, last_t{}, none_w{});
    return;
  }
  direction(0, ca, cb, pf_t{}, first_w{});  // direction k's row is in cb at the top of each trip
  int k = 1;
  for (; k + 2 < g.K; k += 2) {
    direction(k, cb, ca, pf_t{}, next_w{});
    direction(k + 1, ca, cb, pf_t{}, next_w{});
  }
  if (k + 1 < g.K) {
    direction(k, cb, ca, pf_t{}, next_w{});
    direction(k + 1, ca, cb, last_t{}, none_w{});
  } else {
    direction(k, cb, ca, last_t{}, none_w{});
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
  const bool full = g.V == 256 * MAXC;
  if (g.rows && full)
    hipLaunchKernelGGL((probe_kernel<true, MAXC>), dim3((unsigned)grid), dim3(256), 0, stream, g);
  else if (g.rows)
    hipLaunchKernelGGL((probe_kernel<true, 0>), dim3((unsigned)grid), dim3(256), 0, stream, g);
  else if (full)
    hipLaunchKernelGGL((probe_kernel<false, MAXC>), dim3((unsigned)grid), dim3(256), 0, stream, g);
  else
    hipLaunchKernelGGL((probe_kernel<false, 0>), dim3((unsigned)grid), dim3(256), 0, stream, g);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}
