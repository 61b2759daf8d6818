// Credit scoring around the attention reruns (train/val/run.py:186-211, used by `query_key_errors`,
// :594-634): the moved heads of a batch of draws, each draw's output change scored against a target, and the
// score-weighted sum of the draws.
//
// moved_heads: row (draw j, batch b, position t, head h) of 64 dims, x = raw[b, t, h] + sigma a[j, b, t, h];
//   rotary (utils/model.py:55-58: halves d and d + 32, cos / sin of position t) then RMSNorm over the 64 dims
//   (eps = finfo(float32).eps), in fp32, rounded to bf16. Lane l of a 32-lane half-wave owns the rotary pair
//   (l, l + 32), so the rotation needs no exchange and the norm is one 32-lane sum.
// head_scores: score[b, h, t, j] = sum_d (out[j, b, t, h, d] - baseline[b, t, h, d]) hub[b, t, h, d].
// code_estimate: est[b, t, h, d] = sum_j credited[b, h, t, j] a[j, b, t, h, d], draws in order.
// key_filter: the key scores of `query_key_errors` (:622-623), (K.to(bf16) @ score.to(bf16)).float(): per (b, h), the
//   matched filter K [T, T] times the query scores [T, n] on bf16 MFMA with fp32 accumulation, rounded to bf16 as
//   the reference's bf16 matmul returns it.
#include "common.h"
#include "credit.h"

namespace {

constexpr int HD = 64;
constexpr float EPS = 1.1920928955078125e-07f;

// sum over the 32 lanes of each half-wave
__device__ __forceinline__ float half_sum(float v) {
  v = group_sum<16>(v);
  const f32pair r = rowpair16(v);  // rows 0 + 1 (lanes 0-31) and rows 2 + 3 (lanes 32-63)
  return r.lo + r.hi;
}

__global__ void __launch_bounds__(256) moved_heads_kernel(const MovedHeadsArgs g) {
  const int lane = threadIdx.x & 31;
  const long r = (long)blockIdx.x * 8 + (threadIdx.x >> 5);  // (j, b, t, h) row
  if (r >= g.rows) return;
  const int h = (int)(r % g.H);
  const long jbt = r / g.H, t = jbt % g.T, bt = jbt % (g.B * (long)g.T);
  const float* raw = g.raw + (bt * g.H + h) * HD;
  const __bf16* a = g.a + r * HD;
  const float x1 = raw[lane] + g.sigma * (float)a[lane];
  const float x2 = raw[lane + 32] + g.sigma * (float)a[lane + 32];
  const float c = g.cos[t * 32 + lane], s = g.sin[t * 32 + lane];
  const float y1 = x1 * c + x2 * s, y2 = -x1 * s + x2 * c;
  const float inv = rsqrtf(half_sum(y1 * y1 + y2 * y2) * (1.f / HD) + EPS);
  __bf16* o = g.out + jbt * g.ldo + h * HD;
  o[lane] = to_bf16(y1 * inv);
  o[lane + 32] = to_bf16(y2 * inv);
}

__global__ void __launch_bounds__(256) head_scores_kernel(const HeadScoresArgs g) {
  const int lane = threadIdx.x & 31;
  const long r = (long)blockIdx.x * 8 + (threadIdx.x >> 5);  // (j, b, t, h) row
  if (r >= g.rows) return;
  const int h = (int)(r % g.H);
  const long jbt = r / g.H, j = jbt / (g.B * (long)g.T), bt = jbt % (g.B * (long)g.T);
  const long b = bt / g.T, t = bt % g.T;
  const __bf16* out = g.out + jbt * g.ld_out + h * HD;
  const long base_off = (bt * g.H + h) * HD;
  float d = 0.f;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int e = lane + 32 * q;
    d += ((float)out[e] - g.baseline[base_off + e]) * g.hub[base_off + e];
  }
  d = half_sum(d);
  if (lane == 0) g.score[((b * g.H + h) * g.T + t) * g.n + j] = d;
}

__global__ void __launch_bounds__(256) code_estimate_kernel(const CodeEstimateArgs g) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;  // (b, t, h, d)
  if (i >= g.elems) return;
  const int d = (int)(i % HD);
  const long bth = i / HD, h = bth % g.H, bt = bth / g.H, b = bt / g.T, t = bt % g.T;
  const float* cr = g.credited + ((b * g.H + h) * g.T + t) * g.n;
  const long stride = g.elems;  // one draw of a
  float acc = 0.f;
  for (int j = 0; j < g.n; ++j) acc += cr[j] * (float)g.a[j * stride + bth * HD + d];
  g.est[i] = acc;
}

}  // namespace

namespace {
// One workgroup = 64 rows t x 64 draws j of one (b, h); 4 waves of 16 rows. The contraction over s walks 32 at a
// time through LDS: the K tile [64 t][32 s] as loaded (16-byte rows of 8), the scores [32 s][64 j] rounded to bf16
// and stored transposed [64 j][32 s] so both MFMA operands are 16-byte reads along s. Lane l of wave w ends with
// rows 16 w + 4 (l / 16) + e, column l % 16 of each 16-column block.
constexpr int KF_LD = 32 + 8;  // LDS row pitch (bf16): 80 bytes, so 16 rows of a fragment read hit distinct banks
__global__ void __launch_bounds__(256) key_filter_kernel(const KeyFilterArgs g) {
  __shared__ __attribute__((aligned(16))) bf16 sa[64 * KF_LD];
  __shared__ __attribute__((aligned(16))) bf16 sb[64 * KF_LD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int t0 = blockIdx.x * 64, j0 = blockIdx.y * 64, bh = blockIdx.z;
  const bf16* filt = g.filt + (long)bh * g.T * g.T;
  const float* score = g.score + (long)bh * g.T * g.n;
  f32x4 acc[4] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f},
                  f32x4{0.f, 0.f, 0.f, 0.f}};
  // loaders: K row tid / 4, s chunk tid % 4 (8 values); scores row s = tid / 8, columns 8 (tid % 8) .. + 7
  const int ar = tid >> 2, ac = (tid & 3) * 8, bs = tid >> 3, bc = (tid & 7) * 8;
  for (int s0 = 0; s0 < g.T; s0 += 32) {
    const bf16x8 kv = *reinterpret_cast<const bf16x8*>(filt + (long)(t0 + ar) * g.T + s0 + ac);
    float sv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int j = j0 + bc + e;
      sv[e] = j < g.n ? score[(long)(s0 + bs) * g.n + j] : 0.f;
    }
    __syncthreads();  // the previous chunk's fragments have been read
    *reinterpret_cast<bf16x8*>(&sa[ar * KF_LD + ac]) = kv;
#pragma unroll
    for (int e = 0; e < 8; ++e) sb[(bc + e) * KF_LD + bs] = to_bf16(sv[e]);
    __syncthreads();
    const bf16x8 af = *reinterpret_cast<const bf16x8*>(&sa[(16 * wave + (lane & 15)) * KF_LD + 8 * (lane >> 4)]);
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      const bf16x8 bfr = *reinterpret_cast<const bf16x8*>(&sb[(16 * cb + (lane & 15)) * KF_LD + 8 * (lane >> 4)]);
      acc[cb] = mfma16x16x32(af, bfr, acc[cb]);
    }
  }
#pragma unroll
  for (int cb = 0; cb < 4; ++cb) {
    const int j = j0 + 16 * cb + (lane & 15);
    if (j >= g.n) continue;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = t0 + 16 * wave + 4 * (lane >> 4) + e;
      g.out[((long)bh * g.T + t) * g.n + j] = bf16r(acc[cb][e]);
    }
  }
}
}  // namespace

int key_filter_launch(const KeyFilterArgs& g, hipStream_t s) {
  if (!g.filt || !g.score || !g.out || g.BH <= 0 || g.T <= 0 || g.n <= 0 || g.T % 64 ||
      ((uintptr_t)g.filt & 15))
    return NOISE_EINVAL;
  if (g.BH > 65535 || (g.n + 63) / 64 > 65535) return NOISE_ENOTSUP;
  hipLaunchKernelGGL(key_filter_kernel, dim3((unsigned)(g.T / 64), (unsigned)((g.n + 63) / 64), (unsigned)g.BH),
                     dim3(256), 0, s, g);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}

int moved_heads_launch(const MovedHeadsArgs& g, hipStream_t s) {
  if (!g.raw || !g.a || !g.cos || !g.sin || !g.out || g.n <= 0 || g.B <= 0 || g.T <= 0 || g.H <= 0 ||
      g.ldo < (long)g.H * HD)
    return NOISE_EINVAL;
  const long grid = (g.rows + 7) / 8;
  if (grid > 0x7fffffffL) return NOISE_ENOTSUP;
  hipLaunchKernelGGL(moved_heads_kernel, dim3((unsigned)grid), dim3(256), 0, s, g);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}

int head_scores_launch(const HeadScoresArgs& g, hipStream_t s) {
  if (!g.out || !g.baseline || !g.hub || !g.score || g.n <= 0 || g.B <= 0 || g.T <= 0 || g.H <= 0 ||
      g.ld_out < (long)g.H * HD)
    return NOISE_EINVAL;
  const long grid = (g.rows + 7) / 8;
  if (grid > 0x7fffffffL) return NOISE_ENOTSUP;
  hipLaunchKernelGGL(head_scores_kernel, dim3((unsigned)grid), dim3(256), 0, s, g);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}

int code_estimate_launch(const CodeEstimateArgs& g, hipStream_t s) {
  if (!g.credited || !g.a || !g.est || g.n <= 0 || g.elems <= 0 || g.H <= 0 || g.T <= 0) return NOISE_EINVAL;
  const long grid = (g.elems + 255) / 256;
  if (grid > 0x7fffffffL) return NOISE_ENOTSUP;
  hipLaunchKernelGGL(code_estimate_kernel, dim3((unsigned)grid), dim3(256), 0, s, g);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}
