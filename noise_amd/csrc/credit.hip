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
// The three take 16- and 8-byte vector accesses when the pointers and strides allow (8 lanes per 64-dim row; 4 dims
// per thread): at 64 draws x 2048 tokens x 8 heads, moved heads 2.5 -> 6.6 TB/s, head scores 1.2 -> 5.5 TB/s, code
// estimate 3.2 -> 6.8 TB/s of their algorithmic bytes. Otherwise the scalar kernels (32 lanes per row, one
// element per thread) run; the vector estimate is bit for bit the scalar one, the other two sum in another order.
// key_filter: the key scores of `query_key_errors` (:622-623), (K.to(bf16) @ score.to(bf16)).float(): per (b, h), the
//   matched filter K [T, T] times the query scores [T, n] on bf16 MFMA with fp32 accumulation, rounded to bf16 as
//   the reference's bf16 matmul returns it. 64-deep chunks with the next chunk prefetched into registers, and
//   32-draw blocks when 64-draw ones would leave fewer than two workgroups per CU: at 64 draws x 2048 tokens x 8
//   heads, 110 -> 45 -> 33 us (2.3 TB/s of its algorithmic bytes), bit for bit the 32-deep unprefetched loop (the same
//   products in the same order).
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

typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
// The same rows with 8 lanes per row (32 rows per workgroup): lane q owns the rotary pairs (d, d + 32) for
// d = 4 q .. 4 q + 3, so every access is a 16-byte (fp32) or 8-byte (bf16) vector and the norm is an 8-lane sum.
// Taken when every pointer and the output stride allow those accesses.
__global__ void __launch_bounds__(256) moved_heads_vec_kernel(const MovedHeadsArgs g) {
  const int q = threadIdx.x & 7;
  const long r = (long)blockIdx.x * 32 + (threadIdx.x >> 3);  // (j, b, t, h) row
  if (r >= g.rows) return;
  const int h = (int)(r % g.H);
  const long jbt = r / g.H, t = jbt % g.T, bt = jbt % (g.B * (long)g.T);
  const float* raw = g.raw + (bt * g.H + h) * HD + 4 * q;
  const __bf16* a = g.a + r * HD + 4 * q;
  const float4 r1 = *reinterpret_cast<const float4*>(raw), r2 = *reinterpret_cast<const float4*>(raw + 32);
  const bf16x4_t a1 = *reinterpret_cast<const bf16x4_t*>(a), a2 = *reinterpret_cast<const bf16x4_t*>(a + 32);
  const float4 c4 = *reinterpret_cast<const float4*>(g.cos + t * 32 + 4 * q);
  const float4 s4 = *reinterpret_cast<const float4*>(g.sin + t * 32 + 4 * q);
  const float x1[4] = {r1.x + g.sigma * (float)a1[0], r1.y + g.sigma * (float)a1[1], r1.z + g.sigma * (float)a1[2],
                       r1.w + g.sigma * (float)a1[3]};
  const float x2[4] = {r2.x + g.sigma * (float)a2[0], r2.y + g.sigma * (float)a2[1], r2.z + g.sigma * (float)a2[2],
                       r2.w + g.sigma * (float)a2[3]};
  const float c[4] = {c4.x, c4.y, c4.z, c4.w}, s[4] = {s4.x, s4.y, s4.z, s4.w};
  float y1[4], y2[4], ss = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    y1[e] = x1[e] * c[e] + x2[e] * s[e];
    y2[e] = -x1[e] * s[e] + x2[e] * c[e];
    ss += y1[e] * y1[e] + y2[e] * y2[e];
  }
  const float inv = rsqrtf(group_sum<8>(ss) * (1.f / HD) + EPS);
  bf16x4_t o1, o2;
#pragma unroll
  for (int e = 0; e < 4; ++e) o1[e] = to_bf16(y1[e] * inv), o2[e] = to_bf16(y2[e] * inv);
  __bf16* o = g.out + jbt * g.ldo + h * HD + 4 * q;
  *reinterpret_cast<bf16x4_t*>(o) = o1;
  *reinterpret_cast<bf16x4_t*>(o + 32) = o2;
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

// 8 lanes per row, lane q owning dims 8 q .. 8 q + 7 (16-byte bf16 and fp32 vector loads); the same sums otherwise.
// Workgroup (x, y) takes the tile of 8 consecutive (b, t, h) rows bth = 8 x .. 8 x + 7 by 32 draws j = 32 y ..
// 32 y + 31. Pass it of 8-lane group g reads row (8 x + g % 8, 32 y + g / 8 + 4 it): a wave's 8 rows are consecutive
// in memory (1 KiB per load instruction), and each group keeps its (b, t, h)'s baseline and target in registers. The
// scores go through LDS so that each (b, t, h) leaves its 32 draws as one whole 128-byte line.
__global__ void __launch_bounds__(256) head_scores_vec_kernel(const HeadScoresArgs g) {
  __shared__ float sc[8][33];
  const int q = threadIdx.x & 7, grp = threadIdx.x >> 3;
  const long bth_all = g.rows / g.n, bth = (long)blockIdx.x * 8 + (grp & 7);
  const long j0 = (long)blockIdx.y * 32;
  if (bth < bth_all) {
    const int h = (int)(bth % g.H);
    const long bt = bth / g.H;
    const long base_off = (bt * g.H + h) * HD + 8 * q;
    const float4 b0 = *reinterpret_cast<const float4*>(g.baseline + base_off);
    const float4 b1 = *reinterpret_cast<const float4*>(g.baseline + base_off + 4);
    const float4 h0 = *reinterpret_cast<const float4*>(g.hub + base_off);
    const float4 h1 = *reinterpret_cast<const float4*>(g.hub + base_off + 4);
    const float bv[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
    const float hv[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
    const long jstride = g.B * (long)g.T;
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int jl = (grp >> 3) + 4 * it;
      const long j = j0 + jl;
      float d = 0.f;
      if (j < g.n) {
        const bf16x8 ov = *reinterpret_cast<const bf16x8*>(g.out + (j * jstride + bt) * g.ld_out + h * HD + 8 * q);
#pragma unroll
        for (int e = 0; e < 8; ++e) d += ((float)ov[e] - bv[e]) * hv[e];
      }
      d = group_sum<8>(d);
      if (q == 0) sc[grp & 7][jl] = d;
    }
  }
  __syncthreads();
  // thread i: draw 32 y + i % 32 of row 8 x + i / 32
  const int rl = threadIdx.x >> 5, jl = threadIdx.x & 31;
  const long row = (long)blockIdx.x * 8 + rl, j = j0 + jl;
  if (row < bth_all && j < g.n) {
    const int h = (int)(row % g.H);
    const long bt = row / g.H, b = bt / g.T, t = bt % g.T;
    g.score[((b * g.H + h) * g.T + t) * g.n + j] = sc[rl][jl];
  }
}

// Four consecutive dims per thread (8-byte bf16 loads of a); each element's sum over the draws in order, as below.
__global__ void __launch_bounds__(256) code_estimate_vec_kernel(const CodeEstimateArgs g) {
  const long i = ((long)blockIdx.x * 256 + threadIdx.x) * 4;  // (b, t, h, d .. d + 3)
  if (i >= g.elems) return;
  const long bth = i / HD, h = bth % g.H, bt = bth / g.H, b = bt / g.T, t = bt % g.T;
  const float* cr = g.credited + ((b * g.H + h) * g.T + t) * g.n;
  const long stride = g.elems;  // one draw of a
  const __bf16* a = g.a + i;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int j = 0; j < g.n; ++j) {
    const bf16x4_t av = *reinterpret_cast<const bf16x4_t*>(a + j * stride);
    const float c = cr[j];
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] += c * (float)av[e];
  }
  *reinterpret_cast<float4*>(g.est + i) = make_float4(acc[0], acc[1], acc[2], acc[3]);
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
// One workgroup = 64 rows t x 64 draws j of one (b, h); 4 waves of 16 rows. The contraction over s walks 64 at a
// time through LDS: the K tile [64 t][64 s] as loaded (16-byte rows of 8), the scores [64 s][64 j] rounded to bf16
// and stored transposed [64 j][64 s] so both MFMA operands are 16-byte reads along s. Lane l of wave w ends with
// rows 16 w + 4 (l / 16) + e, column l % 16 of each 16-column block. The next chunk's K and score values are loaded
// into registers while the current chunk's MFMAs run (the loop was load-latency bound: one workgroup per CU).
constexpr int KF_BK = 64;
constexpr int KF_LD = KF_BK + 8;  // LDS row pitch (bf16): 144 bytes, so 16 rows of a fragment read hit distinct banks
// JB draws per workgroup (64, or 32 when the 64-wide grid leaves fewer than two workgroups per CU: each output's
// products and their order are the same either way).
template <int JB>
__global__ void __launch_bounds__(256) key_filter_kernel(const KeyFilterArgs g) {
  constexpr int JC = JB / 4, NCB = JB / 16;  // scores per loader thread, 16-column MFMA blocks
  __shared__ __attribute__((aligned(16))) bf16 sa[64 * KF_LD];
  __shared__ __attribute__((aligned(16))) bf16 sb[JB * KF_LD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int t0 = blockIdx.x * 64, j0 = blockIdx.y * JB, bh = blockIdx.z;
  const bf16* filt = g.filt + (long)bh * g.T * g.T;
  const float* score = g.score + (long)bh * g.T * g.n;
  f32x4 acc[NCB];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) acc[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
  // loaders: K row tid / 4, s columns 16 (tid % 4) .. + 15; scores row s = tid / 4, columns JC (tid % 4) .. + JC - 1
  const int ar = tid >> 2, ac = (tid & 3) * 16, bs = tid >> 2, bc = (tid & 3) * JC;
  // whole float4 groups of scores when n % 4 == 0 (a group is then either all below n or all above)
  const bool vec = (g.n & 3) == 0 && !((uintptr_t)g.score & 15);
  auto load = [&](int s0, bf16x8 (&kv)[2], float (&sv)[JC]) {
    const bf16* kr = filt + (long)(t0 + ar) * g.T + s0 + ac;
    kv[0] = *reinterpret_cast<const bf16x8*>(kr);
    kv[1] = *reinterpret_cast<const bf16x8*>(kr + 8);
    const float* sr = score + (long)(s0 + bs) * g.n + j0 + bc;
    if (vec) {
#pragma unroll
      for (int q = 0; q < JC / 4; ++q) {
        const float4 v = j0 + bc + 4 * q < g.n ? *reinterpret_cast<const float4*>(sr + 4 * q)
                                               : make_float4(0.f, 0.f, 0.f, 0.f);
        sv[4 * q] = v.x, sv[4 * q + 1] = v.y, sv[4 * q + 2] = v.z, sv[4 * q + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < JC; ++e) sv[e] = j0 + bc + e < g.n ? sr[e] : 0.f;
    }
  };
  bf16x8 kv[2];
  float sv[JC];
  load(0, kv, sv);
  for (int s0 = 0; s0 < g.T; s0 += KF_BK) {
    __syncthreads();  // the previous chunk's fragments have been read
    *reinterpret_cast<bf16x8*>(&sa[ar * KF_LD + ac]) = kv[0];
    *reinterpret_cast<bf16x8*>(&sa[ar * KF_LD + ac + 8]) = kv[1];
#pragma unroll
    for (int e = 0; e < JC; ++e) sb[(bc + e) * KF_LD + bs] = to_bf16(sv[e]);
    __syncthreads();
    if (s0 + KF_BK < g.T) load(s0 + KF_BK, kv, sv);
#pragma unroll
    for (int kk = 0; kk < KF_BK / 32; ++kk) {
      const bf16x8 af =
          *reinterpret_cast<const bf16x8*>(&sa[(16 * wave + (lane & 15)) * KF_LD + 32 * kk + 8 * (lane >> 4)]);
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        const bf16x8 bfr =
            *reinterpret_cast<const bf16x8*>(&sb[(16 * cb + (lane & 15)) * KF_LD + 32 * kk + 8 * (lane >> 4)]);
        acc[cb] = mfma16x16x32(af, bfr, acc[cb]);
      }
    }
  }
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
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
  if (g.BH > 65535 || (g.n + 31) / 32 > 65535) return NOISE_ENOTSUP;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  const long wide = (long)(g.T / 64) * ((g.n + 63) / 64) * g.BH;
  if (wide < 2L * cus)
    hipLaunchKernelGGL(key_filter_kernel<32>, dim3((unsigned)(g.T / 64), (unsigned)((g.n + 31) / 32), (unsigned)g.BH),
                       dim3(256), 0, s, g);
  else
    hipLaunchKernelGGL(key_filter_kernel<64>, dim3((unsigned)(g.T / 64), (unsigned)((g.n + 63) / 64), (unsigned)g.BH),
                       dim3(256), 0, s, g);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}

int moved_heads_launch(const MovedHeadsArgs& g, hipStream_t s) {
  if (!g.raw || !g.a || !g.cos || !g.sin || !g.out || g.n <= 0 || g.B <= 0 || g.T <= 0 || g.H <= 0 ||
      g.ldo < (long)g.H * HD)
    return NOISE_EINVAL;
  if (g.ldo % 4 == 0 && !(((uintptr_t)g.raw | (uintptr_t)g.cos | (uintptr_t)g.sin) & 15) &&
      !(((uintptr_t)g.a | (uintptr_t)g.out) & 7)) {
    const long grid = (g.rows + 31) / 32;
    if (grid > 0x7fffffffL) return NOISE_ENOTSUP;
    hipLaunchKernelGGL(moved_heads_vec_kernel, dim3((unsigned)grid), dim3(256), 0, s, g);
    NOISE_CHECK_LAUNCH();
    return NOISE_OK;
  }
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
  if (g.ld_out % 8 == 0 && !(((uintptr_t)g.out | (uintptr_t)g.baseline | (uintptr_t)g.hub) & 15)) {
    const long tiles = (g.rows / g.n + 7) / 8, chunks = (g.n + 31) / 32;  // rows = n B T H
    if (tiles > 0x7fffffffL || chunks > 65535) return NOISE_ENOTSUP;
    hipLaunchKernelGGL(head_scores_vec_kernel, dim3((unsigned)tiles, (unsigned)chunks), dim3(256), 0, s, g);
    NOISE_CHECK_LAUNCH();
    return NOISE_OK;
  }
  const long grid = (g.rows + 7) / 8;
  if (grid > 0x7fffffffL) return NOISE_ENOTSUP;
  hipLaunchKernelGGL(head_scores_kernel, dim3((unsigned)grid), dim3(256), 0, s, g);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}

int code_estimate_launch(const CodeEstimateArgs& g, hipStream_t s) {
  if (!g.credited || !g.a || !g.est || g.n <= 0 || g.elems <= 0 || g.H <= 0 || g.T <= 0) return NOISE_EINVAL;
  if (!(((uintptr_t)g.a | (uintptr_t)g.est) & 15)) {  // elems = B T H 64: whole 4-dim groups
    const long grid = (g.elems / 4 + 255) / 256;
    if (grid > 0x7fffffffL) return NOISE_ENOTSUP;
    hipLaunchKernelGGL(code_estimate_vec_kernel, dim3((unsigned)grid), dim3(256), 0, s, g);
    NOISE_CHECK_LAUNCH();
    return NOISE_OK;
  }
  const long grid = (g.elems + 255) / 256;
  if (grid > 0x7fffffffL) return NOISE_ENOTSUP;
  hipLaunchKernelGGL(code_estimate_kernel, dim3((unsigned)grid), dim3(256), 0, s, g);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}
