// EGGROLL update path: fitness from the antithetic losses, the weighted sum of perturbation outer
// products (the gradient estimate), and Adam.
//
// Reference: Eggroll.step (train/val/eggroll.py:151-167) and torch.optim.AdamW(lr, betas=(0.5, 0.95),
// eps=1e-8, weight_decay=0) (:205). All fp32.
#include <algorithm>

#include "common.h"
#include "eggroll.h"

namespace {

// Z-score fitness in one workgroup (O(n) work): f_j = L[2j+1] - L[2j], divided by (unbiased std + 1e-8) with no
// centering (:151-152).
__global__ void __launch_bounds__(1024) zscore_fitness_kernel(const float* __restrict__ losses, int nf,
                                                              float* __restrict__ fit) {
  __shared__ float red[1024];
  __shared__ float stat;
  const int tid = threadIdx.x;
  for (int j = tid; j < nf; j += 1024) fit[j] = losses[2 * j + 1] - losses[2 * j];
  __syncthreads();
  {
    float s = 0.f;
    for (int j = tid; j < nf; j += 1024) s += fit[j];
    red[tid] = s;
    __syncthreads();
    for (int w = 512; w > 0; w >>= 1) {
      if (tid < w) red[tid] += red[tid + w];
      __syncthreads();
    }
    const float mean = red[0] / (float)nf;
    __syncthreads();
    float q = 0.f;
    for (int j = tid; j < nf; j += 1024) {
      const float d = fit[j] - mean;
      q += d * d;
    }
    red[tid] = q;
    __syncthreads();
    for (int w = 512; w > 0; w >>= 1) {
      if (tid < w) red[tid] += red[tid + w];
      __syncthreads();
    }
    if (tid == 0) stat = sqrtf(red[0] / (float)(nf - 1)) + 1e-8f;
    __syncthreads();
    const float den = stat;
    for (int j = tid; j < nf; j += 1024) fit[j] = fit[j] / den;
  }
}

// Rank fitness (config-4 option; no reference function), spread over the GPU: thread j owns f_j and counts
// #{i : f_i < f_j or (f_i == f_j and i < j)} over every f_i, which the workgroup stages through LDS RTILE at a
// time (every lane reads the same LDS word: a broadcast). fit_j = rank / (n - 1) - 0.5, ties broken by index.
// n^2 comparisons in n / 256 workgroups: 131,072 pairs (the reference's population) are 512 workgroups of 131,072
// broadcast-compare steps each.
constexpr int RTILE = 2048;
__global__ void __launch_bounds__(256) rank_fitness_kernel(const float* __restrict__ losses, int nf,
                                                           float* __restrict__ fit) {
  __shared__ float tile[RTILE];
  const int j = blockIdx.x * 256 + threadIdx.x;
  const float fj = j < nf ? losses[2 * j + 1] - losses[2 * j] : 0.f;
  int r = 0;
  for (int i0 = 0; i0 < nf; i0 += RTILE) {
    const int n = min(RTILE, nf - i0);
    __syncthreads();  // the previous tile has been read by every thread
    for (int i = threadIdx.x; i < n; i += 256) tile[i] = losses[2 * (i0 + i) + 1] - losses[2 * (i0 + i)];
    __syncthreads();
    const int lt = j - i0;  // tile entries i < lt have index i0 + i < j
    for (int i = 0; i < n; ++i) {
      const float fi = tile[i];
      r += (fi < fj) || (fi == fj && i < lt);
    }
  }
  if (j < nf) fit[j] = nf > 1 ? (float)r / (float)(nf - 1) - 0.5f : 0.f;
}

// weight[d] = sum of fit_j over j = d mod pairs, in increasing j (:153-154): one thread per direction.
__global__ void __launch_bounds__(256) fold_fitness_kernel(const float* __restrict__ fit, int nf, int pairs,
                                                           float* __restrict__ weight) {
  const int d = blockIdx.x * 256 + threadIdx.x;
  if (d >= pairs) return;
  float s = 0.f;
  for (int j = d; j < nf; j += pairs) s += fit[j];
  weight[d] = s;
}

// G[o, i] = scale * sum_j (w_j a_j[o]) b_j[i] over ndir directions (a null: a_j[o] = 1, out = 1), for up
// to OUTER_MAX matrices in one launch (every perturbed parameter of the model: ~9k 64 x 64 tiles fill the
// GPU, where one 512 x 512 matrix alone is 64 workgroups). On the fp32 MFMA (v_mfma_f32_16x16x4_f32): a
// 64 x 64 output tile per workgroup of 4 waves (32 x 32 each); directions pass through a double-buffered
// LDS stage 32 at a time with w_j folded into the a rows, the next 32 loaded into registers while the
// current ones feed the MFMAs.
__global__ void __launch_bounds__(256) outer_update_kernel(const OuterBatchArgs g) {
  constexpr int TK = 32, LD = 64 + 4;
  __shared__ __attribute__((aligned(16))) float sa[2][TK][LD];
  __shared__ __attribute__((aligned(16))) float sb[2][TK][LD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  // this workgroup's matrix and tile (uniform scan over the prefix sums of tile counts)
  const int t = blockIdx.x;
  int mi = 0;
  while (mi + 1 < g.n && t >= g.m[mi].tile_end) ++mi;
  const OuterMat& M = g.m[mi];
  const int lt = t - (mi ? g.m[mi - 1].tile_end : 0);
  const int o0 = (lt / M.tiles_i) * 64, i0 = (lt % M.tiles_i) * 64;
  // loader: thread tid fills direction jj = tid / 8 (of 32), columns 8 (tid % 8) .. + 7 of a and of b
  const int ljj = tid >> 3, lc = 8 * (tid & 7);
  const bool a_full = M.a && o0 + 64 <= M.out && M.a_ld % 4 == 0, b_full = i0 + 64 <= M.in && M.b_ld % 4 == 0;
  float ra[8], rb[8];
  auto load = [&](int j0) {
    const int j = j0 + ljj;
    const bool live = j < g.ndir;
    const float wj = live ? g.w[j] : 0.f;
    if (live && a_full) {
      const float4 x0 = *reinterpret_cast<const float4*>(M.a + (long)j * M.a_ld + o0 + lc);
      const float4 x1 = *reinterpret_cast<const float4*>(M.a + (long)j * M.a_ld + o0 + lc + 4);
      ra[0] = x0.x, ra[1] = x0.y, ra[2] = x0.z, ra[3] = x0.w, ra[4] = x1.x, ra[5] = x1.y, ra[6] = x1.z, ra[7] = x1.w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        ra[e] = live && o0 + lc + e < M.out ? (M.a ? M.a[(long)j * M.a_ld + o0 + lc + e] : 1.f) : 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) ra[e] *= wj;
    if (live && b_full) {
      const float4 x0 = *reinterpret_cast<const float4*>(M.b + (long)j * M.b_ld + i0 + lc);
      const float4 x1 = *reinterpret_cast<const float4*>(M.b + (long)j * M.b_ld + i0 + lc + 4);
      rb[0] = x0.x, rb[1] = x0.y, rb[2] = x0.z, rb[3] = x0.w, rb[4] = x1.x, rb[5] = x1.y, rb[6] = x1.z, rb[7] = x1.w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) rb[e] = live && i0 + lc + e < M.in ? M.b[(long)j * M.b_ld + i0 + lc + e] : 0.f;
    }
  };
  auto stage = [&](int buf) {
    *reinterpret_cast<float4*>(&sa[buf][ljj][lc]) = make_float4(ra[0], ra[1], ra[2], ra[3]);
    *reinterpret_cast<float4*>(&sa[buf][ljj][lc + 4]) = make_float4(ra[4], ra[5], ra[6], ra[7]);
    *reinterpret_cast<float4*>(&sb[buf][ljj][lc]) = make_float4(rb[0], rb[1], rb[2], rb[3]);
    *reinterpret_cast<float4*>(&sb[buf][ljj][lc + 4]) = make_float4(rb[4], rb[5], rb[6], rb[7]);
  };
  f32x4 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
  load(0);
  stage(0);
  __syncthreads();
  int buf = 0;
  for (int j0 = 0; j0 < g.ndir; j0 += TK) {
    const bool more = j0 + TK < g.ndir;
    if (more) load(j0 + TK);  // in flight during this chunk's MFMAs
#pragma unroll
    for (int ks = 0; ks < TK / 4; ++ks) {
      const int jj = 4 * ks + (lane >> 4);
      float af[2], bf[2];
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        af[f] = sa[buf][jj][wm * 32 + 16 * f + (lane & 15)];
        bf[f] = sb[buf][jj][wn * 32 + 16 * f + (lane & 15)];
      }
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[a], bf[b], acc[a][b], 0, 0, 0);
    }
    if (more) {
      // the other buffer was last read in the previous chunk, before the barrier that ended it
      stage(buf ^ 1);
      __syncthreads();
      buf ^= 1;
    }
  }
  // lane holds C[row = 4 (lane / 16) + e][col = lane % 16] of each 16 x 16 block
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int o = o0 + wm * 32 + 16 * a + 4 * (lane >> 4) + e, i = i0 + wn * 32 + 16 * b + (lane & 15);
        if (o < M.out && i < M.in) M.grad[(long)o * M.in + i] = g.scale * acc[a][b][e];
      }
}

// torch.optim.AdamW (single-tensor path) with weight_decay = 0:
// m = lerp(m, g, 1 - b1); v = b2 v + (1 - b2) g^2; p -= (lr / bc1) m / (sqrt(v) / sqrt(bc2) + eps).
__device__ __forceinline__ void adam_element(float* param, const float* grad, float* mp, float* vp, long i,
                                             float step_size, float bc2_sqrt, float beta1, float beta2, float eps) {
  const float gr = grad[i];
  float m = mp[i], v = vp[i];
  const float w = 1.f - beta1;
  m = w < 0.5f ? m + w * (gr - m) : gr - (gr - m) * (1.f - w);
  v = v * beta2 + (1.f - beta2) * gr * gr;
  mp[i] = m;
  vp[i] = v;
  const float denom = sqrtf(v) / bc2_sqrt + eps;
  param[i] = param[i] + (-step_size) * (m / denom);
}
__global__ void __launch_bounds__(256) adam_kernel(AdamArgs g) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= g.n) return;
  adam_element(g.param, g.grad, g.m, g.v, i, g.step_size, g.bc2_sqrt, g.beta1, g.beta2, g.eps);
}
// Every tensor of an optimizer step in one launch (the same arithmetic per element as adam_kernel): block b
// serves the tensor whose range of 256-element blocks holds it (a uniform scan over the running totals).
__global__ void __launch_bounds__(256) adam_batch_kernel(const AdamBatchArgs g) {
  const long b = blockIdx.x;
  int k = 0;
  while (k + 1 < g.n && b >= g.t[k].block_end) ++k;
  const AdamTensor& t = g.t[k];
  const long i = (b - (k ? g.t[k - 1].block_end : 0)) * 256 + threadIdx.x;
  if (i >= t.n) return;
  adam_element(t.param, t.grad, t.m, t.v, i, t.step_size, t.bc2_sqrt, g.beta1, g.beta2, g.eps);
}

}  // namespace

int fitness_launch(const float* losses, int n, int pairs, int mode, float* fit, float* weight, hipStream_t s) {
  if (!losses || !fit || !weight || n < 4 || n % 2 || pairs <= 0 ||
      (mode != NOISE_FITNESS_ZSCORE && mode != NOISE_FITNESS_RANK))
    return NOISE_EINVAL;
  const int nf = n / 2;
  if (mode == NOISE_FITNESS_ZSCORE)
    hipLaunchKernelGGL(zscore_fitness_kernel, dim3(1), dim3(1024), 0, s, losses, nf, fit);
  else
    hipLaunchKernelGGL(rank_fitness_kernel, dim3((unsigned)((nf + 255) / 256)), dim3(256), 0, s, losses, nf, fit);
  NOISE_CHECK_LAUNCH();
  hipLaunchKernelGGL(fold_fitness_kernel, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0, s, fit, nf, pairs,
                     weight);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}

namespace {
// One workgroup per (direction j, parameter k): copies the out + in floats of the parameter's slice for pair
// directions[j]. A direction or offset outside its range writes NaN rows (never an out-of-bounds read).
__global__ void __launch_bounds__(256) gather_rows_kernel(const GatherArgs g) {
  const int j = blockIdx.x, k = blockIdx.y, tid = threadIdx.x;
  const GatherParam& q = g.p[k];
  const long d = g.directions[j];
  const long off = (d >= 0 && d < g.pairs) ? q.offsets[d] : -1;
  const bool ok = off >= 0 && off <= g.buffer_len - (long)(q.out + q.in);
  const float* src = g.buffer + (ok ? off : 0);
  for (int c = tid; c < q.out; c += 256) q.a[(long)j * q.out + c] = ok ? src[c] : __builtin_nanf("");
  for (int c = tid; c < q.in; c += 256) q.b[(long)j * q.in + c] = ok ? src[q.out + c] : __builtin_nanf("");
}
}  // namespace

int gather_rows_launch(const GatherParam* params, int n, const float* buffer, long buffer_len,
                       const int64_t* directions, int ndir, int pairs, hipStream_t s) {
  if (n <= 0 || !params || !buffer || buffer_len <= 0 || !directions || ndir <= 0 || pairs <= 0) return NOISE_EINVAL;
  if (ndir > 0x7fffffff) return NOISE_ENOTSUP;
  for (int base = 0; base < n; base += GATHER_MAX) {
    GatherArgs g{};
    g.n = std::min(GATHER_MAX, n - base);
    g.buffer = buffer;
    g.buffer_len = buffer_len;
    g.directions = directions;
    g.ndir = ndir;
    g.pairs = pairs;
    for (int k = 0; k < g.n; ++k) {
      const GatherParam& q = params[base + k];
      if (!q.offsets || !q.a || q.out <= 0 || q.in < 0 || (q.in > 0 && !q.b)) return NOISE_EINVAL;
      g.p[k] = q;
    }
    hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)ndir, (unsigned)g.n), dim3(256), 0, s, g);
    NOISE_CHECK_LAUNCH();
  }
  return NOISE_OK;
}

int outer_update_launch(const OuterUpdateArgs* mats, int n, const float* w, int ndir, float scale, hipStream_t s) {
  if (n <= 0 || !mats || !w || ndir <= 0) return NOISE_EINVAL;
  for (int base = 0; base < n; base += OUTER_MAX) {
    OuterBatchArgs g{};
    g.n = std::min(OUTER_MAX, n - base);
    g.w = w;
    g.ndir = ndir;
    g.scale = scale;
    long tiles = 0;
    for (int k = 0; k < g.n; ++k) {
      const OuterUpdateArgs& u = mats[base + k];
      if (!u.b || !u.grad || u.out <= 0 || u.in <= 0 || (!u.a && u.out != 1) || u.b_ld < u.in ||
          (u.a && u.a_ld < u.out))
        return NOISE_EINVAL;
      OuterMat& m = g.m[k];
      m.a = u.a, m.b = u.b, m.grad = u.grad, m.a_ld = u.a_ld, m.b_ld = u.b_ld, m.out = u.out, m.in = u.in;
      m.tiles_i = (u.in + 63) / 64;
      tiles += (long)((u.out + 63) / 64) * m.tiles_i;
      if (tiles > 0x7fffffffL) return NOISE_ENOTSUP;
      m.tile_end = (int)tiles;
    }
    hipLaunchKernelGGL(outer_update_kernel, dim3((unsigned)tiles), dim3(256), 0, s, g);
    NOISE_CHECK_LAUNCH();
  }
  return NOISE_OK;
}

int adam_batch_launch(const AdamTensor* tensors, int n, float beta1, float beta2, float eps, hipStream_t s) {
  if (n <= 0 || !tensors) return NOISE_EINVAL;
  // every tensor and every chunk's block count is checked before the first launch: a rejected call updates nothing
  for (int base = 0; base < n; base += ADAM_MAX) {
    long blocks = 0;
    for (int k = base; k < std::min(n, base + ADAM_MAX); ++k) {
      const AdamTensor& t = tensors[k];
      if (!t.param || !t.grad || !t.m || !t.v || t.n <= 0 || !(t.bc2_sqrt > 0.f)) return NOISE_EINVAL;
      blocks += (t.n + 255) / 256;
    }
    if (blocks > 0x7fffffffL) return NOISE_ENOTSUP;
  }
  for (int base = 0; base < n; base += ADAM_MAX) {
    AdamBatchArgs g{};
    g.n = std::min(ADAM_MAX, n - base);
    g.beta1 = beta1, g.beta2 = beta2, g.eps = eps;
    long blocks = 0;
    for (int k = 0; k < g.n; ++k) {
      g.t[k] = tensors[base + k];
      blocks += (g.t[k].n + 255) / 256;
      g.t[k].block_end = blocks;
    }
    hipLaunchKernelGGL(adam_batch_kernel, dim3((unsigned)blocks), dim3(256), 0, s, g);
    NOISE_CHECK_LAUNCH();
  }
  return NOISE_OK;
}

int adam_launch(const AdamArgs& g, hipStream_t s) {
  if (!g.param || !g.grad || !g.m || !g.v || g.n <= 0 || !(g.bc2_sqrt > 0.f)) return NOISE_EINVAL;
  hipLaunchKernelGGL(adam_kernel, dim3((unsigned)((g.n + 255) / 256)), dim3(256), 0, s, g);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}
