// EGGROLL update path: fitness from the antithetic losses, the weighted sum of perturbation outer
// products (the gradient estimate), and Adam.
//
// Reference: Eggroll.step (train/val/eggroll.py:151-167) and torch.optim.AdamW(lr, betas=(0.5, 0.95),
// eps=1e-8, weight_decay=0) (:205). All fp32.
#include "common.h"
#include "eggroll.h"

namespace {

// One workgroup: f_j = L[2j+1] - L[2j]; z-score mode divides by (unbiased std + 1e-8) with no
// centering (:151-152); rank mode maps f to centred ranks in [-0.5, 0.5] (ties broken by index).
// weight[d] = sum of f_j over j = d mod pairs in increasing j (:153-154).
__global__ void __launch_bounds__(1024) fitness_kernel(const float* __restrict__ losses, int nf, int pairs, int mode,
                                                       float* __restrict__ fit, float* __restrict__ weight) {
  __shared__ float red[1024];
  __shared__ float stat;
  const int tid = threadIdx.x;
  for (int j = tid; j < nf; j += 1024) fit[j] = losses[2 * j + 1] - losses[2 * j];
  __syncthreads();
  if (mode == NOISE_FITNESS_ZSCORE) {
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
  } else {
    // centred rank of f_j: #{i : f_i < f_j or (f_i == f_j and i < j)} / (nf - 1) - 0.5
    for (int j = tid; j < nf; j += 1024) {
      const float fj = losses[2 * j + 1] - losses[2 * j];
      int r = 0;
      for (int i = 0; i < nf; ++i) {
        const float fi = losses[2 * i + 1] - losses[2 * i];
        r += (fi < fj) || (fi == fj && i < j);
      }
      fit[j] = nf > 1 ? (float)r / (float)(nf - 1) - 0.5f : 0.f;
    }
  }
  __syncthreads();
  for (int d = tid; d < pairs; d += 1024) {
    float s = 0.f;
    for (int j = d; j < nf; j += pairs) s += fit[j];
    weight[d] = s;
  }
}

// G[o, i] = scale * sum_j (w_j a_j[o]) b_j[i] over ndir directions (a null: a_j[o] = 1, out = 1),
// on the fp32 MFMA (v_mfma_f32_16x16x4_f32): a 64 x 64 output tile per workgroup of 4 waves (32 x 32
// each), directions staged through LDS 32 at a time with w_j folded into the a rows.
__global__ void __launch_bounds__(256) outer_update_kernel(OuterUpdateArgs g) {
  constexpr int TK = 32;
  __shared__ float sa[TK][64 + 4];
  __shared__ float sb[TK][64 + 4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int o0 = blockIdx.y * 64, i0 = blockIdx.x * 64;
  f32x4 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int j0 = 0; j0 < g.ndir; j0 += TK) {
#pragma unroll
    for (int s = 0; s < TK * 64 / 256; ++s) {
      const int e = tid + s * 256, jj = e >> 6, c = e & 63, j = j0 + jj;
      float av = 0.f, bv = 0.f;
      if (j < g.ndir) {
        if (o0 + c < g.out) av = g.w[j] * (g.a ? g.a[(long)j * g.a_ld + o0 + c] : 1.f);
        if (i0 + c < g.in) bv = g.b[(long)j * g.b_ld + i0 + c];
      }
      sa[jj][c] = av;
      sb[jj][c] = bv;
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < TK / 4; ++ks) {
      const int jj = 4 * ks + (lane >> 4);
      float af[2], bf[2];
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        af[f] = sa[jj][wm * 32 + 16 * f + (lane & 15)];
        bf[f] = sb[jj][wn * 32 + 16 * f + (lane & 15)];
      }
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[a], bf[b], acc[a][b], 0, 0, 0);
    }
    __syncthreads();
  }
  // lane holds C[row = 4 (lane / 16) + e][col = lane % 16] of each 16 x 16 block
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int o = o0 + wm * 32 + 16 * a + 4 * (lane >> 4) + e, i = i0 + wn * 32 + 16 * b + (lane & 15);
        if (o < g.out && i < g.in) g.grad[(long)o * g.in + i] = g.scale * acc[a][b][e];
      }
}

// torch.optim.AdamW (single-tensor path) with weight_decay = 0:
// m = lerp(m, g, 1 - b1); v = b2 v + (1 - b2) g^2; p -= (lr / bc1) m / (sqrt(v) / sqrt(bc2) + eps).
__global__ void __launch_bounds__(256) adam_kernel(AdamArgs g) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= g.n) return;
  const float gr = g.grad[i];
  float m = g.m[i], v = g.v[i];
  const float w = 1.f - g.beta1;
  m = w < 0.5f ? m + w * (gr - m) : gr - (gr - m) * (1.f - w);
  v = v * g.beta2 + (1.f - g.beta2) * gr * gr;
  g.m[i] = m;
  g.v[i] = v;
  const float denom = sqrtf(v) / g.bc2_sqrt + g.eps;
  g.param[i] = g.param[i] + (-g.step_size) * (m / denom);
}

}  // namespace

int fitness_launch(const float* losses, int n, int pairs, int mode, float* fit, float* weight, hipStream_t s) {
  if (!losses || !fit || !weight || n < 4 || n % 2 || pairs <= 0 ||
      (mode != NOISE_FITNESS_ZSCORE && mode != NOISE_FITNESS_RANK))
    return NOISE_EINVAL;
  hipLaunchKernelGGL(fitness_kernel, dim3(1), dim3(1024), 0, s, losses, n / 2, pairs, mode, fit, weight);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}

int outer_update_launch(const OuterUpdateArgs& g, hipStream_t s) {
  if (!g.b || !g.w || !g.grad || g.ndir <= 0 || g.out <= 0 || g.in <= 0 || (!g.a && g.out != 1) ||
      g.b_ld < g.in || (g.a && g.a_ld < g.out))
    return NOISE_EINVAL;
  hipLaunchKernelGGL(outer_update_kernel, dim3((g.in + 63) / 64, (g.out + 63) / 64), dim3(256), 0, s, g);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}

int adam_launch(const AdamArgs& g, hipStream_t s) {
  if (!g.param || !g.grad || !g.m || !g.v || g.n <= 0 || !(g.bc2_sqrt > 0.f)) return NOISE_EINVAL;
  hipLaunchKernelGGL(adam_kernel, dim3((unsigned)((g.n + 255) / 256)), dim3(256), 0, s, g);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}
