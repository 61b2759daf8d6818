// Row kernels of the clean forward at the rounding points of GPT.forward under torch's bf16 autocast with bf16
// embedding tables: the speedrun's scorer (utils/eval.py:44-45 runs utils/model.py:193-210 that way; the tables
// are bf16 because init_weights stores them so on a GPU, utils/model.py:171-175).
//
// Under that autocast every tensor of the residual stream is bf16, and each elementwise op of the forward rounds
// its result to bf16 (torch computes it in fp32 and casts back):
//   x0 = bf16(norm(wte[idx]))                        rms_norm of a bf16 input: fp32 compute, eps = 2^-23 (torch
//                                                     2.10's default for a bf16 input), bf16 out
//   x  = bf16(bf16(l_r x) + bf16(l_0 x0))            the 0-d fp32 lambda is cast to bf16 first (type promotion
//                                                     of a 0-d tensor against a bf16 tensor)
//   x  = bf16(x + y)                                  each block output added to the bf16 stream
//   gate = 2 bf16(sigmoid(bf16(h[:32] W_g^T)))        the gate linear is a bf16 GEMM, sigmoid is bf16, x2 exact
//   q, k: rotary with every product and sum rounded, then norm -> bf16
//   v = bf16(v + bf16(gate ve))
// The GEMMs (bf16 operands, fp32 accumulation, bf16 output), the attention and the head run on the library's
// other kernels.
#include "autocast.h"
#include "common.h"

namespace {

constexpr int D = 512;
constexpr float NORM_EPS = 1.1920928955078125e-07f;  // finfo(float32).eps: rms_norm's default for bf16 input too

__device__ __forceinline__ void load8_bf(const bf16* p, float (&v)[8]) {
  const bf16x8 x = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = (float)x[e];
}
__device__ __forceinline__ void store8_bf(bf16* p, const float (&v)[8]) {
  bf16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = to_bf16(v[e]);
  *reinterpret_cast<bf16x8*>(p) = o;
}
__device__ __forceinline__ void load8_f(const float* p, float (&v)[8]) {
  const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
  v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
}
// bf16(norm(v)) of a row whose WIDTH values lie 8 per lane over WIDTH / 8 lanes (utils/model.py:46-47 on a bf16
// input: fp32 mean of squares, rsqrt, product, cast back)
template <int WIDTH>
__device__ __forceinline__ void norm_bf(float (&v)[8]) {
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += v[e] * v[e];
  ss = group_sum<WIDTH / 8>(ss);
  const float r = rsqrtf(ss * (1.f / WIDTH) + NORM_EPS);
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = bf16r(v[e] * r);
}

// One wave per row: x0, the adds, the mix, the norm and the value gate of AcStreamArgs.
__global__ void __launch_bounds__(256) ac_stream_kernel(AcStreamArgs g) {
  const int lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= g.M) return;
  const int p = (int)(row / g.T), t = (int)(row % g.T);
  float x0[8] = {}, x[8];
  if (!g.x_in || g.lambda_r) {
    const long tok = g.idx[(long)p * g.idx_mstride + t];
    load8_f(g.emb_w + tok * D + lane * 8, x0);
#pragma unroll
    for (int e = 0; e < 8; ++e) x0[e] = bf16r(x0[e]);  // the table's bf16 storage
    norm_bf<D>(x0);
  }
  if (g.x_in) {
    load8_bf(g.x_in + row * D + lane * 8, x);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = x0[e];
  }
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    if (g.add[k]) {
      float y[8];
      load8_bf(g.add[k] + row * D + lane * 8, y);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = bf16r(x[e] + y[e]);
    }
  }
  if (g.lambda_r) {
    const float lr = bf16r(*g.lambda_r), l0 = bf16r(*g.lambda_0);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = bf16r(bf16r(lr * x[e]) + bf16r(l0 * x0[e]));
  }
  if (g.x_out) store8_bf(g.x_out + row * D + lane * 8, x);
  if (!g.h) return;
  norm_bf<D>(x);
  store8_bf(g.h + row * D + lane * 8, x);
  if (g.gate_w) {
    // head hh = lane / 8 sums channels 4 c .. 4 c + 3 (c = lane % 8), held by lane c / 2 at elements 4 (c % 2) ..
    const int hh = lane >> 3, c = lane & 7, src = c >> 1;
    float part = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = __shfl(x[e], src, 64), hi = __shfl(x[4 + e], src, 64);
      part += ((c & 1) ? hi : lo) * bf16r(g.gate_w[hh * 32 + 4 * c + e]);
    }
    const float z = bf16r(group_sum<8>(part));
    const float sg = bf16r(1.f / (1.f + expf(-z)));
    if (c == 0) g.gate[row * 8 + hh] = 2.f * sg;
  }
}

// One wave per row of q | k | v: rotary and norm of the q and k heads, the gated value embedding of v.
__global__ void __launch_bounds__(256) ac_qkv_kernel(AcQkvArgs g) {
  const int lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= g.M) return;
  const int p = (int)(row / g.T), t = (int)(row % g.T);
  bf16* r = g.qkv + row * (3 * D);
  // lane: head lane / 8, dims 8 j .. 8 j + 7 (j = lane % 8); its rotary partners (d +- 32) are in lane ^ 4
  const int hh = lane >> 3, j = lane & 7;
  float cs[8], sn[8];
  {
    const bf16x8 c8 = *reinterpret_cast<const bf16x8*>(g.rot_cos + (long)t * 32 + 8 * (j & 3));
    const bf16x8 s8 = *reinterpret_cast<const bf16x8*>(g.rot_sin + (long)t * 32 + 8 * (j & 3));
#pragma unroll
    for (int e = 0; e < 8; ++e) cs[e] = (float)c8[e], sn[e] = (float)s8[e];
  }
#pragma unroll
  for (int seg = 0; seg < 2; ++seg) {
    bf16* q = r + seg * D + hh * 64 + 8 * j;
    float v[8], o[8];
    load8_bf(q, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float w = __shfl_xor(v[e], 4, 64);
      // [x1 cos + x2 sin, x1 (-sin) + x2 cos] (utils/model.py:55-58), each product and sum rounded to bf16
      o[e] = j < 4 ? bf16r(bf16r(v[e] * cs[e]) + bf16r(w * sn[e])) : bf16r(bf16r(w * -sn[e]) + bf16r(v[e] * cs[e]));
    }
    norm_bf<64>(o);
    store8_bf(q, o);
  }
  if (g.gate) {
    bf16* vp = r + 2 * D + lane * 8;
    const long tok = g.idx[(long)p * g.idx_mstride + t];
    float v[8], ve[8];
    load8_bf(vp, v);
    load8_f(g.ve_w + tok * D + lane * 8, ve);
    const float gt = g.gate[row * 8 + hh];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = bf16r(v[e] + bf16r(gt * bf16r(ve[e])));
    store8_bf(vp, v);
  }
}

int grid_of(long M) { return (int)((M + 3) / 4); }

}  // namespace

int ac_stream_launch(const AcStreamArgs& g, hipStream_t s) {
  if (g.M <= 0 || g.T <= 0) return NOISE_EINVAL;
  const bool need_x0 = !g.x_in || g.lambda_r;
  if (need_x0 && (!g.emb_w || !g.idx || g.V <= 0 || g.idx_mstride < 0)) return NOISE_EINVAL;
  if ((g.lambda_r == nullptr) != (g.lambda_0 == nullptr)) return NOISE_EINVAL;
  if (g.gate_w && (!g.h || !g.gate)) return NOISE_EINVAL;
  if (!g.x_out && !g.h) return NOISE_EINVAL;
  if (((uintptr_t)g.x_in | (uintptr_t)g.emb_w | (uintptr_t)g.add[0] | (uintptr_t)g.add[1] | (uintptr_t)g.x_out |
       (uintptr_t)g.h) & 15)
    return NOISE_EINVAL;
  hipLaunchKernelGGL(ac_stream_kernel, dim3(grid_of(g.M)), dim3(256), 0, s, g);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}

int ac_qkv_launch(const AcQkvArgs& g, hipStream_t s) {
  if (g.M <= 0 || g.T <= 0 || !g.qkv || !g.rot_cos || !g.rot_sin) return NOISE_EINVAL;
  if (g.gate && (!g.ve_w || !g.idx || g.V <= 0 || g.idx_mstride < 0)) return NOISE_EINVAL;
  if (((uintptr_t)g.qkv | (uintptr_t)g.rot_cos | (uintptr_t)g.rot_sin | (uintptr_t)g.ve_w) & 15) return NOISE_EINVAL;
  hipLaunchKernelGGL(ac_qkv_kernel, dim3(grid_of(g.M)), dim3(256), 0, s, g);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}
