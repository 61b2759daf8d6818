// Row-wise kernels of the population forward (HBM-bound; one wave per row group).
#include "common.h"
#include "gemm.h"

namespace {

// u[row] = bf16(sum_k x[row, k] * bf16(b[dir, k])): the rank-1 GEMV `x @ b` of `lowrank`
// (train/val/eggroll.py:58) under autocast (bf16 operands, fp32 accumulation, bf16 result).
__global__ void __launch_bounds__(256)
rowdot_kernel(const bf16* __restrict__ x, long ldx, long x_mstride, int M, int K, int T, int pair_shift,
              const float* __restrict__ b, long ldb, float* __restrict__ u) {
  const int lane = threadIdx.x & 63;
  const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int nwaves = (gridDim.x * blockDim.x) >> 6;
  for (int row = wave; row < M; row += nwaves) {
    const int p = row / T;
    const bf16* xr = x + (long)p * x_mstride + (long)(row % T) * ldx;
    const float* br = b + (long)(p >> pair_shift) * ldb;
    float acc = 0.f;
    for (int k = lane * 8; k < K; k += 512) {
      const bf16x8 xv = *reinterpret_cast<const bf16x8*>(xr + k);
      const float4 b0 = *reinterpret_cast<const float4*>(br + k);
      const float4 b1 = *reinterpret_cast<const float4*>(br + k + 4);
      acc += (float)xv[0] * bf16r(b0.x) + (float)xv[1] * bf16r(b0.y) + (float)xv[2] * bf16r(b0.z) +
             (float)xv[3] * bf16r(b0.w) + (float)xv[4] * bf16r(b1.x) + (float)xv[5] * bf16r(b1.y) +
             (float)xv[6] * bf16r(b1.z) + (float)xv[7] * bf16r(b1.w);
    }
    acc = group_sum<64>(acc);
    if (lane == 0) u[row] = bf16r(acc);
  }
}

}  // namespace

int rowdot_launch(const bf16* x, long ldx, long x_mstride, int M, int K, int T, int pair_shift, const float* b,
                  long ldb, float* u, hipStream_t stream) {
  if (!x || !b || !u || M <= 0 || K <= 0 || K % 8 || ldx % 8 || x_mstride % 8 || ldb % 4 || T <= 0)
    return NOISE_EINVAL;
  const int blocks = min((M + 3) / 4, 8192);
  hipLaunchKernelGGL(rowdot_kernel, dim3(blocks), dim3(256), 0, stream, x, ldx, x_mstride, M, K, T, pair_shift,
                     b, ldb, u);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}
