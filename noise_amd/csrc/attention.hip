// Windowed causal attention of the population forward on gfx950 bf16 MFMA, with the c_proj
// input-side dot and optional per-head output moments fused into the epilogue.
//
// Reference: `attention` / `window_mask` (utils/model.py:14-31) called from population_loss
// (train/val/eggroll.py:91): softmax(q k^T / sqrt(64)) v, a query at s seeing keys k with
// s - window <= k <= s. q, k, v arrive bf16 (rotary and QK-norm already applied by the QKV GEMM).
//
// One workgroup = one (member, head, 128-query block); 4 waves of 32 queries. K/V blocks of 64 keys
// go through a double-buffered LDS ring (K rows, V transposed to V^T so the key dimension is the
// MFMA contraction dimension of both products). Per wave and key block:
//   S^T = K Q^T   (MFMA A = K rows, B = Q rows): lane l holds 16 scores of query l % 16;
//   online softmax in fp32 (exp2, row max/sum across the 4 lanes of a query by two shuffles);
//   O^T += V^T P^T (MFMA A = V^T rows, B = P): the scores' register layout IS the B operand once
//   the K rows of each 16-row MFMA block are interleaved (block kb, row r <-> key
//   32 (kb / 2) + 8 (r / 4) + 4 (kb % 2) + r % 4), so P never leaves registers. P enters as the bf16
//   pair hi = bf16(P), lo = bf16(P - hi) (two MFMAs): the probabilities keep ~16 mantissa bits,
//   so the only rounding of the attention path is that of q, k, v and y to bf16.
// V^T rows are interleaved the same way (block db, row r <-> dim 16 (r / 4) + 4 db + r % 4), so each
// lane ends with 16 contiguous output dims of one query: 16-byte stores, and the c_proj dot
// y . b_proj over the head's 64 dims is a 4-lane reduction.
#include "attention.h"
#include "common.h"

namespace {

constexpr int HD = 64, BQ = 128, BKV = 64, NWAVE = 4, NTH = NWAVE * 64;

// Element offset of (row r, 16-byte chunk c) in a [64 x 64] bf16 LDS tile, chunk XOR-swizzled.
__device__ __forceinline__ int tswz(int r, int c) { return r * 64 + ((c ^ (r & 7)) << 3); }

// LDS row of key k (0..63) in the interleaved K tile, and of dim d in the interleaved V^T tile.
__device__ __forceinline__ int krow(int k) {
  const int grp = k >> 5, w = k & 31;
  const int kb = 2 * grp + ((w & 7) >> 2), r = 4 * (w >> 3) + (w & 3);
  return 16 * kb + r;
}
__device__ __forceinline__ int drow(int d) {
  const int db = (d & 15) >> 2, r = 4 * (d >> 4) + (d & 3);
  return 16 * db + r;
}

__device__ __forceinline__ unsigned pack2(float a, float b) {
  bf16x2 p = {to_bf16(a), to_bf16(b)};
  return *reinterpret_cast<unsigned*>(&p);
}

__global__ void __launch_bounds__(NTH, 2) attention_kernel(AttnArgs g) {
  __shared__ __attribute__((aligned(16))) bf16 sk[2][BKV * HD];
  __shared__ __attribute__((aligned(16))) bf16 sv[2][HD * BKV];
  __shared__ float smom[NWAVE][2][HD];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, grp = lane >> 4;
  // heavier (later) query blocks first
  const int qblk = gridDim.x - 1 - blockIdx.x, h = blockIdx.y, p = blockIdx.z;
  const int q0 = qblk * BQ;
  const long rbase = (long)p * g.T;
  const bf16* qkv = g.qkv;
  const int qcol = h * HD, kcol = g.koff + h * HD, vcol = g.voff + h * HD;

  // Q fragments (MFMA B operand): query q0 + 32 wave + 16 qb + lane % 16, dims 32 kk + 8 grp ..
  bf16x8 qf[2][2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
      qf[qb][kk] = *reinterpret_cast<const bf16x8*>(
          qkv + (rbase + q0 + 32 * wave + 16 * qb + (lane & 15)) * g.ldq + qcol + 32 * kk + 8 * grp);

  const int k_lo = max(0, q0 - g.window), k_hi = min(g.T - 1, q0 + BQ - 1);
  const int j0 = k_lo / BKV, j1 = k_hi / BKV;

  // global -> register staging of one K/V block: 2 K chunks and one V key pair per thread
  uint4 rk[2], rv[2];
  auto gload = [&](int j) {
    const int kstart = j * BKV;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int item = tid + s * NTH, k = item >> 3, c = item & 7;
      rk[s] = *reinterpret_cast<const uint4*>(qkv + (rbase + kstart + k) * g.ldq + kcol + 8 * c);
    }
    const int kp = tid >> 3, c = tid & 7;
#pragma unroll
    for (int s = 0; s < 2; ++s)
      rv[s] = *reinterpret_cast<const uint4*>(qkv + (rbase + kstart + 2 * kp + s) * g.ldq + vcol + 8 * c);
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int item = tid + s * NTH, k = item >> 3, c = item & 7;
      *reinterpret_cast<uint4*>(&sk[buf][tswz(krow(k), c)]) = rk[s];
    }
    const int kp = tid >> 3, c = tid & 7;
    const bf16* v0 = reinterpret_cast<const bf16*>(&rv[0]);
    const bf16* v1 = reinterpret_cast<const bf16*>(&rv[1]);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int R = drow(8 * c + e);
      // keys 2 kp, 2 kp + 1 of V^T row R: chunk kp / 4, element 2 (kp % 4)
      bf16x2 pr = {v0[e], v1[e]};
      *reinterpret_cast<bf16x2*>(&sv[buf][R * 64 + (((kp >> 2) ^ (R & 7)) << 3) + 2 * (kp & 3)]) = pr;
    }
  };

  const float scale = 0.125f * 1.4426950408889634f;  // 1/sqrt(64) * log2(e)
  float m2[2] = {-1e30f, -1e30f}, lsum[2] = {0.f, 0.f};
  f32x4 o[2][4];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int db = 0; db < 4; ++db) o[qb][db] = f32x4{0.f, 0.f, 0.f, 0.f};

  gload(j0);
  sstore(0);
  __syncthreads();
  for (int j = j0; j <= j1; ++j) {
    const int buf = (j - j0) & 1;
    if (j < j1) gload(j + 1);
    const int kstart = j * BKV;
    const bf16* kt = sk[buf];
    const bf16* vt = sv[buf];
    // S^T = K Q^T for 4 key blocks x 2 query blocks
    f32x4 s[2][4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      bf16x8 kf[2];
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) kf[kk] = *reinterpret_cast<const bf16x8*>(&kt[tswz(16 * kb + (lane & 15), 4 * kk + grp)]);
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        f32x4 a = f32x4{0.f, 0.f, 0.f, 0.f};
        a = mfma16x16x32(kf[0], qf[qb][0], a);
        a = mfma16x16x32(kf[1], qf[qb][1], a);
        s[qb][kb] = a;
      }
    }
    // mask (only blocks touching the causal edge or the window edge need it), online softmax
    const bool full = kstart + BKV - 1 <= q0 && q0 + BQ - 1 - kstart <= g.window;
    bf16x8 pf[2][2], pl[2][2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const int q = q0 + 32 * wave + 16 * qb + (lane & 15);
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float v = s[qb][kb][e] * scale;
          if (!full) {
            const int key = kstart + 32 * (kb >> 1) + 8 * grp + 4 * (kb & 1) + e;
            if (key > q || q - key > g.window) v = -INFINITY;
          }
          s[qb][kb][e] = v;
          mx = fmaxf(mx, v);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mnew = fmaxf(m2[qb], mx);
      const float alpha = exp2f(m2[qb] - mnew);
      m2[qb] = mnew;
      float ps = 0.f;
      float pv[4][4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          pv[kb][e] = exp2f(s[qb][kb][e] - mnew);
          ps += pv[kb][e];
        }
      lsum[qb] = lsum[qb] * alpha + ps;
#pragma unroll
      for (int db = 0; db < 4; ++db) o[qb][db] *= alpha;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bf16 h0 = to_bf16(pv[2 * c][e]), h1 = to_bf16(pv[2 * c + 1][e]);
          pf[qb][c][e] = h0;
          pf[qb][c][4 + e] = h1;
          pl[qb][c][e] = to_bf16(pv[2 * c][e] - (float)h0);
          pl[qb][c][4 + e] = to_bf16(pv[2 * c + 1][e] - (float)h1);
        }
      }
    }
    // O^T += V^T P^T
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const bf16x8 vf = *reinterpret_cast<const bf16x8*>(&vt[tswz(16 * db + (lane & 15), 4 * c + grp)]);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          o[qb][db] = mfma16x16x32(vf, pf[qb][c], o[qb][db]);
          o[qb][db] = mfma16x16x32(vf, pl[qb][c], o[qb][db]);
        }
      }
    if (j < j1) {
      __syncthreads();  // everyone is done with buf ^ 1 (read two blocks ago)
      sstore(buf ^ 1);
      __syncthreads();
    }
  }

  // ---- epilogue: y = O / l, bf16; c_proj dot partial; optional moments
  const int dir = p >> g.pair_shift;
  float mom1[16], mom2[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) mom1[e] = mom2[e] = 0.f;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    float l = lsum[qb];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const float inv = 1.f / l;
    const int q = q0 + 32 * wave + 16 * qb + (lane & 15);
    const long row = rbase + q;
    float yv[16];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int e = 0; e < 4; ++e) yv[4 * db + e] = bf16r(o[qb][db][e] * inv);
    uint4* out = reinterpret_cast<uint4*>(g.y + row * g.ldy + h * HD + 16 * grp);
    out[0] = make_uint4(pack2(yv[0], yv[1]), pack2(yv[2], yv[3]), pack2(yv[4], yv[5]), pack2(yv[6], yv[7]));
    out[1] = make_uint4(pack2(yv[8], yv[9]), pack2(yv[10], yv[11]), pack2(yv[12], yv[13]), pack2(yv[14], yv[15]));
    if (g.upart) {
      const float* br = g.b_proj + (long)dir * g.b_ld + h * HD + 16 * grp;
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) d += yv[e] * bf16r(br[e]);
      d += __shfl_xor(d, 16, 64);
      d += __shfl_xor(d, 32, 64);
      if (grp == 0) g.upart[row * g.upart_ld + h] = d;
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      mom1[e] += yv[e];
      mom2[e] += yv[e] * yv[e];
    }
  }
  if (g.mom) {
    // sum over the wave's 32 queries (lanes sharing lane / 16), then over the 4 waves
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      mom1[e] = group_sum<16>(mom1[e]);
      mom2[e] = group_sum<16>(mom2[e]);
    }
    if ((lane & 15) == 0) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        smom[wave][0][16 * grp + e] = mom1[e];
        smom[wave][1][16 * grp + e] = mom2[e];
      }
    }
    __syncthreads();
    if (tid < 2 * HD) {
      const int k = tid / HD, d = tid % HD;
      const float v = smom[0][k][d] + smom[1][k][d] + smom[2][k][d] + smom[3][k][d];
      g.mom[((((long)p * gridDim.y + h) * gridDim.x + qblk) * 2 + k) * HD + d] = v;
    }
  }
}

// moments[p, h, k, d] = (1 / T) sum over query blocks of the partials (fixed order).
__global__ void moments_reduce_kernel(const float* part, float* out, int nqb, int T, long n) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const long ph = i / (2 * HD), kd = i % (2 * HD);
  float s = 0.f;
  for (int b = 0; b < nqb; ++b) s += part[(ph * nqb + b) * 2 * HD + kd];
  out[i] = s / (float)T;
}

}  // namespace

long attention_moment_partials(int members, int T, int H) { return (long)members * H * (T / BQ) * 2 * HD; }

int attention_launch(const AttnArgs& g, hipStream_t s) {
  if (!g.qkv || !g.y || g.members <= 0 || g.T <= 0 || g.T % BQ || g.H <= 0 || g.window < 0 || g.ldq % 8 ||
      g.ldy % 8 || g.koff % 8 || g.voff % 8 || ((uintptr_t)g.qkv & 15) || ((uintptr_t)g.y & 15))
    return NOISE_EINVAL;
  if (g.upart && (!g.b_proj || g.upart_ld < g.H || g.b_ld < g.H * HD)) return NOISE_EINVAL;
  if (g.mom && !g.mom_out) return NOISE_EINVAL;
  if ((long)g.members > 65535 || g.H > 65535) return NOISE_ENOTSUP;
  hipLaunchKernelGGL(attention_kernel, dim3(g.T / BQ, g.H, g.members), dim3(NTH), 0, s, g);
  NOISE_CHECK_LAUNCH();
  if (g.mom) {
    const long n = (long)g.members * g.H * 2 * HD;
    hipLaunchKernelGGL(moments_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, g.mom, g.mom_out,
                       g.T / BQ, g.T, n);
    NOISE_CHECK_LAUNCH();
  }
  return NOISE_OK;
}
