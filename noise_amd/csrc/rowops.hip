// Row kernels of the population forward: embedding gather + RMSNorm, the per-block residual mix +
// RMSNorm + rank-1 dots, the final RMSNorm feeding the head, and the cross-entropy finalisation.
//
// All of them are HBM-bound: one wave owns one 512-wide row (8 contiguous elements per lane), reads
// it once and writes what the next GEMM needs (bf16 operand, the x.b dots its epilogue adds).
// Rounding points follow the reference under bf16 autocast (train/val/eggroll.py:144): the residual
// stream and norms are fp32, a GEMM operand is the bf16 rounding of its fp32 input, and the rank-1
// GEMV x @ b is bf16 x bf16 with fp32 accumulation, rounded to bf16.
#include "common.h"
#include "gemm.h"
#include "rowops.h"

namespace {

constexpr int D = 512;
constexpr float NORM_EPS = 1.1920928955078125e-07f;  // finfo(float32).eps: F.rms_norm default

struct Row8 {
  float v[8];
};

__device__ __forceinline__ Row8 load8(const float* p) {
  const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
  return Row8{{a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w}};
}
__device__ __forceinline__ void store8(float* p, const Row8& r) {
  *reinterpret_cast<float4*>(p) = make_float4(r.v[0], r.v[1], r.v[2], r.v[3]);
  *reinterpret_cast<float4*>(p + 4) = make_float4(r.v[4], r.v[5], r.v[6], r.v[7]);
}
// RMSNorm of a 512-wide row spread 8 per lane over one wave: x * rsqrt(mean(x^2) + eps), fp32.
__device__ __forceinline__ void rms_norm_row(Row8& r) {
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += r.v[e] * r.v[e];
  ss = group_sum<64>(ss);
  const float s = rsqrtf(ss * (1.f / D) + NORM_EPS);
#pragma unroll
  for (int e = 0; e < 8; ++e) r.v[e] *= s;
}
// A row's 8 values of a lane rounded to bf16 (round to nearest even) as 4 packed pairs: the GEMM operand that
// is stored, and the operand of the rank-1 dots.
struct RowBf {
  unsigned p[4];
};
__device__ __forceinline__ unsigned pack_bf16x2(float a, float b) {
  bf16x2 p = {to_bf16(a), to_bf16(b)};
  return *reinterpret_cast<unsigned*>(&p);
}
__device__ __forceinline__ RowBf pack_row(const Row8& r) {
  return RowBf{{pack_bf16x2(r.v[0], r.v[1]), pack_bf16x2(r.v[2], r.v[3]), pack_bf16x2(r.v[4], r.v[5]),
                pack_bf16x2(r.v[6], r.v[7])}};
}
__device__ __forceinline__ void store_bf(bf16* p, const RowBf& h) { store_stream_x4(p, h.p[0], h.p[1], h.p[2], h.p[3]); }
// bf16(sum_c bf16(h_c) bf16(b_c)) over the row: the autocast rank-1 GEMV, on v_dot2_f32_bf16 (exact bf16
// products, fp32 accumulation).
__device__ __forceinline__ float dot_bf16(const RowBf& h, const Row8& bv) {
  float acc = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, h.p[e]),
                                          __builtin_bit_cast(bf16x2, pack_bf16x2(bv.v[2 * e], bv.v[2 * e + 1])), acc,
                                          false);
  return bf16r(group_sum<64>(acc));
}

// x += the deferred c_proj outputs (`x = x + lowrank(...)`, train/val/eggroll.py:92-93): the same fp32
// operations the GEMM epilogue would have done, v = fma(s bf16(u), a, bf16 dense) then x + v, in order.
// Loads and arithmetic are split: every pending row, partial and vector of a row is loaded before any is
// used, so a row waits for one memory round trip instead of one per deferred residual.
struct PendRow {
  bf16x8 y[MAX_PENDING];
  float uq[MAX_PENDING];  // lane q: partial q
  Row8 a[MAX_PENDING];
};
// a0, a1: the deferred residuals' a vectors of the row's direction
__device__ __forceinline__ void load_pending(PendRow& L, const Pending* pend, int npend, long row, int lane,
                                             const float* a0, const float* a1) {
#pragma unroll
  for (int k = 0; k < MAX_PENDING; ++k) {
    if (k < npend) {
      const Pending& pd = pend[k];
      L.y[k] = *reinterpret_cast<const bf16x8*>(pd.y + row * D + lane * 8);
      L.uq[k] = lane < pd.u_parts ? pd.u[row * pd.u_ld + lane * pd.u_qstride] : 0.f;
      if (k ? a1 : a0) L.a[k] = load8((k ? a1 : a0) + lane * 8);
    }
  }
}
__device__ __forceinline__ void load_pending(PendRow& L, const Pending* pend, int npend, long row, int dir, int lane) {
  load_pending(L, pend, npend, row, lane, npend > 0 ? pend[0].a + (long)dir * D : nullptr,
               npend > 1 ? pend[1].a + (long)dir * D : nullptr);
}
__device__ __forceinline__ void add_pending(Row8& x, const PendRow& L, const Pending* pend, int npend, float s) {
#pragma unroll
  for (int k = 0; k < MAX_PENDING; ++k) {
    if (k < npend) {
      // the sum runs q = 0, 1, ... on the broadcast partials (a fixed order)
      const int parts = pend[k].u_parts;
      float u = 0.f;
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (q < parts) u += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(L.uq[k]), q));
      for (int q = 8; q < parts; ++q) u += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(L.uq[k]), q));
      const float su = s * bf16r(u);
#pragma unroll
      for (int e = 0; e < 8; ++e) x.v[e] = x.v[e] + fmaf(su, L.a[k].v[e], (float)L.y[k][e]);
    }
  }
}

// x0 = norm(W[idx] + s a[:, idx] b) (train/val/eggroll.py:61-63, :74).
// x0 row t of member p (sign s, direction dir): norm(w[tok] + s a[dir, tok] b[dir]) with tok the member's
// token id at position t, 8 values per lane.
__device__ __forceinline__ Row8 embed_finish(const EmbedSrc& e, long tok, int dir, float s, const Row8& b, int lane) {
  const float sa = s * e.a[(long)dir * e.V + tok];
  Row8 w = load8(e.w + tok * D + lane * 8);
#pragma unroll
  for (int k = 0; k < 8; ++k) w.v[k] = w.v[k] + sa * b.v[k];
  rms_norm_row(w);
  return w;
}
__device__ __forceinline__ Row8 embed_row(const EmbedSrc& e, int p, int t, int dir, float s, int lane) {
  const long tok = e.idx[(long)p * e.mstride + t];
  return embed_finish(e, tok, dir, s, load8(e.b + (long)dir * D + lane * 8), lane);
}

__global__ void __launch_bounds__(256) embed_norm_kernel(EmbedNormArgs g) {
  const int lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= g.M) return;
  const int p = (int)(row / g.T), t = (int)(row % g.T), dir = p >> g.pair_shift;
  const EmbedSrc e{g.w, g.a, g.b, g.V, g.idx, 0};
  store8(g.x0 + row * D + lane * 8, embed_row(e, p, t, dir, g.sign[p], lane));
}

// Block entry (train/val/eggroll.py:77-88): x = (l_r + s e_r) x + (l_0 + s e_0) x0; h = norm(x);
// q/k/v input-side dots; the value-embedding gate 2 sigmoid(lowrank(h[:32], ve_gate)).
// One row per wave. FIRST: block 0 (no incoming stream, no deferred residuals, x0 recomputed): fewer live registers,
// twice the waves.
// LATE: the vectors live in LDS and each is read just before its use (compiler barriers keep the reads there), so
// a wave holds only its row's data.
template <bool FIRST, bool LATE = false>
__device__ __forceinline__ void block_entry_row(const BlockEntryArgs& g, long row, int lane, const float* const (&vec)[6]) {
  // vec: the member's vectors for this row (global memory or the workgroup's LDS copy): the embedding's b, b_q,
  // b_k, b_v, and the deferred residuals' a
  const int p = (int)(row / g.T), t = (int)(row % g.T), dir = p >> g.pair_shift;
  // Every load that depends on no other is issued first (the row then waits for its longest chain of dependent
  // loads, the token id before the embedding row, not for the sum of all of them).
  // x0: stored, or recomputed from the embedding (2 KiB gathered from an L2-resident table instead of 2 KiB
  // streamed from HBM); block 0 mixes x0 with itself
  const bool recompute = FIRST || !g.x0;
  long tok = 0;
  Row8 x0, xin, eb, bqkv[3];
  if (recompute) {
    tok = g.emb.idx[(long)p * g.emb.mstride + t];
    if (!LATE) eb = load8(vec[0] + lane * 8);
  } else {
    x0 = load8(g.x0 + row * D + lane * 8);
  }
  if (!FIRST && g.x_in) xin = load8(g.x_in + row * D + lane * 8);
  PendRow pr;
  if (!FIRST) load_pending(pr, g.pend, g.npend, row, lane, LATE ? nullptr : vec[4], LATE ? nullptr : vec[5]);
  if (!LATE) {
#pragma unroll
    for (int k = 0; k < 3; ++k) bqkv[k] = load8(vec[1 + k] + lane * 8);
  }
  const float s = g.sign[p];
  const float lr = g.lambda_r[0] + s * g.eps_r[(long)dir * g.eps_ld];
  const float l0 = g.lambda_0[0] + s * g.eps_0[(long)dir * g.eps_ld];
  if (LATE) asm volatile("" ::: "memory");
  if (recompute) x0 = embed_finish(g.emb, tok, dir, s, LATE ? load8(vec[0] + lane * 8) : eb, lane);
  Row8 x = (!FIRST && g.x_in) ? xin : x0;
  if (LATE) {
    asm volatile("" ::: "memory");
#pragma unroll
    for (int k = 0; k < MAX_PENDING; ++k)
      if (k < g.npend) pr.a[k] = load8(vec[4 + k] + lane * 8);
  }
  if (!FIRST) add_pending(x, pr, g.pend, g.npend, s);
  // one fixed contraction (an fma with the x0 product rounded first), the same in every instance
#pragma unroll
  for (int e = 0; e < 8; ++e) x.v[e] = fmaf(lr, x.v[e], l0 * x0.v[e]);
  store8(g.x_out + row * D + lane * 8, x);
  rms_norm_row(x);
  const RowBf hb = pack_row(x);
  store_bf(g.h + row * D + lane * 8, hb);
  float u[3];
  if (LATE) asm volatile("" ::: "memory");
#pragma unroll
  for (int k = 0; k < 3; ++k) u[k] = dot_bf16(hb, LATE ? load8(vec[1 + k] + lane * 8) : bqkv[k]);
  if (lane == 0) {
    float* ur = g.u_qkv + row * 4;
    ur[0] = u[0], ur[1] = u[1], ur[2] = u[2], ur[3] = s;  // the member's sign rides with the dots
  }
  if (g.gate_w) {
    // gate = 2 sigmoid(lowrank(h[:32], ve_gate)) (train/val/eggroll.py:87) under autocast: bf16 h[:32] against
    // bf16 rows of W_g and bf16 b_g, exact products, fp32 sums, each rounded to bf16. Every lane takes part:
    // lane l forms head l / 8's products over channels 4 c .. 4 c + 3 (c = l % 8) and the dot with b over the
    // same channels; each group of 8 lanes then sums. h[4 c .. 4 c + 3] (two bf16 pairs) comes from lane c / 2,
    // which holds channels 8 (c / 2) .. + 7.
    const int hh = lane >> 3, c = lane & 7, src = (c >> 1) << 2;
    const unsigned w0 = __builtin_amdgcn_ds_bpermute(src, hb.p[0]), w1 = __builtin_amdgcn_ds_bpermute(src, hb.p[1]);
    const unsigned w2 = __builtin_amdgcn_ds_bpermute(src, hb.p[2]), w3 = __builtin_amdgcn_ds_bpermute(src, hb.p[3]);
    const unsigned h01 = (c & 1) ? w2 : w0, h23 = (c & 1) ? w3 : w1;
    const float4 wg = *reinterpret_cast<const float4*>(g.gate_w + hh * 32 + 4 * c);
    const float4 bg = *reinterpret_cast<const float4*>(g.gate_b + (long)dir * 32 + 4 * c);
    auto dot4 = [&](const float4& v) {
      const float d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, h01),
                                                      __builtin_bit_cast(bf16x2, pack_bf16x2(v.x, v.y)), 0.f, false);
      return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, h23),
                                             __builtin_bit_cast(bf16x2, pack_bf16x2(v.z, v.w)), d, false);
    };
    const float z = group_sum<8>(dot4(wg));   // head hh's dense logit in lanes 8 hh .. 8 hh + 7
    const float ub = group_sum<8>(dot4(bg));  // h[:32] . b in every lane
    if (c == 0) {
      const float gl = bf16r(z) + s * bf16r(ub) * g.gate_a[(long)dir * 8 + hh];
      g.gate[row * 8 + hh] = 2.f / (1.f + __expf(-gl));
    }
  }
}
template <bool FIRST>
__global__ void __launch_bounds__(256) block_entry_kernel(BlockEntryArgs g) {
  const int lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= g.M) return;
  const int dir = (int)(row / g.T) >> g.pair_shift;
  const long vo = (long)dir * D;
  const float* const vec[6] = {!g.x0 ? g.emb.b + vo : nullptr, g.b_qkv[0] + vo, g.b_qkv[1] + vo,
                               g.b_qkv[2] + vo, g.npend > 0 ? g.pend[0].a + vo : nullptr,
                               g.npend > 1 ? g.pend[1].a + vo : nullptr};
  block_entry_row<FIRST>(g, row, lane, vec);
}
// GROUP_ROWS rows of one member per workgroup (T % GROUP_ROWS == 0), GROUP_ROWS / 4 per wave in turn: the member's
// vectors (up to six, 12 KiB) are staged in LDS once per workgroup (1.5 KiB per row) instead of being read from L2 by
// every row (12 KiB per row); the result is bit for bit the per-row kernel's. Block 0 takes it too (FIRST, 61 VGPRs):
// entry stage 68.9 → 67.4 ms per step (three runs each, one box).
// Measured (entry stage per step): 8 rows 66.5-66.7 ms, 4 rows 66.6-67.1, 16 rows 69.1-71.4, 32 rows 68.9-70.9.
constexpr int GROUP_ROWS = 8;
template <bool FIRST>
__global__ void __launch_bounds__(256) block_entry_group_kernel(BlockEntryArgs g) {
  __shared__ __attribute__((aligned(16))) float svec[6][D];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // XCD-aware order: workgroup b runs on XCD b % 8, which takes a contiguous range of row groups (a member's groups
  // then share one XCD's L2 for its vectors): entry stage 68.1 -> 66.6 ms per step (three runs each, one box)
  const unsigned G = gridDim.x, b = blockIdx.x, x = b & 7, qg = G >> 3, rg = G & 7;
  const long row0 = (long)(x * qg + min(x, rg) + (b >> 3)) * GROUP_ROWS;
  const int dir = (int)(row0 / g.T) >> g.pair_shift;
  const long vo = (long)dir * D;
  const float* src[6] = {!g.x0 ? g.emb.b : nullptr, g.b_qkv[0], g.b_qkv[1], g.b_qkv[2],
                         g.npend > 0 ? g.pend[0].a : nullptr, g.npend > 1 ? g.pend[1].a : nullptr};
  for (int i = threadIdx.x; i < 6 * (D / 4); i += 256) {
    const int v = i / (D / 4), q = i - v * (D / 4);
    if (src[v]) *reinterpret_cast<float4*>(&svec[v][4 * q]) = *reinterpret_cast<const float4*>(src[v] + vo + 4 * q);
  }
  __syncthreads();
  const float* const vec[6] = {svec[0], svec[1], svec[2], svec[3], svec[4], svec[5]};
  // one row at a time; the compiler barrier keeps each row's vector reads from LDS inside its iteration (hoisted, the
  // six vectors would stay live in registers across the loop)
#pragma unroll 1
  for (int k = 0; k < GROUP_ROWS / 4; ++k) {
    asm volatile("" ::: "memory");
    block_entry_row<FIRST, true>(g, row0 + wave * (GROUP_ROWS / 4) + k, lane, vec);
  }
}

// h = norm(x) as the bf16 operand of the next GEMM, plus its input-side dot (MLP entry,
// train/val/eggroll.py:93).
__global__ void __launch_bounds__(256) norm_dot_kernel(NormDotArgs g) {
  const int lane = threadIdx.x & 63;
  // XCD-aware order (as the block entry's): a member's rows share one XCD's L2 for its b and a vectors (MLP entries
  // 34.5 -> 34.0 ms per step, three runs each, one box)
  const unsigned G = gridDim.x, b = blockIdx.x, xcd = b & 7, qg = G >> 3, rg = G & 7;
  const long row = (long)(xcd * qg + min(xcd, rg) + (b >> 3)) * 4 + (threadIdx.x >> 6);
  if (row >= g.M) return;
  const int p = (int)(row / g.T), dir = p >> g.pair_shift;
  Row8 x = load8(g.x + row * D + lane * 8);
  PendRow pr;
  load_pending(pr, g.pend, g.npend, row, dir, lane);
  const Row8 bv = load8(g.b + (long)dir * D + lane * 8);
  if (g.npend) add_pending(x, pr, g.pend, g.npend, g.sign[p]);
  rms_norm_row(x);
  const RowBf hb = pack_row(x);
  store_bf(g.h + row * D + lane * 8, hb);
  const float u = dot_bf16(hb, bv);
  if (lane == 0) g.u[row] = u;
}

// Final norm feeding the head (train/val/eggroll.py:94-99). Three operand formats (HeadNormArgs::fp32_head):
//   2: fp16(h) (|h| <= sqrt(512) after the norm, so fp16's range holds it; 11 significant bits) for the fp16
//      head GEMM, which forms h W_hi + h W_lo against a 22-bit split of the weight (with the gain folded into the
//      weight, so the operand carries none); the dot (h gain).b is fp32;
//   1: the bf16 split [hi | lo] of h gain (hi = bf16(h), lo = bf16(h - hi)); the head GEMM forms
//      hi W_hi + hi W_lo + lo W_hi from them (its a_fold), ~2^-16 relative; the dot h.b is fp32;
//   0: bf16(h gain) (the bf16 head), the dot following autocast.
// One row of the head's norm: x (plus the deferred residuals) and RMSNorm, without the gain; 8 values per lane.
__device__ __forceinline__ Row8 head_row(const HeadNormArgs& g, long row, int lane, int p, int dir) {
  Row8 x;
  if (g.x_bf16) {
    const bf16x8 xv = *reinterpret_cast<const bf16x8*>(static_cast<const bf16*>(g.x) + row * D + lane * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) x.v[e] = (float)xv[e];
  } else {
    x = load8(static_cast<const float*>(g.x) + row * D + lane * 8);
    PendRow pr;
    load_pending(pr, g.pend, g.npend, row, dir, lane);
    if (g.npend) add_pending(x, pr, g.pend, g.npend, g.sign[p]);
  }
  rms_norm_row(x);
  return x;
}
__device__ __forceinline__ Row8 with_gain(const HeadNormArgs& g, Row8 x, int lane) {
  if (g.gain) {
    const Row8 gv = load8(g.gain + lane * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) x.v[e] *= gv.v[e];
  }
  return x;
}
__device__ __forceinline__ u32x4 pack_row_x4(const Row8& r) {
  bf16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = to_bf16(r.v[e]);
  return __builtin_bit_cast(u32x4, o);
}
__device__ __forceinline__ u32x4 pack_row_f16_x4(const Row8& r) {
  _Float16 __attribute__((ext_vector_type(8))) o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = (_Float16)r.v[e];
  return __builtin_bit_cast(u32x4, o);
}
// fp32 dot of the lane's 8 values with the row's b, summed over the wave
__device__ __forceinline__ float dot_f32_row(const Row8& x, const float* b, int lane) {
  const Row8 bv = load8(b + lane * 8);
  float acc = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) acc += x.v[e] * bv.v[e];
  return group_sum<64>(acc);
}
// The row's operand units (unit 0 in op[0]; [hi | lo]: unit 64 + lane in op[1]) and its dot with b.
__device__ __forceinline__ float head_operand(const HeadNormArgs& g, const Row8& h, int lane, int dir, u32x4 (&op)[2]) {
  const float* b = g.b + (long)dir * D;
  if (g.fp32_head == 2) {
    op[0] = pack_row_f16_x4(h);
    return dot_f32_row(with_gain(g, h, lane), b, lane);
  }
  const Row8 x = with_gain(g, h, lane);
  if (g.fp32_head) {
    Row8 lo;
#pragma unroll
    for (int e = 0; e < 8; ++e) lo.v[e] = x.v[e] - bf16r(x.v[e]);
    op[0] = pack_row_x4(x);
    op[1] = pack_row_x4(lo);
    return dot_f32_row(x, b, lane);
  }
  const RowBf hb = pack_row(x);
  op[0] = u32x4{hb.p[0], hb.p[1], hb.p[2], hb.p[3]};
  return dot_bf16(hb, load8(b + lane * 8));
}

__global__ void __launch_bounds__(256) head_norm_kernel(HeadNormArgs g) {
  const int lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= g.M) return;
  const int p = (int)(row / g.T), dir = p >> g.pair_shift;
  u32x4 op[2];
  const float u = head_operand(g, head_row(g, row, lane, p, dir), lane, dir, op);
  const int W = g.fp32_head == 1 ? 2 * D : D;
  bf16* o = g.h + row * W + lane * 8;
  store_stream_x4(o, op[0]);
  if (g.fp32_head == 1) store_stream_x4(o + D, op[1]);
  if (lane == 0) g.u[row] = u;
}

// The same rows written in TILE16 (the tile GEMM's whole-line operand layout): element (r, c) of the [M, W]
// operand (W = 1024 for [hi | lo], 512 otherwise) at (r / 16) 16 W + (c / 32) 512 + 8 q + c % 8 with
// q = 4 (r % 16) + ((c % 32) / 8 ^ ((r % 16) / 2) % 4). A workgroup of 16 waves normalises one 16-row group, a row
// per wave as above, into LDS, then writes the group's 16 W 16-bit values (one contiguous 32 or 16 KiB run) as
// whole lines: row by row, four lanes would fill half a line each and the stores would scatter over 16 or 32 tiles.
__global__ void __launch_bounds__(1024) head_norm_tiled_kernel(HeadNormArgs g) {
  constexpr int UNITS = 2 * D / 8;           // 16-byte units per row of [hi | lo]
  // + 4 units: consecutive rows start 16 banks apart, so the 4 rows of one 16-lane read pass cover all 64 banks
  __shared__ u32x4 rows16[16][UNITS + 4];
  const int lane = threadIdx.x & 63, r16 = threadIdx.x >> 6;
  const long r0 = (long)blockIdx.x * 16, row = r0 + r16;
  const int W = g.fp32_head == 1 ? 2 * D : D, units = W / 8;
  const int p = (int)(row / g.T), dir = p >> g.pair_shift;
  u32x4 op[2];
  const float u = head_operand(g, head_row(g, row, lane, p, dir), lane, dir, op);
  rows16[r16][lane] = op[0];
  if (g.fp32_head == 1) rows16[r16][64 + lane] = op[1];
  if (lane == 0) g.u[row] = u;
  __syncthreads();
  // unit n of the group: tile n / 64, q = n % 64 -> row q / 4, 8-column chunk (q % 4) ^ ((q / 8) % 4) of the tile
  bf16* out = g.h + r0 * W;
  for (int n = threadIdx.x; n < 16 * units; n += 1024) {
    const int q = n & 63, rq = q >> 2, ch = (q & 3) ^ ((rq >> 1) & 3);
    store_stream_x4(out + 8L * n, rows16[rq][4 * (n >> 6) + ch]);
  }
}

// Cross-entropy of the soft-capped logits: row r's loss is log(sum_j part[r, j]) - z[r, target]. Sixteen lanes
// share a row: lane j of the group loads partials 4 j .. 4 j + 3, + 64, ... (parts a multiple of 4), so a wave
// reads four whole 256-byte runs per instruction.
__device__ __forceinline__ float ce_row_loss(const CeFinalizeArgs& g, long row, int gl) {
  float s = 0.f;
  for (int c = 4 * gl; c < g.parts; c += 64) {
    const float4 v = *reinterpret_cast<const float4*>(g.part + row * g.parts + c);
    s += (v.x + v.y) + (v.z + v.w);
  }
  s = group_sum<16>(s);
  return __logf(s) - g.tgt[row];
}
// ignore_index = -1 (utils/model.py:206-207)
__device__ __forceinline__ bool ce_row_valid(const CeFinalizeArgs& g, long row) {
  return g.targets[(row / g.T) * g.tgt_mstride + row % g.T] != -1;
}

// CE_MEMBER_MEAN (population_loss, train/val/eggroll.py:101-102): workgroup p sums member p's T rows.
// CE_NONE / CE_SUM / CE_MEAN (F.cross_entropy's reductions with ignore_index = -1, utils/model.py:205-208):
// per row; or one workgroup sums every valid row. Each 16-lane group sums a fixed stride of rows, then the 16
// group sums add in a fixed order: the result does not depend on scheduling.
__global__ void __launch_bounds__(256) ce_finalize_kernel(CeFinalizeArgs g) {
  __shared__ float red[16], cnt[16];
  const int tid = threadIdx.x, gl = tid & 15, gid = tid >> 4;
  if (g.reduction == CE_NONE) {
    const long row = (long)blockIdx.x * 16 + gid;
    if (row < (long)g.members * g.T) {
      const float l = ce_row_loss(g, row, gl);
      if (gl == 0) g.loss[row] = ce_row_valid(g, row) ? l : 0.f;
    }
    return;
  }
  const bool all = g.reduction != CE_MEMBER_MEAN;
  const long r0 = all ? 0 : (long)blockIdx.x * g.T, n = all ? (long)g.members * g.T : g.T;
  float acc = 0.f, c = 0.f;
  for (long i = gid; i < n; i += 16) {
    const long row = r0 + i;
    const float l = ce_row_loss(g, row, gl);
    if (!all || ce_row_valid(g, row)) {
      acc += l;
      c += 1.f;
    }
  }
  if (gl == 0) {
    red[gid] = acc;
    cnt[gid] = c;
  }
  __syncthreads();
  if (tid == 0) {
    float t = 0.f, k = 0.f;
    for (int q = 0; q < 16; ++q) {
      t += red[q];
      k += cnt[q];
    }
    if (!all) g.loss[blockIdx.x] = t / (float)g.T;
    else g.loss[0] = g.reduction == CE_SUM ? t : t / k;  // 0 / 0 = NaN, as torch's mean
  }
}

// fp32 -> bf16 (round to nearest even); with split != 0 also writes [hi | lo | hi] rows of width
// `cols` (the fp32 head operand): out row r = [bf16(w_r) | bf16(w_r - bf16(w_r)) | bf16(w_r)].
__global__ void __launch_bounds__(256) cast_kernel(const float* __restrict__ in, bf16* __restrict__ out, long n, int cols,
                                                   int split) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = in[i];
  const bf16 hi = to_bf16(v);
  if (!split) {
    out[i] = hi;
    return;
  }
  const long r = i / cols, c = i % cols;
  bf16* o = out + r * 3 * cols + c;
  o[0] = hi;
  o[cols] = to_bf16(v - (float)hi);
  o[2 * cols] = hi;
}

int grid_rows(long M) { return (int)((M + 3) / 4); }

// HBM calibration: one wave per row reads in_kib KiB of the row's source and writes out_kib KiB, with the row
// kernels' 16-byte vector loads and stores (ordinary stores for the full lines). The written values are a function
// of the read ones, so no load is dead.
template <int IN, int OUT>
__global__ void __launch_bounds__(256) hbm_stream_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                         long rows) {
  const int lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const u32x4* s = src + row * IN * 64 + lane;
  u32x4 v[IN];
#pragma unroll
  for (int k = 0; k < IN; ++k) v[k] = s[k * 64];  // every load issued before any is used
  u32x4 acc = v[0];
#pragma unroll
  for (int k = 1; k < IN; ++k) acc ^= v[k];
  u32x4* d = dst + row * OUT * 64 + lane;
#pragma unroll
  for (int k = 0; k < OUT; ++k) d[k * 64] = acc + u32x4{(unsigned)k, 0u, 0u, 0u};
}
template <int IN>
int hbm_stream_out(const void* src, void* dst, int out_kib, long rows, hipStream_t s) {
  const dim3 grid((unsigned)((rows + 3) / 4));
  const u32x4* a = static_cast<const u32x4*>(src);
  u32x4* b = static_cast<u32x4*>(dst);
  switch (out_kib) {
    case 1: hipLaunchKernelGGL((hbm_stream_kernel<IN, 1>), grid, dim3(256), 0, s, a, b, rows); break;
    case 2: hipLaunchKernelGGL((hbm_stream_kernel<IN, 2>), grid, dim3(256), 0, s, a, b, rows); break;
    case 3: hipLaunchKernelGGL((hbm_stream_kernel<IN, 3>), grid, dim3(256), 0, s, a, b, rows); break;
    default: hipLaunchKernelGGL((hbm_stream_kernel<IN, 4>), grid, dim3(256), 0, s, a, b, rows); break;
  }
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}

bool bad_pending(const Pending* pend, int npend) {
  if (npend < 0 || npend > MAX_PENDING) return true;
  for (int k = 0; k < npend; ++k) {
    const Pending& pd = pend[k];
    if (!pd.y || !pd.u || !pd.a || pd.u_parts < 1 || pd.u_parts > 64 || pd.u_ld < 1 || pd.u_qstride < 1 ||
        (((uintptr_t)pd.y | (uintptr_t)pd.a) & 15))
      return true;
  }
  return false;
}

}  // namespace

int hbm_stream_launch(const void* src, int in_kib, void* dst, int out_kib, long rows, hipStream_t s) {
  if (!src || !dst || in_kib < 1 || in_kib > 4 || out_kib < 1 || out_kib > 4 || rows <= 0 || (rows + 3) / 4 > 0x7fffffffL ||
      (((uintptr_t)src | (uintptr_t)dst) & 15))
    return NOISE_EINVAL;
  switch (in_kib) {
    case 1: return hbm_stream_out<1>(src, dst, out_kib, rows, s);
    case 2: return hbm_stream_out<2>(src, dst, out_kib, rows, s);
    case 3: return hbm_stream_out<3>(src, dst, out_kib, rows, s);
    default: return hbm_stream_out<4>(src, dst, out_kib, rows, s);
  }
}

int embed_norm_launch(const EmbedNormArgs& g, hipStream_t s) {
  if (g.M <= 0 || g.T <= 0 || !g.w || !g.a || !g.b || !g.sign || !g.idx || !g.x0 || g.V <= 0) return NOISE_EINVAL;
  hipLaunchKernelGGL(embed_norm_kernel, dim3(grid_rows(g.M)), dim3(256), 0, s, g);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}

int block_entry_launch(const BlockEntryArgs& g, hipStream_t s) {
  if (!g.x0 && (!g.emb.w || !g.emb.a || !g.emb.b || !g.emb.idx || g.emb.V <= 0)) return NOISE_EINVAL;
  if (g.M <= 0 || g.T <= 0 || !g.x_out || !g.h || !g.u_qkv || !g.sign || !g.eps_r || !g.eps_0 ||
      !g.lambda_r || !g.lambda_0 || !g.b_qkv[0] || !g.b_qkv[1] || !g.b_qkv[2])
    return NOISE_EINVAL;
  if (g.gate_w && (!g.gate_a || !g.gate_b || !g.gate || (((uintptr_t)g.gate_w | (uintptr_t)g.gate_b) & 15)))
    return NOISE_EINVAL;
  if (bad_pending(g.pend, g.npend)) return NOISE_EINVAL;
  const bool first = !g.x_in && !g.x0 && !g.npend, grouped = g.T % GROUP_ROWS == 0 && g.M % GROUP_ROWS == 0;
  if (first && grouped)
    hipLaunchKernelGGL(block_entry_group_kernel<true>, dim3((unsigned)(g.M / GROUP_ROWS)), dim3(256), 0, s, g);
  else if (first)
    hipLaunchKernelGGL(block_entry_kernel<true>, dim3(grid_rows(g.M)), dim3(256), 0, s, g);
  else if (grouped)
    hipLaunchKernelGGL(block_entry_group_kernel<false>, dim3((unsigned)(g.M / GROUP_ROWS)), dim3(256), 0, s, g);
  else
    hipLaunchKernelGGL(block_entry_kernel<false>, dim3(grid_rows(g.M)), dim3(256), 0, s, g);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}

int norm_dot_launch(const NormDotArgs& g, hipStream_t s) {
  if (g.M <= 0 || g.T <= 0 || !g.x || !g.h || !g.b || !g.u || !g.sign || bad_pending(g.pend, g.npend))
    return NOISE_EINVAL;
  hipLaunchKernelGGL(norm_dot_kernel, dim3(grid_rows(g.M)), dim3(256), 0, s, g);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}

int head_norm_launch(const HeadNormArgs& g, hipStream_t s) {
  if (g.M <= 0 || g.T <= 0 || !g.x || !g.h || !g.b || !g.u || !g.sign || bad_pending(g.pend, g.npend) ||
      (g.x_bf16 && g.npend) || g.fp32_head < 0 || g.fp32_head > 2)
    return NOISE_EINVAL;
  if (g.tiled) {
    if (g.M % 16) return NOISE_EINVAL;
    hipLaunchKernelGGL(head_norm_tiled_kernel, dim3((unsigned)(g.M / 16)), dim3(1024), 0, s, g);
  } else {
    hipLaunchKernelGGL(head_norm_kernel, dim3(grid_rows(g.M)), dim3(256), 0, s, g);
  }
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}

int ce_finalize_launch(const CeFinalizeArgs& g, hipStream_t s) {
  if (g.members <= 0 || g.T <= 0 || g.parts <= 0 || !g.part || !g.tgt || !g.loss || g.reduction < CE_MEMBER_MEAN ||
      g.reduction > CE_MEAN || (g.reduction != CE_MEMBER_MEAN && !g.targets))
    return NOISE_EINVAL;
  const long rows = (long)g.members * g.T;
  if (g.parts % 4 || ((uintptr_t)g.part & 15)) return NOISE_ENOTSUP;
  const long grid = g.reduction == CE_MEMBER_MEAN ? g.members : g.reduction == CE_NONE ? (rows + 15) / 16 : 1;
  if (grid > 0x7fffffffL) return NOISE_ENOTSUP;
  hipLaunchKernelGGL(ce_finalize_kernel, dim3((unsigned)grid), dim3(256), 0, s, g);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}

int cast_launch(const float* in, bf16* out, long n, int cols, int split, hipStream_t s) {
  if (!in || !out || n <= 0 || (split && (cols <= 0 || n % cols))) return NOISE_EINVAL;
  hipLaunchKernelGGL(cast_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, in, out, n, cols, split);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}

// ---- rank-1 GEMV for a bf16 activation (config-1 MLP entry): u[row] = bf16(x.bf16(b_dir)).
namespace {
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
