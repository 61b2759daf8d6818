// Windowed causal attention of the population forward on gfx950 MFMA, with the c_proj input-side
// dot and optional per-head output moments fused into the epilogue.
//
// Reference: `attention` / `window_mask` (utils/model.py:14-31) called from population_loss
// (train/val/eggroll.py:91): softmax(q k^T / sqrt(64)) v, a query at s seeing keys k with
// s - window <= k <= s. In the population forward q, k and v arrive as fp16 written from the fp32 values the
// reference feeds flex (rotary and QK-norm already applied by the QKV kernels): an 11-bit significand, the
// precision class of the TF32 attention the reference runs under set_float32_matmul_precision('high')
// (train/val/eggroll.py:184). The credit reruns (train/val/run.py:594-634) run attention on bf16 q and k, as
// the reference does there; the q/k element type is a template parameter, v is fp16 in both. The clean forward at
// torch's bf16 autocast rounding (the speedrun's scorer, utils/eval.py:44-45) runs it on bf16 q, k and v with the
// probabilities rounded to bf16 for P V, as torch's attention on bf16 operands does.
//
// One workgroup = one (member, head, 128-query block); 4 waves of 32 queries; four workgroups per CU (122
// VGPRs, 34 KiB of LDS each: 4 waves per SIMD hide the LDS and transcendental latencies).
// K/V blocks of 64 keys go through a double-buffered LDS ring filled by direct global -> LDS loads
// (global_load_lds_dwordx4, issued from inline assembly so the compiler adds no LDS-wide waits): while block j
// is computed, block j + 1 lands; one s_waitcnt vmcnt(0) + s_barrier per block (the loads are the only
// vector memory operations in the loop). Nothing passes through registers on the way in.
//   S^T = K Q^T (fp16 or bf16 MFMA, A = K rows, B = Q rows): lane l holds 16 scores of query l % 16. The K rows
//   of each 16-row MFMA block are interleaved at load time (block kb, row r <-> key
//   32 (kb / 2) + 8 (r / 4) + 4 (kb % 2) + r % 4), so the scores' register layout IS the B operand of P V;
//   P never leaves registers.
//   Softmax in fp32: exp2 on the FMA-folded argument; P rounded to fp16 (11-bit significand, the precision
//   class of the reference's TF32 attention). With RMS-normalised q, k (QKN) the scores are bounded and no
//   running maximum is kept; otherwise a lazy running maximum (moves only beyond 2^8 of headroom).
//   O^T += V^T P^T (fp16 MFMA): V stays row-major [key][dim] in LDS and its A fragments (8 consecutive keys
//   of one dim per lane) come from ds_read_b64_tr_b16, which transposes 16-bit elements across each group
//   of 16 lanes: with source lane 4 t + a of group g pointing at key 32 c + 8 g + 4 h + t, dims
//   16 db + 4 a .. + 3, output lane 16 g + 4 a + b receives keys 32 c + 8 g + 4 h + (0..3) of dim
//   16 db + 4 a + b, so block db of the output is dims 16 db .. 16 db + 15 in order. The four lanes of a
//   key row read both 8-byte halves of two adjacent 16-byte chunks (32 bytes), and the rows' chunk pairs are
//   XOR-swizzled so that the rows read together cover the banks once (no conflicts for 16 lanes on 32
//   banks, nor for 32 lanes on 64 banks). Each lane ends with dims 16 db + 4 (lane / 16) .. + 3 of one
//   query for db = 0..3: 8-byte stores, and the c_proj dot y . b_proj over the head's 64 dims is a 4-lane
//   reduction.
#include <type_traits>

#include "attention.h"
#include "common.h"

namespace {

constexpr int HD = 64, BQ = 128, BKV = 64, NWAVE = 4, NTH = NWAVE * 64;
constexpr int DH = BKV * HD * 2 / 1024 / NWAVE;  // K (and V) load instructions per wave and block
constexpr int KB = BKV / 16;       // 16-key MFMA blocks per key block
constexpr int KC = BKV / 32;       // 32-key contraction steps of P V
constexpr float LAZY = 8.f;        // max moves only beyond 2^8 of headroom

typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4_t;

__device__ __forceinline__ f32x4 mfma16x16x32_f16(const f16x8& a, const f16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
// The score MFMA on 8 16-bit q / k elements per lane, fp16 (F16) or bf16.
template <bool F16>
__device__ __forceinline__ f32x4 mfma_qk(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  if constexpr (F16)
    return mfma16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c);
  else
    return mfma16x16x32(a, b, c);
}

// K tile [BKV keys][64 dims] bf16, 128-byte rows, 16-byte chunks XOR-swizzled by row.
__device__ __forceinline__ int kswz(int r, int c) { return r * HD + ((c ^ (r & 7)) << 3); }
// key held by LDS row R of the interleaved K tile (inverse of the row interleave above)
__device__ __forceinline__ int key_of_krow(int R) {
  const int kb = R >> 4, r = R & 15;
  return 32 * (kb >> 1) + 8 * (r >> 2) + 4 * (kb & 1) + (r & 3);
}
// V tile [BKV keys][64 dims] fp16, 128-byte rows in key order; chunk c of row R sits at chunk c ^ vsw(R). A
// transposing read takes one aligned chunk pair of each of the rows 8 g + 4 h + t (t = 0..3) of four groups g;
// with R = 8 g + 4 h + t the pair index is XORed with (t / 2) | ((g ^ t) % 2) << 1, distinct over t for one g
// (16 lanes x 8 bytes over 32 banks) and over (t / 2, g % 2) for one t % 2 (32 lanes x 8 bytes over 64 banks,
// where rows of one parity share a bank half).
__device__ __forceinline__ int vsw(int R) { return 2 * (((R >> 1) & 1) | ((((R >> 3) ^ R) & 1) << 1)); }

// Edge-block masks as lane masks. A lane (query row r = lane % 16, lane group g = lane / 16) holds, for MFMA key block
// kb and element e, the key kstart + 8 g + ko with ko = 32 (kb / 2) + 4 (kb % 2) + e. Against its query
// q0 + 32 wave + 16 qb + r the causal test key <= q reads v >= t with v = r - 8 g (a per-lane constant, -24 .. 15) and
// t = ko + t0, t0 = kstart - q0 - 32 wave - 16 qb (uniform); the window test key >= q - window reads the complement
// v < t + window + 1. The set of lanes with v >= t depends on t alone: LANES_GE[t + 64] holds it as a 64-bit lane
// mask for t in [-64, 80) (all lanes below -24, none above 15), so a block's 16 masks per query block come from two
// scalar loads of 8 consecutive entries (ko = 0..7 and 32..39, t0 clamped to [-64, 40] where the masks saturate) and
// each score costs one v_cndmask on an SGPR-pair condition instead of a compare and a select.
constexpr int LANES_T0 = -64, LANES_N = 144;
struct LaneMaskTable {
  uint64_t m[LANES_N];
};
constexpr LaneMaskTable make_lane_masks() {
  LaneMaskTable t{};
  for (int i = 0; i < LANES_N; ++i) {
    uint64_t m = 0;
    for (int l = 0; l < 64; ++l)
      if ((l & 15) - 8 * (l >> 4) >= i + LANES_T0) m |= uint64_t(1) << l;
    t.m[i] = m;
  }
  return t;
}
__constant__ LaneMaskTable LANES_GE = make_lane_masks();
// v in the lanes whose bit of `lanes` is set, w in the others
__device__ __forceinline__ float select_lanes(float v, float w, uint64_t lanes) {
  float r;
  asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(r) : "v"(w), "v"(v), "s"(lanes));
  return r;
}

__device__ __forceinline__ unsigned pack2(float a, float b) {
  bf16x2 p = {to_bf16(a), to_bf16(b)};
  return *reinterpret_cast<unsigned*>(&p);
}

// QKN: q and k rows are RMS-normalised (||q||, ||k|| <= 8 up to 16-bit rounding), so every score s = q.k / 8
// satisfies |s| <= 8.03 and 2^(s log2(e) / 8) <= 3.1e3: the probabilities need no running maximum (they stay
// normal fp16 numbers and their sums stay far from fp32 overflow), which removes the max reduction, its
// cross-lane shuffles and the rescaling from the loop. Softmax is shift-invariant, so the result is the same.
// F16: q and k are fp16 (bf16 otherwise); they travel as raw 16-bit lanes and only the score MFMA reads their type.
// QL2: q arrives pre-multiplied by log2(e) / 8 (noise_qkv writes it so), so the MFMA returns scores in base-2 units
// and the softmax takes exp2 of them directly: one VALU multiply per score less (with QKN no max is subtracted).
// VB: v is bf16 and the probabilities are rounded to bf16 for P V (the operands of torch's attention on bf16 q, k, v:
// the autocast clean forward); fp16 otherwise.
template <bool QKN, bool F16, bool QL2, bool VB>
__global__ void __launch_bounds__(NTH, 4) attention_kernel(AttnArgs g) {
  static_assert(!QL2 || QKN, "pre-scaled q is the population forward's QK-normalised format");
  static_assert(!VB || !F16, "bf16 v comes with bf16 q and k");
  // element type of v and of the probabilities
  using PT = typename std::conditional<VB, bf16, f16>::type;
  typedef PT pt8 __attribute__((ext_vector_type(8)));
  typedef PT pt4 __attribute__((ext_vector_type(4)));
  auto mfma_pv = [](const pt8& a, const pt8& b, const f32x4& c) {
    if constexpr (VB)
      return mfma16x16x32(a, b, c);
    else
      return mfma16x16x32_f16(a, b, c);
  };
  __shared__ __attribute__((aligned(1024))) bf16 sk[2][BKV * HD];
  __shared__ __attribute__((aligned(1024))) PT sv[2][BKV * HD];
  __shared__ float smom[NWAVE][2][HD];

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), grp = lane >> 4;
  // XCD-aware order. Workgroups reach the 8 XCDs round-robin (workgroup b runs on XCD b % 8), so XCD x takes
  // a contiguous range of logical indices n: the query blocks of one (member, head) run together on one XCD
  // and read its K/V through that XCD's L2 once from HBM. Heavier (later) query blocks first.
  const int nq = g.T / BQ;
  const unsigned G = gridDim.x, b = blockIdx.x, x = b & 7, qg = G >> 3, rg = G & 7;
  const unsigned n = x * qg + min(x, rg) + (b >> 3);
  const int ph = (int)(n / nq), qblk = nq - 1 - (int)(n % nq), h = ph % g.H, p = ph / g.H;
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

  // ---- loads of key block j into ring slot buf: 8 K and 8 V instructions of 1 KiB, 2 + 2 per wave.
  // Instruction d fills LDS rows 8 d .. 8 d + 7; lane L -> row R = 8 d + L / 8, physical chunk L % 8.
  // The block's first key row is a wave-uniform base (SGPRs); each lane's byte offset from it is fixed.
  const int lrow = lane >> 3, lchunk = lane & 7;
  unsigned koffs[DH], voffs[DH];
#pragma unroll
  for (int q = 0; q < DH; ++q) {
    const int R = 8 * (DH * wave + q) + lrow;
    koffs[q] = 2u * (unsigned)(key_of_krow(R) * g.ldq + kcol + 8 * (lchunk ^ (R & 7)));
    voffs[q] = 2u * (unsigned)(R * g.ldq + vcol + 8 * (lchunk ^ vsw(R)));
  }
  auto issue = [&](int j, int buf) {
    const bf16* kv0 = qkv + (rbase + (long)j * BKV) * g.ldq;
#pragma unroll
    for (int q = 0; q < DH; ++q)
      dma_x4_s(kv0, koffs[q], reinterpret_cast<const char*>(sk[buf]) + (DH * wave + q) * 1024);
#pragma unroll
    for (int q = 0; q < DH; ++q)
      dma_x4_s(kv0, voffs[q], reinterpret_cast<const char*>(sv[buf]) + (DH * wave + q) * 1024);
  };

  const float c2 = QL2 ? 1.f : 0.125f * 1.4426950408889634f;  // scores -> log2 units: 1/sqrt(64) * log2(e)
  float mref[2] = {-1e30f, -1e30f};  // running max (score units)
  // O^T accumulators, and the row sums of the fp16 probabilities actually used in P V, accumulated on the
  // MFMA pipe (an all-ones A operand: every element of osum[qb] in lane l is the sum for query l % 16)
  f32x4 o[2][4], osum[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int db = 0; db < 4; ++db) o[qb][db] = f32x4{0.f, 0.f, 0.f, 0.f};

  // per-lane LDS offsets of the MFMA operand reads (the block / step index adds a constant)
  // K block kb: row 16 kb + lane % 16, chunk grp and 4 + grp
  const int kofs0 = kswz(lane & 15, grp), kofs1 = kswz(lane & 15, 4 + grp);
  // V fragment (step c, dim block db, half hh): source row 32 c + 8 grp + 4 hh + t, dims 16 db + 4 a ..
  // (t = (lane % 16) / 4, a = lane % 4), i.e. half a % 2 of chunk 2 db + a / 2; byte offset within the tile,
  // without the 4096 c of the step
  int vofs[2][4];
  {
    const int t = (lane & 15) >> 2, a = lane & 3;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const int R = 8 * grp + 4 * hh + t;
        vofs[hh][db] = R * 128 + 16 * ((2 * db + (a >> 1)) ^ vsw(R)) + 8 * (a & 1);
      }
  }
  const pt8 ones = {(PT)1.f, (PT)1.f, (PT)1.f, (PT)1.f, (PT)1.f, (PT)1.f, (PT)1.f, (PT)1.f};

  // Scores of keys a query may not see become -inf (branch-free): keys after it when the block touches the
  // causal edge, keys more than `window` before it when the block touches the window edge (the lane masks of
  // LANES_GE).
  const float neg_inf = -INFINITY;
  auto mask_edge = [&](f32x4 (&sq)[KB], int t0, bool keep_ge) {
    // masks of t = t0 + ko: entries t0 .. t0 + 7 (kb 0, 1) and t0 + 32 .. t0 + 39 (kb 2, 3)
    const uint64_t* lm = LANES_GE.m + (min(max(t0, LANES_T0), 40) - LANES_T0);
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint64_t m = lm[32 * (kb >> 1) + 4 * (kb & 1) + e];
        sq[kb][e] = keep_ge ? select_lanes(sq[kb][e], neg_inf, m) : select_lanes(neg_inf, sq[kb][e], m);
      }
  };
  auto apply_mask = [&](f32x4 (&s)[2][KB], int kstart, bool causal_edge, bool window_edge) {
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const int t0 = kstart - q0 - 32 * wave - 16 * qb;
      // causal: keep the lanes with v >= t; window: drop the lanes with v >= t + window + 1
      if (causal_edge) mask_edge(s[qb], t0, true);
      if (window_edge) mask_edge(s[qb], t0 + g.window + 1, false);
    }
  };
  // Online softmax of one key block for query block qb of this wave.
  auto softmax = [&](f32x4 (&s)[2][KB], pt8 (&pf)[2][KC], int qb) {
    float mc = 0.f;
    if constexpr (!QKN) {
      float m0 = -INFINITY, m1 = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < KB; kb += 2) {
        m0 = fmaxf(m0, fmaxf(fmaxf(s[qb][kb][0], s[qb][kb][1]), fmaxf(s[qb][kb][2], s[qb][kb][3])));
        m1 = fmaxf(m1, fmaxf(fmaxf(s[qb][kb + 1][0], s[qb][kb + 1][1]), fmaxf(s[qb][kb + 1][2], s[qb][kb + 1][3])));
      }
      float mx = fmaxf(m0, m1);
      mx = max_rows4(mx);
      const bool move = mx * c2 > mref[qb] * c2 + LAZY;
      if (__any(move)) {
        const float mnew = move ? mx : mref[qb];
        const float alpha = __builtin_amdgcn_exp2f((mref[qb] - mnew) * c2);
        mref[qb] = mnew;
        osum[qb] *= alpha;
#pragma unroll
        for (int db = 0; db < 4; ++db) o[qb][db] *= alpha;
      }
      mc = mref[qb] * c2;
    }
#pragma unroll
    for (int c = 0; c < KC; ++c)
#pragma unroll
      for (int hlf = 0; hlf < 2; ++hlf)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          pf[qb][c][4 * hlf + e] =
              (PT)__builtin_amdgcn_exp2f(QL2 ? s[qb][2 * c + hlf][e] : fmaf(s[qb][2 * c + hlf][e], c2, -mc));
  };

  // One key block j from ring slot BUF (a compile-time constant: the slot's LDS base folds into the reads'
  // offsets instead of costing an address VALU operation per read group).
  auto block = [&](int j, auto bufc) {
    constexpr int buf = decltype(bufc)::value;
    // block j + 1 into the slot block j - 1 used (every wave finished it before the last barrier)
    if (j < j1) issue(j + 1, buf ^ 1);
    const int kstart = j * BKV;
    const bf16* kt = sk[buf];
    const char* vt = reinterpret_cast<const char*>(sv[buf]);
    // S^T = K Q^T
    f32x4 s[2][KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const bf16x8 k0 = *reinterpret_cast<const bf16x8*>(&kt[kofs0 + 1024 * kb]);
      const bf16x8 k1 = *reinterpret_cast<const bf16x8*>(&kt[kofs1 + 1024 * kb]);
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        f32x4 a = f32x4{0.f, 0.f, 0.f, 0.f};
        a = mfma_qk<F16>(k0, qf[qb][0], a);
        s[qb][kb] = mfma_qk<F16>(k1, qf[qb][1], a);
      }
    }
    // blocks away from the causal edge and the window edge need no mask
    const bool causal_edge = kstart + BKV - 1 > q0, window_edge = q0 + BQ - 1 - kstart > g.window;
    if (causal_edge || window_edge) apply_mask(s, kstart, causal_edge, window_edge);
    pt8 pf[2][KC];
    softmax(s, pf, 0);
    softmax(s, pf, 1);
    // O^T += V^T P^T
#pragma unroll
    for (int c = 0; c < KC; ++c)
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(vt + 4096 * c + vofs[0][db]));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(vt + 4096 * c + vofs[1][db]));
        const pt4 lo16 = __builtin_bit_cast(pt4, lo), hi16 = __builtin_bit_cast(pt4, hi);
        const pt8 vf = {lo16[0], lo16[1], lo16[2], lo16[3], hi16[0], hi16[1], hi16[2], hi16[3]};
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) o[qb][db] = mfma_pv(vf, pf[qb][c], o[qb][db]);
      }
#pragma unroll
    for (int c = 0; c < KC; ++c)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) osum[qb] = mfma_pv(ones, pf[qb][c], osum[qb]);
    // block j + 1 has landed for this wave (the only vector memory operations in flight are its loads);
    // the barrier makes every wave's part visible and retires slot buf
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  };

  issue(j0, 0);
  __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0) expcnt(0) lgkmcnt(0)
  __syncthreads();
  // blocks j0, j0 + 2, ... use slot 0, the others slot 1: the loop runs two blocks per trip (measured against one
  // block per trip with the slot in a register: config 2 1.635 -> 1.622 ms, attention 107.2 -> 105.7 ms per step)
  for (int j = j0; j <= j1; j += 2) {
    block(j, std::integral_constant<int, 0>{});
    if (j + 1 <= j1) block(j + 1, std::integral_constant<int, 1>{});
  }

  // ---- epilogue: y = O / l, bf16; c_proj dot partial; optional moments
  const int dir = p >> g.pair_shift;
  float mom1[16], mom2[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) mom1[e] = mom2[e] = 0.f;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const float inv = 1.f / osum[qb][0];
    const int q = q0 + 32 * wave + 16 * qb + (lane & 15);
    const long row = rbase + q;
    // yv[4 db + e] is dim 16 db + 4 grp + e
    float yv[16];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int e = 0; e < 4; ++e) yv[4 * db + e] = bf16r(o[qb][db][e] * inv);
    // ordinary stores: the four lane groups fill 32 bytes of each row per instruction, which L2 merges
    bf16* out = g.y + row * g.ldy + h * HD + 4 * grp;
#pragma unroll
    for (int db = 0; db < 4; ++db)
      *reinterpret_cast<uint2*>(out + 16 * db) = make_uint2(pack2(yv[4 * db], yv[4 * db + 1]), pack2(yv[4 * db + 2], yv[4 * db + 3]));
    if (g.upart) {
      const float* br = g.b_proj + (long)dir * g.b_ld + h * HD + 4 * grp;
      float d = 0.f;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int e = 0; e < 4; ++e) d += yv[4 * db + e] * bf16r(br[16 * db + e]);
      d = sum_rows4(d);
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
        smom[wave][0][16 * (e >> 2) + 4 * grp + (e & 3)] = mom1[e];
        smom[wave][1][16 * (e >> 2) + 4 * grp + (e & 3)] = mom2[e];
      }
    }
    __syncthreads();
    if (tid < 2 * HD) {
      const int k = tid / HD, d = tid % HD;
      const float v = smom[0][k][d] + smom[1][k][d] + smom[2][k][d] + smom[3][k][d];
      g.mom[((((long)p * g.H + h) * nq + qblk) * 2 + k) * HD + d] = v;
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
  if (!g.qkv || !g.y || g.members <= 0 || g.T <= 0 || g.T % BQ || g.T % BKV || g.H <= 0 || g.window < 0 ||
      g.ldq % 8 || g.ldy % 8 || g.koff % 8 || g.voff % 8 || ((uintptr_t)g.qkv & 15) || ((uintptr_t)g.y & 15))
    return NOISE_EINVAL;
  if (g.upart && (!g.b_proj || g.upart_ld < g.H || g.b_ld < g.H * HD)) return NOISE_EINVAL;
  if (g.mom && !g.mom_out) return NOISE_EINVAL;
  if (g.qk_format < QK_BF16 || g.qk_format > QK_BF16_V_BF16 ||
      ((g.qk_format == QK_F16_Q_LOG2 || g.qk_format == QK_BF16_V_BF16) && !g.qk_norm))
    return NOISE_EINVAL;
  const long grid = (long)(g.T / BQ) * g.H * g.members;
  if (grid > 0x7fffffffL) return NOISE_ENOTSUP;
  if (g.qk_format == QK_F16_Q_LOG2)
    hipLaunchKernelGGL((attention_kernel<true, true, true, false>), dim3((unsigned)grid), dim3(NTH), 0, s, g);
  else if (g.qk_format == QK_BF16_V_BF16)
    hipLaunchKernelGGL((attention_kernel<true, false, false, true>), dim3((unsigned)grid), dim3(NTH), 0, s, g);
  else if (g.qk_norm && g.qk_format == QK_F16)
    hipLaunchKernelGGL((attention_kernel<true, true, false, false>), dim3((unsigned)grid), dim3(NTH), 0, s, g);
  else if (g.qk_norm)
    hipLaunchKernelGGL((attention_kernel<true, false, false, false>), dim3((unsigned)grid), dim3(NTH), 0, s, g);
  else if (g.qk_format == QK_F16)
    hipLaunchKernelGGL((attention_kernel<false, true, false, false>), dim3((unsigned)grid), dim3(NTH), 0, s, g);
  else
    hipLaunchKernelGGL((attention_kernel<false, false, false, false>), dim3((unsigned)grid), dim3(NTH), 0, s, g);
  NOISE_CHECK_LAUNCH();
  if (g.mom) {
    const long n = (long)g.members * g.H * 2 * HD;
    hipLaunchKernelGGL(moments_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, g.mom, g.mom_out,
                       g.T / BQ, g.T, n);
    NOISE_CHECK_LAUNCH();
  }
  return NOISE_OK;
}
