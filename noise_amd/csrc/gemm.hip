// Low-rank-perturbed GEMM on gfx950 bf16 MFMA: out = x W^T + s_p (x.b_p) a_p^T per member p.
//
// Reference: `lowrank` (train/val/eggroll.py:56-58) under bf16 autocast (:144). The dense part runs
// on v_mfma_f32_16x16x32_bf16; the rank-1 part never touches the MFMA pipe: the input-side dot
// u = bf16(x.b_p) arrives per row (computed by the kernel that produced x) and the epilogue adds
// (s_p u) a_p[col] in fp32 on top of the bf16-rounded GEMM output, exactly the autocast rounding
// points (bf16 GEMM output, fp32 correction).
//
// Layouts (row-major, K contiguous): A [M, K] bf16 with M = members x T rows (member p owns rows
// p*T .. p*T+T-1); W [N, K] bf16 in the reference's nn.Linear orientation [out, in].
//
// Schedule. The kernel is persistent: one workgroup per CU walks a list of BM x BN output tiles.
// Hardware deals workgroups round-robin over the 8 XCDs, so workgroup b serves XCD b % 8; each XCD
// owns one contiguous range of tiles (N fastest), which keeps the x rows shared by neighbouring
// tiles in that XCD's L2.
//
// Main loop. K is walked in 32-deep MFMA steps through a STAGES-deep LDS ring of BK-deep stages,
// filled by direct global->LDS loads (global_load_lds_dwordx4, no VGPR staging). The refill of a
// stage is issued right after the barrier that retires it, so STAGES - 1 stages are in flight while
// one feeds the MFMAs. MFMA operands are double-buffered in registers: step t + 1's W fragments and
// x fragments are read from LDS while step t's MFMAs run (x fragment i right after row i's MFMAs,
// when its register is dead), so the MFMA pipe never waits on LDS latency. Rows of BK bf16 are
// stored with their 16-byte chunks XOR-swizzled per 128-byte LDS line: the ds_read_b128 operand
// fetches (16 consecutive rows, one chunk) are bank-conflict free.
//
// Transposed product. The MFMA computes C^T = W x^T: W rows are the MFMA "A" operand and x rows the
// "B" operand, so each lane ends up holding one token row and CW = 4 x FN output columns. LDS row
// R of the W tile holds W row band + (r / 4) * CW + 4 j + r % 4 (band = R - R % WN, j = (R % WN) / 16,
// r = R % 16), so MFMA block j reads 16 consecutive LDS rows and each lane's CW columns are
// contiguous: the epilogue stores 16-byte vectors from registers and reduces row dots over the 4
// lanes that share a row.
//
// Epilogue overlap. When a tile's last MFMAs are issued, the workgroup issues the global loads of the
// next tile's epilogue vectors (a_p, b_next, x.b partial sums, sign) and the DMA of the next tile's
// first STAGES stages, then runs this tile's epilogue from LDS-staged vectors; the stores drain
// while the next tile's operands land.
#include <algorithm>

#include <type_traits>

#include "common.h"
#include "gemm.h"

namespace {

typedef _Float16 h16x8 __attribute__((ext_vector_type(8)));

template <int BM, int BN, int BK, int STAGES, int WGM, int WGN>
struct Cfg {
  static constexpr int NW = WGM * WGN, NTH = NW * 64;
  static constexpr int WM = BM / WGM, WN = BN / WGN;
  static constexpr int FM = WM / 16, FN = WN / 16;
  static constexpr int CW = 4 * FN;              // contiguous output columns per lane
  static constexpr int CPR = BK / 8;             // 16-byte chunks per LDS row
  static constexpr int RPL = 8 / CPR;            // rows per 128-byte LDS line
  static constexpr int ROWS_PER_DMA = 64 / CPR;  // rows one wave-wide 1 KiB DMA fills
  static constexpr int LA = BM / ROWS_PER_DMA / NW;  // DMA instructions per wave per stage (x tile)
  static constexpr int LB = BN / ROWS_PER_DMA / NW;  // (W tile)
  static constexpr int L = LA + LB;
  static constexpr int STAGE = (BM + BN) * BK;   // bf16 elements per LDS stage
  static constexpr int UGROUPS = NTH / BM;       // threads summing one row's x.b partials
  static_assert(BK == 32 || BK == 64, "BK must be 32 or 64");
  static_assert(WM % 16 == 0 && WN % 16 == 0 && FN % 2 == 0, "wave tile must be a multiple of 16 x 32");
  static_assert(LA * ROWS_PER_DMA * NW == BM && LB * ROWS_PER_DMA * NW == BN, "DMA must tile evenly");
  static_assert((STAGES - 1) * L <= 63, "vmcnt range");
  static_assert(STAGES >= 2 && STAGES <= 4, "wait_stage handles up to 3 stages ahead");
  static_assert(NTH % BM == 0 && NTH >= BN / 2, "epilogue vector staging");
};

// Element offset of (row r, logical 16-byte chunk c) in a swizzled LDS tile with BK-wide rows.
template <int BK>
__device__ __forceinline__ int swz(int r, int c) {
  constexpr int CPR = BK / 8, RPL = 8 / CPR;
  return r * BK + ((c ^ ((r / RPL) % CPR)) << 3);
}

// s_waitcnt with vmcnt(n) (n <= 63), lgkmcnt(0), expcnt untouched.
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(N >= 0 && N <= 63, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | ((N >> 4) << 14));
}
// Wait until every DMA older than the last `ahead` stages (L instructions each) has landed. Vector
// memory operations complete in issue order, so counting only the unconditionally issued DMA of
// later stages is safe: any other operation issued after them only makes the wait stricter.
template <int L, int MAXAHEAD>
__device__ __forceinline__ void wait_stage(int ahead) {
  if constexpr (MAXAHEAD >= 3) {
    if (ahead >= 3) { wait_vm_lgkm0<3 * L>(); return; }
  }
  if constexpr (MAXAHEAD >= 2) {
    if (ahead >= 2) { wait_vm_lgkm0<2 * L>(); return; }
  }
  if constexpr (MAXAHEAD >= 1) {
    if (ahead >= 1) { wait_vm_lgkm0<L>(); return; }
  }
  wait_vm_lgkm0<0>();
}

// Epilogue stores of the tile GEMM are ordinary (write-back) stores: a lane's 16-byte stores cover half of
// each 128-byte line per instruction, and as non-temporal stores those halves reach memory separately
// (measured: twice the written bytes in WRITE_SIZE); through L2 they merge into whole lines.
__device__ __forceinline__ void store_x4(void* p, unsigned a, unsigned b, unsigned c, unsigned d) {
  *reinterpret_cast<uint4*>(p) = make_uint4(a, b, c, d);
}
__device__ __forceinline__ void store_f4(void* p, float a, float b, float c, float d) {
  *reinterpret_cast<float4*>(p) = make_float4(a, b, c, d);
}

__device__ __forceinline__ unsigned pack_bf16(float a, float b) {
  bf16x2 p = {to_bf16(a), to_bf16(b)};
  return *reinterpret_cast<unsigned*>(&p);
}
// fp16 pair (round to nearest even) of two fp32 values: q, k and v enter attention with an 11-bit significand,
// the precision class of the reference's TF32 flex attention on fp32 operands (|v| must stay below 65504)
__device__ __forceinline__ unsigned pack_f16(float a, float b) {
  _Float16 __attribute__((ext_vector_type(2))) p = {(_Float16)a, (_Float16)b};
  return *reinterpret_cast<unsigned*>(&p);
}

template <int BM, int BN, int BK, int STAGES, int WGM, int WGN, int OCC, int EPI>
__global__ void __launch_bounds__(WGM * WGN * 64, WGM * WGN * OCC / 4)
lowrank_gemm_kernel(const LowrankGemmArgs g) {
  using C = Cfg<BM, BN, BK, STAGES, WGM, WGN>;
  constexpr int FM = C::FM, FN = C::FN, WM = C::WM, WN = C::WN, CW = C::CW;
  constexpr int SUB = BK / 32;
  // the head's cross-entropy epilogue, on bf16 or (F16) fp16 operands
  constexpr bool CE = EPI == EPI_CE || EPI == EPI_CE_F16, F16 = EPI == EPI_CE_F16;
  __shared__ __attribute__((aligned(1024))) bf16 smem[STAGES * C::STAGE];
  __shared__ __attribute__((aligned(16))) float ep_a[BN];             // a_p over the tile's columns (F16: a_p scaled)
  __shared__ __attribute__((aligned(16))) float ep_m[F16 ? BN : 4];   // F16: the exp argument's factor per column
  __shared__ float ep_u[C::UGROUPS][BM];                               // partial sums of x.b per row
  __shared__ float ep_sign;
  __shared__ int ep_t[CE ? BM : 1];                                    // the head: target token per row (-1: none)

  // (a wave index made uniform with readfirstlane measured slower here: config 1 2.20 -> 2.50 ms, head +6%)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int tiles_m = (g.M + BM - 1) / BM, tiles_n = g.N / BN, ntiles = tiles_m * tiles_n;
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3, nslots = gridDim.x >> 3;
  const int t_lo = (int)((long)xcd * ntiles / 8), t_hi = (int)((long)(xcd + 1) * ntiles / 8);
  const int KT = g.K / BK, KS = KT * SUB;

  // ---- per-tile DMA sources. Instruction d of this wave fills LDS rows
  // R = (wave * L + d) * ROWS_PER_DMA + lane / CPR at physical chunk lane % CPR, i.e. logical k chunk
  // (lane % CPR) ^ ((R / RPL) % CPR).
  const int lrow = lane / C::CPR;
  long a_src[C::LA];
  const bf16* b_src[C::LB];
  auto set_sources = [&](int m0, int n0) {
#pragma unroll
    for (int d = 0; d < C::LA; ++d) {
      if (g.a_tiled) {
        // the 16 rows of this instruction are one 1 KiB TILE16 tile per 32-deep stage
        const int G = min(m0 + (wave * C::LA + d) * C::ROWS_PER_DMA, g.M - 16) >> 4;
        a_src[d] = (long)G * 16 * g.lda + 8 * lane;
      } else {
        const int r = (wave * C::LA + d) * C::ROWS_PER_DMA + lrow;
        const int c = (lane % C::CPR) ^ ((r / C::RPL) % C::CPR);
        const int row = min(m0 + r, g.M - 1);
        a_src[d] = (long)(row / g.T) * g.a_mstride + (long)(row % g.T) * g.lda + c * 8;
      }
    }
#pragma unroll
    for (int d = 0; d < C::LB; ++d) {
      if (g.w_tiled) {
        // WTILE: these 16 LDS rows are one 1 KiB block per 32-deep stage, already in LDS order
        b_src[d] = g.W + (long)((n0 >> 4) + wave * C::LB + d) * KT * 512 + 8 * lane;
        continue;
      }
      const int R = (wave * C::LB + d) * C::ROWS_PER_DMA + lrow;
      const int c = (lane % C::CPR) ^ ((R / C::RPL) % C::CPR);
      const int loc = R % WN, r = loc & 15;
      const int n = n0 + (R - loc) + (r >> 2) * CW + (loc >> 4) * 4 + (r & 3);
      b_src[d] = g.W + (long)n * g.ldw + c * 8;
    }
  };
  // elements one stage advances the A and W sources by: BK columns, or one 512-element block per 32 columns for
  // a TILE16 A and a WTILE W (both require BK = 32)
  const int a_step = g.a_tiled ? 16 * BK : BK, w_step = g.w_tiled ? 512 : BK;
  auto issue = [&](int kt, int buf) {
    bf16* sx = smem + buf * C::STAGE;
    bf16* sw = sx + BM * BK;
    // The fp32 head (a_fold): A = [hi | lo] and W = [W_hi | W_lo | W_hi]; its three products hi W_hi, hi W_lo and
    // lo W_hi run interleaved per 32-deep block b (stages 3 b, 3 b + 1, 3 b + 2), so the second read of an A_hi
    // block and of a W_hi block comes one or two stages after the first, from L2.
    int ks = kt, kwt = kt;
    if constexpr (EPI == EPI_CE) {
      if (g.a_fold) {
        const int blk = kt / 3, pass = kt - 3 * blk, nb = g.a_fold / BK;
        ks = pass == 2 ? nb + blk : blk;
        kwt = pass == 1 ? nb + blk : blk;
      }
    } else if constexpr (F16) {
      // h W_hi and h W_lo interleaved per 32-deep block: the second read of each A block comes from L2
      const int blk = kt >> 1;
      ks = blk;
      kwt = (kt & 1) ? g.a_fold / BK + blk : blk;
    }
    const long ka = ks * a_step, kw = kwt * w_step;
    // The dense product issues its loads from inline assembly, which the compiler's wait insertion does not see:
    // with the builtin it waits vmcnt(0) before the next LDS read at a tile's first and last steps (measured: MLP
    // pair 23.83 -> 23.62 ms). The loop's own waits (open) order every stage read after its loads. The other
    // epilogues keep the builtin: their M0 saves and restores cost more than the waits (config 3 13.27 -> 13.75 ms).
    if constexpr (EPI == EPI_DENSE) {
#pragma unroll
      for (int d = 0; d < C::LA; ++d) dma_x4(g.A + a_src[d] + ka, sx + (wave * C::LA + d) * 512);
#pragma unroll
      for (int d = 0; d < C::LB; ++d) dma_x4(b_src[d] + kw, sw + (wave * C::LB + d) * 512);
    } else {
#pragma unroll
      for (int d = 0; d < C::LA; ++d)
        __builtin_amdgcn_global_load_lds((const void*)(g.A + a_src[d] + ka),
                                         (lds_void_t*)(sx + (wave * C::LA + d) * 512), 16, 0, 0);
#pragma unroll
      for (int d = 0; d < C::LB; ++d)
        __builtin_amdgcn_global_load_lds((const void*)(b_src[d] + kw),
                                         (lds_void_t*)(sw + (wave * C::LB + d) * 512), 16, 0, 0);
    }
  };

  // ---- epilogue vectors of a tile, loaded into registers ahead of time and staged through LDS.
  // Thread tid sums x.b partial group tid / BM of row tid % BM; threads [0, BN/4) fetch a float4 of
  // a_p (EPI_CE_F16: and of the weight rows' scales); thread 0 the sign (whole tile in one member only).
  float4 pre_ab = make_float4(0.f, 0.f, 0.f, 0.f), pre_sc = make_float4(1.f, 1.f, 1.f, 1.f);
  float pre_u = 0.f, pre_sign = 0.f;
  int pre_t = -1;
  auto prefetch_ep = [&](int m0, int n0) {
    if constexpr (EPI == EPI_DENSE) return;
    const int pfirst = m0 / g.T, plast = min(m0 + BM - 1, g.M - 1) / g.T;
    const int dir = pfirst >> g.pair_shift, sl = n0 / g.seg_n, seg = g.seg0 + sl, ncol = n0 - sl * g.seg_n;
    if (tid < BN / 4) pre_ab = *reinterpret_cast<const float4*>(g.ra[seg] + (long)dir * g.ra_ld + ncol + 4 * tid);
    if (F16 && tid < BN / 4) pre_sc = *reinterpret_cast<const float4*>(g.col_scale + n0 + 4 * tid);
    if (tid == 0) pre_sign = pfirst == plast ? g.sign[pfirst] : 0.f;
    const int row = min(m0 + tid % BM, g.M - 1), grp = tid / BM;
    const int q0 = grp * g.u_parts / C::UGROUPS, q1 = (grp + 1) * g.u_parts / C::UGROUPS;
    const float* up = g.u + (long)row * g.u_ld + (long)seg * g.u_parts * g.u_qstride;
    float u = 0.f;
    for (int q = q0; q < q1; ++q) u += up[q * g.u_qstride];
    pre_u = u;
    // the head: the tile's target tokens, so that its epilogue makes no global load (a load there, issued after the
    // next tile's stage loads, would wait for all of them: vector memory operations complete in issue order)
    // (a token id past the int range, like a negative one, matches no column)
    if (CE && g.targets && tid < BM) {
      const long tk = g.targets[(long)(row / g.T) * g.tok_mstride + row % g.T];
      pre_t = tk < 0 || tk > 0x7fffffffL ? -1 : (int)tk;
    }
  };
  auto stage_ep = [&]() {
    if constexpr (EPI == EPI_DENSE) return;
    if constexpr (F16) {
      // the weight rows arrive scaled by sc (a power of two): a sc and the exp argument's factor / sc are exact
      constexpr float K2 = 2.f * 1.4426950408889634f / 15.f;
      if (tid < BN / 4) {
        *reinterpret_cast<float4*>(&ep_a[4 * tid]) =
            make_float4(pre_ab.x * pre_sc.x, pre_ab.y * pre_sc.y, pre_ab.z * pre_sc.z, pre_ab.w * pre_sc.w);
        *reinterpret_cast<float4*>(&ep_m[4 * tid]) =
            make_float4(K2 / pre_sc.x, K2 / pre_sc.y, K2 / pre_sc.z, K2 / pre_sc.w);
      }
    } else {
      if (tid < BN / 4) *reinterpret_cast<float4*>(&ep_a[4 * tid]) = pre_ab;
    }
    if (tid == 0) ep_sign = pre_sign;
    ep_u[tid / BM][tid % BM] = pre_u;
    if (CE && tid < BM) ep_t[tid] = pre_t;
  };

  // ---- MFMA operands of one 32-deep k step: x rows wm*WM + 16 i + (lane & 15) and W rows
  // wn*WN + 16 j + (lane & 15), k chunk kk * 4 + lane / 16.
  const int xrow0 = wm * WM + (lane & 15), wrow0 = wn * WN + (lane & 15);
  // the MFMA of the operand type (the registers hold 8 raw 16-bit elements either way)
  auto mma = [](const bf16x8& w, const bf16x8& x, const f32x4& c) {
    if constexpr (F16)
      return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h16x8, w), __builtin_bit_cast(h16x8, x), c, 0,
                                                     0, 0);
    else
      return mfma16x16x32(w, x, c);
  };
  auto read_w = [&](bf16x8 (&w)[FN], int buf, int kk) {
    const bf16* sw = smem + buf * C::STAGE + BM * BK;
    const int c = kk * 4 + (lane >> 4);
#pragma unroll
    for (int j = 0; j < FN; ++j) w[j] = *reinterpret_cast<const bf16x8*>(&sw[swz<BK>(wrow0 + j * 16, c)]);
  };
  auto read_x = [&](bf16x8& x, int buf, int kk, int i) {
    const bf16* sx = smem + buf * C::STAGE;
    x = *reinterpret_cast<const bf16x8*>(&sx[swz<BK>(xrow0 + i * 16, kk * 4 + (lane >> 4))]);
  };
  f32x4 acc[FM][FN];
  bf16x8 wa[FN], wb[FN], xf[FM];

  // Make step t's stage readable: when t opens a new stage, wait for its DMA, barrier, and refill the
  // stage retired by the previous step. Before the wait for stage kt, the stages issued are
  // 0 .. STAGES-1 (prologue) and kt-2+STAGES at most (refills of the earlier opens), so
  // min(KT-1, max(STAGES-1, kt-2+STAGES)) - kt later stages may stay in flight. A steady open (`steady`,
  // 1 <= kt <= KT - STAGES) has STAGES - 2 later stages in flight and refills, both known at compile time (the
  // general form selects its s_waitcnt through scalar compares and branches).
  auto open = [&](int t, auto steady) {
    constexpr bool ST = decltype(steady)::value;
    if (t % SUB == 0) {
      const int kt = t / SUB;
      if constexpr (ST)
        wait_vm_lgkm0<(STAGES - 2) * C::L>();
      else
        wait_stage<C::L, STAGES - 1>(min(KT - 1, max(STAGES - 1, kt - 2 + STAGES)) - kt);
      __builtin_amdgcn_s_barrier();
      if (ST || (kt >= 1 && kt - 1 + STAGES < KT)) issue(kt - 1 + STAGES, (kt - 1) % STAGES);
    }
  };
  constexpr std::true_type steady{};
  constexpr std::false_type general{};
  // the dense product and the head run their steady steps from a loop of their own; the other epilogues keep
  // one loop (with a second one, config 1's EPI_STORE product measured 4% slower)
  constexpr bool STEADY_LOOP = SUB == 1 && (EPI == EPI_DENSE || CE);
  // Step t's MFMAs with (wc, xf) while step t + 1's operands are read into (wn_, xf).
  auto step_read = [&](int t, const bf16x8 (&wc)[FN], bf16x8 (&wn_)[FN], auto st) {
    open(t + 1, st);
    const int buf = ((t + 1) / SUB) % STAGES, kk = (t + 1) % SUB;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = mma(wc[j], xf[i], acc[i][j]);
      if (i == 0) read_w(wn_, buf, kk);
      read_x(xf[i], buf, kk, i);
    }
  };
  auto step_last = [&](const bf16x8 (&wc)[FN]) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = mma(wc[j], xf[i], acc[i][j]);
  };

  // Tile order: row block outer, column tile inner, except for the head (EPI_CE: 16 column tiles of a W that
  // does not fit an XCD's L2), which walks groups of CE_GROUP row blocks per column tile so each W column tile
  // is read once per group rather than once per row block (measured: config 3 15.4 -> 14.7 ms; groups of 4:
  // 14.8, 16: 15.3, 32: 17.4).
  constexpr int CE_GROUP = 8;
  auto tile_mn = [&](int t, int which) {
    if (CE) {
      const int span = CE_GROUP * tiles_n, grp = t / span, rem = t % span;
      const int gm = min(CE_GROUP, tiles_m - grp * CE_GROUP);
      return which == 0 ? (grp * CE_GROUP + rem % gm) * BM : (rem / gm) * BN;
    }
    return which == 0 ? (t / tiles_n) * BM : (t % tiles_n) * BN;
  };
  int tile = t_lo + slot;
  if (tile >= t_hi) return;
  {
    const int m0 = tile_mn(tile, 0), n0 = tile_mn(tile, 1);
    prefetch_ep(m0, n0);
    set_sources(m0, n0);
#pragma unroll
    for (int s = 0; s < STAGES; ++s)
      if (s < KT) issue(s, s);
  }
  while (true) {
    const int m0 = tile_mn(tile, 0), n0 = tile_mn(tile, 1);
    // the previous tile's epilogue has finished reading the staged vectors
    wait_vm_lgkm0<63>();
    __builtin_amdgcn_s_barrier();
    stage_ep();

#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    open(0, general);
    read_w(wa, 0, 0);
#pragma unroll
    for (int i = 0; i < FM; ++i) read_x(xf[i], 0, 0, i);
    // KS is even (K % 64 == 0): pairs of steps alternate the W register sets; the last step reads
    // nothing.
    int t = 0;
    if constexpr (STEADY_LOOP) {
      // pairs whose two opens (k stages t + 1, t + 2; one step per stage) are both steady
      for (; t + 2 <= KT - STAGES && t < KS - 2; t += 2) {
        step_read(t, wa, wb, steady);
        step_read(t + 1, wb, wa, steady);
      }
    }
    for (; t < KS - 2; t += 2) {
      step_read(t, wa, wb, general);
      step_read(t + 1, wb, wa, general);
    }
    step_read(KS - 2, wa, wb, general);
    step_last(wb);

    // every wave has read the ring for the last time: prefetch the next tile
    const int next = tile + nslots;
    wait_vm_lgkm0<63>();
    __builtin_amdgcn_s_barrier();
    if (next < t_hi) {
      const int nm0 = tile_mn(next, 0), nn0 = tile_mn(next, 1);
      prefetch_ep(nm0, nn0);
      set_sources(nm0, nn0);
#pragma unroll
      for (int s = 0; s < STAGES; ++s)
        if (s < KT) issue(s, s);
    }

    // ---- epilogue. Lane holds, for token row m0 + wm*WM + i*16 + (lane & 15), the output columns
    // cb .. cb + CW - 1 with cb = n0 + wn*WN + (lane >> 4) * CW; acc[i][j][e] is column cb + 4j + e.
    const int lcol = wn * WN + (lane >> 4) * CW, cb = n0 + lcol;
    const int sl = n0 / g.seg_n, seg = g.seg0 + sl, scol = cb - sl * g.seg_n;  // column inside the segment
    const bool uniform = m0 / g.T == min(m0 + BM - 1, g.M - 1) / g.T;
    const float s_uni = ep_sign;
    if constexpr (EPI == EPI_DENSE) {
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int row = m0 + wm * WM + i * 16 + (lane & 15);
        if (row < g.M) {
          bf16* o = g.out_bf16 + (long)row * g.ldo + cb;
#pragma unroll
          for (int e = 0; e < CW; e += 8)
            store_x4(o + e, pack_bf16(acc[i][e / 4][0], acc[i][e / 4][1]), pack_bf16(acc[i][e / 4][2], acc[i][e / 4][3]),
                            pack_bf16(acc[i][e / 4 + 1][0], acc[i][e / 4 + 1][1]),
                            pack_bf16(acc[i][e / 4 + 1][2], acc[i][e / 4 + 1][3]));
        }
      }
      if (next >= t_hi) break;
      tile = next;
      continue;
    }
    // bf16 rounding of the product and of u (the bf16 paths); the fp16 head never rounds
    const bool rnd = !F16 && g.round_bf16;
    // The epilogue, instantiated for a tile inside one member (UNI: its vectors from LDS and no global load, so no
    // wait on the next tile's stage loads issued above) and for a tile that straddles members.
    auto epilogue = [&](auto uni_c) {
      constexpr bool UNI = decltype(uni_c)::value;
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int lr = wm * WM + i * 16 + (lane & 15), row = m0 + lr;
        const bool live = row < g.M;
        const int rrow = live ? row : g.M - 1;
        float u = 0.f;
#pragma unroll
        for (int q = 0; q < C::UGROUPS; ++q) u += ep_u[q][lr];
        // the row's member: for a tile that straddles members (per-row vectors from global memory) and for the value
        // embedding's gather; a tile inside one member takes its vectors from LDS
        int p = 0;
        if (EPI == EPI_QKV || !UNI) p = rrow / g.T;
        const int dir = p >> g.pair_shift;
        float sgn = s_uni;
        if constexpr (!UNI) sgn = g.sign[p];
        const float su = sgn * (rnd ? bf16r(u) : u);
        // v = dense + s u a over the lane's CW columns
        float v[CW];
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          float av[4];
          if constexpr (UNI) {
            const float4 a4 = *reinterpret_cast<const float4*>(&ep_a[lcol + 4 * j]);
            av[0] = a4.x, av[1] = a4.y, av[2] = a4.z, av[3] = a4.w;
          } else {
            const float* arow = g.ra[seg] + (long)dir * g.ra_ld + scol + 4 * j;
#pragma unroll
            for (int e = 0; e < 4; ++e) av[e] = F16 ? arow[e] * g.col_scale[cb + 4 * j + e] : arow[e];
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) v[4 * j + e] = (rnd ? bf16r(acc[i][j][e]) : acc[i][j][e]) + su * av[e];
        }
        if constexpr (EPI == EPI_STORE) {
          if (live) {
            if (g.out_f32) {
              float* o = g.out_f32 + (long)row * g.ldo + cb;
#pragma unroll
              for (int j = 0; j < FN; ++j) store_f4(o + 4 * j, v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
            }
            if (g.out_bf16) {
              bf16* o = g.out_bf16 + (long)row * g.ldo + cb;
#pragma unroll
              for (int e = 0; e < CW; e += 8)
                store_x4(o + e, pack_bf16(v[e], v[e + 1]), pack_bf16(v[e + 2], v[e + 3]), pack_bf16(v[e + 4], v[e + 5]),
                                pack_bf16(v[e + 6], v[e + 7]));
            }
          }
        } else if constexpr (EPI == EPI_RESID) {
          if (live) {
            float4* o = reinterpret_cast<float4*>(g.out_f32 + (long)row * g.ldo + cb);
#pragma unroll
            for (int j = 0; j < FN; ++j) {
              float4 r = o[j];
              r.x += v[4 * j];
              r.y += v[4 * j + 1];
              r.z += v[4 * j + 2];
              r.w += v[4 * j + 3];
              o[j] = r;
            }
          }
        } else if constexpr (EPI == EPI_QKV) {
          // the wave's WN = 64 columns are one head; lane group lane / 16 holds head dims 16 (lane / 16) ..
          const int t = rrow % g.T;
          if (seg < 2) {
            // rotary (utils/model.py:55-58): dims d and d + 32 pair up, held by lanes l and l ^ 32 (exchanged by
            // v_permlane32_swap)
            const int dd = (lane >> 4) * CW & 31;
            const bool first = (lane >> 4) < 2;
            const __bf16* cr = g.rot_cos + (long)t * 32 + dd;
            const __bf16* sr = g.rot_sin + (long)t * 32 + dd;
            float ss = 0.f;
#pragma unroll
            for (int e = 0; e < CW; ++e) {
              const f32pair hv = halves32(v[e]);  // dims d (lanes 0-31) and d + 32 (lanes 32-63)
              const float c = (float)cr[e], sn = (float)sr[e];
              const float y = first ? hv.lo * c + hv.hi * sn : hv.hi * c - hv.lo * sn;
              v[e] = y;
              ss += y * y;
            }
            // QK RMSNorm over the head's 64 dims (eps = 2^-23, utils/model.py:46-47)
            ss = sum_rows4(ss);
            // q (segment 0) leaves pre-multiplied by log2(e) / 8, the attention's score scale in base-2 units
            const float r = rsqrtf(ss * (1.f / 64.f) + 1.1920928955078125e-07f) * (seg ? 1.f : 0.18033688011112042f);
#pragma unroll
            for (int e = 0; e < CW; ++e) v[e] *= r;
          } else if (g.gate) {
            // value embedding (train/val/eggroll.py:85-89): v += 2 sigmoid(gate) (W[idx] + s a[idx] b)
            const long tok = g.idx[(long)p * g.tok_mstride + t];
            const float gt = g.gate[(long)rrow * 8 + scol / 64];
            const float sa = sgn * g.ve_a[(long)dir * g.ve_v + tok];
            const float* wr = g.ve_w + tok * 512 + scol;
            const float* br = g.ve_b + (long)dir * 512 + scol;
#pragma unroll
            for (int e = 0; e < CW; ++e) v[e] += gt * (wr[e] + sa * br[e]);
          }
          if (live) {
            // q, k and v: fp16 of the fp32 values (the reference feeds flex fp32 operands, train/val/eggroll.py:91)
            bf16* o = g.out_bf16 + (long)row * g.ldo + cb;
#pragma unroll
            for (int e = 0; e < CW; e += 8)
              store_x4(o + e, pack_f16(v[e], v[e + 1]), pack_f16(v[e + 2], v[e + 3]), pack_f16(v[e + 4], v[e + 5]),
                              pack_f16(v[e + 6], v[e + 7]));
          }
        } else {  // EPI_CE
          // soft cap 15 tanh(z / 15) (train/val/eggroll.py:100) with tanh(y) = 1 - 2 / (exp(2y) + 1); |z'| <= 15,
          // so the sum of exp(z') over 4096 columns needs no running maximum.
          // Everything in log2 units: ez = exp(2 z / 15) = 2^(z 2 log2(e) / 15); zl = z' log2(e) =
          // 15 log2(e) - 30 log2(e) / (ez + 1); exp(z') = 2^zl. The reciprocal is the hardware one
          // (v_rcp_f32, 1 ulp): an IEEE division would cost ~10 VALU operations per logit.
          constexpr float L2E = 1.4426950408889634f;
          // the target's column among the lane's CW, if any (a target of -1, or none, matches no column)
          const int tk = ep_t[lr];
          const int te = tk < 0 ? -1 : (int)(tk - cb);
          float se = 0.f, zt = 0.f;
          float* lg = g.logits && live ? g.logits + (long)row * g.ldo + cb : nullptr;
#pragma unroll
          for (int j = 0; j < FN; ++j) {
            float zq[4], m[4] = {2.f * L2E / 15.f, 2.f * L2E / 15.f, 2.f * L2E / 15.f, 2.f * L2E / 15.f};
            if constexpr (F16) {
              // v is the logit times the weight row's scale; m divides it out
              const float4 m4 = *reinterpret_cast<const float4*>(&ep_m[lcol + 4 * j]);
              m[0] = m4.x, m[1] = m4.y, m[2] = m4.z, m[3] = m4.w;
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float ez = __builtin_amdgcn_exp2f(v[4 * j + e] * m[e]);
              const float zl = fmaf(__builtin_amdgcn_rcpf(ez + 1.f), -30.f * L2E, 15.f * L2E);
              se += __builtin_amdgcn_exp2f(zl);
              zt = 4 * j + e == te ? zl : zt;
              zq[e] = zl;
            }
            // the capped logits themselves (utils/model.py:203-204, returned when no targets are given)
            if (lg) store_f4(lg + 4 * j, zq[0] * 0.6931471805599453f, zq[1] * 0.6931471805599453f,
                             zq[2] * 0.6931471805599453f, zq[3] * 0.6931471805599453f);
          }
          if (live && te >= 0 && te < CW) g.ce_tgt[row] = zt * 0.6931471805599453f;
          se = sum_rows4(se);
          if (live && (lane >> 4) == 0) g.upart_out[(long)row * g.upart_ld + (n0 + wn * WN) / WN] = se;
        }
      }
    };
    if (uniform) epilogue(std::true_type{});
    else epilogue(std::false_type{});
    if (next >= t_hi) break;
    tile = next;
  }
}

// Tile configurations: <BM, BN, BK, STAGES, WGM, WGN>.
#ifndef NOISE_GEMM_CFG
#define NOISE_GEMM_CFG 0
#endif
// <BM, BN, BK, STAGES, WGM, WGN, OCC>: OCC workgroups of WGM x WGN waves share a CU.
#if NOISE_GEMM_CFG == 0
#define CFG_BIG 256, 256, 32, 4, 2, 4, 1
#define CFG_SMALL 256, 128, 32, 4, 4, 2, 1
#elif NOISE_GEMM_CFG == 1
#define CFG_BIG 256, 256, 64, 2, 2, 4, 1
#define CFG_SMALL 256, 128, 64, 2, 4, 2, 1
#elif NOISE_GEMM_CFG == 3
#define CFG_BIG 256, 256, 32, 3, 2, 4, 1
#define CFG_SMALL 256, 128, 32, 3, 4, 2, 1
#elif NOISE_GEMM_CFG == 5
#define CFG_BIG 256, 128, 32, 3, 2, 2, 2
#define CFG_SMALL 256, 128, 32, 3, 2, 2, 2
#elif NOISE_GEMM_CFG == 6
#define CFG_BIG 256, 128, 32, 2, 2, 2, 2
#define CFG_SMALL 256, 128, 32, 2, 2, 2, 2
#elif NOISE_GEMM_CFG == 7
#define CFG_BIG 128, 256, 32, 3, 2, 2, 2
#define CFG_SMALL 128, 128, 32, 4, 2, 2, 2
#endif

template <int BM, int BN, int BK, int STAGES, int WGM, int WGN, int OCC>
constexpr int cfg_wave_n() { return BN / WGN; }

int num_cus() {
  static int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    return n;
  }();
  return cus;
}

template <int BM, int BN, int BK, int STAGES, int WGM, int WGN, int OCC, int EPI>
int launch_cfg(const LowrankGemmArgs& g, hipStream_t stream) {
  using C = Cfg<BM, BN, BK, STAGES, WGM, WGN>;
  if (g.N % BN || g.K % 64) return NOISE_ENOTSUP;
  // a TILE16 A operand is one tile per 16-row DMA instruction and 32-deep stage; a WTILE W one block, whose row
  // order is the one of 64-column wave tiles with 16 contiguous columns per lane
  if (g.a_tiled && (BK != 32 || C::ROWS_PER_DMA != 16)) return NOISE_ENOTSUP;
  if (g.w_tiled && (BK != 32 || C::ROWS_PER_DMA != 16 || C::WN != 64 || C::CW != 16)) return NOISE_ENOTSUP;
  const long tiles = (long)((g.M + BM - 1) / BM) * (g.N / BN);
  if (tiles > 0x7fffffffL) return NOISE_ENOTSUP;
  // OCC persistent workgroups per CU, a multiple of 8 for the XCD split
  long grid = std::min<long>((long)OCC * num_cus(), tiles);
  grid = (grid + 7) / 8 * 8;
  hipLaunchKernelGGL((lowrank_gemm_kernel<BM, BN, BK, STAGES, WGM, WGN, OCC, EPI>), dim3((unsigned)grid),
                     dim3(WGM * WGN * 64), 0, stream, g);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}

bool use_big(int N) { return N % 256 == 0; }

template <int EPI>
int launch_epi(const LowrankGemmArgs& g, hipStream_t stream) {
  if (use_big(g.N)) return launch_cfg<CFG_BIG, EPI>(g, stream);
  return launch_cfg<CFG_SMALL, EPI>(g, stream);
}

}  // namespace

namespace {
// WTILE copy of a row-major bf16 weight: thread q writes the 16-byte output chunk q (block q / 64, row r and
// physical chunk p of the block), read from the weight row and logical chunk the layout assigns to it.
__global__ void __launch_bounds__(256) weight_tiles_kernel(const bf16* __restrict__ in, long ld, int K, long chunks,
                                                           bf16* __restrict__ out) {
  const long q = (long)blockIdx.x * 256 + threadIdx.x;
  if (q >= chunks) return;
  const long blk = q >> 6, kt = K >> 5, g = blk / kt, st = blk - g * kt;
  const int u = (int)(q & 63), r = u >> 2, c = (u & 3) ^ ((r >> 1) & 3);
  const long i = 16 * g + r;
  const long n = (i & ~63L) + (r >> 2) * 16 + ((i & 63) >> 4) * 4 + (r & 3);
  *reinterpret_cast<uint4*>(out + 8 * q) = *reinterpret_cast<const uint4*>(in + n * ld + 32 * st + 8 * c);
}
}  // namespace

int weight_tiles_launch(const bf16* in, long ld, int N, int K, bf16* out, hipStream_t stream) {
  if (!in || !out || N <= 0 || K <= 0 || N % 64 || K % 32 || ld < K || ld % 8 ||
      (((uintptr_t)in | (uintptr_t)out) & 15))
    return NOISE_EINVAL;
  const long chunks = (long)N * K / 8;
  hipLaunchKernelGGL(weight_tiles_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, stream, in, ld, K,
                     chunks, out);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}

namespace {
// One wave per weight row n: lane l holds columns 8 l .. 8 l + 7 of (w * gain), scaled by 2^e so that the row's
// largest magnitude lies in [2^14, 2^15), then split into hi = fp16(v) and lo = fp16(v - hi). fp16 keeps 11
// significant bits for magnitudes down to 2^-14, i.e. for every element within 2^-28 of the row's largest; the
// smaller ones lose relative precision but keep an absolute error below 2^-24, which a 512-term dot does not see.
__global__ void __launch_bounds__(256) head_weight_f16_kernel(const float* __restrict__ w, long ldw,
                                                              const float* __restrict__ gain, int N, int tiled,
                                                              _Float16* __restrict__ out, float* __restrict__ scale) {
  const int lane = threadIdx.x & 63;
  const long n = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const float4 w0 = *reinterpret_cast<const float4*>(w + n * ldw + 8 * lane);
  const float4 w1 = *reinterpret_cast<const float4*>(w + n * ldw + 8 * lane + 4);
  float v[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
  if (gain) {
    const float4 g0 = *reinterpret_cast<const float4*>(gain + 8 * lane);
    const float4 g1 = *reinterpret_cast<const float4*>(gain + 8 * lane + 4);
    const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] *= gv[e];
  }
  float mx = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(v[e]));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  int ex = 0;
  if (mx > 0.f) {
    frexpf(mx, &ex);  // mx = f 2^ex, f in [0.5, 1)
    ex = min(max(15 - ex, -120), 120);
  }
  const float sc = ldexpf(1.f, ex);
  _Float16 hi[8], lo[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float s = v[e] * sc;
    hi[e] = (_Float16)s;
    lo[e] = (_Float16)(s - (float)hi[e]);
  }
  const long k = 8 * lane;
  const long oh = tiled ? wtile_offset(n, k, 1024) : n * 1024 + k;
  const long ol = tiled ? wtile_offset(n, 512 + k, 1024) : n * 1024 + 512 + k;
  *reinterpret_cast<uint4*>(out + oh) = __builtin_bit_cast(uint4, hi);
  *reinterpret_cast<uint4*>(out + ol) = __builtin_bit_cast(uint4, lo);
  if (lane == 0) scale[n] = sc;
}
}  // namespace

int head_weight_f16_launch(const float* w, long ldw, const float* gain, int N, int tiled, bf16* out, float* scale,
                           hipStream_t stream) {
  if (!w || !out || !scale || N <= 0 || N % 64 || ldw < 512 || ldw % 4 ||
      (((uintptr_t)w | (uintptr_t)gain | (uintptr_t)out) & 15))
    return NOISE_EINVAL;
  hipLaunchKernelGGL(head_weight_f16_kernel, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, stream, w, ldw, gain, N,
                     tiled, reinterpret_cast<_Float16*>(out), scale);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}

int lowrank_gemm_parts(int N) {
  if (N <= 0 || N % 128) return 0;
  return use_big(N) ? N / cfg_wave_n<CFG_BIG>() : N / cfg_wave_n<CFG_SMALL>();
}

int lowrank_gemm_launch(int epi, const LowrankGemmArgs& g, hipStream_t stream) {
  if (g.a_tiled && (epi == EPI_RELU2 || g.M % 16 || g.T % 16 || g.lda % 32 || g.a_mstride != (long)g.T * g.lda))
    return NOISE_EINVAL;
  if (g.out_tiled && (epi != EPI_RELU2 || g.M % 16 || g.ldo % 32)) return NOISE_EINVAL;
  if (epi == EPI_DENSE) {
    if (g.M <= 0 || g.N <= 0 || g.K <= 0 || g.T <= 0 || !g.A || !g.W || !g.out_bf16 || g.lda % 8 ||
        (!g.w_tiled && (g.ldw % 8 || g.ldw < g.K)) || g.a_mstride % 8 || g.lda < g.K || g.ldo % 8 || g.ldo < g.N ||
        g.N % 128 || g.K % 64 ||
        (((uintptr_t)g.A | (uintptr_t)g.W | (uintptr_t)g.out_bf16) & 15))
      return NOISE_EINVAL;
    // K = 512 (the attention c_proj): the weight-resident kernel streams x once per 256 output columns
    if (xs_dense_supported(g)) return xs_dense_launch(g, stream);
    return launch_epi<EPI_DENSE>(g, stream);
  }
  if (g.a_fold && ((epi != EPI_CE && epi != EPI_CE_F16) || g.a_fold < 0 || g.a_fold % 64 ||
                   g.K != (epi == EPI_CE ? 3 : 2) * g.a_fold))
    return NOISE_EINVAL;
  if (epi == EPI_CE_F16 && (!g.a_fold || !g.col_scale || ((uintptr_t)g.col_scale & 15) || g.round_bf16))
    return NOISE_EINVAL;
  if (g.M <= 0 || g.N <= 0 || g.K <= 0 || g.T <= 0 || !g.A || !g.W || !g.sign || !g.u || g.u_parts <= 0 ||
      g.u_ld < 1 || g.lda % 8 || (!g.w_tiled && (g.ldw % 8 || g.ldw < g.K)) || g.a_mstride % 8 ||
      g.lda < g.K - g.a_fold ||
      g.pair_shift < 0 || g.pair_shift > 1 || g.ra_ld % 4 || g.ldo % 8 || g.N % 128 || g.K % 64 ||
      g.seg_n <= 0 || g.seg_n % 128 || g.N % g.seg_n || g.seg0 < 0 || g.seg0 + g.N / g.seg_n > 3 || g.u_qstride < 1)
    return NOISE_EINVAL;
  const int nseg = g.N / g.seg_n;
  if (g.u_qstride == 1 && g.u_ld < (g.seg0 + nseg) * g.u_parts) return NOISE_EINVAL;
  for (int s = g.seg0; s < g.seg0 + nseg; ++s)
    if (!g.ra[s] || ((uintptr_t)g.ra[s] & 15)) return NOISE_EINVAL;
  if (((uintptr_t)g.A | (uintptr_t)g.W) & 15) return NOISE_EINVAL;
  if (((uintptr_t)g.out_f32 | (uintptr_t)g.out_bf16) & 15) return NOISE_EINVAL;
  switch (epi) {
    case EPI_STORE:
      if (!g.out_f32 && !g.out_bf16) return NOISE_EINVAL;
      return launch_epi<EPI_STORE>(g, stream);
    case EPI_RELU2:
      if (!xs_relu2_supported(g)) return NOISE_ENOTSUP;
      return xs_relu2_launch(g, stream);
    case EPI_RESID:
      if (!g.out_f32) return NOISE_EINVAL;
      return launch_epi<EPI_RESID>(g, stream);
    case EPI_QKV:
      if (!g.out_bf16 || g.seg_n != 512 || g.seg0 + nseg != 3 || !g.rot_cos || !g.rot_sin ||
          (g.gate && (!g.ve_w || !g.ve_a || !g.ve_b || !g.idx || g.ve_v <= 0)))
        return NOISE_EINVAL;
      return launch_epi<EPI_QKV>(g, stream);
    case EPI_CE:
    case EPI_CE_F16:
      if ((!g.targets && !g.logits) || !g.ce_tgt || !g.upart_out || g.upart_ld != lowrank_gemm_parts(g.N) ||
          (g.logits && g.ldo < g.N) || g.tok_mstride < 0)
        return NOISE_EINVAL;
      return epi == EPI_CE ? launch_epi<EPI_CE>(g, stream) : launch_epi<EPI_CE_F16>(g, stream);
  }
  return NOISE_EINVAL;
}
