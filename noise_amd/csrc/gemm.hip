// Low-rank-perturbed GEMM on gfx950 bf16 MFMA: out = x W^T + s_p (x.b_p) a_p^T per member p.
//
// Reference: `lowrank` (train/val/eggroll.py:56-58) under bf16 autocast (:144). The dense part runs
// on v_mfma_f32_16x16x32_bf16 with LDS-staged, XOR-swizzled tiles; the rank-1 part never touches the
// MFMA pipe: the input-side dot u = bf16(x.b_p) arrives per row (computed by the kernel that produced
// x) and the epilogue adds (s_p u) a_p[col] in fp32 on top of the bf16-rounded GEMM output, exactly
// the autocast rounding points (bf16 GEMM output, fp32 correction).
//
// Layouts (row-major, K contiguous): A [M, K] bf16 with M = members x T rows (member p owns rows
// p*T .. p*T+T-1); W [N, K] bf16 in the reference's nn.Linear orientation [out, in].
#include "common.h"
#include "gemm.h"

namespace {

// Epilogue kinds.
enum : int {
  EPI_STORE = 0,   // out = lowrank(x)            -> fp32 and/or bf16 store
  EPI_RELU2 = 1,   // h = bf16(relu(lowrank(x))^2) -> bf16 store + partial dots h.b_next per row
  EPI_RESID = 2,   // resid += lowrank(x)          -> fp32 read-modify-write
};

template <int BM, int BN, int BK, int WGM, int WGN>
struct Tile {
  static constexpr int NTH = WGM * WGN * 64;
  static constexpr int WM = BM / WGM, WN = BN / WGN;
  static constexpr int FM = WM / 16, FN = WN / 16;
  static constexpr int CH = BK / 8;  // 16-byte chunks per LDS row
  static constexpr int A_LOADS = BM * CH / NTH;
  static constexpr int B_LOADS = BN * CH / NTH;
  static_assert(BK == 64, "swizzle assumes 128-byte LDS rows");
  static_assert(WM % 16 == 0 && WN % 16 == 0, "wave tile must be a multiple of 16");
  static_assert(BM * CH % NTH == 0 && BN * CH % NTH == 0, "tile loads must divide evenly");
};

// 16-byte chunk c of LDS row r is stored at chunk c ^ (r & 7): the 8 lanes of a ds_read_b128 phase
// (consecutive rows, same k chunk) then hit 8 distinct 16-byte bank groups.
__device__ __forceinline__ int swz(int r, int c) { return r * 64 + ((c ^ (r & 7)) << 3); }

template <int BM, int BN, int BK, int WGM, int WGN, int EPI>
__global__ void __launch_bounds__(WGM * WGN * 64)
lowrank_gemm_kernel(const LowrankGemmArgs g) {
  using TL = Tile<BM, BN, BK, WGM, WGN>;
  constexpr int NTH = TL::NTH, WM = TL::WM, WN = TL::WN, FM = TL::FM, FN = TL::FN, CH = TL::CH;
  __shared__ __attribute__((aligned(16))) bf16 sA[2][BM * BK];
  __shared__ __attribute__((aligned(16))) bf16 sB[2][BN * BK];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int tiles_n = g.N / BN;
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int m0 = (tile / tiles_n) * BM, n0 = (tile % tiles_n) * BN;

  // Per-thread source rows of the global->LDS copies (fixed across the K loop): thread tid copies
  // chunk (tid % CH) of rows tid / CH + i * (NTH / CH).
  constexpr int RSTEP = NTH / CH;
  const int cchunk = tid % CH, r0 = tid / CH;
  const bf16* a_src = nullptr;
  long a_step[TL::A_LOADS];
#pragma unroll
  for (int i = 0; i < TL::A_LOADS; ++i) {
    const int row = min(m0 + r0 + i * RSTEP, g.M - 1);
    const long off = (long)(row / g.T) * g.a_mstride + (long)(row % g.T) * g.lda + cchunk * 8;
    a_step[i] = off;
  }
  a_src = g.A;
  const bf16* b_src = g.W + (long)(n0 + r0) * g.ldw + cchunk * 8;
  const long b_rstep = (long)RSTEP * g.ldw;
  u32x4 ra[TL::A_LOADS], rb[TL::B_LOADS];
#define GLOAD(k0)                                                                                   \
  do {                                                                                              \
    _Pragma("unroll") for (int i = 0; i < TL::A_LOADS; ++i)                                        \
      ra[i] = *reinterpret_cast<const u32x4*>(a_src + a_step[i] + (k0));                            \
    _Pragma("unroll") for (int i = 0; i < TL::B_LOADS; ++i)                                        \
      rb[i] = *reinterpret_cast<const u32x4*>(b_src + i * b_rstep + (k0));                          \
  } while (0)
#define SSTORE(buf)                                                                                 \
  do {                                                                                              \
    _Pragma("unroll") for (int i = 0; i < TL::A_LOADS; ++i)                                        \
      *reinterpret_cast<u32x4*>(&sA[buf][swz(r0 + i * RSTEP, cchunk)]) = ra[i];                     \
    _Pragma("unroll") for (int i = 0; i < TL::B_LOADS; ++i)                                        \
      *reinterpret_cast<u32x4*>(&sB[buf][swz(r0 + i * RSTEP, cchunk)]) = rb[i];                     \
  } while (0)

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int KT = g.K / BK;
  GLOAD(0);
  SSTORE(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < KT) GLOAD((kt + 1) * BK);
    const bf16* a_s = sA[buf];
    const bf16* b_s = sB[buf];
#pragma unroll
    for (int kk = 0; kk < BK / 32; ++kk) {
      const int c = kk * 4 + (lane >> 4);
      bf16x8 af[FM], bw[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int r = wm * WM + i * 16 + (lane & 15);
        af[i] = *reinterpret_cast<const bf16x8*>(&a_s[swz(r, c)]);
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int r = wn * WN + j * 16 + (lane & 15);
        bw[j] = *reinterpret_cast<const bf16x8*>(&b_s[swz(r, c)]);
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = mfma16x16x32(af[i], bw[j], acc[i][j]);
    }
    if (kt + 1 < KT) SSTORE(buf ^ 1);
    __syncthreads();
  }

#undef GLOAD
#undef SSTORE
  // ---- epilogue. Lane holds C[row = 4*(lane>>4) + e][col = lane & 15] of each 16x16 block.
  const int col_base = n0 + wn * WN + (lane & 15);
#pragma unroll
  for (int i = 0; i < FM; ++i) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = m0 + wm * WM + i * 16 + 4 * (lane >> 4) + e;
      const bool live = row < g.M;
      const int rrow = live ? row : g.M - 1;
      const int p = rrow / g.T;
      const int dir = p >> g.pair_shift;
      float u = 0.f;
      for (int j = 0; j < g.u_parts; ++j) u += g.u[(long)rrow * g.u_parts + j];
      const float su = g.sign[p] * bf16r(u);
      const float* arow = g.ra + (long)dir * g.ra_ld;
      float dot = 0.f;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int col = col_base + j * 16;
        const float v = bf16r(acc[i][j][e]) + su * arow[col];
        if constexpr (EPI == EPI_STORE) {
          if (live) {
            if (g.out_f32) g.out_f32[(long)row * g.ldo + col] = v;
            if (g.out_bf16) g.out_bf16[(long)row * g.ldo + col] = to_bf16(v);
          }
        } else if constexpr (EPI == EPI_RELU2) {
          const float r = fmaxf(v, 0.f);
          const bf16 hb = to_bf16(r * r);
          if (live) g.out_bf16[(long)row * g.ldo + col] = hb;
          dot += (float)hb * bf16r(g.rb_next[(long)dir * g.rb_next_ld + col]);
        } else {
          if (live) g.out_f32[(long)row * g.ldo + col] += v;
        }
      }
      if constexpr (EPI == EPI_RELU2) {
        dot = group_sum<16>(dot);
        if (live && (lane & 15) == 0) g.upart_out[(long)row * g.upart_ld + (n0 + wn * WN) / WN] = dot;
      }
    }
  }
}

template <int BM, int BN, int BK, int WGM, int WGN, int EPI>
int launch_cfg(const LowrankGemmArgs& g, hipStream_t stream) {
  if (g.N % BN || g.K % BK) return NOISE_ENOTSUP;
  const int tiles = ((g.M + BM - 1) / BM) * (g.N / BN);
  hipLaunchKernelGGL((lowrank_gemm_kernel<BM, BN, BK, WGM, WGN, EPI>), dim3(tiles), dim3(WGM * WGN * 64), 0,
                     stream, g);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}

template <int EPI>
int launch_epi(const LowrankGemmArgs& g, hipStream_t stream) {
  return launch_cfg<128, 128, 64, 2, 2, EPI>(g, stream);
}

}  // namespace

int lowrank_gemm_wave_n() { return 64; }

int lowrank_gemm_launch(int epi, const LowrankGemmArgs& g, hipStream_t stream) {
  if (g.M <= 0 || g.N <= 0 || g.K <= 0 || g.T <= 0 || !g.A || !g.W || !g.sign || !g.ra || !g.u ||
      g.u_parts <= 0 || g.lda % 8 || g.ldw % 8 || g.a_mstride % 8 || g.lda < g.K || g.ldw < g.K ||
      g.pair_shift < 0 || g.pair_shift > 1)
    return NOISE_EINVAL;
  if (((uintptr_t)g.A | (uintptr_t)g.W) & 15) return NOISE_EINVAL;
  switch (epi) {
    case EPI_STORE:
      if (!g.out_f32 && !g.out_bf16) return NOISE_EINVAL;
      return launch_epi<EPI_STORE>(g, stream);
    case EPI_RELU2:
      if (!g.out_bf16 || !g.rb_next || !g.upart_out || g.upart_ld != g.N / lowrank_gemm_wave_n())
        return NOISE_EINVAL;
      return launch_epi<EPI_RELU2>(g, stream);
    case EPI_RESID:
      if (!g.out_f32) return NOISE_EINVAL;
      return launch_epi<EPI_RESID>(g, stream);
  }
  return NOISE_EINVAL;
}
