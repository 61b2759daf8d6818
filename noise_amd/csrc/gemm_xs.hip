// Weight-resident low-rank-perturbed GEMM for K = 512 on gfx950 bf16 MFMA, with the relu^2 epilogue of the
// MLP c_fc: h = bf16(relu(bf16(x W^T) + s_p bf16(x.b_p) a_p)^2) and the partial dots h . bf16(b_next).
//
// Reference: `lowrank` (train/val/eggroll.py:56-58) feeding `F.relu(...).square()` of the MLP
// (utils/model.py:106-107, train/val/eggroll.py:93) under bf16 autocast (:144); the dot with the c_proj
// input-side vector is the `(x @ b)` of the following `lowrank`, computed here from the bf16 h the kernel
// already holds.
//
// Why this shape. With 256 x 256 output tiles every tile re-reads both operands from L2: K = 512 GEMMs then
// need (256 + 256) rows of K per 256^2 outputs, and the L2 -> CU path (about 17 TB/s measured on MI355X)
// caps the c_fc GEMM near the MFMA time. Here a workgroup owns one 256-column slice of W for the whole
// launch and keeps it in registers (wave w: columns 32 w .. 32 w + 31, all 512 K = 128 VGPRs as MFMA A
// fragments), so only x streams: half the L2 traffic per FLOP.
//
// Schedule. 8 waves (2 per SIMD), one workgroup per CU. Workgroup b serves XCD b % 8; on each XCD the
// N / 256 slices form groups that walk the same 32-row blocks of x in the same order (the XCD's contiguous
// range of blocks, strided over the groups), so each x block is fetched from HBM once and served from that
// XCD's L2 to every slice.
//
// x path. Blocks of 32 rows x 512 K (32 KiB) stream through a 4-deep LDS ring with direct global -> LDS
// loads (global_load_lds_dwordx4), one whole 1 KiB row per instruction: every request is a full 128-byte
// line (a 16 rows x 64 bytes pattern, half lines, measured 8.9 TB/s from L2 into LDS against 15.9 TB/s for
// whole rows). LDS rows are 1040 bytes apart, so the 16 rows of an MFMA fragment fall in 16 different bank
// groups. The contraction order inside K is permuted to make the fragment reads affine: MFMA k step s,
// lane group g (lanes 16 g .. 16 g + 15) contracts k = 128 g + 8 s .. + 7, i.e. LDS chunk 16 g + s of the
// lane's row, and the resident W fragments use the same k. The loads are issued from inline assembly: the
// compiler would otherwise make every LDS read wait for every outstanding LDS-bound load (vmcnt(0)), which
// drains the ring. The kernel waits for them itself: vector memory operations complete in issue order, so
// "block k landed" is s_waitcnt vmcnt(n) with n = the operations issued after block k's loads, followed by
// s_barrier.
//
// Epilogue overlap. Iteration k runs the MFMAs of block k and, interleaved one stage per MFMA k step (a
// scheduling barrier between steps keeps the interleave), the epilogue of block k - 1 from the other
// accumulator set: the epilogue VALU work issues in the shadow of the MFMAs.
//
// h . b_next. Each lane holds 8 consecutive bf16 h of a row and the matching bf16(b_next) pairs: 4
// v_dot2_f32_bf16 per row, two VALU lane swaps (v_permlane16/32_swap) give the wave's 32-column partial, and the 8 wave partials of a
// row are summed in LDS (fixed order) by wave 0, which stores one partial per (slice, row): upart_out is
// part-major [N / 256][M], 128 contiguous bytes per block.
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "gemm.h"

namespace {

constexpr int R = 32;                 // rows per block
constexpr int NBUF = 4;               // LDS ring depth (blocks)
constexpr int NW = 8;                 // waves per workgroup
constexpr int BN = 256;               // columns per workgroup slice (32 per wave)
constexpr int KD = 512;               // K
constexpr int KS = KD / 32;           // MFMA k steps per block
constexpr int XROW = KD * 2 + 16;     // LDS bytes per x row (1 KiB + 16: bank-group skew between rows)
constexpr int XBYTES = R * XROW;      // LDS bytes of one x block
constexpr int VEC = 512;              // per-wave vector area: a (128 B) | b_next (128 B) | u (128 B) | .. | sign
constexpr int SIGN_OFF = VEC - 8;
// Epilogue modes of the kernel.
enum : int {
  XS_RELU2 = 0,  // MLP c_fc: bf16(relu(lowrank)^2) + partial dots with b_next
  XS_DENSE = 1,  // c_proj dense product y = bf16(x W^T), row-major
  XS_QK = 2,     // c_q | c_k: lowrank + rotary + RMSNorm over each 64-dim head, fp16 of the fp32 result (q times
                 // log2(e) / 8)
  XS_V = 3,      // c_v without value embedding: lowrank, fp16 of the fp32 result
  XS_VE = 4,     // c_v with the gated value embedding: lowrank + gate (ve_w[tok] + s ve_a[tok] ve_b), fp16
};
// LDS ring depth per mode: the value-embedding mode gives one ring slot to its gathered embedding rows
template <int MODE>
constexpr int RING = MODE == XS_VE ? 3 : NBUF;
// per wave and block: 4 x rows, then the mode's vectors (relu^2: a|b_next|u and the sign; q|k: a, and one
// of cos / sin / u|sign / padding)
template <int MODE>
constexpr int DMA_PER_BLOCK = MODE == XS_DENSE ? 4 : 6;
constexpr int VE_DMA = 6;  // value embedding: loads of one block's gather per wave (4 rows of W, b, a[tok])

// value-embedding mode: the per-block vectors of one ring slot, and one wave's gathered embedding block.
struct VeVec {
  float av[NW][32];   // a_v over each wave's 32 columns
  float uq[R][4];     // u_qkv rows: bf16 dots with b_q, b_k, b_v and the member's sign
  float gate[R][8];   // the block's gate rows, 2 sigmoid(ve_gate(h[:32])) per head
  int64_t tok[R];     // token ids of the NEXT block's rows (they address that block's embedding gather)
};
struct VeRows {
  float w[R][32];     // ve_w[tok] over the wave's 32 columns, one row per block row; the 16-byte chunk c of row r
                      // sits at chunk c ^ ((r / 2) % 8), so the 16 rows one read instruction touches fall in
                      // distinct banks
  float b[32];        // ve_b[dir] over the wave's 32 columns
  float a[R];         // ve_a[dir, tok] per block row
};

// q|k mode: the per-block vectors shared by the workgroup's 8 waves (5.5 KiB per ring slot).
struct QkVec {
  // rotary cos / sin rows of the block's 32 tokens; the 16-byte chunk c of row r sits at chunk c ^ ((r / 4) % 4),
  // so the 16 rows one read instruction touches fall in distinct banks
  bf16 cs[2][R][32];
  float uq[R][4];     // u_qkv rows: bf16 dots with b_q, b_k, b_v and the member's sign
  float av[NW][32];   // a over each wave's 32 columns
};
constexpr int STORES_PER_EPI = 2;     // lower bound on an epilogue's store instructions (two h rows)

template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(N >= 0 && N <= 63, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | ((N >> 4) << 14));
}

__device__ __forceinline__ unsigned pack_bf16(float a, float b) {
  bf16x2 p = {to_bf16(a), to_bf16(b)};
  return *reinterpret_cast<unsigned*>(&p);
}
__device__ __forceinline__ bf16x2 as_bf16x2(unsigned v) { return *reinterpret_cast<bf16x2*>(&v); }
// fp16 pair (round to nearest even) of two fp32 values: q, k and v enter attention with an 11-bit significand
__device__ __forceinline__ unsigned pack_f16(float a, float b) {
  _Float16 __attribute__((ext_vector_type(2))) p = {(_Float16)a, (_Float16)b};
  return *reinterpret_cast<unsigned*>(&p);
}

// q|k mode column map: slice s covers segment s / 2 (q, k), heads 4 (s % 2) .. + 3; wave w takes head
// 4 (s % 2) + w / 2 and, of its 64 dims, the 16 rotary pairs (d, d + 32) with d in 16 h .. 16 h + 15, h = w % 2.
// Local column 8 g + 4 j + e (lane group g, MFMA column block j, element e) is dim 32 j + 16 h + 4 g + e: a lane's
// 8 columns are dims d0 .. d0 + 3 and their partners d0 + 32 .. d0 + 35 (d0 = 16 h + 4 g), so the rotation stays
// inside the lane, and the head's RMSNorm needs only the partner wave w ^ 1.
__device__ __forceinline__ int qk_col(int nslice, int wave, int lc) {
  const int seg = nslice >> 1, head = 4 * (nslice & 1) + (wave >> 1), half = wave & 1;
  const int dim = 32 * ((lc >> 2) & 1) + 16 * half + 4 * (lc >> 3) + (lc & 3);
  return seg * 512 + head * 64 + dim;
}

// DENSE: the c_proj dense product y = bf16(x W^T) only (no rank-1 term, no vectors, no partial dots), row-major.
template <int MODE>
__global__ void __launch_bounds__(512, 2) xs_kernel(const LowrankGemmArgs g) {
  constexpr bool DENSE = MODE == XS_DENSE, QK = MODE == XS_QK, VV = MODE == XS_V, VE = MODE == XS_VE;
  constexpr int NB = RING<MODE>;
  constexpr int FIRST_STORE = QK ? 2 : 1;
  __shared__ __attribute__((aligned(16))) char smem[NB * XBYTES];
  __shared__ __attribute__((aligned(16))) char svec[NB][NW][VEC];
  // per-row partials padded to 12 floats: the 16 rows one instruction touches fall in distinct banks
  __shared__ __attribute__((aligned(16))) float red[2][R][NW + 4];
  __shared__ __attribute__((aligned(16))) QkVec qv[NB];
  __shared__ __attribute__((aligned(16))) float ssq[2][R][NW + 4];  // q|k: per-row partial sums of squares
  __shared__ __attribute__((aligned(16))) float qpad[R][4];     // q|k: landing area of the padding loads
  __shared__ __attribute__((aligned(16))) VeVec vv[NB];         // value embedding: per-block vectors
  __shared__ __attribute__((aligned(16))) VeRows ver[NW];       // value embedding: each wave's gathered rows
  __shared__ float vpad[NW];                                    // value embedding: landing area of padding loads

  // the wave index is uniform: keeping it in an SGPR keeps every per-wave address on the scalar unit
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), grp = lane >> 4;
  const int nslices = g.N / BN;
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const int streams = (gridDim.x >> 3) / nslices;
  const int nslice = slot % nslices, stream = slot / nslices;
  const int nb_all = g.M / R;
  const int lo = (int)((long)xcd * nb_all / 8), hi = (int)((long)(xcd + 1) * nb_all / 8);
  // this workgroup's blocks: lo + stream + k * streams, k = 0 .. nb - 1 (the same for every wave)
  const int nb = stream < streams && lo + stream < hi ? (hi - lo - stream + streams - 1) / streams : 0;
  if (nb == 0) return;
  const int fw = nslice * BN + wave * 32;  // first column of this wave (relu^2 / dense)

  // ---- resident W: fragment [j][s] holds W row fw + 8 (r >> 2) + 4 j + (r & 3), r = lane & 15,
  // k = 128 grp + 8 s. MFMA output element e of column block j in lane l is then column
  // fw + 8 (l >> 4) + 4 j + e: the lane's 8 columns are contiguous.
  bf16x8 wr[2][KS];
  {
    const int r = lane & 15;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int lcol = 8 * (r >> 2) + 4 * j + (r & 3);
      const long n = QK ? qk_col(nslice, wave, lcol) : fw + lcol;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const long k = 128 * grp + 8 * s;  // 8 columns of one 16-byte chunk, in either layout
        wr[j][s] = *reinterpret_cast<const bf16x8*>(g.W + (g.w_tiled ? wtile_offset(n, k, KD) : n * g.ldw + k));
      }
    }
  }
  // the resident fragments have landed before any LDS-bound load is issued, so no wait below covers them
  wait_vm_lgkm0<0>();

  auto blk_of = [&](int k) { return lo + stream + k * streams; };

  // ---- loads of block k into ring slot k % NB. Wave w fills x rows 4 w + q: lane L loads k 8 L .. 8 L + 7.
  // Lanes 0-7 load a_p, 8-15 b_next over the wave's 32 columns, 16-23 the block's 32 input-side dots; lane 0
  // the member's sign.
  // Blocks are issued in order k = 0, 1, 2, ...: the next one's first row, member and token, its x rows and
  // (relu^2) the lane's vector source advance by streams * R rows per call, with no integer division or 64-bit
  // multiply per block; the vector source is recomputed only when the block starts a new member.
  int nx_row = blk_of(0) * R;
  int nx_p = nx_row / g.T, nx_t0 = nx_row - nx_p * g.T;
  const int step_rows = streams * R;
  const unsigned lane16 = 16u * lane;  // the lane's byte offset in a 1 KiB row load
  const bf16* nx_x = g.A + (long)nx_p * g.a_mstride + (long)(nx_t0 + 4 * wave) * g.lda;
  const long x_step = (long)step_rows * g.lda, x_wrap = g.a_mstride - (long)g.T * g.lda;
  const long x_row = 2 * g.lda;  // bytes between the x rows one wave loads
  // relu^2: lanes 0-7 load a_p, 8-15 b_next (the wave's 32 columns of direction p >> pair_shift), 16-23 the
  // block's 32 input-side dots (rows row0 ..)
  auto vsrc_at = [&](int p, int row0) -> const float* {
    const int dir = p >> g.pair_shift;
    return lane < 8    ? g.ra[0] + (long)dir * g.ra_ld + fw + 4 * lane
           : lane < 16 ? g.rb_next + (long)dir * g.rb_next_ld + fw + 4 * (lane - 8)
                       : g.u + row0 + 4 * (lane - 16);
  };
  const float* nx_v = MODE == XS_RELU2 ? vsrc_at(nx_p, nx_row) : nullptr;
  const int v_step = lane >= 16 ? step_rows : 0;
  auto issue = [&](int k) {
    const int buf = k % NB, row0 = nx_row, p = nx_p, t0 = nx_t0, dir = p >> g.pair_shift;
    const char* xb = reinterpret_cast<const char*>(nx_x);
    const float* vsrc = nx_v;
    nx_row += step_rows;
    nx_t0 += step_rows;
    nx_x += x_step;
    if (nx_t0 >= g.T) {
      do {
        nx_t0 -= g.T;
        ++nx_p;
        nx_x += x_wrap;
      } while (nx_t0 >= g.T);
      if constexpr (MODE == XS_RELU2) nx_v = vsrc_at(nx_p, nx_row);
    } else if constexpr (MODE == XS_RELU2) {
      nx_v += v_step;
    }
    char* xsl = smem + buf * XBYTES + 4 * wave * XROW;
    dma_x4_s4<XROW>(xb, xb + x_row, xb + 2 * x_row, xb + 3 * x_row, lane16, xsl);
    // u_qkv rows of the block: 16 bytes per row (lanes 0-31)
    const float* urows = g.u + (long)row0 * 4;
    if constexpr (VV) {
      // a over the wave's 32 columns (lanes 0-7); wave 4: the block's u_qkv rows, the others the same rows
      // into a padding area (every wave issues DMA_PER_BLOCK loads per block)
      if (lane < 8) dma_x4_s(g.ra[2] + (long)dir * g.ra_ld + fw, lane16, &qv[buf].av[wave][0]);
      if (lane < R) dma_x4_s(urows, lane16, wave == 4 ? &qv[buf].uq[0][0] : &qpad[0][0]);
      return;
    }
    if constexpr (VE) {
      // a over the wave's 32 columns (lanes 0-7); one more load per wave: wave 4 the block's u_qkv rows, wave 5
      // its gate rows, wave 6 the token ids of the next block (when there is one), the others 4 padding bytes
      // (every wave issues DMA_PER_BLOCK loads per block)
      if (lane < 8) dma_x4_s(g.ra[2] + (long)dir * g.ra_ld + fw, lane16, &vv[buf].av[wave][0]);
      if (wave == 4) {
        if (lane < R) dma_x4_s(urows, lane16, &vv[buf].uq[0][0]);
      } else if (wave == 5) {
        dma_x4_s(g.gate + (long)row0 * 8, lane16, &vv[buf].gate[0][0]);
      } else if (wave == 6 && k + 1 < nb) {
        if (lane < R / 2) dma_x4_s(g.idx + (long)nx_p * g.tok_mstride + nx_t0, lane16, &vv[buf].tok[0]);
      } else if (lane == 0) {
        dma_x1(g.u, &vpad[wave]);
      }
      return;
    }
    if constexpr (QK) {
      // a over the wave's columns (lanes 0-7: local columns 4 L .. 4 L + 3 = dims 16 h + 4 (L / 2) + 32 (L % 2)
      // .. + 3); then wave 0-3: cos / sin rows (1 KiB each), wave 4: the block's u_qkv rows, waves 5-7: the same rows
      // into a padding area (every wave issues DMA_PER_BLOCK loads per block)
      const int seg = nslice >> 1;
      if (lane < 8)
        dma_x4_s(g.ra[seg] + (long)dir * g.ra_ld + qk_col(nslice, wave, 0) - seg * 512, 128u * (lane & 1) + 16u * (lane >> 1),
                 &qv[buf].av[wave][0]);
      if (wave < 4) {
        const bf16* tab = (wave >> 1) ? g.rot_sin : g.rot_cos;
        dma_x4_s(tab + (long)(t0 + 16 * (wave & 1)) * 32, 64u * (lane >> 2) + 16u * ((lane & 3) ^ ((lane >> 4) & 3)),
                 &qv[buf].cs[wave >> 1][16 * (wave & 1)][0]);
      } else if (lane < R) {
        dma_x4_s(urows, lane16, wave == 4 ? &qv[buf].uq[0][0] : &qpad[0][0]);
      }
      return;
    }
    if constexpr (MODE == XS_RELU2) {
      if (lane < 24) dma_x4(vsrc, &svec[buf][wave][0]);
      if (lane == 0) dma_x1(g.sign + p, &svec[buf][wave][SIGN_OFF]);
    }
  };

  // Block k has landed for this wave once at most nd * DMA_PER_BLOCK + ne * STORES_PER_EPI later operations
  // are outstanding: the nd later load groups and the stores of the ne epilogues issued since.
  auto wait_block = [&](int nd, int ne) {
    constexpr int D = DMA_PER_BLOCK<MODE>, S = STORES_PER_EPI;
    switch (nd * 3 + ne) {
      case 0: wait_vm_lgkm0<0>(); break;
      case 1: wait_vm_lgkm0<S>(); break;
      case 2: wait_vm_lgkm0<2 * S>(); break;
      case 3: wait_vm_lgkm0<D>(); break;
      case 4: wait_vm_lgkm0<D + S>(); break;
      case 5: wait_vm_lgkm0<D + 2 * S>(); break;
      case 6: wait_vm_lgkm0<2 * D>(); break;
      case 7: wait_vm_lgkm0<2 * D + S>(); break;
      default: wait_vm_lgkm0<2 * D + 2 * S>(); break;
    }
  };

  f32x4 accA[2][2], accB[2][2];
  float ev_a[8], ev_u[2], ev_dot[2];
  unsigned ev_bp[4], ev_h[2][4];
  float ev_v[2][8], ev_ss[2];   // q|k: rotated values and the wave's sums of squares per row half
  // value embedding: block k's term gate (W[idx] + s a[idx] b) per lane, read in iteration k (after its gather
  // landed) and added by block k's epilogue in iteration k + 1: ve_x = W[idx] + s a[idx] b over the lane's 8
  // columns of rows r and r + 16, ve_g = the rows' gates for the wave's head
  float ve_x[2][8], ve_g[2];

  // The gather of block k's embedding rows into this wave's VeRows (VE_DMA loads): tk[q] is the token of block
  // row r = 8 q + lane / 8, whose physical chunk lane % 8 receives logical chunk (lane % 8) ^ ((r / 2) % 8)
  // (columns 4 c .. 4 c + 3 of the wave's 32); tka the token of row lane % 32 (lanes 0-31 load a[dir, tok]).
  auto ve_issue = [&](int k, const int64_t(&tk)[4], int64_t tka) {
    const int p = blk_of(k) * R / g.T, dir = p >> g.pair_shift;
    VeRows& vr = ver[wave];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = 8 * q + (lane >> 3);
      dma_x4(g.ve_w + tk[q] * 512 + fw + 4 * ((lane & 7) ^ ((r >> 1) & 7)), &vr.w[8 * q][0]);
    }
    if (lane < 8) dma_x4_s(g.ve_b + (long)dir * 512 + fw, lane16, &vr.b[0]);
    if (lane < R) dma_x1(g.ve_a + (long)dir * g.ve_v + tka, &vr.a[0]);
  };
  // ... of block k + 1, from the token ids that arrived with block k
  auto ve_next = [&](int k) {
    const int64_t* tt = vv[k % NB].tok;
    int64_t tk[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) tk[q] = tt[8 * q + (lane >> 3)];
    ve_issue(k + 1, tk, tt[lane & 31]);
  };
  // block k's term from its landed gather and its gate / sign rows (EPI_QKV's arithmetic, per element)
  auto ve_read = [&](int k) {
    const VeVec& q = vv[k % NB];
    const VeRows& vr = ver[wave];
    const int r = lane & 15, head = fw >> 6;
    const float4 b0 = *reinterpret_cast<const float4*>(&vr.b[8 * grp]);
    const float4 b1 = *reinterpret_cast<const float4*>(&vr.b[8 * grp + 4]);
    const float bb[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = 16 * i + r;
      const float sa = q.uq[row][3] * vr.a[row];
      ve_g[i] = q.gate[row][head];
      const int sw = (row >> 1) & 7;
      const float4 w0 = *reinterpret_cast<const float4*>(&vr.w[row][4 * ((2 * grp) ^ sw)]);
      const float4 w1 = *reinterpret_cast<const float4*>(&vr.w[row][4 * ((2 * grp + 1) ^ sw)]);
      const float ww[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
      for (int c = 0; c < 8; ++c) ve_x[i][c] = ww[c] + sa * bb[c];
    }
  };
  bf16x4 ev_cs[2][2];           // q|k: cos / sin of the lane's 4 rotary pairs for rows r, r + 16
  const int qk_ocol = QK ? qk_col(nslice, wave, 8 * grp) : 0;  // the lane's first output column
  // Stores of a row half go to a uniform base (the half's first row, the wave's first column) plus a per-lane
  // byte offset fixed for the kernel: row lane % 16, the lane's 8 columns.
  const int col0 = QK ? qk_col(nslice, wave, 0) : fw;
  const unsigned st_off = 2u * (unsigned)((lane & 15) * g.ldo + (QK ? qk_ocol - col0 : 8 * grp));

  // TILE16 (c_fc h): the half's 1 KiB tile of the wave's 32 columns, 16-byte unit 4 r + (grp ^ ((r / 2) % 4))
  const unsigned tile_off = 16u * (unsigned)(4 * (lane & 15) + (grp ^ (((lane & 15) >> 1) & 3)));
  // the block's first output row at the wave's first column; row half i adds 16 i rows (one base per block for
  // both halves' stores)
  auto blk_base = [&](int blk) { return g.out_bf16 + (long)blk * (R * g.ldo) + col0; };
  auto half_base = [&](int blk, int i) { return blk_base(blk) + 16 * i * g.ldo; };
  // relu^2 h, the lane's byte offset from half_base: row-major (st_off) or TILE16 (tile_off into the wave's 1 KiB
  // tile of each 16-row half, which starts (fw / 32) * 512 elements into the half's first row)
  const unsigned h_lane = g.out_tiled ? tile_off + 2u * (unsigned)((fw >> 5) * 512 - col0) : st_off;
  // The epilogues of blocks 0, 1, 2, ... run in order, one per iteration k >= 1 and the last after the loop:
  // ep_base is the base of the next one (every mode but q|k, which stores a block one iteration later), advanced
  // by one block of rows after each, with no 64-bit multiply per block.
  bf16* ep_base = blk_base(blk_of(0));
  const long ep_step = (long)streams * R * g.ldo;
  auto store_half = [&](int i, u32x4 v) {
    *reinterpret_cast<u32x4*>(reinterpret_cast<char*>(ep_base + 16 * i * g.ldo) + st_off) = v;
  };
  // q|k: the lane's dims d0 .. d0 + 3 at st_off, their partners d0 + 32 .. at st_off + 64 bytes
  auto store_half_qk = [&](int blk, int i, u32x4 v) {
    char* b = reinterpret_cast<char*>(half_base(blk, i)) + st_off;
    *reinterpret_cast<uint2*>(b) = make_uint2(v[0], v[1]);
    *reinterpret_cast<uint2*>(b + 64) = make_uint2(v[2], v[3]);
  };

  // Stage st (0 .. 15) of the epilogue of block pk (ring slot pbuf) from acc:
  //   0: vectors from LDS; 1-4 / 7-10: column pairs of row half 0 / 1; 5 / 11: h store and first shuffle;
  //   6 / 12: second shuffle and the wave partial into LDS.
  auto epi_stage = [&](const f32x4 (&acc)[2][2], int pk, int pbuf, int st) {
    const char* vw = &svec[pbuf][wave][0];
    if constexpr (VV || VE) {
      // stages 0: the wave's a; 1-4 / 6-9: v = bf16(dense) + s bf16(u_v) a of row half 0 / 1 (fp32, as the
      // reference's lowrank output), plus the gated embedding term in VE mode, as fp16 pairs; 5 / 10: the row
      // half's store
      const float* avw = VE ? &vv[pbuf].av[wave][0] : &qv[pbuf].av[wave][0];
      if (st == 0) {
        // a over the wave's own columns (this wave's own load); ev_u was read in the block's own iteration
        const float4 a0 = *reinterpret_cast<const float4*>(avw + 8 * grp);
        const float4 a1 = *reinterpret_cast<const float4*>(avw + 8 * grp + 4);
        ev_a[0] = a0.x, ev_a[1] = a0.y, ev_a[2] = a0.z, ev_a[3] = a0.w;
        ev_a[4] = a1.x, ev_a[5] = a1.y, ev_a[6] = a1.z, ev_a[7] = a1.w;
        return;
      }
      if (st > 10) return;
      const int i = st < 6 ? 0 : 1, sub = st - (i ? 6 : 1);
      if (sub < 4) {
        const int j = sub >> 1, e0 = (sub & 1) * 2, c = 4 * j + e0;
        float v0, v1;
        bf16r2(acc[i][j][e0], acc[i][j][e0 + 1], v0, v1);
        v0 += ev_u[i] * ev_a[c];
        v1 += ev_u[i] * ev_a[c + 1];
        if constexpr (VE) {
          // value embedding (train/val/eggroll.py:85-89): v += 2 sigmoid(gate) (W[idx] + s a[idx] b)
          v0 += ve_g[i] * ve_x[i][c];
          v1 += ve_g[i] * ve_x[i][c + 1];
        }
        ev_h[i][sub] = pack_f16(v0, v1);
      } else {
        store_half(i, u32x4{ev_h[i][0], ev_h[i][1], ev_h[i][2], ev_h[i][3]});
      }
      return;
    }
    if constexpr (QK) {
      // Iteration k runs, for block pk - 1 (held from iteration k - 1): stages 0 / 1, the head's RMSNorm
      // (utils/model.py:46-47, eps = 2^-23) of row half 0 / 1 from both waves' sums of squares, written
      // to LDS last iteration and visible since this iteration's barrier, and the fp16 store; for block pk:
      // stage 2 the wave's a, 3-6 / 8-11 v = bf16(dense) + s bf16(u) a of row half 0 / 1, 7 / 12 rotary
      // (utils/model.py:55-58) and the wave's sum of squares into LDS.
      const QkVec& q = qv[pbuf];
      const int r = lane & 15, seg = nslice >> 1;
      if (st < 2) {
        if (pk < 1) return;
        const int i = st;
        const float tot = ev_ss[i] + ssq[(pk - 1) & 1][16 * i + r][wave ^ 1];
        // q (segment 0) leaves pre-multiplied by log2(e) / 8, the attention's score scale in base-2 units
        const float rn = rsqrtf(tot * (1.f / 64.f) + 1.1920928955078125e-07f) * (seg ? 1.f : 0.18033688011112042f);
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = pack_f16(ev_v[i][2 * e] * rn, ev_v[i][2 * e + 1] * rn);
        store_half_qk(blk_of(pk - 1), i, o);
        return;
      }
      if (pk < 0 || st > 12) return;
      if (st == 2) {
        // a over the wave's own columns (this wave's own load); ev_u and ev_cs were read in the block's own
        // iteration
        const float4 a0 = *reinterpret_cast<const float4*>(&q.av[wave][8 * grp]);
        const float4 a1 = *reinterpret_cast<const float4*>(&q.av[wave][8 * grp + 4]);
        ev_a[0] = a0.x, ev_a[1] = a0.y, ev_a[2] = a0.z, ev_a[3] = a0.w;
        ev_a[4] = a1.x, ev_a[5] = a1.y, ev_a[6] = a1.z, ev_a[7] = a1.w;
        return;
      }
      const int i = st < 8 ? 0 : 1, sub = st - (i ? 8 : 3);
      if (sub < 4) {
        const int j = sub >> 1, e0 = (sub & 1) * 2, c = 4 * j + e0;
        bf16r2(acc[i][j][e0], acc[i][j][e0 + 1], ev_v[i][c], ev_v[i][c + 1]);
        ev_v[i][c] += ev_u[i] * ev_a[c];
        ev_v[i][c + 1] += ev_u[i] * ev_a[c + 1];
      } else {
        // pair (d, d + 32) = (x1, x2) of elements e, e + 4: [x1 cos + x2 sin, -x1 sin + x2 cos]
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x1 = ev_v[i][e], x2 = ev_v[i][e + 4];
          const float cv = (float)ev_cs[i][0][e], sv = (float)ev_cs[i][1][e];
          const float y1 = x1 * cv + x2 * sv, y2 = x2 * cv - x1 * sv;
          ev_v[i][e] = y1;
          ev_v[i][e + 4] = y2;
          ss += y1 * y1 + y2 * y2;
        }
        ss = sum_rows4(ss);
        ev_ss[i] = ss;
        if (grp == 0) ssq[pk & 1][16 * i + r][wave] = ss;
      }
      return;
    }
    if constexpr (DENSE) {
      // stages 1-4 / 7-10: bf16 pairs of row half 0 / 1; 5 / 11: the row half's store
      if (st == 0 || st > 11 || st == 6) return;
      const int i = st < 7 ? 0 : 1, sub = st - (i ? 7 : 1);
      if (sub < 4) {
        const int j = sub >> 1, e0 = (sub & 1) * 2;
        ev_h[i][sub] = pack_bf16(acc[i][j][e0], acc[i][j][e0 + 1]);
      } else {
        store_half(i, u32x4{ev_h[i][0], ev_h[i][1], ev_h[i][2], ev_h[i][3]});
      }
      return;
    }
    if (st == 0) {
      const float4 a0 = *reinterpret_cast<const float4*>(vw + 32 * grp);
      const float4 a1 = *reinterpret_cast<const float4*>(vw + 32 * grp + 16);
      ev_a[0] = a0.x, ev_a[1] = a0.y, ev_a[2] = a0.z, ev_a[3] = a0.w;
      ev_a[4] = a1.x, ev_a[5] = a1.y, ev_a[6] = a1.z, ev_a[7] = a1.w;
      const float4 b0 = *reinterpret_cast<const float4*>(vw + 128 + 32 * grp);
      const float4 b1 = *reinterpret_cast<const float4*>(vw + 128 + 32 * grp + 16);
      ev_bp[0] = pack_bf16(b0.x, b0.y), ev_bp[1] = pack_bf16(b0.z, b0.w);
      ev_bp[2] = pack_bf16(b1.x, b1.y), ev_bp[3] = pack_bf16(b1.z, b1.w);
      const float sg = *reinterpret_cast<const float*>(vw + SIGN_OFF);
      const float* uw = reinterpret_cast<const float*>(vw + 256);
      ev_u[0] = sg * bf16r(uw[lane & 15]);
      ev_u[1] = sg * bf16r(uw[16 + (lane & 15)]);
      return;
    }
    if (st > 12) return;
    const int i = st < 7 ? 0 : 1, sub = st - (i ? 7 : 1);
    const int lr = 16 * i + (lane & 15);
    if (sub < 4) {
      // columns c, c + 1 of the lane's 8: dense part rounded to bf16 (autocast GEMM output), fp32
      // rank-1 correction, relu^2, bf16
      const int j = sub >> 1, e0 = (sub & 1) * 2, c = 4 * j + e0;
      float v0, v1;
      bf16r2(acc[i][j][e0], acc[i][j][e0 + 1], v0, v1);
      v0 += ev_u[i] * ev_a[c];
      v1 += ev_u[i] * ev_a[c + 1];
      const unsigned h2 = relu2_bf16x2(v0, v1);
      ev_h[i][sub] = h2;
      ev_dot[i] = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(h2), as_bf16x2(ev_bp[sub]), sub == 0 ? 0.f : ev_dot[i], false);
    } else if (sub == 4) {
      // row-major: 16 rows x 64 bytes per instruction; TILE16: one contiguous 1 KiB tile (16 rows, the
      // wave's 32 columns), eight whole 128-byte lines
      const u32x4 hv = u32x4{ev_h[i][0], ev_h[i][1], ev_h[i][2], ev_h[i][3]};
      store_stream_x4_s(ep_base + 16 * i * g.ldo, h_lane, hv);
      const f32pair a = rowpair16(ev_dot[i]);  // rows 0 + 1 and 2 + 3 of the 16-lane rows
      ev_dot[i] = a.lo + a.hi;
    } else {
      const f32pair b = halves32(ev_dot[i]);
      ev_dot[i] = b.lo + b.hi;
      red[pk & 1][lr][wave] = ev_dot[i];  // the row's four lanes write the same value
    }
  };
  // The per-block vectors one wave loads for all eight (the u_qkv rows, whose u and sign give ev_u; q|k: also the
  // rotary rows, loaded by waves 0-3) are read into registers in the iteration of their own block k, after the
  // epilogue of block k - 1 has used the previous ones (MFMA step 13). Block k's ring slot is refilled at the end
  // of iteration k + 1, after that iteration's barrier, which every wave passes only once its reads of iteration
  // k are complete; an epilogue read of iteration k + 1 would race with a faster wave's refill.
  auto read_shared = [&](int k) {
    const int buf = k % NB, r = lane & 15;
    if constexpr (VV || VE) {
      const float(*uqr)[4] = VE ? vv[buf].uq : qv[buf].uq;
      const float4 u0 = *reinterpret_cast<const float4*>(&uqr[r][0]);
      const float4 u1 = *reinterpret_cast<const float4*>(&uqr[16 + r][0]);
      ev_u[0] = u0.w * bf16r(u0.z);
      ev_u[1] = u1.w * bf16r(u1.z);
    } else if constexpr (QK) {
      const QkVec& q = qv[buf];
      const int seg = nslice >> 1;
      const float4 u0 = *reinterpret_cast<const float4*>(&q.uq[r][0]);
      const float4 u1 = *reinterpret_cast<const float4*>(&q.uq[16 + r][0]);
      ev_u[0] = u0.w * bf16r(seg ? u0.y : u0.x);
      ev_u[1] = u1.w * bf16r(seg ? u1.y : u1.x);
      const int dd = (qk_ocol & 63) & 31;  // the lane's first dim d0 (< 32): 4 dims, half of a 16-byte chunk
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int c = 0; c < 2; ++c)
          ev_cs[i][c] = *reinterpret_cast<const bf16x4*>(&q.cs[c][16 * i + r][8 * ((dd >> 3) ^ ((r >> 2) & 3)) + (dd & 7)]);
    }
  };
  // wave 0: the 8 wave partials of block pk's rows (written before the last barrier) -> one partial per row
  float* const up_lane = g.upart_out + (long)nslice * g.M + (long)blk_of(0) * R + lane;
  auto sum_partials = [&](int pk) {
    if (wave == 0 && lane < R) {
      const float4 p0 = *reinterpret_cast<const float4*>(&red[pk & 1][lane][0]);
      const float4 p1 = *reinterpret_cast<const float4*>(&red[pk & 1][lane][4]);
      const float s = ((((((p0.x + p0.y) + p0.z) + p0.w) + p1.x) + p1.y) + p1.z) + p1.w;
      up_lane[pk * step_rows] = s;
    }
  };

  // One iteration: wait for block k, MFMAs of block k into acc, interleaved step by step with the epilogue
  // of block k - 1 (epi) and the partial sums of block k - 2 (sum); then the loads of block k + NB - 1
  // into the slot block k - 1 used. A steady iteration (`steady`) is one with FIRST_STORE + 2 <= k <= nb - NB:
  // the previous iterations' stores and the later blocks' loads are all outstanding, so its waits, the sums and
  // the refill need no run-time case analysis (a cascade of scalar compares and branches otherwise). The q|k
  // and value-embedding modes keep the general form only: with a second copy of the loop hipcc spills their
  // registers to scratch.
  auto iter = [&](f32x4 (&acc)[2][2], const f32x4 (&prev)[2][2], int k, bool epi, bool sum, auto steady) {
    constexpr bool ST = decltype(steady)::value;
    // stores are issued in iterations j >= FIRST_STORE (q|k stores block j - 2's rows, the others block j - 1's)
    if constexpr (VE) {
      // Block k has landed once the operations issued after its loads are the only ones outstanding: in
      // iteration k - 1 the two stores of block k - 2's epilogue (k >= 2), block k's gather (VE_DMA) and block
      // k + 1's loads (when issued); block k's gather then has landed too.
      constexpr int D = DMA_PER_BLOCK<MODE>, E = VE_DMA;
      const bool xn = k + 1 < nb;
      if (k == 0) {
        if (xn) wait_vm_lgkm0<D>(); else wait_vm_lgkm0<0>();
      } else if (k == 1) {
        if (xn) wait_vm_lgkm0<E + D>(); else wait_vm_lgkm0<E>();
      } else {
        if (xn) wait_vm_lgkm0<2 + E + D>(); else wait_vm_lgkm0<2 + E>();
      }
    } else if constexpr (ST) {
      wait_vm_lgkm0<(NB - 2) * DMA_PER_BLOCK<MODE> + 2 * STORES_PER_EPI>();
    } else {
      wait_block(min(NB - 2, nb - 1 - k), min(2, max(0, k - FIRST_STORE)));
    }
    __builtin_amdgcn_s_barrier();
    const int pbuf = (k + NB - 1) % NB;
    // lane (row r = lane & 15, group grp): row-half i at LDS row 16 i + r, step s at chunk 16 grp + s
    const char* xsb = smem + (k % NB) * XBYTES + (lane & 15) * XROW + 256 * grp;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    bf16x8 xa[2], xb[2];
    xa[0] = *reinterpret_cast<const bf16x8*>(xsb);
    xa[1] = *reinterpret_cast<const bf16x8*>(xsb + 16 * XROW);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      bf16x8(&xc)[2] = (s & 1) ? xb : xa;
      bf16x8(&xn)[2] = (s & 1) ? xa : xb;
      if (s + 1 < KS) {
        xn[0] = *reinterpret_cast<const bf16x8*>(xsb + 16 * (s + 1));
        xn[1] = *reinterpret_cast<const bf16x8*>(xsb + 16 * XROW + 16 * (s + 1));
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma16x16x32(wr[j][s], xc[i], acc[i][j]);
      if (epi) epi_stage(prev, k - 1, pbuf, s);
      if constexpr (VE) {
        if (s == 11) {
          // block k's gather (issued in iteration k - 1, or before the ring for k = 0) has landed once block
          // k + 1's loads (when issued) and this iteration's two stores are the only later operations left
          if (k >= 1) {
            if (k + 1 < nb) wait_vm_lgkm0<DMA_PER_BLOCK<MODE> + 2>(); else wait_vm_lgkm0<2>();
          }
          ve_read(k);
        } else if (s == 12 && k + 1 < nb) {
          // this wave's reads of its gathered rows are complete before the next gather overwrites them
          wait_vm_lgkm0<63>();
          ve_next(k);
        }
      }
      if constexpr (MODE == XS_RELU2) {
        if (s == 13 && (ST || sum)) sum_partials(k - 2);
      }
      if constexpr (VV || VE || QK) {
        if (s == 13) read_shared(k);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (epi) ep_base += ep_step;
    if (ST || k + NB - 1 < nb) issue(k + NB - 1);
  };
  constexpr std::true_type steady{};
  constexpr std::false_type general{};
  constexpr bool STEADY_LOOP = !QK && !VE;

  if constexpr (VE) {
    // block 0's embedding gather goes out before the ring's loads, from token ids read straight from memory
    const int64_t* tt = g.idx + (long)nx_p * g.tok_mstride + nx_t0;
    int64_t tk[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) tk[q] = tt[8 * q + (lane >> 3)];
    ve_issue(0, tk, tt[lane & 31]);
  }
#pragma unroll
  for (int k = 0; k < NB - 1; ++k)
    if (k < nb) issue(k);

  iter(accA, accB, 0, false, false, general);
  int k = 1;
  for (; k + 1 < nb; k += 2) {
    if (STEADY_LOOP && k >= FIRST_STORE + 2 && k + 1 <= nb - NB) {
      if constexpr (STEADY_LOOP) {
        iter(accB, accA, k, true, true, steady);
        iter(accA, accB, k + 1, true, true, steady);
      }
    } else {
      iter(accB, accA, k, true, k >= 2, general);
      iter(accA, accB, k + 1, true, true, general);
    }
  }
  // tail: the last block's epilogue; partial sums of the last two blocks, each after a barrier
  int last = k - 1;
  if (k < nb) {
    iter(accB, accA, k, true, k >= 2, general);
    last = k;
  }
  wait_vm_lgkm0<0>();
  __builtin_amdgcn_s_barrier();
  if constexpr (MODE == XS_RELU2) {
    if (last >= 1) sum_partials(last - 1);
  }
#pragma unroll
  for (int st = 0; st < KS; ++st) {
    if (last == k) epi_stage(accB, last, last % NB, st);
    else epi_stage(accA, last, last % NB, st);
  }
  if constexpr (MODE == XS_RELU2) {
    wait_vm_lgkm0<0>();
    __builtin_amdgcn_s_barrier();
    sum_partials(last);
  }
  if constexpr (QK) {
    // the last block's normalisation, once every wave's sums of squares are in LDS
    __builtin_amdgcn_s_barrier();
    epi_stage(accA, last + 1, 0, 0);
    epi_stage(accA, last + 1, 0, 1);
  }
}

}  // namespace

int xs_relu2_parts(int N) { return (N > 0 && N % BN == 0) ? N / BN : 0; }

namespace {
bool xs_shape_ok(const LowrankGemmArgs& g) {
  return g.K == KD && g.N % BN == 0 && g.N > 0 && g.M % R == 0 && g.T % R == 0 && !g.a_tiled && g.lda % 8 == 0 &&
         (g.w_tiled || (g.ldw % 8 == 0 && g.ldw >= g.K)) && g.a_mstride % 8 == 0 && g.ldo % 8 == 0 && g.lda >= g.K &&
         g.ldo >= g.N &&
         g.A && g.W && g.out_bf16 && !(((uintptr_t)g.A | (uintptr_t)g.W | (uintptr_t)g.out_bf16) & 15);
}
template <int MODE>
int xs_launch(const LowrankGemmArgs& g, hipStream_t stream) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  const int nslices = g.N / BN, per_xcd = std::max(1, cus / 8);
  const int streams = std::max(1, per_xcd / nslices);
  hipLaunchKernelGGL((xs_kernel<MODE>), dim3(8 * streams * nslices), dim3(512), 0, stream, g);
  NOISE_CHECK_LAUNCH();
  return NOISE_OK;
}
}  // namespace

bool xs_relu2_supported(const LowrankGemmArgs& g) {
  return xs_shape_ok(g) && g.u_parts == 1 && g.u_ld == 1 && (!g.out_tiled || g.ldo % 32 == 0) && g.ra_ld % 4 == 0 &&
         g.rb_next_ld % 4 == 0;
}

int xs_relu2_launch(const LowrankGemmArgs& g, hipStream_t stream) {
  if (!xs_relu2_supported(g) || !g.sign || !g.u || !g.ra[0] || !g.rb_next || !g.upart_out || g.pair_shift < 0 ||
      g.pair_shift > 1)
    return NOISE_EINVAL;
  if (((uintptr_t)g.ra[0] | (uintptr_t)g.rb_next | (uintptr_t)g.u) & 15) return NOISE_EINVAL;
  return xs_launch<XS_RELU2>(g, stream);
}

bool xs_dense_supported(const LowrankGemmArgs& g) { return xs_shape_ok(g) && !g.out_tiled; }

int xs_dense_launch(const LowrankGemmArgs& g, hipStream_t stream) {
  if (!xs_dense_supported(g)) return NOISE_EINVAL;
  return xs_launch<XS_DENSE>(g, stream);
}

bool xs_qk_supported(const LowrankGemmArgs& g) {
  return xs_shape_ok(g) && !g.out_tiled && g.N == 1024 && g.u_ld == 4 && g.ra_ld % 4 == 0 && g.T % R == 0;
}

bool xs_v_supported(const LowrankGemmArgs& g) {
  return xs_shape_ok(g) && !g.out_tiled && g.N == 512 && g.u_ld == 4 && g.ra_ld % 4 == 0 && !g.gate;
}

int xs_v_launch(const LowrankGemmArgs& g, hipStream_t stream) {
  if (!xs_v_supported(g) || !g.u || !g.ra[2] || g.pair_shift < 0 || g.pair_shift > 1) return NOISE_EINVAL;
  if (((uintptr_t)g.ra[2] | (uintptr_t)g.u) & 15) return NOISE_EINVAL;
  return xs_launch<XS_V>(g, stream);
}

bool xs_ve_supported(const LowrankGemmArgs& g) {
  return xs_shape_ok(g) && !g.out_tiled && g.N == 512 && g.u_ld == 4 && g.ra_ld % 4 == 0 && g.gate && g.ve_w &&
         g.ve_a && g.ve_b && g.idx && g.ve_v > 0 && g.tok_mstride >= 0 && g.tok_mstride % 2 == 0 &&
         !(((uintptr_t)g.gate | (uintptr_t)g.ve_w | (uintptr_t)g.ve_b | (uintptr_t)g.idx) & 15);
}

int xs_ve_launch(const LowrankGemmArgs& g, hipStream_t stream) {
  if (!xs_ve_supported(g) || !g.u || !g.ra[2] || g.pair_shift < 0 || g.pair_shift > 1) return NOISE_EINVAL;
  if (((uintptr_t)g.ra[2] | (uintptr_t)g.u) & 15) return NOISE_EINVAL;
  return xs_launch<XS_VE>(g, stream);
}

int xs_qk_launch(const LowrankGemmArgs& g, hipStream_t stream) {
  if (!xs_qk_supported(g) || !g.u || !g.ra[0] || !g.ra[1] || !g.rot_cos || !g.rot_sin || g.pair_shift < 0 ||
      g.pair_shift > 1)
    return NOISE_EINVAL;
  if (((uintptr_t)g.ra[0] | (uintptr_t)g.ra[1] | (uintptr_t)g.u | (uintptr_t)g.rot_cos | (uintptr_t)g.rot_sin) & 15)
    return NOISE_EINVAL;
  return xs_launch<XS_QK>(g, stream);
}
