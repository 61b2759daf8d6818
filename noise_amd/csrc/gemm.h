// Internal interface of the low-rank-perturbed GEMM (not part of the C ABI).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

// Epilogue kinds of lowrank_gemm_launch.
enum : int {
  EPI_STORE = 0,  // out = lowrank(x)                       -> fp32 and/or bf16 store
  EPI_RELU2 = 1,  // h = bf16(relu(lowrank(x))^2)            -> bf16 store + partial dots h.b_next per row
                  //                                         (weight-resident kernel of gemm_xs.hip, K = 512)
  EPI_RESID = 2,  // resid += lowrank(x)                     -> fp32 read-modify-write
  EPI_QKV = 3,    // q|k|v = lowrank(x) per 512-column segment; rotary + RMSNorm on q and k, gated value
                  // embedding added to v                   -> fp16 store of the fp32 values
  EPI_CE = 4,     // z = 15 tanh(lowrank(x) / 15); per row partial sum of exp(z) over each wave's columns
                  // and z at the target column             -> fp32 partials
  EPI_DENSE = 5,  // y = bf16(x W^T) only: the rank-1 term and the residual add are left to the row kernel
                  // that consumes y (a deferred residual)  -> bf16 store
  EPI_CE_F16 = 6, // EPI_CE on fp16 operands: A = fp16 h [M, a_fold], W = fp16 [W_hi | W_lo] (K = 2 a_fold), row n
                  // of W scaled by col_scale[n] (a power of two); the fp32 head at an 11-bit h and a 22-bit W
};

// TILE16 layout of a bf16 matrix [rows, cols] with leading dimension ld (rows % 16 == 0, ld % 32 == 0):
// element (r, c) lives at (r / 16) * 16 * ld + (c / 32) * 512 + 8 * p + c % 8, with
// p = 4 (r % 16) + (((c % 32) / 8) ^ (((r % 16) >> 1) & 3)). Each 1 KiB tile (16 rows x 32 columns) is
// contiguous and already in the order of the GEMM's swizzled 32-deep LDS stage, so one wave-wide LDS-DMA
// instruction moves one tile as eight whole 128-byte lines.
__host__ __device__ inline long tile16_offset(long r, long c, long ld) {
  const long rr = r & 15, p = 4 * rr + (((c & 31) >> 3) ^ ((rr >> 1) & 3));
  return (r >> 4) * 16 * ld + (c >> 5) * 512 + 8 * p + (c & 7);
}

// WTILE layout of a bf16 weight W [N, K] (N % 64 == 0, K % 32 == 0), the order in which the tile GEMM's
// 32-deep LDS stages hold it: the 1 KiB block (g, s) at element (g * K / 32 + s) * 512 holds columns
// 32 s .. 32 s + 31 of the 16 rows with tiled index i = 16 g + r (r < 16), row r of the block being weight row
// (i & ~63) + (r >> 2) * 16 + ((i & 63) >> 4) * 4 + (r & 3), its 16-byte chunk c at chunk c ^ ((r >> 1) & 3).
// Within each 64-row band, MFMA block j of a wave's 64 output columns then reads 16 consecutive LDS rows and
// a lane's 16 output columns are contiguous (the tile GEMM's transposed product). One wave-wide LDS-DMA
// instruction moves one block as eight whole 128-byte lines (row-major rows give 64-byte half lines, which
// the L2 -> LDS path serves at about half the rate).
__host__ __device__ inline long wtile_offset(long n, long k, long K) {
  const long loc = n & 63;
  const long i = (n & ~63L) + ((loc >> 2) & 3) * 16 + ((loc >> 4) << 2) + (loc & 3), r = i & 15;
  return ((i >> 4) * (K >> 5) + (k >> 5)) * 512 + 32 * r + 8 * (((k & 31) >> 3) ^ ((r >> 1) & 3)) + (k & 7);
}

struct LowrankGemmArgs {
  // A operand: row r (member p = r / T, token t = r % T) starts at A + p * a_mstride + t * lda.
  // a_mstride = T * lda for per-member activations, 0 for one activation broadcast to all members.
  // a_tiled: A is TILE16 with leading dimension lda over all M rows (requires a_mstride = T * lda).
  // a_fold > 0 (the fp32 head, K = 3 a_fold): A rows are [hi | lo] and W rows [W_hi | W_lo | W_hi]; the GEMM
  // forms hi W_hi + hi W_lo + lo W_hi with the three products interleaved per 32-deep block b: stage 3 b reads A
  // block b and W block b, stage 3 b + 1 A block b and W block a_fold / 32 + b, stage 3 b + 2 A block
  // a_fold / 32 + b and W block b (no stored second copy of hi; the repeated blocks come from L2).
  // EPI_CE_F16 (K = 2 a_fold): A rows are fp16 h and W rows [W_hi | W_lo]; stage 2 b reads A block b and W block
  // b, stage 2 b + 1 A block b again and W block a_fold / 32 + b.
  const __bf16* A;
  long lda;
  long a_mstride;
  int a_tiled;
  int a_fold;
  const __bf16* W;  // [N, K], K contiguous (nn.Linear orientation), or WTILE when w_tiled
  long ldw;         // row stride of a row-major W (ignored when w_tiled)
  int w_tiled;
  int M, N, K;
  int T;              // rows per member
  int pair_shift;     // perturbation row of member p is p >> pair_shift (1: antithetic pairs share a, b)
  const float* sign;  // [members] +-sigma
  // Output-side rank-1 vectors, per column segment of seg_n columns: column n of member p uses
  // ra[n / seg_n][dir(p) * ra_ld + n % seg_n]. One segment unless EPI_QKV.
  const float* ra[3];
  int seg_n;
  int seg0;           // EPI_QKV: index of the first segment this launch covers (2: v only)
  long ra_ld;
  // Input-side dots x.b, as u_parts partial sums: row r, segment s: sum_q u[r * u_ld + (s * u_parts + q) * u_qstride]
  // (u_qstride = 1: row-major partials; u_ld = 1, u_qstride = rows: part-major).
  const float* u;
  int u_parts;
  int u_ld;
  long u_qstride;
  // 1: autocast rounding points (the dense product and the dot rounded to bf16); 0: fp32 throughout.
  int round_bf16;
  // outputs
  float* out_f32;     // EPI_STORE (optional) / EPI_RESID (accumulated in place)
  __bf16* out_bf16;   // EPI_STORE (optional) / EPI_RELU2 / EPI_QKV
  long ldo;
  int out_tiled;      // EPI_RELU2: out_bf16 is TILE16 with leading dimension ldo
  // EPI_RELU2: partial dots of the bf16 output with the next layer's input-side vector b_next, part-major
  // [xs_relu2_parts(N), M]. EPI_CE: per-row partial sums, row-major [M, upart_ld].
  const float* rb_next;
  long rb_next_ld;
  float* upart_out;
  int upart_ld;       // EPI_CE: = lowrank_gemm_parts(N)
  // EPI_QKV: rotary tables (bf16 [>= T, 32]); optional gated value embedding for the v segment:
  // v += gate[r, head] * (ve_w[idx[t]] + s_p ve_a[dir, idx[t]] ve_b[dir]).
  const __bf16* rot_cos;
  const __bf16* rot_sin;
  const float* gate;     // [M, 8] (null: no value embedding)
  const float* ve_w;     // [V, 512]
  const float* ve_a;     // [dirs, V]
  const float* ve_b;     // [dirs, 512]
  long ve_v;             // V (row stride of ve_a)
  const int64_t* idx;    // token ids: member p, position t reads idx[p * tok_mstride + t]
  // EPI_CE: targets (member p, position t: targets[p * tok_mstride + t]; -1 = ignored; may be null when
  // logits is set); partial sums of exp(z) [M, upart_ld]; z at the target [M]; optionally the capped logits
  // z' fp32 [M, ldo]
  const int64_t* targets;
  float* ce_tgt;
  long tok_mstride;      // 0: one sequence shared by every member; T: one sequence per member
  float* logits;
  // EPI_CE_F16: W row n holds the weight row times col_scale[n] (a power of two), so that its fp16 halves keep
  // 22 significant bits whatever the row's magnitude; the epilogue divides it out exactly.
  const float* col_scale;
};

// WTILE copy (out, N * K bf16) of a row-major bf16 weight in [N, K] with row stride ld.
int weight_tiles_launch(const __bf16* in, long ld, int N, int K, __bf16* out, hipStream_t stream);
// The fp16 operand of EPI_CE_F16 from an fp32 weight w [N, 512] (row stride ldw) and an optional gain [512]
// folded in along K: row n of (w * gain) times scale[n] = 2^e (its largest magnitude in [2^14, 2^15)), split into
// fp16 hi = fp16(row) and lo = fp16(row - hi): out [N, 1024] = [hi | lo], WTILE when tiled, else row-major.
int head_weight_f16_launch(const float* w, long ldw, const float* gain, int N, int tiled, __bf16* out,
                           float* scale, hipStream_t stream);

// Number of per-row partials EPI_CE writes for an N-column output (0: N unsupported).
int lowrank_gemm_parts(int N);
int lowrank_gemm_launch(int epi, const LowrankGemmArgs& g, hipStream_t stream);

// The weight-resident K = 512 relu^2 GEMM (gemm_xs.hip): partials per row it writes for N columns (0: N
// unsupported), whether it tiles the shape, and the launch.
int xs_relu2_parts(int N);
bool xs_relu2_supported(const LowrankGemmArgs& g);
int xs_relu2_launch(const LowrankGemmArgs& g, hipStream_t stream);
// The same weight-resident kernel for the dense c_proj product y = bf16(x W^T) at K = 512 (row-major A and y).
bool xs_dense_supported(const LowrankGemmArgs& g);
int xs_dense_launch(const LowrankGemmArgs& g, hipStream_t stream);
// ... and for q | k (N = 1024 = c_q ; c_k): rank-1 term, rotary and the per-head RMSNorm in the epilogue.
// u rows [M, 4] = the bf16 dots with b_q, b_k, b_v and the member's sign; ra[0] / ra[1] = a_q / a_k.
bool xs_qk_supported(const LowrankGemmArgs& g);
int xs_qk_launch(const LowrankGemmArgs& g, hipStream_t stream);
// ... and for c_v without value embedding (N = 512, W and out already offset to the v segment; a = ra[2]).
bool xs_v_supported(const LowrankGemmArgs& g);
int xs_v_launch(const LowrankGemmArgs& g, hipStream_t stream);
// ... and for c_v with the gated value embedding (gate, ve_w, ve_a, ve_b, idx set; T a multiple of 32).
bool xs_ve_supported(const LowrankGemmArgs& g);
int xs_ve_launch(const LowrankGemmArgs& g, hipStream_t stream);
