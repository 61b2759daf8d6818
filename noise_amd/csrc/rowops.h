// Internal interface of the row kernels (not part of the C ABI). Rows are [M = members x T, 512];
// member p = row / T uses perturbation row dir = p >> pair_shift and sign[p].
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

// A c_proj output not yet added to the residual stream (deferred residual): row r receives
// y[r, c] + s_p bf16(sum_q u[r * u_ld + q * u_qstride]) a[dir * 512 + c], with y = bf16(x W^T) from an
// EPI_DENSE GEMM. y == null: nothing pending.
struct Pending {
  const __bf16* y;
  const float* u;
  int u_parts;
  long u_ld, u_qstride;
  const float* a;
};
constexpr int MAX_PENDING = 2;

struct EmbedNormArgs {
  const float* w;        // [V, 512] embedding table
  const float* a;        // [dirs, V] output-side (row) vectors
  const float* b;        // [dirs, 512] input-side vectors
  long V;
  const float* sign;
  const int64_t* idx;    // [T]
  int M, T, pair_shift;
  float* x0;             // [M, 512] fp32 out
};

// Source of x0 = norm(lowrank_embed(w, a, b)) rows, recomputed where they are read instead of stored.
struct EmbedSrc {
  const float* w;        // [V, 512] embedding table
  const float* a;        // [dirs, V]
  const float* b;        // [dirs, 512]
  long V;
  const int64_t* idx;    // token ids: member p, position t reads idx[p * mstride + t]
  long mstride;          // 0: every member reads the same T ids; T: one sequence per member
};

struct BlockEntryArgs {
  const float* x_in;     // [M, 512] residual stream before the mix; null: x0 itself (block 0)
  const float* x0;       // [M, 512]; null: recomputed from emb
  EmbedSrc emb;
  float* x_out;          // mixed stream (may alias x_in)
  __bf16* h;             // [M, 512] bf16(norm(x))
  float* u_qkv;          // [M, 4] bf16-rounded dots with b_q, b_k, b_v (4th slot zero)
  const float* b_qkv[3];  // [dirs, 512] each
  const float* lambda_r;  // this block's resid_lambdas / x0_lambdas entries
  const float* lambda_0;
  const float* eps_r;    // resid_lambdas noise: eps_r[dir * eps_ld]
  const float* eps_0;
  long eps_ld;
  const float* sign;
  int M, T, pair_shift;
  // value-embedding gate (null gate_w: none at this block)
  const float* gate_w;   // [8, 32]
  const float* gate_a;   // [dirs, 8]
  const float* gate_b;   // [dirs, 32]
  float* gate;           // [M, 8] 2 sigmoid(...)
  // deferred residuals added (in order) to x_in before the mix
  Pending pend[MAX_PENDING];
  int npend;
};

struct NormDotArgs {
  const float* x;
  __bf16* h;
  const float* b;        // [dirs, 512]
  float* u;              // [M]
  const float* sign;
  int M, T, pair_shift;
  // deferred residuals added (in order) to x before the norm; x itself is not written back
  Pending pend[MAX_PENDING];
  int npend;
};

struct HeadNormArgs {
  const void* x;         // [M, 512] fp32, or bf16 when x_bf16
  int x_bf16;
  const float* gain;     // [512] or null
  __bf16* h;             // fp32_head 1: bf16 [M, 1024] = [hi | lo]; 2: fp16 [M, 512]; 0: bf16 [M, 512]
  const float* b;        // [dirs, 512]
  float* u;              // [M]
  const float* sign;
  int M, T, pair_shift;
  int fp32_head;         // operand format: 0 bf16(h gain), 1 bf16 [hi | lo] of h gain, 2 fp16(h) (no gain)
  // deferred residuals added (in order) to x (fp32 only) before the norm
  Pending pend[MAX_PENDING];
  int npend;
  int tiled;             // the operand rows written in TILE16 (M % 16 == 0)
};

// Reductions of the per-token losses logsumexp(z'_t) - z'_t[target_t].
enum : int {
  CE_MEMBER_MEAN = 0,  // loss[p] = mean over member p's T tokens (every target valid)
  CE_NONE = 1,         // loss[row] per token; 0 where the target is -1 (ignored)
  CE_SUM = 2,          // loss[0] = sum over the tokens whose target is not -1
  CE_MEAN = 3,         // loss[0] = that sum / their count (NaN when every target is -1)
};
struct CeFinalizeArgs {
  const float* part;     // [members * T, parts] sums of exp(z)
  const float* tgt;      // [members * T] z at the target (written only where the target is valid)
  int parts, members, T;
  float* loss;           // [members] / [members * T] / [1] by reduction
  const int64_t* targets;  // member p, position t: targets[p * tgt_mstride + t]
  long tgt_mstride;
  int reduction;
};

int embed_norm_launch(const EmbedNormArgs& g, hipStream_t s);
// HBM streaming calibration: rows of in_kib KiB read and out_kib KiB written (1..4 each), one wave per row.
int hbm_stream_launch(const void* src, int in_kib, void* dst, int out_kib, long rows, hipStream_t s);
int block_entry_launch(const BlockEntryArgs& g, hipStream_t s);
int norm_dot_launch(const NormDotArgs& g, hipStream_t s);
int head_norm_launch(const HeadNormArgs& g, hipStream_t s);
int ce_finalize_launch(const CeFinalizeArgs& g, hipStream_t s);
int cast_launch(const float* in, __bf16* out, long n, int cols, int split, hipStream_t s);
// Row dots u[row] = bf16(sum_k x[row, k] * bf16(b[dir, k])) for a bf16 activation.
int rowdot_launch(const __bf16* x, long ldx, long x_mstride, int M, int K, int T, int pair_shift,
                  const float* b, long ldb, float* u, hipStream_t stream);
