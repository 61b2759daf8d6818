// Internal interface of the low-rank-perturbed GEMM (not part of the C ABI).
#pragma once
#include <hip/hip_runtime.h>

struct LowrankGemmArgs {
  // A operand: row r (member p = r / T, token t = r % T) starts at A + p * a_mstride + t * lda.
  // a_mstride = T * lda for per-member activations, 0 for one activation broadcast to all members.
  const __bf16* A;
  long lda;
  long a_mstride;
  const __bf16* W;  // [N, K], K contiguous (nn.Linear orientation)
  long ldw;
  int M, N, K;
  int T;           // rows per member
  int pair_shift;  // perturbation row of member p is p >> pair_shift (1: antithetic pairs share a, b)
  const float* sign;  // [members] +-sigma
  const float* ra;    // output-side vectors a, row dir at ra + dir * ra_ld, N entries
  long ra_ld;
  const float* u;     // input-side dots x.b per row, as u_parts partial sums: u[row * u_parts + j]
  int u_parts;
  // outputs
  float* out_f32;     // EPI_STORE (optional) / EPI_RESID (accumulated in place)
  __bf16* out_bf16;   // EPI_STORE (optional) / EPI_RELU2
  long ldo;
  // EPI_RELU2: partial dots of the bf16 output with the next layer's input-side vector b_next
  const float* rb_next;
  long rb_next_ld;
  float* upart_out;   // [M, upart_ld]
  int upart_ld;       // = lowrank_gemm_parts(N)
};

// Number of partial row dots EPI_RELU2 writes per row for an N-column output (0: N unsupported).
int lowrank_gemm_parts(int N);
int lowrank_gemm_launch(int epi, const LowrankGemmArgs& g, hipStream_t stream);

// Row dots u[row] = bf16(sum_k x[row, k] * bf16(b[dir, k])) for a bf16 activation (rowops.hip).
int rowdot_launch(const __bf16* x, long ldx, long x_mstride, int M, int K, int T, int pair_shift,
                  const float* b, long ldb, float* u, hipStream_t stream);
