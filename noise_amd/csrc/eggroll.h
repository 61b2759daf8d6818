// Internal interface of the EGGROLL update kernels (not part of the C ABI).
#pragma once
#include <hip/hip_runtime.h>

#define NOISE_FITNESS_ZSCORE 0
#define NOISE_FITNESS_RANK 1

// One matrix of an update: grad [out, in] = scale * sum_j (w_j a_j[o]) b_j[i].
struct OuterUpdateArgs {
  const float* a;  // [ndir, a_ld] output-side vectors (null: scalar 1, out must be 1)
  long a_ld;
  const float* b;  // [ndir, b_ld] input-side vectors
  long b_ld;
  int out, in;
  float* grad;     // [out, in]
};

// Kernel-side form: up to OUTER_MAX matrices per launch, passed by value (under the 4 KiB argument limit),
// with the running total of 64 x 64 tiles.
constexpr int OUTER_MAX = 56;
struct OuterMat {
  const float* a;
  const float* b;
  float* grad;
  long a_ld, b_ld;
  int out, in, tiles_i, tile_end;
};
struct OuterBatchArgs {
  OuterMat m[OUTER_MAX];
  int n;
  const float* w;  // [ndir] direction weights, shared by every matrix
  int ndir;
  float scale;
};

// Rows of the noise buffer per (parameter, direction): buffer[offsets[directions[j]] ..] split into a [out]
// and b [in] (train/val/eggroll.py:122-128). Up to GATHER_MAX parameters per launch, passed by value.
constexpr int GATHER_MAX = 64;
struct GatherParam {
  const int64_t* offsets;  // [pairs] slice starts of this parameter
  float* a;                // [ndir, out]
  float* b;                // [ndir, in] (null when in == 0: a 1-D parameter's eps rows)
  int out, in;
};
struct GatherArgs {
  GatherParam p[GATHER_MAX];
  int n;
  const float* buffer;
  long buffer_len;
  const int64_t* directions;  // [ndir] pair indices
  int ndir, pairs;
};
int gather_rows_launch(const GatherParam* params, int n, const float* buffer, long buffer_len,
                       const int64_t* directions, int ndir, int pairs, hipStream_t s);

struct AdamArgs {
  float* param;
  const float* grad;
  float* m;
  float* v;
  long n;
  float step_size;  // lr / (1 - beta1^step)
  float beta1, beta2, eps;
  float bc2_sqrt;   // sqrt(1 - beta2^step)
};

int fitness_launch(const float* losses, int n, int pairs, int mode, float* fit, float* weight, hipStream_t s);
int outer_update_launch(const OuterUpdateArgs* mats, int n, const float* w, int ndir, float scale, hipStream_t s);
int adam_launch(const AdamArgs& g, hipStream_t s);

// Several tensors' Adam steps in one launch: up to ADAM_MAX tensors per launch, passed by value, with the running
// total of 256-element blocks (block b belongs to the first tensor whose block_end exceeds b).
constexpr int ADAM_MAX = 64;
struct AdamTensor {
  float* param;
  const float* grad;
  float* m;
  float* v;
  long n;
  float step_size, bc2_sqrt;
  long block_end;
};
struct AdamBatchArgs {
  AdamTensor t[ADAM_MAX];
  int n;
  float beta1, beta2, eps;
};
int adam_batch_launch(const AdamTensor* tensors, int n, float beta1, float beta2, float eps, hipStream_t s);
