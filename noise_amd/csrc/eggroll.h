// Internal interface of the EGGROLL update kernels (not part of the C ABI).
#pragma once
#include <hip/hip_runtime.h>

#define NOISE_FITNESS_ZSCORE 0
#define NOISE_FITNESS_RANK 1

struct OuterUpdateArgs {
  const float* a;  // [ndir, a_ld] output-side vectors (null: scalar 1, out must be 1)
  long a_ld;
  const float* b;  // [ndir, b_ld] input-side vectors
  long b_ld;
  const float* w;  // [ndir] direction weights
  int ndir, out, in;
  float scale;
  float* grad;     // [out, in]
};

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
int outer_update_launch(const OuterUpdateArgs& g, hipStream_t s);
int adam_launch(const AdamArgs& g, hipStream_t s);
