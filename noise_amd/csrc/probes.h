// Internal interface of the readout-probe kernel (not part of the C ABI).
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

struct ProbeArgs {
  const float* base;        // [n, base_ld] logits W x of the clean streams
  long base_ld;
  const float* C;           // [P, c_ld] row j = W D_j
  long c_ld;
  const int64_t* rows;      // [n, K] directions of each token, or null: every direction (K == P)
  int K;
  const int64_t* y;         // [n] targets, -1 = none
  const float* steps;       // [n]
  const float* sq;          // [n] |x|^2
  const float* dots;        // [n, dots_ld] x . D (the K directions of the token)
  long dots_ld;
  const float* dir_sq;      // [P] |D_j|^2, or [n, K] per token (dir_sq_tok != 0)
  int dir_sq_tok;
  int n, V, P, width;
  float* out;               // [n, K]
};

int probe_launch(const ProbeArgs& g, hipStream_t stream);
