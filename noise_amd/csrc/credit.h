// Internal interface of the credit-scoring kernels (not part of the C ABI).
#pragma once
#include <hip/hip_runtime.h>

struct MovedHeadsArgs {
  const float* raw;    // [B, T, H, 64]
  const __bf16* a;     // [n, B, T, H, 64]
  float sigma;
  const float* cos;    // [>= T, 32]
  const float* sin;
  __bf16* out;         // row (j, b, t) at out + ((j * B + b) * T + t) * ldo, head h at columns h * 64
  long ldo;
  int n, B, T, H;
  long rows;           // n * B * T * H
};

struct HeadScoresArgs {
  const __bf16* out;       // attention output of the draws, row (j, b, t) at out + ((j * B + b) * T + t) * ld_out
  long ld_out;
  const float* baseline;   // [B, T, H, 64]
  const float* hub;        // [B, T, H, 64]
  float* score;            // [B, H, T, n]
  int n, B, T, H;
  long rows;               // n * B * T * H
};

struct CodeEstimateArgs {
  const float* credited;   // [B, H, T, n]
  const __bf16* a;         // [n, B, T, H, 64]
  float* est;              // [B, T, H, 64]
  int n, T, H;
  long elems;              // B * T * H * 64
};

struct KeyFilterArgs {
  const __bf16* filt;      // [BH, T, T] matched filter (attention map transposed and row-normalised)
  const float* score;      // [BH, T, n] query scores
  float* out;              // [BH, T, n] bf16-rounded key scores, as fp32
  int BH, T, n;
};

int moved_heads_launch(const MovedHeadsArgs& g, hipStream_t s);
int key_filter_launch(const KeyFilterArgs& g, hipStream_t s);
int head_scores_launch(const HeadScoresArgs& g, hipStream_t s);
int code_estimate_launch(const CodeEstimateArgs& g, hipStream_t s);
