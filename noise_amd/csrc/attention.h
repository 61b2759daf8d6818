// Internal interface of the attention kernel (not part of the C ABI).
#pragma once
#include <hip/hip_runtime.h>

// Formats of the q and k columns (values of the C ABI's qk_format).
// QK_BF16_V_BF16: q, k and v bf16 and the probabilities rounded to bf16 for P V (torch's bf16 attention operands)
enum : int { QK_BF16 = 0, QK_F16 = 1, QK_F16_Q_LOG2 = 2, QK_BF16_V_BF16 = 3 };

struct AttnArgs {
  const __bf16* qkv;  // [members * T, ldq] 16-bit rows; q at column h*64, k at koff + h*64, v (fp16; bf16 for QK_BF16_V_BF16) at
                      // voff + h*64
  long ldq;
  int koff, voff;
  __bf16* y;          // [members * T, ldy], head h at columns h*64 .. h*64+63
  long ldy;
  int members, T, H, window;
  int qk_norm;        // q and k rows are RMS-normalised (scores bounded by 8.03): no running maximum
  int qk_format;      // QK_BF16, QK_F16, QK_F16_Q_LOG2 (fp16, q pre-multiplied by log2(e) / 8: noise_qkv's output) or
                      // QK_BF16_V_BF16 (bf16 q, k, v and probabilities)
  // c_proj input-side dot partials: upart[row * upart_ld + h] = sum_d y[row, h*64+d] bf16(b_proj[dir, h*64+d])
  const float* b_proj;
  long b_ld;
  int pair_shift;
  float* upart;       // nullable
  int upart_ld;
  // per-(member, head) moments of y over tokens: partials [members, H, T/128, 2, 64] reduced into
  // mom_out [members, H, 2, 64] (mean of y, mean of y^2); nullable
  float* mom;
  float* mom_out;
};

// Floats of the moment partials workspace.
long attention_moment_partials(int members, int T, int H);
int attention_launch(const AttnArgs& g, hipStream_t s);
