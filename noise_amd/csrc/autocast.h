// Internal interface of the bf16-autocast row kernels (not part of the C ABI): the clean forward at the rounding
// points utils/eval.py gives GPT.forward (torch bf16 autocast, bf16 embedding tables). Rows are [M, 512] (the
// stream) or [M, 1536] (q | k | v), one 64-lane wave per row.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

struct AcStreamArgs {
  const __bf16* x_in;     // [M, 512] bf16 residual stream; null: x0 itself (block 0)
  const float* emb_w;     // [V, 512] token-embedding table holding bf16 values; x0 = bf16(norm(emb_w[tok]))
  long V;
  const int64_t* idx;     // row r = (p, t) reads token idx[p * idx_mstride + t]
  long idx_mstride;
  const __bf16* add[2];   // bf16 block outputs added in order, each sum rounded to bf16 (null: none)
  const float* lambda_r;  // 0-d fp32 scalars of the mix; null: no mix
  const float* lambda_0;
  __bf16* x_out;          // [M, 512] the stream after the adds and the mix; nullable
  __bf16* h;              // [M, 512] bf16(norm(x)); nullable
  const float* gate_w;    // [8, 32] ve_gate weight, or null
  float* gate;            // [M, 8] the bf16 gate values 2 sigmoid(ve_gate(h[:32]))
  int M, T;
};

struct AcQkvArgs {
  __bf16* qkv;            // [M, 1536] bf16 GEMM output q | k | v, updated in place
  const __bf16* rot_cos;  // [>= T, 32] bf16 rotary tables
  const __bf16* rot_sin;
  const float* gate;      // [M, 8] or null (no value embedding)
  const float* ve_w;      // [V, 512] value-embedding table holding bf16 values
  long V;
  const int64_t* idx;
  long idx_mstride;
  int M, T;
};

int ac_stream_launch(const AcStreamArgs& g, hipStream_t s);
int ac_qkv_launch(const AcQkvArgs& g, hipStream_t s);
