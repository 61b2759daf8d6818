// Shared device helpers for the gfx950 kernels of libnoise_hip.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Status codes returned by every entry point (0 = ok; positive = hipError_t).
#define NOISE_OK 0
#define NOISE_EINVAL (-1)     // bad shape / stride / pointer
#define NOISE_ENOSPC (-2)     // workspace too small
#define NOISE_ENOTSUP (-3)    // shape outside what the kernels tile

#define NOISE_CHECK_LAUNCH()                                   \
  do {                                                         \
    hipError_t e_ = hipGetLastError();                         \
    if (e_ != hipSuccess) return (int)e_;                      \
  } while (0)

// Round-to-nearest-even float -> bf16 (v_cvt_pk_bf16_f32 on gfx950), the same rounding torch uses.
__device__ __forceinline__ bf16 to_bf16(float x) { return (bf16)x; }
__device__ __forceinline__ float bf16r(float x) { return (float)(bf16)x; }

__device__ __forceinline__ f32x4 mfma16x16x32(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32x32x16(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Butterfly reductions inside groups of lanes.
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = WIDTH / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
template <int WIDTH>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int o = WIDTH / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// XCD-aware workgroup remap: the hardware deals consecutive workgroup ids round-robin over the 8 XCDs;
// this returns a logical tile id such that each XCD works on one contiguous range of tiles (shared
// operand rows then stay in that XCD's L2).
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
  constexpr int XCDS = 8;
  if (nblocks % XCDS != 0) return bid;
  return (bid % XCDS) * (nblocks / XCDS) + bid / XCDS;
}

// 16-byte non-temporal vector store (global_store_dwordx4 ... nt, the encoding the compiler gives
// __builtin_nontemporal_store on gfx950): the line is marked for early eviction instead of staying dirty in
// L2, so later L2 fills of the same kernel wait less on write-backs. Measured on MI355X: a kernel that
// streams its operand from HBM while writing 4x as many bytes runs about 10% faster with these stores.
// Issued from inline assembly so a 16-byte vector keeps one instruction; a vmcnt wait the compiler places
// for its own loads only becomes stricter for it (vector memory operations complete in issue order). The
// trailing s_nop 1 is the hazard wait the compiler would insert itself: a VALU write to the data VGPRs of a
// preceding store wider than 8 bytes needs 2 wait states on gfx940+, or the store may pick up the new value.
__device__ __forceinline__ void store_stream_x4(void* p, u32x4 v) {
  asm volatile("global_store_dwordx4 %0, %1, off nt\n\ts_nop 1" : : "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store_stream_x4(void* p, unsigned a, unsigned b, unsigned c, unsigned d) {
  store_stream_x4(p, u32x4{a, b, c, d});
}
__device__ __forceinline__ void store_stream_f4(void* p, float a, float b, float c, float d) {
  store_stream_x4(p, u32x4{__float_as_uint(a), __float_as_uint(b), __float_as_uint(c), __float_as_uint(d)});
}
