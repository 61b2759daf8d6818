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
// float(bf16(x)) in one instruction: v_cvt_pk_bf16_f32 with +0 as the low half leaves bf16(x) in the high half
// and zeros below it, which are the fp32 bits of bf16(x). (From C++ the compiler emits a conversion and a shift.)
__device__ __forceinline__ float bf16r(float x) {
  unsigned u;
  asm("v_cvt_pk_bf16_f32 %0, 0, %1" : "=v"(u) : "v"(x));
  return __uint_as_float(u);
}
// bf16r of two values (one instruction each).
__device__ __forceinline__ void bf16r2(float a, float b, float& ra, float& rb) {
  ra = bf16r(a);
  rb = bf16r(b);
}
typedef short s16x2 __attribute__((ext_vector_type(2)));
// The bf16 pair {bf16(relu(a)^2), bf16(relu(b)^2)} (low half a): a |a| and b |b| rounded as a pair, whose halves
// with the sign bit set (a < 0, or -0) become +0 by one packed 16-bit integer max with 0. For a > 0, a |a| is the
// same fp32 product as relu(a)^2; a NaN keeps its sign, so a positive NaN stays NaN (relu propagates NaN).
__device__ __forceinline__ unsigned relu2_bf16x2(float a, float b) {
  const bf16x2 p = {to_bf16(a * fabsf(a)), to_bf16(b * fabsf(b))};
  const s16x2 m = __builtin_elementwise_max(__builtin_bit_cast(s16x2, p), s16x2{0, 0});
  return __builtin_bit_cast(unsigned, m);
}

__device__ __forceinline__ f32x4 mfma16x16x32(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32x32x16(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// A DPP lane permutation of a float inside each row of 16 lanes (every lane reads a valid source).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int DPP_QUAD_XOR1 = 0xB1;        // quad_perm [1, 0, 3, 2]
constexpr int DPP_QUAD_XOR2 = 0x4E;        // quad_perm [2, 3, 0, 1]
constexpr int DPP_ROW_HALF_MIRROR = 0x141;  // lane i <- 7 - i inside each 8
constexpr int DPP_ROW_MIRROR = 0x140;       // lane i <- 15 - i inside each 16

// Sum over aligned groups of WIDTH lanes, every lane of a group receiving it. Inside a row of 16 lanes the
// partial sums combine through DPP operands of the adds (after the two quad steps all lanes of a quad hold
// its sum, so the mirrors pair whole quads, then whole halves); the four row sums of a 64-lane group meet
// through gfx950's lane swaps. No LDS permute: ds_bpermute costs an LDS round trip per step.
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(WIDTH == 2 || WIDTH == 4 || WIDTH == 8 || WIDTH == 16 || WIDTH == 64, "group width");
  v += dpp_f32<DPP_QUAD_XOR1>(v);
  if constexpr (WIDTH >= 4) v += dpp_f32<DPP_QUAD_XOR2>(v);
  if constexpr (WIDTH >= 8) v += dpp_f32<DPP_ROW_HALF_MIRROR>(v);
  if constexpr (WIDTH >= 16) v += dpp_f32<DPP_ROW_MIRROR>(v);
  if constexpr (WIDTH == 64) {
    // the four row sums r0..r3 meet as (r0 + r1) + (r2 + r3) through two VALU lane swaps (v_permlane16_swap,
    // v_permlane32_swap: no SGPR round trip and none of the wait states a v_readlane result needs)
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const float pr = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(pr), __float_as_uint(pr), false, false);
    v = __uint_as_float(b[0]) + __uint_as_float(b[1]);
  }
  return v;
}
// gfx950 VALU lane swaps. v_permlane32_swap(x, x) returns {x[l % 32], x[l % 32 + 32]} in lane l: the values of
// the lower and the upper half-wave side by side; v_permlane16_swap(x, x) likewise {x of row 2 (r / 2),
// x of row 2 (r / 2) + 1} for lane l of 16-lane row r. No LDS round trip (ds_bpermute) and no address VGPR.
struct f32pair {
  float lo, hi;
};
__device__ __forceinline__ f32pair halves32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return {__uint_as_float(r[0]), __uint_as_float(r[1])};
}
__device__ __forceinline__ f32pair rowpair16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return {__uint_as_float(r[0]), __uint_as_float(r[1])};
}
// Sum over lanes l, l ^ 16, l ^ 32, l ^ 48 (the four 16-lane rows' lane l % 16), in the butterfly order
// (x[r0] + x[r1]) + (x[r2] + x[r3]) in every lane.
__device__ __forceinline__ float sum_rows4(float x) {
  const f32pair a = rowpair16(x);
  const f32pair b = halves32(a.lo + a.hi);
  return b.lo + b.hi;
}
__device__ __forceinline__ float max_rows4(float x) {
  const f32pair a = rowpair16(x);
  const f32pair b = halves32(fmaxf(a.lo, a.hi));
  return fmaxf(b.lo, b.hi);
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
// Direct global -> LDS loads, issued from inline assembly (the compiler would otherwise make every later LDS
// read wait for every outstanding LDS-bound load). The kernels wait for them themselves: vector memory
// operations complete in issue order.
typedef __attribute__((address_space(3))) void lds_void_t;
// The LDS byte offset of a generic pointer into __shared__ memory: the low 32 bits of its flat address (the shared
// aperture's base is 4 GiB aligned). A cast to the LDS address space would add a null-pointer check on every use.
__device__ __forceinline__ unsigned lds_offset(const void* p) { return (unsigned)(uintptr_t)p; }
// global_load_lds_dword{x4}: each active lane's bytes land at lds + size * lane. M0 is saved and restored.
__device__ __forceinline__ void dma_x4(const void* src, const void* lds) {
  const unsigned off = __builtin_amdgcn_readfirstlane(lds_offset(lds));
  unsigned saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
               : "=&s"(saved)
               : "v"(src), "s"(off)
               : "memory");
}
// The same load from a wave-uniform base (SGPR pair) plus a per-lane 32-bit byte offset: the address arithmetic
// stays on the scalar unit and the offset VGPR is computed once.
__device__ __forceinline__ void dma_x4_s(const void* base, unsigned voff, const void* lds) {
  const unsigned off = __builtin_amdgcn_readfirstlane(lds_offset(lds));
  unsigned saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
               : "=&s"(saved)
               : "v"(voff), "s"(base), "s"(off)
               : "memory");
}
// Four such loads from the bases b[0..3] (same lane offset) into LDS lds, lds + STEP, lds + 2 STEP, lds + 3 STEP
// bytes, with one save and restore of M0 for the four. The s_add_u32 that advances M0 writes SCC, which the
// clobber list declares, so the compiler keeps no scalar condition live across the block.
template <unsigned STEP>
__device__ __forceinline__ void dma_x4_s4(const void* b0, const void* b1, const void* b2, const void* b3, unsigned voff,
                                          const void* lds) {
  const unsigned off = __builtin_amdgcn_readfirstlane(lds_offset(lds));
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %3\n\t"
      "s_add_u32 m0, m0, %7\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %4\n\t"
      "s_add_u32 m0, m0, %7\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %5\n\t"
      "s_add_u32 m0, m0, %7\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %6\n\ts_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(off), "s"(b0), "s"(b1), "s"(b2), "s"(b3), "i"(STEP)
      : "memory", "scc");
}
__device__ __forceinline__ void dma_x1(const void* src, const void* lds) {
  const unsigned off = __builtin_amdgcn_readfirstlane(lds_offset(lds));
  unsigned saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
               : "=&s"(saved)
               : "v"(src), "s"(off)
               : "memory");
}

// The same store at a wave-uniform base (SGPR pair) plus a per-lane 32-bit byte offset.
__device__ __forceinline__ void store_stream_x4_s(void* base, unsigned voff, u32x4 v) {
  asm volatile("global_store_dwordx4 %0, %1, %2 nt\n\ts_nop 1" : : "v"(voff), "v"(v), "s"(base) : "memory");
}
__device__ __forceinline__ void store_stream_x4(void* p, unsigned a, unsigned b, unsigned c, unsigned d) {
  store_stream_x4(p, u32x4{a, b, c, d});
}
__device__ __forceinline__ void store_stream_f4(void* p, float a, float b, float c, float d) {
  store_stream_x4(p, u32x4{__float_as_uint(a), __float_as_uint(b), __float_as_uint(c), __float_as_uint(d)});
}
