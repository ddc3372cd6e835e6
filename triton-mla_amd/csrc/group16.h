// Device helpers of the 16-head-group decode kernels (mla_decode_fp8.hip,
// mla_decode_g16.hip): LDS operand fetches issued as asm, waits that tie
// registers, cross-row reductions of the 16x16 MFMA layouts, register-class
// pins and the in-place rescale of AGPR accumulators.
#pragma once

#include "cdna.h"

namespace tmla {
namespace grp {

typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

// LDS operand fetches as asm: the compiler cannot tell them from reads of
// the LDS-DMA destinations and would otherwise drain every copy in flight
// (vmcnt(0)) before each. Completion is awaited with lgkm_tie.
template <int OFF>
__device__ __forceinline__ i32x4 ds_read_x4(const char LDS_AS* p) {
  return __builtin_bit_cast(i32x4, ds_read_b128<OFF>(p));
}
template <int OFF>
__device__ __forceinline__ i32x2 ds_read_tr8(const char LDS_AS* p) {
  i32x2 r;
  asm volatile("ds_read_b64_tr_b8 %0, %1 offset:%2" : "=v"(r) : "v"(p), "i"(OFF));
  return r;
}
// Wait until at most N LDS/scalar operations are outstanding, tying x there.
template <int N>
__device__ __forceinline__ void lgkm_tie(f32x4& x) {
  static_assert(N >= 0 && N <= 15, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(x) : "i"(N));
}
template <int N>
__device__ __forceinline__ void lgkm_tie(i32x4& x) {
  static_assert(N >= 0 && N <= 15, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(x) : "i"(N));
}
template <int N>
__device__ __forceinline__ void lgkm_tie(i32x2& x) {
  static_assert(N >= 0 && N <= 15, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(x) : "i"(N));
}

__device__ __forceinline__ float rows_max(float x) {
  float a = x, b = x;
  swap_rows16(a, b);
  x = fmaxf(a, b);
  a = x;
  b = x;
  swap_rows32(a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float rows_sum(float x) {
  float a = x, b = x;
  swap_rows16(a, b);
  x = a + b;
  a = x;
  b = x;
  swap_rows32(a, b);
  return a + b;
}

// Register-class pins (empty asm): O^T stays in AGPRs and Q^T in VGPRs
// across the loop instead of being shuttled between the two files.
__device__ __forceinline__ void pin_acc(f32x4& x) { asm volatile("" : "+a"(x)); }
template <class T>
__device__ __forceinline__ void pin_v(T& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void mfma_fence(f32x4& x) { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(x)); }
__device__ __forceinline__ void mfma_fence_a(f32x4& x) { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+a"(x)); }

// acc *= f in place in the AGPRs (the rare lazy rescale): written as asm so
// that the accumulators never need VGPR copies around the loop. The MFMAs
// that last wrote them completed long before (a softmax lies between).
__device__ __forceinline__ void scale_acc(f32x4& acc, float f) {
  float e0 = acc[0], e1 = acc[1], e2 = acc[2], e3 = acc[3], t;
  asm volatile(
      "v_accvgpr_read_b32 %4, %0\n\tv_mul_f32 %4, %4, %5\n\tv_accvgpr_write_b32 %0, %4\n\t"
      "v_accvgpr_read_b32 %4, %1\n\tv_mul_f32 %4, %4, %5\n\tv_accvgpr_write_b32 %1, %4\n\t"
      "v_accvgpr_read_b32 %4, %2\n\tv_mul_f32 %4, %4, %5\n\tv_accvgpr_write_b32 %2, %4\n\t"
      "v_accvgpr_read_b32 %4, %3\n\tv_mul_f32 %4, %4, %5\n\tv_accvgpr_write_b32 %3, %4\n\ts_nop 1"
      : "+a"(e0), "+a"(e1), "+a"(e2), "+a"(e3), "=&v"(t)
      : "v"(f));
  acc = f32x4{e0, e1, e2, e3};
}

}  // namespace grp
}  // namespace tmla
