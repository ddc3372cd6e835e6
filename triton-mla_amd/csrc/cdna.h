// Device helpers shared by the decode and layer kernels of triton_mla
// (gfx950 / CDNA4): vector types, LDS operand fetches issued as asm, the
// LDS-DMA copy, the element-type traits and the LDS piece swizzle.
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>

#include <utility>

#include "triton_mla.h"

namespace tmla {

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#define LDS_AS __attribute__((address_space(3)))

// s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

// Transposed operand fetch (ds_read_b64_tr_b16: four 16-bit elements of one
// column from four rows per lane). Issued as asm because the builtin carries
// no alias information and the compiler would otherwise drain every
// in-flight LDS-DMA copy (vmcnt(0)) before it; completion is awaited with an
// explicit s_waitcnt lgkmcnt that also ties the destination registers.
template <int OFF>
__device__ __forceinline__ i16x4 ds_read_tr(const char LDS_AS* p) {
  i16x4 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(p), "i"(OFF));
  return r;
}

// 16-byte operand fetch, asm for the same reason as ds_read_tr.
template <int OFF>
__device__ __forceinline__ i16x8 ds_read_b128(const char LDS_AS* p) {
  i16x8 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(p), "i"(OFF));
  return r;
}
// One LDS-DMA copy: 16 bytes per lane from src + OFF into LDS at
// dst + 16 * lane (global_load_lds_dwordx4; completion counts in vmcnt). The
// instruction's immediate offset applies to both addresses, so the LDS base
// (M0, a scalar) is lowered by OFF and the per-lane address needs no add.
template <int OFF>
__device__ __forceinline__ void lds_copy16(const char* src, char LDS_AS* dst) {
  static_assert(OFF >= 0 && OFF < 4096, "immediate offset range");
  __builtin_amdgcn_global_load_lds(src, (void LDS_AS*)(dst - OFF), 16, OFF, 0);
}

// Workgroup barrier that the compiler treats as a full memory-ordering point
// but that adds no counter waits of its own: the producer side waits for its
// LDS-DMA copies with wait_vmcnt first.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_barrier" ::: "memory"); }

template <int DT>
struct Elt;
template <>
struct Elt<TMLA_BF16> {
  __device__ static __forceinline__ f32x16 mfma(i16x8 a, i16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  __device__ static __forceinline__ short from_float(float x) {
    return __builtin_bit_cast(short, (__bf16)x);
  }
  __device__ static __forceinline__ float to_float(short x) {
    return __builtin_bit_cast(float, (unsigned)(unsigned short)x << 16);
  }
};
template <>
struct Elt<TMLA_FP16> {
  __device__ static __forceinline__ f32x16 mfma(i16x8 a, i16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ static __forceinline__ short from_float(float x) {
    return __builtin_bit_cast(short, (_Float16)x);
  }
  __device__ static __forceinline__ float to_float(short x) { return (float)__builtin_bit_cast(_Float16, x); }
};

// XOR swizzle of the 16-byte piece index inside an 8-row x 128-byte LDS
// block. Row r of row-group rg: keeps the S^T operand reads (16 lanes = 16
// rows, one piece) and the V^T transpose reads (32 lanes = 4 rows x 4 pieces)
// on distinct banks.
__device__ __forceinline__ int piece_swizzle(int r, int rg) {
  return (((r >> 1) & 1) << 2) | ((r >> 2) & 1) | ((rg & 1) << 1);
}

// Reductions over the four 16-lane rows of a wave without the LDS pipe.
// v_permlane16_swap_b32 a, b swaps the odd 16-lane rows of a with the even
// rows of b, v_permlane32_swap_b32 the upper 32 lanes of a with the lower 32
// of b: with x in both, a and b then hold x of the two rows (halves) of each
// pair, so combining them reduces over the pair. As asm, with both registers
// read and written (the builtins' second result is not usable here); the
// s_nop is the wait state a VALU result needs before the swap reads it.
__device__ __forceinline__ void swap_rows16(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap_rows32(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}

// Compile-time loop: f(std::integral_constant<int, I>) for I = 0..N-1, so
// LDS offsets can be instruction immediates.
template <class F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

}  // namespace tmla
