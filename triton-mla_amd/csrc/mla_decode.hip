// MLA decode attention for MI355X (gfx950): split-KV partial kernel, log-sum-exp
// combine kernel and the C ABI declared in include/triton_mla.h.
//
// Reference behaviour: src/triton_mla/kernel.py (stage 1 kernel.py:43-138,
// stage 2 kernel.py:141-181, host wrapper kernel.py:204-323).
//
// Design (one workgroup = one worker, 4 waves = one per SIMD, 32 * NHB heads
// with NHB = 1, 2 or 4 blocks of 32):
//  * Each worker owns a range of 64-token tiles; it walks them as 32-token
//    sub-tiles through LDS rings (V dims: 4 entries, rope dims: 3). Rows are
//    copied HBM -> LDS with global_load_lds_dwordx4 (no VGPR staging): one
//    instruction moves eight full 128-byte lines into 1 KiB of LDS; the
//    copies of sub-tile i+3 are spread over the MFMA steps of iteration i.
//  * S^T = K . Q^T by head: wave w < NHB keeps Q^T of its 32 heads in VGPRs,
//    reads K (all 576 dims) from LDS and runs the softmax of those heads.
//  * O^T += V^T . P^T by value dimension: wave w owns 128 of the 512 dims of
//    every head of the workgroup (fp32 accumulators in AGPRs); P^T and the
//    per-head rescale factors go through LDS, so each V^T operand (read
//    straight from the row-major tile with ds_read_b64_tr_b16) feeds NHB
//    MFMAs. Both products run on v_mfma_f32_32x32x16_{bf16,f16}.
//  * Online softmax in the base-2 domain with a lazy rescale: the running
//    reference max only moves when a new score exceeds it by more than 2^8,
//    so probabilities stay <= 256 and the O^T rescale is rare.
//  * A worker writes its normalised result through LDS as whole rows: the
//    final output when it covers a sequence alone, else a partial (input
//    dtype) and a base-2 log-sum-exp that the combine kernel merges exactly
//    like the reference's stage 2.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <utility>

#include "cdna.h"
#include "decode_common.h"
#include "merge.h"
#include "triton_mla.h"

namespace tmla {

constexpr int kSubTokens = 32;      // LDS stage unit: M of the 32x32x16 MFMA
// Schedule of the partial kernel's tile loop (build-time knobs): LDS operand
// reads issued this many MFMA steps ahead of their use; PV MFMAs beside the
// S chain, in units of NHB of the 2 * 4 * NHB PV MFMAs of a sub-tile (the
// rest run beside the softmax); the spacing of those PV MFMAs among the S
// steps; exponentials per step of the softmax pass.
#ifndef TMLA_READ_AHEAD
#define TMLA_READ_AHEAD 3
#endif
#ifndef TMLA_PV1_EIGHTHS
#define TMLA_PV1_EIGHTHS 4
#endif
#ifndef TMLA_PV_STRIDE
#define TMLA_PV_STRIDE 2
#endif
#ifndef TMLA_EXP_PER_STEP
#define TMLA_EXP_PER_STEP 2
#endif
// start-up order: 0 = Q and sub-tile 0, then sub-tile 1; 1 = Q, sub-tiles 0
// and 1, then wait for Q and sub-tile 0; 2 = sub-tile 0, Q, sub-tile 1
#ifndef TMLA_STARTUP
#define TMLA_STARTUP 1
#endif
// L2 domains the workers of one sequence are grouped by (1: no grouping)
#ifndef TMLA_XCDS
#define TMLA_XCDS 8
#endif
// 1: Q staged through LDS in the KV layout before the first KV copies
#ifndef TMLA_Q_LDS
#define TMLA_Q_LDS 1
#endif
// 1: one LDS wait per two MFMA steps (for the operands of both)
#ifndef TMLA_WAIT_PAIR
#define TMLA_WAIT_PAIR 1
#endif
// step order inside a pass: 0 = reads, wait, S MFMA, PV MFMA, hook;
// 1 = wait, S MFMA, reads, hook, PV MFMA (the two MFMAs of a step apart)
#ifndef TMLA_STEP_ORDER
#define TMLA_STEP_ORDER 0
#endif
// 1: the S and PV MFMAs are volatile asm, so they keep their places among
// the LDS reads and waits instead of being grouped by the scheduler
#ifndef TMLA_MFMA_VOLATILE
#define TMLA_MFMA_VOLATILE 0
#endif
// 1: probabilities rounded two at a time (v_cvt_pk_*_f32, same rounding)
#ifndef TMLA_PACK_PK
#define TMLA_PACK_PK 1
#endif
// 1: phase stamps (profiling builds only; see tmla_debug_stamps)
#ifndef TMLA_STAMPS
#define TMLA_STAMPS 0
#endif
constexpr int kStages = 4;          // LDS ring depth (3 sub-tiles in flight)
constexpr int kHeadsPerWave = 32;   // N of the 32x32x16 MFMA
// 16-bit cache: up to this many heads (virtual heads of a multi-token call)
// the 16-head-group kernel runs (mla_decode_g16.hip); 0 disables it
#ifndef TMLA_G16_HEADS
#define TMLA_G16_HEADS 16
#endif
// fp8 cache: up to this many heads the 16-head-group kernel runs (its
// workgroups stream the cache on their own); above, the 16-bit kernel with the
// cache widened once per workgroup into its ring
#ifndef TMLA_FP8_GROUP_HEADS
#define TMLA_FP8_GROUP_HEADS 16
#endif
// combine: four heads per wave when one head per wave would take more than
// this many workgroups
#ifndef TMLA_COMBINE_WIDE_WGS
#define TMLA_COMBINE_WIDE_WGS 1024
#endif
constexpr int kFp8GroupHeads = TMLA_FP8_GROUP_HEADS;
constexpr int kG16Heads = TMLA_G16_HEADS;
constexpr int64_t kCombineWideWgs = TMLA_COMBINE_WIDE_WGS;
static_assert(kG16Heads <= 16, "one head group per workgroup");

struct CombineArgs {
  const int32_t* seqlens;
  int32_t batch, num_heads;
  int32_t num_splits, num_workers;
  char* out;
  int64_t out_sb, out_sh;
  float* lse;
  const short* mid_o;
  const float* mid_lse;
};

// ---------------------------------------------------------------------------
// small device helpers
// ---------------------------------------------------------------------------

// Phase stamps of a profiling build (TMLA_STAMPS=1): lane 0 of wave 0 of
// workgroups (x, 0), x < kStampWorkers, stores the 100 MHz wall clock and the
// shader clock when it reaches a phase: 0 entry, 1 work range known, 2 loop
// start, 3 loop end, 4 finalize end of its first segment, and inside
// iteration kStampIter of that segment 5 start (after the barrier), 6 after
// the first pass, 7 after the second pass, 8 start of the next iteration.
// Compiled out otherwise.
constexpr int kStampWorkers = 4096;
constexpr int kStampSlots = 9;
constexpr int kStampIter = 8;
#if TMLA_STAMPS
__device__ unsigned long long g_stamps[kStampWorkers * kStampSlots * 2];
#endif
// The clocks are read where the phase is reached (stamp_now) and stored
// later (stamp_store), where the code waits for its LDS and scalar
// operations anyway, so reading them adds no wait inside a phase.
struct StampRec {
  unsigned long long rt, ck;
};
__device__ __forceinline__ StampRec stamp_now() {
#if TMLA_STAMPS
  return StampRec{__builtin_amdgcn_s_memrealtime(), __builtin_amdgcn_s_memtime()};
#else
  return StampRec{0, 0};
#endif
}
__device__ __forceinline__ void stamp_store(int slot, StampRec r) {
#if TMLA_STAMPS
  if (threadIdx.x == 0 && blockIdx.y == 0 && blockIdx.x < kStampWorkers) {
    unsigned long long* p = g_stamps + ((size_t)blockIdx.x * kStampSlots + slot) * 2;
    asm volatile("global_store_dwordx2 %0, %1, off" : : "v"(p), "v"(r.rt) : "memory");
    asm volatile("global_store_dwordx2 %0, %1, off offset:8" : : "v"(p), "v"(r.ck) : "memory");
  }
#else
  (void)slot;
  (void)r;
#endif
}
__device__ __forceinline__ void phase_stamp(int slot) { stamp_store(slot, stamp_now()); }

// Register-class pins: an empty asm that requires its operand in VGPRs /
// AGPRs at that point. They keep the PV accumulators in AGPRs and the S tile
// in VGPRs instead of letting the allocator shuttle blocks between files.
__device__ __forceinline__ void pin_vgpr(f32x16& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void pin_agpr(f32x16& x) { asm volatile("" : "+a"(x)); }
// (Operand-constrained asm lives in __device__ helpers only: the host pass
// of the compiler rejects GPU register constraints inside a kernel body.)
__device__ __forceinline__ void pin_f1(float& a) { asm volatile("" : "+v"(a)); }
__device__ __forceinline__ void pin_f2(float& a, float& b) { asm volatile("" : "+v"(a), "+v"(b)); }
__device__ __forceinline__ void pin_f3(float& a, float& b, float& c) { asm volatile("" : "+v"(a), "+v"(b), "+v"(c)); }
__device__ __forceinline__ void pin_f4(f32x4& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void pin_f16(f32x16& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void pin_f8(float* x) {
  asm volatile("" : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]), "+v"(x[6]), "+v"(x[7]));
}


// LDS stores of this kernel's own P^T / factor buffers, as asm so that
// they keep their place among the asm reads whose lgkmcnt counts they share.
template <int OFF>
__device__ __forceinline__ void ds_write_b128(char LDS_AS* p, i16x8 v) {
  asm volatile("ds_write_b128 %0, %1 offset:%2" : : "v"(p), "v"(v), "i"(OFF));
}
__device__ __forceinline__ void ds_write_b32(char LDS_AS* p, float v) {
  asm volatile("ds_write_b32 %0, %1" : : "v"(p), "v"(v));
}
__device__ __forceinline__ f32x4 ds_read_f32x4(const char LDS_AS* p) {
  f32x4 r;
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(p));
  return r;
}
template <int N>
__device__ __forceinline__ void lgkm_tie_f4(f32x4& x) {
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(x) : "i"(N));
}

// Wait until at most N LDS/scalar-memory operations are outstanding and tie
// the operands fetched for one pass step (K, V^T halves, P^T; each present or
// not) to that point, so no use of them is scheduled above the wait.
template <int N, bool HK, bool HV, bool HP>
__device__ __forceinline__ void lgkm_tie(i16x8& k, i16x4& vl, i16x4& vh, i16x8& p) {
  static_assert(N >= 0 && N <= 15, "lgkmcnt range");
  if constexpr (HK && HV && HP)
    asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(k), "+v"(vl), "+v"(vh), "+v"(p) : "i"(N));
  else if constexpr (HK && HV)
    asm volatile("s_waitcnt lgkmcnt(%3)" : "+v"(k), "+v"(vl), "+v"(vh) : "i"(N));
  else if constexpr (HK && HP)
    asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(k), "+v"(p) : "i"(N));
  else if constexpr (HV && HP)
    asm volatile("s_waitcnt lgkmcnt(%3)" : "+v"(vl), "+v"(vh), "+v"(p) : "i"(N));
  else if constexpr (HK)
    asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(k) : "i"(N));
  else if constexpr (HV)
    asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(vl), "+v"(vh) : "i"(N));
  else if constexpr (HP)
    asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(p) : "i"(N));
}

// Tie operands to the preceding wait without waiting again (an empty asm
// that takes them as read-write, so no use of them moves above it).
template <bool HK, bool HV, bool HP>
__device__ __forceinline__ void tie_ops(i16x8& k, i16x4& vl, i16x4& vh, i16x8& p) {
  if constexpr (HK) asm volatile("" : "+v"(k));
  if constexpr (HV) asm volatile("" : "+v"(vl), "+v"(vh));
  if constexpr (HP) asm volatile("" : "+v"(p));
}
template <int N>
__device__ __forceinline__ void lgkm_wait() {
  static_assert(N >= 0 && N <= 15, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%0)" : : "i"(N));
}

// Step t of a pass carries PV step PV0 + (t - PVOFF) / PVS when t >= PVOFF
// and (t - PVOFF) is a multiple of PVS below NV * PVS.
constexpr bool pass_has_pv(int t, int NV, int PVOFF, int PVS) {
  return t >= PVOFF && (t - PVOFF) % PVS == 0 && (t - PVOFF) / PVS < NV;
}

// LDS reads issued by fetch(t) of a pass (one K operand per S step, and a
// Q^T operand beside it for k-chunks SLO + t >= QR0; on the PV steps, two
// V^T halves at the first head block of a PV column block and one P^T
// operand at the first column block of a (token half, head block)).
template <int NS, int NV, int PV0, int NHB, int PVOFF, int PVS, int SLO, int QR0>
constexpr int pass_reads(int t) {
  int n = t < NS ? (SLO + t >= QR0 ? 2 : 1) : 0;
  if (pass_has_pv(t, NV, PVOFF, PVS)) {
    const int g = PV0 + (t - PVOFF) / PVS;
    n += (g % NHB == 0 ? 2 : 0) + ((g % (4 * NHB)) / NHB == 0 ? 1 : 0);
  }
  return n;
}

// S^T accumulation in VGPRs (the PV accumulators own every AGPR). After the
// chain, mfma_vgpr_fence waits out the MFMA result latency before any VALU
// instruction reads the accumulator.
template <int DT>
__device__ __forceinline__ f32x16 mfma_vgpr_first(const i16x8& a, const i16x8& b) {
  f32x16 d;
  if constexpr (TMLA_MFMA_VOLATILE) {
    if constexpr (DT == TMLA_BF16)
      asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "v"(b));
    else
      asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "v"(b));
  } else {
    if constexpr (DT == TMLA_BF16)
      asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=v"(d) : "v"(a), "v"(b));
    else
      asm("v_mfma_f32_32x32x16_f16 %0, %1, %2, 0" : "=v"(d) : "v"(a), "v"(b));
  }
  return d;
}
template <int DT>
__device__ __forceinline__ void mfma_vgpr_acc(f32x16& d, const i16x8& a, const i16x8& b) {
  if constexpr (TMLA_MFMA_VOLATILE) {
    if constexpr (DT == TMLA_BF16)
      asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "v"(b));
    else
      asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "v"(b));
  } else {
    if constexpr (DT == TMLA_BF16)
      asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "v"(b));
    else
      asm("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "v"(b));
  }
}
// O^T += V^T . P^T with the accumulator in AGPRs. The volatile asm form
// keeps its place among the reads and waits; its operands come straight
// from LDS reads (no VALU writes them just before), and the accumulators are
// read by VALU code only after mfma_agpr_fence or long after their last MFMA
// (the lazy rescale, one softmax and one barrier later).
template <int DT>
__device__ __forceinline__ void mfma_agpr_acc(f32x16& acc, const i16x8& v, const i16x8& p) {
  if constexpr (TMLA_MFMA_VOLATILE) {
    if constexpr (DT == TMLA_BF16)
      asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(v), "v"(p));
    else
      asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(v), "v"(p));
  } else {
    acc = Elt<DT>::mfma(v, p, acc);
    asm volatile("" : "+a"(acc));
  }
}
__device__ __forceinline__ void mfma_agpr_fence(f32x16& acc) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+a"(acc));
}
__device__ __forceinline__ void mfma_vgpr_fence(f32x16& d) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(d));
}

// Exact widening of 8 fp8 (e4m3) bytes, half H of a 16-byte chunk, to 8
// elements of the 16-bit type (every e4m3 value is a bf16 and an fp16 value;
// the conversion's scale is 1).
template <int DT, int H>
__device__ __forceinline__ i16x8 widen_half(const i16x8& raw) {
  typedef int i32x4v __attribute__((ext_vector_type(4)));
  const i32x4v x = __builtin_bit_cast(i32x4v, raw);
  const int lo = x[2 * H], hi = x[2 * H + 1];
  if constexpr (DT == TMLA_BF16) {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    const b2 a0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false);
    const b2 a1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true);
    const b2 b0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false);
    const b2 b1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true);
    return __builtin_bit_cast(i16x8, bf16x8{a0[0], a0[1], a1[0], a1[1], b0[0], b0[1], b1[0], b1[1]});
  } else {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 a0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 1.0f, false);
    const h2 a1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 1.0f, true);
    const h2 b0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 1.0f, false);
    const h2 b1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 1.0f, true);
    return __builtin_bit_cast(i16x8, f16x8{a0[0], a0[1], a1[0], a1[1], b0[0], b0[1], b1[0], b1[1]});
  }
}

// Two probabilities rounded to the 16-bit type, packed into one dword (a in
// the low half). The softmax packs its 16 probabilities in place into the
// first 8 registers of the score tile (pair k reads registers 2k and 2k + 1,
// which no earlier pair has overwritten), so P^T needs no registers of its
// own: registers 0-3 hold the first token half, 4-7 the second.
template <int DT>
__device__ __forceinline__ float pack_pair(float a, float b) {
  if constexpr (TMLA_PACK_PK) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    if constexpr (DT == TMLA_BF16)
      return __builtin_bit_cast(float, __builtin_convertvector((f32x2){a, b}, bf16x2));
    else
      return __builtin_bit_cast(float, __builtin_convertvector((f32x2){a, b}, f16x2));
  } else {
    const unsigned lo = (unsigned short)Elt<DT>::from_float(a), hi = (unsigned short)Elt<DT>::from_float(b);
    return __builtin_bit_cast(float, lo | (hi << 16));
  }
}
template <int DT>
__device__ __forceinline__ void pack_probs_in_place(f32x16& p) {
#pragma unroll
  for (int k = 0; k < 8; ++k) p[k] = pack_pair<DT>(p[2 * k], p[2 * k + 1]);
  pin_f16(p);
}
__device__ __forceinline__ i16x8 packed_half(const f32x16& p, int h) {
  const f32x4 v = h == 0 ? f32x4{p[0], p[1], p[2], p[3]} : f32x4{p[4], p[5], p[6], p[7]};
  return __builtin_bit_cast(i16x8, v);
}

// Byte offset of the row of (local) token `tok` of sequence b inside kv.
// Token indices past the sequence end are clamped to its last token so every
// copied row is real cache memory (its scores are masked to -inf later).
template <bool PAGED>
__device__ __forceinline__ int64_t row_offset(const PartialArgs& a, int b, int tok, int n_b,
                                              int page_id) {
  const int t = min(tok, n_b - 1);
  // dense caches hold num_blocks (= capacity) rows per sequence
  if (!PAGED) return (int64_t)b * a.kv_s0 + (int64_t)min(t, (int)(a.num_blocks - 1)) * a.kv_s1;
  const int in_page = a.page_shift >= 0 ? (t & (a.page_size - 1)) : (t % a.page_size);
  return (int64_t)page_id * a.kv_s0 + (int64_t)in_page * a.kv_s1;
}

// Segment of a worker: tiles [t0, t1) of sequence b, result goes to `slot`
// (a partial) or straight to out/lse when `direct`.
struct Segment {
  int b, t0, t1, slot;
  bool direct;
};

// ---------------------------------------------------------------------------
// Stage 1: split-KV partial attention
// ---------------------------------------------------------------------------
//
// LDS layout of one 32-token sub-tile, split by lifetime:
//  * V part (dims 0..DV-1, read by S and by PV): 4 row-groups x NVB column
//    blocks of 1 KiB in a kStages-deep ring;
//  * rope part (dims DV..DQK-1, read by S only): 4 row-groups x NRB blocks in
//    a ring one entry shorter, since it is dead once S of its sub-tile is done.
// Block (rg, cb) holds rows 8rg..8rg+7, bytes [128cb, 128cb+128) of each row,
// 16-byte piece p of row r at position r*8 + (p ^ piece_swizzle(r, rg)).
//
// Work split inside a workgroup of 4 waves (one per SIMD) and NHB blocks of
// 32 heads (NHB = 1, 2, 4):
//  * S and the softmax by head: wave w < NHB owns heads 32w..32w+31 (its Q^T
//    lives in its VGPRs) and writes their probabilities P^T and rescale
//    factors to LDS;
//  * O^T += V^T P^T by value dimension: wave w owns dims [w*DV/4, (w+1)*DV/4)
//    of all 32*NHB heads, so each V^T operand read from LDS feeds NHB MFMAs.
// With fewer than 4 head blocks the waves past NHB only copy and run PV, so
// small head counts still use every SIMD of the CU.
// PAGE_UNIFORM: paged, page size a power of two and a multiple of 32
// F8: the cache holds fp8 (e4m3) codes with one float32 scale per page (or
// per tensor), pages of a multiple of 32 tokens. Each wave copies the fp8
// bytes of its 8 rows of a sub-tile into its own staging slot (LDS-DMA, half
// the bytes of a 16-bit row) and widens them, exactly, into the same 16-bit
// ring layout the 16-bit cache is copied into, once for all heads of the
// workgroup; the page's scale multiplies the scores (folded into the softmax
// scale) and the probabilities before their rounding. The V ring has three
// entries and the rope ring two, which makes room for two staging entries.
template <int DT, int DV, int DR, int NHB, bool PAGED, bool PAGE_UNIFORM, bool F8 = false>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void mla_partial_kernel(PartialArgs a) {
  constexpr int DQK = DV + DR;
  static_assert(DQK % 64 == 0 && DV % 64 == 0, "row must be whole 128-byte blocks");
  constexpr int NCB = DQK / 64;           // 128-byte column blocks per row
  constexpr int NVB = DV / 64;            // ... of which hold V dims
  constexpr int NRB = NCB - NVB;          // ... and rope dims
  constexpr int NKC = DQK / 16;           // k-chunks of QK^T
  constexpr int NDB = DV / 32;            // 32-dim blocks of PV
  constexpr int NW = 4;                   // waves per workgroup
  constexpr int NDBW = NDB / NW;          // ... owned by one wave
  constexpr int NACC = NDBW * NHB;        // 32x32 accumulator blocks per wave
  constexpr int VSLOT = 4 * NVB * 1024;   // V ring entry
  constexpr int RSLOT = 4 * NRB * 1024;   // rope ring entry
  constexpr int VST = F8 ? 3 : kStages;   // V ring entries
  constexpr int kRopeStages = VST - 1;    // rope ring entries
  constexpr int PSLOT = NHB * 2 * 1024;   // P^T of one sub-tile: [hb][c][lane] x 16 bytes
  constexpr int ASLOT = 32 * 4 * 4;       // per-head factors: [head % 32][hb] floats
  constexpr int STG_W = 8 * DQK;          // fp8 staging: one wave's 8 rows of a sub-tile
  constexpr int STG = 4 * STG_W;          // ... one sub-tile
  constexpr int LOADS8 = (STG_W + 1023) / 1024;  // fp8 DMA instructions per wave per sub-tile
  constexpr int OFF_R = VST * VSLOT;
  constexpr int OFF_S = OFF_R + kRopeStages * RSLOT;
  constexpr int OFF_P = OFF_S + (F8 ? 2 * STG : 0);
  constexpr int OFF_A = OFF_P + 2 * PSLOT;
  // With two S waves (64 heads), the rope rows of Q stay in LDS for the
  // whole kernel (RSLOT per S wave) and S reads their Q^T operands from there
  // beside the K rope operands: 16 VGPRs fewer than Q^T all in registers,
  // which the 64-head accumulators need.
  constexpr bool QR = NHB == 2 && TMLA_Q_LDS;
  constexpr int NKQ = QR ? 4 * NVB : NKC;  // k-chunks of Q^T held in VGPRs
  constexpr int OFF_QR = OFF_A + 2 * ASLOT;
  constexpr int SMEM = OFF_QR + (QR ? NHB * RSLOT : 0);
  constexpr int RG_PER_WAVE = 4 / NW;
  constexpr int LOADS = RG_PER_WAVE * NCB;  // DMA instructions per wave per sub-tile
  constexpr int OPITCH = DV * 2 + 16;        // output staging row pitch (bytes)
  static_assert(NHB == 1 || NHB == 2 || NHB == 4, "head blocks per workgroup");
  static_assert(NRB >= 1 && NDB % NW == 0 && NDBW % 2 == 0, "column split");
  static_assert(LOADS < 64, "vmcnt immediate range");
  static_assert(NHB * 32 * OPITCH <= OFF_P, "output staging fits the rings");
  static_assert(DV == 512, "one output row = 64 lanes x 8 elements");
  static_assert(!F8 || (PAGED && PAGE_UNIFORM), "fp8 ring: pages of whole sub-tiles");
  static_assert(!F8 || (DQK == 576 && LOADS8 == 5 && STG_W == 4608), "fp8 staging: 4 full copies + a half (rope)");
  static_assert(SMEM <= 160 * 1024, "LDS");

  __shared__ __attribute__((aligned(1024))) char smem[SMEM];
  char LDS_AS* const lds = (char LDS_AS*)(void LDS_AS*)smem;
  // fused merge: the split segments awaiting their merge ({b, index among
  // b's workers, their count, b's first slot, arrived last}) and the merge
  // decisions wave 0 hands to the other waves
  __shared__ int s_pend[2][5];
  __shared__ int s_msg[4];

  phase_stamp(0);
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar LDS bases
  const int nwg = gridDim.x;
  const int worker = worker_index(a);
  const bool s_owner = NHB == 4 || wave < NHB;  // runs S and the softmax of head block `wave`
  const int head_base = blockIdx.y * (kHeadsPerWave * NHB) + wave * kHeadsPerWave;
  // the wave's first head has its earliest query token: the most tokens unseen
  const int lag_wave = __builtin_amdgcn_readfirstlane(causal_lag(a, head_base));
  // fused merge: this worker clears sequences worker, worker + nwg, ... when
  // they are empty; the first length is requested now, used at the end
  const int pre_len = __builtin_amdgcn_readfirstlane((a.fused && worker < a.batch) ? a.seqlens[worker] : 1);
  // split segments awaiting their merge: at most the first (record 0) and
  // the last (record 1) segment of the worker's range; b < 0 = none
  if (a.fused && tid == 0) s_pend[0][0] = s_pend[1][0] = -1;

  // Q rows of sequence bq for this wave's heads into LDS (the KV copies'
  // swizzled layout; heads past num_heads copy head 0's row): V part at qv,
  // rope part at qrope. The 16-bit cache stages wave w in V ring entry w and
  // rope entry w (wave 3: P buffer 0, written again only after the first
  // barrier of the loop); the fp8 ring (three V and two rope entries) stages
  // wave 3's rows in the staging area and the rope rows of waves 2 and 3 in P
  // buffer 0, which holds two rope entries when all four waves run S.
  const int qv = wave < VST ? wave * VSLOT : OFF_S;
  const int qrope = !s_owner ? 0
                    : QR ? OFF_QR + wave * RSLOT
                         : (wave < kRopeStages ? OFF_R + wave * RSLOT : OFF_P + (wave - kRopeStages) * RSLOT);
  static_assert(!F8 || NHB < 4 || PSLOT >= 2 * RSLOT, "Q rope staging in P buffer 0");
  auto stage_q = [&](int bq) __attribute__((always_inline)) {
    const int ln = lane_id_fresh();
    const int r = ln >> 3;
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      const int hq = head_base + 8 * rg + r;
      const char* src = a.q + ((int64_t)bq * a.q_sb + (int64_t)(hq < a.num_heads ? hq : 0) * a.q_sh) * 2 +
                        ((ln & 7) ^ piece_swizzle(r, rg)) * 16;
      static_for<NCB>([&](auto CB) __attribute__((always_inline)) {
        constexpr int cb = decltype(CB)::value;
        char LDS_AS* dst = cb < NVB ? lds + qv + (rg * NVB + cb) * 1024
                                    : lds + qrope + (rg * NRB + cb - NVB) * 1024;
        lds_copy16<cb * 128>(src, dst);
      });
    }
  };

  // ---- work range -------------------------------------------------------
  WorkRange wr;
  if (!work_range(a, worker, wr)) {
    if (!a.fused) return;  // (the fused tail still clears empty sequences)
  }
  const int b_first = wr.b_first, tile_lo = wr.tile_lo, tile_hi = wr.tile_hi;
  const int off_first = wr.off_first, n_first = wr.n_first;
  if (a.fused) {
    // empty sequences worker, worker + nwg, ...: out = 0, lse = -inf
    // (kernel.py:126-128, 178-181); the first length was requested at entry
    const int lane = lane_id_fresh();
    const int hb0 = blockIdx.y * (kHeadsPerWave * NHB);
    const int nh = min(kHeadsPerWave * NHB, a.num_heads - hb0);
    const MergeView mv{a.mid_o, a.mid_lse, a.num_heads, a.out, a.out_sb, a.out_sh, a.lse};
    for (int bb = worker; bb < a.batch; bb += nwg) {
      const int len = bb == worker ? pre_len : a.seqlens[bb];
      if (tiles_of(len) == 0)
        for (int h = hb0 + wave; h < hb0 + nh; h += 4) merge_zero(mv, bb, h, lane);
    }
  }
  if (tile_lo >= tile_hi) return;
  phase_stamp(1);

  // ---- segments -----------------------------------------------------------
  int b = b_first;
  int t_start = tile_lo;              // local tile index within b
  int remaining = tile_hi - tile_lo;  // tiles left in this worker's range
  int seg_global_off = off_first;     // balanced mode: tile offset of b

  while (remaining > 0) {
    const int n_b = b == b_first ? n_first : a.seqlens[b];
    const int nt_b = tiles_of(n_b);
    if (nt_b == 0) {  // only possible in balanced mode between sequences
      ++b;
      continue;
    }
    const int t_end = min(nt_b, t_start + remaining);
    // this segment's lane-derived values (recomputed per segment, see
    // lane_id_fresh)
    const int lane = lane_id_fresh();
    const int head = head_base + (lane & 31);
    const bool head_ok = s_owner && head < a.num_heads;
    const int hi = lane >> 5;  // which half of the 32-token M block / k slots
    // per-lane LDS read offsets inside a ring entry
    // S^T A operand: token = lane%32 (rg = (lane%32)/8, r = lane%8), piece = 2*(kc%4) + hi
    // (the rope part's offset is the latent part's plus k_rope_delta: the
    // two rings differ only in the row-group stride)
    int k_off_v[4];
    int k_rope_delta;
    // V^T operand via ds_read_b64_tr_b16: group g = lane/16, L = lane%16;
    // read e2 covers tokens 16c + 8e2 + 4(g/2) + L/4, dims 32db + 16(g%2) + 4(L%4).
    // This wave's dims start at block column (wave * NDBW / 2).
    int v_off[2][2];  // [db&1][e2]
    // (set again before the sub-tile loop of an fp8 segment, from a fresh
    // lane id, so that they need not stay live across its start-up)
    auto set_lane_offsets = [&](int ln) __attribute__((always_inline)) {
      {
        const int rg = (ln & 31) >> 3, r = ln & 7;
        const int sw = piece_swizzle(r, rg);
#pragma unroll
        for (int j = 0; j < 4; ++j) k_off_v[j] = rg * NVB * 1024 + (r * 8 + ((2 * j + (ln >> 5)) ^ sw)) * 16;
        k_rope_delta = OFF_R - rg * (NVB - NRB) * 1024;
      }
      {
        const int g = ln >> 4, L = ln & 15;
        const int r = 4 * (g >> 1) + (L >> 2);
#pragma unroll
        for (int dbp = 0; dbp < 2; ++dbp)
#pragma unroll
          for (int e2 = 0; e2 < 2; ++e2) {
            const int piece = 4 * dbp + 2 * (g & 1) + ((L & 3) >> 1);
            v_off[dbp][e2] = e2 * NVB * 1024 + wave * (NDBW / 2) * 1024 +
                             (r * 8 + (piece ^ piece_swizzle(r, e2))) * 16 + 8 * (L & 1);
          }
      }
    };
    set_lane_offsets(lane);
    // DMA: this lane copies, for each of its wave's row-groups, the piece
    // (lane%8) ^ swizzle of token row 8rg + lane/8.
    const int dma_r = lane >> 3;

    Segment seg;
    seg.b = b;
    seg.t0 = t_start;
    seg.t1 = t_end;
    {
      const SegmentSlot ss = segment_slot(a, wr, worker, b, t_start, nt_b, seg_global_off);
      seg.slot = ss.slot;
      seg.direct = ss.direct;
      // fused merge record: b, this worker's index among b's workers, their
      // count, b's first slot
      if (a.fused && !seg.direct && wave == 0 && lane == 0) {
        int* r = s_pend[b == b_first ? 0 : 1];
        r[0] = b;
        r[1] = ss.index;
        r[2] = ss.count;
        r[3] = ss.first_slot;
      }
    }

    // O^T of this wave's dims: block j4 * NHB + hb = dims 32 * j4 (of the
    // wave's slice) x heads 32 * hb of the workgroup
    f32x16 acc[NACC];
#pragma unroll
    for (int d = 0; d < NACC; ++d) acc[d] = (f32x16)0.0f;
    // base-2 reference max (per head); kNoMax until the head has seen a token,
    // so that p = exp2(s * c - m) of a masked score (s = -inf) is 0 even then
    float m_run = kNoMax;
    float l_run = 0.0f;       // sum of p over this lane's half of the tokens
    i16x8 qop[NKQ];           // Q^T operands (B of S^T = K . Q^T), loaded below
    i16x8 pop[2][NHB];        // P^T operands of the sub-tile in PV: [c][hb]

    // sub-tiles of 32 tokens; a trailing fully-invalid half tile is skipped
    const int st0 = 2 * seg.t0;
    const int st1 = min(2 * seg.t1, (n_b + kSubTokens - 1) / kSubTokens);
    const int nst = st1 - st0;

    // Page id of a sub-tile (pages of a multiple of 32 tokens hold whole
    // sub-tiles): a scalar load issued one iteration before the copy that
    // needs it, so its wait is free when it comes.
    const int32_t* bt_row = PAGED ? a.bt + (int64_t)b * a.bt_sb : a.bt;
    auto page_fetch = [&](int st) __attribute__((always_inline)) -> int {
      return s_load_i32(bt_row + page_slot_of<PAGE_UNIFORM>(a, st * kSubTokens));
    };
    auto page_ready = [&](int v) __attribute__((always_inline)) -> int {
      v = s_wait_i32(v);
      return v < 0 ? 0 : min(v, a.max_page);
    };

    // Copies of one sub-tile: per-lane source rows (one per row-group of this
    // wave, already offset to this lane's 16-byte piece), then one
    // global_load_lds per (row-group, column block).
    // A whole sub-tile inside one page (every sub-tile but a sequence's last,
    // partial one) needs no clamping: its rows start at a uniform offset
    // (page, first row in the page) plus a per-lane offset that is the same
    // for every sub-tile of the segment.
    // (32 rows of one page: below 2^31 bytes, which the host checks)
    uint32_t lane_row_off[RG_PER_WAVE];
#pragma unroll
    for (int ri = 0; ri < RG_PER_WAVE; ++ri) {
      const int rg = wave * RG_PER_WAVE + ri;
      lane_row_off[ri] = (uint32_t)((rg * 8 + dma_r) * (uint32_t)a.kv_s1) + ((lane & 7) ^ piece_swizzle(dma_r, rg)) * 16;
    }
    auto copy_src = [&](int st, int page, const char* (&src)[RG_PER_WAVE]) __attribute__((always_inline)) {
      const int tok_base = st * kSubTokens;
      if (PAGED && PAGE_UNIFORM && tok_base + kSubTokens <= n_b) {
        const int in_page = tok_base & (a.page_size - 1);  // PAGE_UNIFORM: power-of-two page
        const char* row0 = a.kv + (int64_t)page * a.kv_s0 + (int64_t)in_page * a.kv_s1;
#pragma unroll
        for (int ri = 0; ri < RG_PER_WAVE; ++ri) src[ri] = row0 + lane_row_off[ri];
        return;
      }
#pragma unroll
      for (int ri = 0; ri < RG_PER_WAVE; ++ri) {
        const int rg = wave * RG_PER_WAVE + ri;
        const int tok = tok_base + rg * 8 + dma_r;
        int pg = page;
        if (PAGED && !PAGE_UNIFORM) pg = load_page(a, b, page_slot_of(a, min(tok, n_b - 1)));
        src[ri] = a.kv + row_offset<PAGED>(a, b, tok, n_b, pg) + ((lane & 7) ^ piece_swizzle(dma_r, rg)) * 16;
      }
    };
    // voff / roff: byte offsets of the destination entries in the V and rope
    // rings (computed once per sub-tile, uniform)
    auto copy_one = [&](int voff, int roff, int ri, auto CB, const char* const (&src)[RG_PER_WAVE])
                        __attribute__((always_inline)) {
      constexpr int cb = decltype(CB)::value;
      const int rg = wave * RG_PER_WAVE + ri;
      char LDS_AS* dst = cb < NVB ? lds + voff + (rg * NVB + cb) * 1024
                                  : lds + OFF_R + roff + (rg * NRB + cb - NVB) * 1024;
      lds_copy16<cb * 128>(src[ri], dst);
    };
    auto issue = [&](int st, int page) __attribute__((always_inline)) {
      const char* src[RG_PER_WAVE];
      copy_src(st, page, src);
      const int k = st - st0;  // >= 0
#pragma unroll
      for (int ri = 0; ri < RG_PER_WAVE; ++ri)
        static_for<NCB>([&](auto CB) __attribute__((always_inline)) {
          copy_one(k % VST * VSLOT, k % kRopeStages * RSLOT, ri, CB, src);
        });
    };

    // fp8 cache. Copy of one sub-tile: this wave's rows 8w .. 8w + 7 into its
    // staging slot of entry (k & 1), where copy j (j < 4) moves the 16-byte
    // chunks 8j + lane / 8 (dims 128j + 16 * (lane / 8) ..) of row lane % 8
    // and copy 4 (lanes < 32) the rope chunks 32 + lane / 8. Lane l thus
    // reads back exactly the chunks it copied, and their places in the ring
    // differ from copy to copy by immediate offsets only.
    // (lane-derived offsets are recomputed where used: kept across the loop
    // they would not fit the register file beside Q^T and the operands)
    auto issue8 = [&](int st, int page) __attribute__((always_inline)) {
      const int k = st - st0;  // >= 0
      const int ln = lane_id_fresh();
      char LDS_AS* stg = lds + OFF_S + (k & 1) * STG + wave * STG_W;
      const int tok_base = st * kSubTokens;
      // a whole sub-tile of one page, or the sequence's last sub-tile, whose
      // rows past its end read its last row
      const int tok = min(tok_base + 8 * wave + (ln & 7), n_b - 1);
      // page_size * kv_s1 may pass 2^32 bytes: the in-page offset in 64 bits
      const char* src = a.kv + (int64_t)page * a.kv_s0 + (int64_t)(tok & (a.page_size - 1)) * a.kv_s1 +
                        16 * (ln >> 3);
      static_for<4>([&](auto J) __attribute__((always_inline)) {
        constexpr int j = decltype(J)::value;
        lds_copy16<128 * j>(src, stg + 1024 * j);
      });
      if (ln < 32) lds_copy16<512>(src, stg + 4096);
    };
    // Widening of the sub-tile copied into staging entry (k & 1) into V ring
    // entry k % VST and rope ring entry k % (VST - 1): conv_read fetches this
    // wave's chunks (its own copies: no barrier needed), conv_write writes
    // them, exactly widened, in the 16-bit ring layout (after the barrier
    // that frees the entries).
    i16x8 raw8[5];
    auto conv_read = [&](int k) __attribute__((always_inline)) {
      const char LDS_AS* stg = lds + OFF_S + (k & 1) * STG + wave * STG_W + lane_id_fresh() * 16;
      static_for<5>([&](auto J) __attribute__((always_inline)) {
        constexpr int j = decltype(J)::value;
        raw8[j] = ds_read_b128<1024 * j>(stg);
      });
      asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(raw8[0]), "+v"(raw8[1]), "+v"(raw8[2]), "+v"(raw8[3]), "+v"(raw8[4]));
    };
    auto conv_write = [&](int k) __attribute__((always_inline)) {
      const int ln = lane_id_fresh();
      const int r8c = ln & 7;
      const int swc = piece_swizzle(r8c, wave);
      const int p0c = 2 * ((ln >> 3) & 3);
      const int relA = (ln >> 5) * 1024 + (r8c * 8 + (p0c ^ swc)) * 16;
      const int relB = (ln >> 5) * 1024 + (r8c * 8 + ((p0c + 1) ^ swc)) * 16;
      char LDS_AS* vA = lds + (k % VST) * VSLOT + wave * NVB * 1024 + relA;
      char LDS_AS* vB = lds + (k % VST) * VSLOT + wave * NVB * 1024 + relB;
      static_for<4>([&](auto J) __attribute__((always_inline)) {
        constexpr int j = decltype(J)::value;
        ds_write_b128<2048 * j>(vA, widen_half<DT, 0>(raw8[j]));
        ds_write_b128<2048 * j>(vB, widen_half<DT, 1>(raw8[j]));
      });
      if (ln < 32) {
        char LDS_AS* r = lds + OFF_R + (k % kRopeStages) * RSLOT + wave * NRB * 1024;
        ds_write_b128<0>(r + relA, widen_half<DT, 0>(raw8[4]));
        ds_write_b128<0>(r + relB, widen_half<DT, 1>(raw8[4]));
      }
    };

    // One pass over a sub-tile pair: S^T of the sub-tile in kst (DO_S) and
    // PV steps [PV0, PV1) of O^T += V^T P^T for the sub-tile in vst, the
    // latter starting at step PVOFF, interleaved step by step so the MFMA
    // pipe alternates between the independent S chain and the PV
    // accumulators. PV step g is MFMA (c, j4, hb) = (g / SPC, (g % SPC) / NHB,
    // g % NHB), SPC = 4 * NHB steps per token half c; its V^T operand is
    // read at the first hb of each j4 and its P^T
    // operand at the first j4 of each c. LDS operands run PD steps ahead;
    // each step waits with an lgkmcnt that counts exactly the reads issued
    // after its own. hook(step) runs after each step's MFMAs (copies of a
    // later sub-tile, the rescale check, softmax pieces), so its VALU and
    // memory work overlaps them.
    // (two steps for the fp8 ring with 64 heads, whose widening leaves too
    // few registers for three steps of operands beside Q^T)
    constexpr int PD = F8 && NHB == 2 && TMLA_READ_AHEAD > 2 ? 2 : TMLA_READ_AHEAD;
    constexpr int SPC = NDBW * NHB;    // PV steps per token half
    // PV steps beside S (pass 1); the rest run beside the softmax (pass 2)
    constexpr int PV_SPLIT = NHB * TMLA_PV1_EIGHTHS;
    constexpr int PV_START = 4;        // S-only steps first: the rescale factors arrive meanwhile
    constexpr int EXP_PER_STEP = TMLA_EXP_PER_STEP;
    constexpr int SM_STEPS = 3 + 16 / EXP_PER_STEP;  // steps the softmax pieces need in pass 2
    static_assert(PV_SPLIT > 0 && PV_SPLIT <= 2 * SPC && 16 % EXP_PER_STEP == 0, "schedule");
    // pass 1 of an S wave: one PV step every PV_STRIDE S steps, so that the
    // time between a read and its use (PD steps) never shrinks to PD bare S
    // steps
    constexpr int PV_STRIDE0 = (NKC - 1 - PV_START) / (PV_SPLIT > 1 ? PV_SPLIT - 1 : 1);
    constexpr int PV_STRIDE = TMLA_PV_STRIDE < PV_STRIDE0 ? TMLA_PV_STRIDE : (PV_STRIDE0 > 0 ? PV_STRIDE0 : 1);
    static_assert(NDBW == 4, "four 32-dim blocks per wave");
    // S runs k-steps [SLO, SHI) of the S^T chain (the whole chain: [0, NKC));
    // the fence after its last k-step makes the scores readable by VALU.
    auto pass = [&](auto SLOC, auto SHIC, auto PVLO, auto PVHI, auto PVOFFC, auto PVSC, auto MINSTEPS,
                    const char LDS_AS* kst_v, const char LDS_AS* kst_r, const char LDS_AS* vst, const char LDS_AS* pst,
                    f32x16& s, auto&& hook) __attribute__((always_inline)) {
      constexpr int SLO = decltype(SLOC)::value, SHI = decltype(SHIC)::value;
      constexpr bool do_s = SHI > SLO;
      constexpr int PV0 = decltype(PVLO)::value;
      constexpr int PVOFF = decltype(PVOFFC)::value;
      constexpr int PVS = decltype(PVSC)::value;
      constexpr int NS = SHI - SLO, NV = decltype(PVHI)::value - PV0;
      constexpr int PV_END = PVOFF + (NV - 1) * PVS + 1;  // one past the last PV step
      constexpr int NSTEPS0 = NS > PV_END ? NS : PV_END;
      constexpr int NSTEPS = NSTEPS0 > decltype(MINSTEPS)::value ? NSTEPS0 : decltype(MINSTEPS)::value;
      const char LDS_AS* kvb[4] = {kst_v + k_off_v[0], kst_v + k_off_v[1], kst_v + k_off_v[2], kst_v + k_off_v[3]};
      const int rope_shift = (int)(kst_r - kst_v) + k_rope_delta;
      const char LDS_AS* krb[4] = {kvb[0] + rope_shift, kvb[1] + rope_shift, kvb[2] + rope_shift, kvb[3] + rope_shift};
      const char LDS_AS* vbase[2][2] = {{vst + v_off[0][0], vst + v_off[0][1]},
                                        {vst + v_off[1][0], vst + v_off[1][1]}};
      const char LDS_AS* pbase = pst + lane * 16;
      // Q^T rope operands (QR): the K rope operand's offsets in this wave's
      // Q rope rows
      const int q_shift = qrope - OFF_R + k_rope_delta;
      const char LDS_AS* qrb[4] = {lds + k_off_v[0] + q_shift, lds + k_off_v[1] + q_shift,
                                   lds + k_off_v[2] + q_shift, lds + k_off_v[3] + q_shift};
      i16x8 kb[PD + 1];
      i16x8 qb[PD + 1];
      i16x4 vl[NDBW * 2], vh[NDBW * 2];  // indexed by V^T operand id c * NDBW + j4
      auto fetch = [&](auto T) __attribute__((always_inline)) {
        constexpr int t = decltype(T)::value;
        if constexpr (t < NS) {
          constexpr int kc = SLO + t, cb = kc >> 2;
          if constexpr (cb < NVB)
            kb[t % (PD + 1)] = ds_read_b128<cb * 1024>(kvb[kc & 3]);
          else
            kb[t % (PD + 1)] = ds_read_b128<(cb - NVB) * 1024>(krb[kc & 3]);
          if constexpr (kc >= NKQ) qb[t % (PD + 1)] = ds_read_b128<(cb - NVB) * 1024>(qrb[kc & 3]);
        }
        if constexpr (pass_has_pv(t, NV, PVOFF, PVS)) {
          constexpr int g = PV0 + (t - PVOFF) / PVS, c = g / SPC, j4 = (g % SPC) / NHB, hb = g % NHB;
          if constexpr (hb == 0) {
            constexpr int off = c * 2 * NVB * 1024 + (j4 >> 1) * 1024;
            vl[c * NDBW + j4] = ds_read_tr<off>(vbase[j4 & 1][0]);
            vh[c * NDBW + j4] = ds_read_tr<off>(vbase[j4 & 1][1]);
          }
          if constexpr (j4 == 0) pop[c][hb] = ds_read_b128<(hb * 2 + c) * 1024>(pbase);
        }
      };
      static_for<PD>([&](auto T) __attribute__((always_inline)) { fetch(T); });
      static_for<NSTEPS>([&](auto J) __attribute__((always_inline)) {
        constexpr int j = decltype(J)::value;
        if constexpr (!TMLA_STEP_ORDER && j + PD < NSTEPS) fetch(std::integral_constant<int, j + PD>{});
        // reads issued after those of step j (before this step's wait)
        constexpr int ahead = TMLA_STEP_ORDER ? PD - 1 : PD;
        constexpr int last = (j + ahead < NSTEPS - 1) ? j + ahead : NSTEPS - 1;
        constexpr int after = [] {
          int n = 0;
          for (int t = j + 1; t <= last; ++t) n += pass_reads<NS, NV, PV0, NHB, PVOFF, PVS, SLO, NKQ>(t);
          return n;
        }();
        constexpr bool pv = pass_has_pv(j, NV, PVOFF, PVS);
        constexpr int g = PV0 + (pv ? (j - PVOFF) / PVS : 0), c = g / SPC, j4 = (g % SPC) / NHB, hb = g % NHB;
        constexpr bool has_k = j < NS;
        constexpr bool has_v = pv && hb == 0;
        constexpr bool has_p = pv && j4 == 0;
        constexpr int vi = c * NDBW + j4;
        constexpr int r = j % (PD + 1);
        // the wait ties the operands read for this step to it (a step that
        // only reuses operands needs none)
        constexpr bool has_q = has_k && SLO + j >= NKQ;  // the Q^T operand comes from LDS too
        if constexpr (!TMLA_WAIT_PAIR) {
          if constexpr (has_k || has_v || has_p)
            lgkm_tie<after, has_k, has_v, has_p>(kb[r], vl[vi], vh[vi], pop[c][hb]);
          if constexpr (has_q) asm volatile("" : "+v"(qb[r]));
        } else if constexpr (j % 2 == 0) {
          // one wait per two steps: the operands of steps j and j + 1
          constexpr int j2 = j + 1 < NSTEPS ? j + 1 : j;
          constexpr int after2 = [] {
            int n = 0;
            for (int t = j2 + 1; t <= last; ++t) n += pass_reads<NS, NV, PV0, NHB, PVOFF, PVS, SLO, NKQ>(t);
            return n;
          }();
          constexpr bool pv1 = pass_has_pv(j2, NV, PVOFF, PVS);
          constexpr int g1 = PV0 + (pv1 ? (j2 - PVOFF) / PVS : 0), c1 = g1 / SPC, j41 = (g1 % SPC) / NHB,
                        hb1 = g1 % NHB;
          constexpr bool has_k1 = j2 != j && j2 < NS, has_v1 = j2 != j && pv1 && hb1 == 0,
                         has_p1 = j2 != j && pv1 && j41 == 0;
          if constexpr (has_k || has_v || has_p || has_k1 || has_v1 || has_p1) {
            lgkm_wait<after2>();
            tie_ops<has_k, has_v, has_p>(kb[r], vl[vi], vh[vi], pop[c][hb]);
            tie_ops<has_k1, has_v1, has_p1>(kb[j2 % (PD + 1)], vl[c1 * NDBW + j41], vh[c1 * NDBW + j41],
                                            pop[c1][hb1]);
            if constexpr (has_q) asm volatile("" : "+v"(qb[r]));
            if constexpr (has_k1 && SLO + j2 >= NKQ) asm volatile("" : "+v"(qb[j2 % (PD + 1)]));
          }
        }
        if constexpr (j < NS) {
          if constexpr (SLO + j == 0)
            s = mfma_vgpr_first<DT>(kb[0], qop[0]);
          else if constexpr (has_q)
            mfma_vgpr_acc<DT>(s, kb[r], qb[r]);
          else
            mfma_vgpr_acc<DT>(s, kb[r], qop[SLO + j]);
        }
        auto pv_mfma = [&]() __attribute__((always_inline)) {
          if constexpr (pv) {
            const i16x4 lo = vl[vi], hi4 = vh[vi];
            const i16x8 vop = {lo[0], lo[1], lo[2], lo[3], hi4[0], hi4[1], hi4[2], hi4[3]};
            mfma_agpr_acc<DT>(acc[j4 * NHB + hb], vop, pop[c][hb]);
          }
        };
        if constexpr (TMLA_STEP_ORDER) {
          // the reads of a later step and this step's hook run under the S
          // MFMA, the PV MFMA follows them
          if constexpr (j + PD < NSTEPS) fetch(std::integral_constant<int, j + PD>{});
          hook(J);
          pv_mfma();
        } else {
          pv_mfma();
          hook(J);
        }
      });
      if constexpr (do_s && SHI == NKC) mfma_vgpr_fence(s);
    };

    // PV side: O^T columns of head block hb scale by the factor its S-owner
    // published; one 16-register block at a time, so the accumulators stay
    // in AGPRs.
    auto rescale = [&](const f32x4& alpha4) __attribute__((always_inline)) {
#pragma unroll
      for (int d = 0; d < NACC; ++d) {
        f32x16 t = acc[d];
        pin_vgpr(t);
        t *= alpha4[d % NHB];
        acc[d] = t;
        pin_agpr(acc[d]);
      }
    };

    // P^T (and factor) buffers of the sub-tile before the first: P = 0 and
    // factor 1, so that iteration -1's PV half adds exactly nothing.
    if (s_owner) {
      char LDS_AS* p1 = lds + OFF_P + PSLOT + wave * 2 * 1024 + lane * 16;
      ds_write_b128<0>(p1, (i16x8)0);
      ds_write_b128<1024>(p1, (i16x8)0);
      ds_write_b32(lds + OFF_A + ASLOT + ((lane & 31) * 4 + wave) * 4, 1.0f);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

    // Start-up: page ids of the first kStages sub-tiles (scalar loads, issued
    // before any vector traffic so they do not queue behind it), Q (needs
    // no page id, so it is in flight while the page ids come back), the copy
    // of sub-tile 0, and once Q and sub-tile 0 have landed the copy of
    // sub-tile 1; iteration -1 then copies sub-tile 2 beside its MFMAs like
    // every later iteration. At start-up every CU requests memory at once,
    // so asking only for what is needed first lets the computation start
    // sooner.
    static_assert(kStages == 4, "prologue page ids");
    static_assert(!F8 || TMLA_Q_LDS, "fp8 ring start-up stages Q through LDS");
    int pro_page[kStages] = {0, 0, 0, 0};
    // fp8 cache: scales of sub-tiles i+1 (used by iteration i), i+2 and i+3
    // (loading); scalar loads, rotated after the wait that completes them
    float sc1 = 1.0f, sc2 = 1.0f, sc3 = 1.0f;
    if (PAGED && PAGE_UNIFORM) {
#pragma unroll
      for (int i = 0; i < kStages; ++i) pro_page[i] = page_fetch(st0 + min(i, nst - 1));
    }
    auto load_q = [&]() __attribute__((always_inline)) {
      if (s_owner) {  // only the S waves use Q
        // heads past num_heads (a partial last block) run on head 0's row:
        // their scores stay finite and their output rows are never stored
        const short* qrow = reinterpret_cast<const short*>(a.q) + (int64_t)b * a.q_sb +
                            (int64_t)(head_ok ? head : 0) * a.q_sh + 8 * hi;
#pragma unroll
        for (int kc = 0; kc < NKQ; ++kc) qop[kc] = *reinterpret_cast<const i16x8*>(qrow + 16 * kc);
      }
      asm volatile("" ::: "memory");  // the copies below are issued after Q
    };
    auto pages_ready = [&]() __attribute__((always_inline)) {
      if (PAGED && PAGE_UNIFORM) {
#pragma unroll
        for (int i = 0; i < kStages; ++i) pro_page[i] = page_ready(pro_page[i]);
      }
    };
    if (TMLA_Q_LDS) {
      // Q through LDS: wave w copies its 32 rows (contiguous 1 KiB pieces,
      // the KV copies' swizzled layout) into V ring entry w and rope entry w
      // (wave 3: P buffer 0, written again only after the first barrier of
      // the loop), reads Q^T back with the K-operand offsets, and only then
      // are the rings handed to the KV copies.
      if (s_owner) stage_q(b);
      wait_vmcnt<0>();
      if (s_owner) {
#pragma unroll
        for (int kc = 0; kc < NKQ; ++kc) {
          const int cb = kc >> 2;
          const char LDS_AS* p = cb < NVB ? lds + qv + k_off_v[kc & 3] + cb * 1024
                                          : lds + qrope - OFF_R + k_off_v[kc & 3] + k_rope_delta + (cb - NVB) * 1024;
          qop[kc] = *reinterpret_cast<const i16x8 LDS_AS*>(p);
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      lds_barrier();  // every wave has its Q^T before the rings are refilled
      pages_ready();
      if constexpr (F8) {
        // sub-tiles 0 and 1 into staging entries 0 and 1, their scales, and
        // sub-tile 0 widened into ring entry 0 (the rings are free: every
        // wave has its Q^T)
        issue8(st0, pro_page[0]);  // nst >= 1
        sc2 = s_load_f32(a.kv_scale + (int64_t)pro_page[0] * a.sc_s0);
        sc3 = s_load_f32(a.kv_scale + (int64_t)pro_page[1] * a.sc_s0);
        if (nst > 1) {
          issue8(st0 + 1, pro_page[1]);
          wait_vmcnt<LOADS8>();
        } else {
          wait_vmcnt<0>();
        }
        conv_read(0);
        conv_write(0);
      } else {
        issue(st0, pro_page[0]);  // nst >= 1
        if (nst > 1) {
          issue(st0 + 1, pro_page[1]);
          wait_vmcnt<LOADS>();
        } else {
          wait_vmcnt<0>();
        }
      }
    } else if (TMLA_STARTUP == 0) {
      load_q();
      pages_ready();
      issue(st0, pro_page[0]);  // nst >= 1
      wait_vmcnt<0>();  // Q and sub-tile 0; the loop then uses Q with no further wait
      if (nst > 1) issue(st0 + 1, pro_page[1]);
    } else {
      // sub-tile 1 is in flight while Q and sub-tile 0 land (mode 1: Q
      // requested first; mode 2: sub-tile 0 first)
      if (TMLA_STARTUP == 1) load_q();
      pages_ready();
      issue(st0, pro_page[0]);  // nst >= 1
      if (TMLA_STARTUP == 2) load_q();
      if (nst > 1) {
        issue(st0 + 1, pro_page[1]);
        wait_vmcnt<LOADS>();  // all but sub-tile 1's copies
      } else {
        wait_vmcnt<0>();
      }
    }
    int next_page = pro_page[2];  // already waited for

    // Iteration i (-1 <= i < nst): PV(i) from ring entry i interleaved with
    // S(i+1) from entry i+1 (and the copies of sub-tile i+3), then the rest
    // of PV(i) interleaved with the softmax of sub-tile i+1, which publishes
    // P^T(i+1) and the factors for the next iteration; sub-tiles i+2 and i+3
    // are in flight. One instance of the passes serves every iteration: at
    // i = -1 the PV half multiplies sub-tile 0 by P = 0 and adds exactly
    // nothing; at i = nst-1 the S half reads a stale entry and its result is
    // discarded. The body is instantiated twice: with the copies of sub-tile
    // i+3 (every iteration with i + 3 < nst, no per-copy condition) and
    // without them (the last three iterations).
    static_assert(kStages == 4 && (F8 ? VST == 3 && kRopeStages == 2 : VST == 4 && kRopeStages == 3),
                  "ring offsets below");
    auto iteration = [&](const int i, auto DOCOPY) __attribute__((always_inline)) {
      constexpr bool do_copy = decltype(DOCOPY)::value;  // sub-tile i+3
      int page = 0;
      if constexpr (F8) {
        // fp8: copy sub-tile i+3 into staging entry (i+3) & 1 (this wave
        // widened its previous content, sub-tile i+1, in iteration i-1),
        // fetch this wave's chunks of sub-tile i+2 (copied in iteration i-1),
        // and once every wave is done with ring entries (i-1) % 3 (V) and
        // i % 2 (rope) widen sub-tile i+2 into them
        if (do_copy) {
          page = page_ready(next_page);
          issue8(st0 + i + 3, page);
        }
        if (i + 2 < nst) {
          if (do_copy) {
            wait_vmcnt<LOADS8>();
          } else {
            wait_vmcnt<0>();
          }
          conv_read(i + 2);
        }
        // every wave's P^T(i) and factors are written; the scale of sub-tile
        // i+2 has arrived
        asm volatile("s_waitcnt lgkmcnt(0)" : "+s"(sc2), "+s"(sc3) : : "memory");
        sc1 = sc2;
        sc2 = sc3;
        lds_barrier();
        if (i + 2 < nst) conv_write(i + 2);
      } else {
        // sub-tile i+1 must have landed; sub-tile i+2 may still be in flight
        if (do_copy) {  // here i + 2 < nst
          if (i >= 0) wait_vmcnt<LOADS>();
        } else if (i >= 0 && i + 1 < nst) {
          if (i + 2 < nst) {
            wait_vmcnt<LOADS>();
          } else {
            wait_vmcnt<0>();
          }
        }
        page = (PAGED && PAGE_UNIFORM && do_copy) ? page_ready(next_page) : 0;
        // every wave's P^T(i) and factors are written and every wave is done
        // with the ring entries refilled during this iteration
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        lds_barrier();
      }
      // the page-id (and scale) loads go out before every counted LDS read of
      // the iteration, so their out-of-order returns can only make the
      // counted waits wait longer
      if (PAGED && PAGE_UNIFORM && i + kStages < nst)
        next_page = i < 0 ? pro_page[kStages - 1] : page_fetch(st0 + i + kStages);
      if (F8 && do_copy) sc3 = s_load_f32(a.kv_scale + (int64_t)page * a.sc_s0);  // sub-tile i+3
      const int pbuf = i & 1;
      f32x4 alpha4 = ds_read_f32x4(lds + OFF_A + pbuf * ASLOT + (lane & 31) * 16);
      // ring entries (i + 1 >= 0): S(i+1) reads entry i+1, PV(i) entry i
      // (entry 0 at i = -1, where P = 0), the copies fill entry i+3 (16-bit
      // cache; the fp8 widening fills entry i+2 above)
      const unsigned k1 = (unsigned)(i + 1);
      const unsigned r1 = F8 ? (k1 & 1u) : k1 % 3u;
      const char LDS_AS* vst = lds + (i < 0 ? 0u : (F8 ? (k1 + 2u) % 3u : (k1 + 3u) & 3u)) * VSLOT;
      const char LDS_AS* kst_v = lds + (F8 ? k1 % 3u : k1 & 3u) * VSLOT;
      const char LDS_AS* kst_r = lds + r1 * RSLOT;
      const int copy_voff = (int)((k1 + 2u) & 3u) * VSLOT;
      const int copy_roff = (int)(r1 == 0u ? 2u : r1 - 1u) * RSLOT;
      const char LDS_AS* pst = lds + OFF_P + pbuf * PSLOT;
      const int st_s = st0 + i + 1;  // sub-tile of this iteration's S
      const bool stamped = TMLA_STAMPS && b == b_first && (i == kStampIter || i == kStampIter + 1);
      StampRec st_begin{}, st_pass1{}, st_pass2{};
      if (stamped) st_begin = stamp_now();

      // pass 1: S(i+1) and PV(i) steps [0, PV_SPLIT) from step PV_START on;
      // the copies of sub-tile i+3 are spread evenly over the pass's steps,
      // and the factors published for PV(i) are applied before its first
      // MFMA (the wait of step PV_START - 1 covers their read, which is older
      // than every read of the pass)
      const char* csrc[RG_PER_WAVE];
      auto pass1_hook = [&](auto NSTEPSC) __attribute__((always_inline)) {
        return [&](auto J) __attribute__((always_inline)) {
          constexpr int j = decltype(J)::value;
          constexpr int NST = decltype(NSTEPSC)::value;
          if constexpr (j == 0 && do_copy && !F8) copy_src(st0 + i + kStages - 1, page, csrc);
          if constexpr (j == PV_START - 1) {
            pin_f4(alpha4);
            bool any = false;
#pragma unroll
            for (int hb = 0; hb < NHB; ++hb) any |= alpha4[hb] != 1.0f;
            if (__builtin_amdgcn_ballot_w64(any) != 0) rescale(alpha4);
          }
          static_for<LOADS>([&](auto K) __attribute__((always_inline)) {
            constexpr int k = decltype(K)::value;
            if constexpr (do_copy && !F8 && k * NST / LOADS == j)
              copy_one(copy_voff, copy_roff, k / NCB, std::integral_constant<int, k % NCB>{}, csrc);
          });

        };
      };

      // S-owner waves: pass 1 with S(i+1); pass 2 = PV(i) steps
      // [PV_SPLIT, 2 * SPC) beside the softmax of sub-tile i+1 (heads of this
      // wave), base-2 with the lazy rescale: the reference max only moves,
      // for the whole wave, when a score exceeds it by 2^kRescaleLog2 (then
      // both token halves of every head agree on the new max through one lane
      // exchange). Scores stay unscaled: the max is taken on s (scale > 0) or
      // -s (scale < 0) and the scale is folded into p = 2^(s * c - m).
      auto owner_iteration = [&]() __attribute__((always_inline)) {
        f32x16 s;
        pass(std::integral_constant<int, 0>{}, std::integral_constant<int, NKC>{}, std::integral_constant<int, 0>{},
             std::integral_constant<int, PV_SPLIT>{}, std::integral_constant<int, PV_START>{},
             std::integral_constant<int, PV_STRIDE>{},
             std::integral_constant<int, 0>{}, kst_v, kst_r, vst, pst, s, pass1_hook(std::integral_constant<int, NKC>{}));
        if (stamped) st_pass1 = stamp_now();
        // no token past the sequence (for the wave's earliest query token)
        const bool full = (st_s + 1) * kSubTokens <= n_b - lag_wave;
        // (fp8 cache: the page's scale multiplies every score; a zero product
        // runs as the smallest normal float of the same sign, as the host does
        // for a zero softmax scale, so masked scores stay -inf)
        float c = a.qk_scale_log2;
        if constexpr (F8) {
          c *= sc1;
          if (c == 0.0f) c = copysignf(1.17549435e-38f, a.qk_scale_log2);
        }
        float m_use = m_run, lsum = 0.0f, alpha = 1.0f;
        auto softmax_hook = [&](auto J) __attribute__((always_inline)) {
          constexpr int j = decltype(J)::value;
          if constexpr (j == 0) {  // mask tokens past the sequence (last sub-tile only)
            if (!full) {
              const int tok0 = st_s * kSubTokens + 4 * hi;
              const float off = c >= 0.0f ? -INFINITY : INFINITY;
#pragma unroll
              for (int r = 0; r < 16; ++r)
                if (tok0 + 8 * (r >> 2) + (r & 3) >= n_b - causal_lag(a, head_base + (lane_id_fresh() & 31))) s[r] = off;
            }
            pin_f16(s);
          } else if constexpr (j == 1) {  // reference max
            float mx = c >= 0.0f ? s[0] : -s[0];
            if (c >= 0.0f) {
#pragma unroll
              for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
            } else {
#pragma unroll
              for (int r = 1; r < 16; ++r) mx = fmaxf(mx, -s[r]);
            }
            mx *= fabsf(c);
            if (__builtin_amdgcn_ballot_w64(mx > m_run + kRescaleLog2) != 0) {
              // the exchange is an LDS operation outside the pass's
              // counting: let every counted read finish first
              asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
              m_use = fmaxf(m_run, fmaxf(mx, __shfl_xor(mx, 32)));
              if (m_run != kNoMax) alpha = fast_exp2(m_run - m_use);
            }
            pin_f2(m_use, alpha);
          } else if constexpr (j >= 2 && j < 2 + 16 / EXP_PER_STEP) {  // EXP_PER_STEP probabilities
#pragma unroll
            for (int e = 0; e < EXP_PER_STEP; ++e) {
              const int r = EXP_PER_STEP * (j - 2) + e;
              s[r] = fast_exp2(fmaf(s[r], c, -m_use));  // masked: +-inf * c = -inf -> 0
              lsum += s[r];
            }
            pin_f16(s);
            pin_f1(lsum);
          } else if constexpr (j == 2 + 16 / EXP_PER_STEP) {
            if constexpr (F8) {  // the value product sees p times the page's scale
#pragma unroll
              for (int r = 0; r < 16; ++r) s[r] *= sc1;
            }
            pack_probs_in_place<DT>(s);
          }
        };
        pass(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, std::integral_constant<int, PV_SPLIT>{},
             std::integral_constant<int, 2 * SPC>{}, std::integral_constant<int, 0>{}, std::integral_constant<int, 1>{},
             std::integral_constant<int, SM_STEPS>{}, kst_v, kst_r, vst, pst, s, softmax_hook);
        if (stamped) st_pass2 = stamp_now();
        {
          char LDS_AS* pw = lds + OFF_P + (pbuf ^ 1) * PSLOT + wave * 2 * 1024 + lane * 16;
          ds_write_b128<0>(pw, packed_half(s, 0));
          ds_write_b128<1024>(pw, packed_half(s, 1));
          ds_write_b32(lds + OFF_A + (pbuf ^ 1) * ASLOT + ((lane & 31) * 4 + wave) * 4, alpha);
        }
        if (i + 1 < nst) {
          l_run = l_run * alpha + lsum;
          m_run = m_use;
        }
        if (stamped) {  // the next iteration starts with this wait anyway
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          if (i == kStampIter) {
            stamp_store(5, st_begin);
            stamp_store(6, st_pass1);
            stamp_store(7, st_pass2);
          } else {
            stamp_store(8, st_begin);
          }
        }
      };
      // the other waves: their share of PV(i) and of the copies
      auto pv_iteration = [&]() __attribute__((always_inline)) {
        f32x16 s;
        pass(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{},
             std::integral_constant<int, PV_SPLIT>{}, std::integral_constant<int, PV_START>{},
             std::integral_constant<int, 1>{}, std::integral_constant<int, 0>{}, kst_v, kst_r, vst, pst, s,
             pass1_hook(std::integral_constant<int, PV_SPLIT + PV_START>{}));
        pass(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, std::integral_constant<int, PV_SPLIT>{},
             std::integral_constant<int, 2 * SPC>{}, std::integral_constant<int, 0>{}, std::integral_constant<int, 1>{},
             std::integral_constant<int, 0>{}, kst_v, kst_r, vst, pst, s, [](auto) {});
      };
      if constexpr (NHB == NW) {
        owner_iteration();
      } else {
        if (s_owner)
          owner_iteration();
        else
          pv_iteration();
      }
    };
    // Iteration -1 always runs with copies: for a segment of fewer than
    // kStages - 1 sub-tiles its copy is of a clamped (valid) row into an
    // entry no iteration reads, and the tail then never starts from the
    // initial accumulators (which would have to be kept live across the
    // first loop).
    if (b == b_first) phase_stamp(2);
    if constexpr (F8) set_lane_offsets(lane_id_fresh());
    int i = -1;
    for (; i < 0 || i + kStages - 1 < nst; ++i) iteration(i, std::true_type{});
    if constexpr (F8) set_lane_offsets(lane_id_fresh());
    for (; i < nst; ++i) iteration(i, std::false_type{});
    // every copy has landed and all waves are done with the rings before the
    // finalize reuses them
    if constexpr (TMLA_MFMA_VOLATILE) mfma_agpr_fence(acc[NACC - 1]);  // the last PV MFMAs have landed
    wait_vmcnt<0>();
    lds_barrier();
    if (b == b_first) phase_stamp(3);

    // ---- finalize: out = acc / l, lse2 = m + log2(l) -------------------------
    {
      const int lane = lane_id_fresh();  // (see lane_id_fresh)
      const int head = head_base + (lane & 31);
      const bool head_ok = s_owner && head < a.num_heads;
      const int hi = lane >> 5;
      const float l_tot = l_run + __shfl_xor(l_run, 32);
      const bool has = l_tot > 0.0f;
      const float inv = has ? 1.0f / l_tot : 0.0f;
      const float lse2 = has ? m_run + fast_log2(l_tot) : -INFINITY;
      {
        // 1/l of every head of the workgroup, for the waves' column slices
        ds_write_b32(lds + OFF_A + ((lane & 31) * 4 + wave) * 4, inv);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        lds_barrier();
        f32x4 inv4 = ds_read_f32x4(lds + OFF_A + (lane & 31) * 16);
        lgkm_tie_f4<0>(inv4);
        // The normalised rows go through the idle rings (32*NHB padded rows;
        // the 16-byte pad spreads the lanes' 8-byte writes over all banks),
        // so that every global store then writes one whole row of DV elements.
#pragma unroll
        for (int j4 = 0; j4 < NDBW; ++j4)
#pragma unroll
          for (int hb = 0; hb < NHB; ++hb)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
              i16x4 v;
#pragma unroll
              for (int e = 0; e < 4; ++e) v[e] = Elt<DT>::from_float(acc[j4 * NHB + hb][4 * q4 + e] * inv4[hb]);
              const int dim = wave * (DV / NW) + 32 * j4 + 8 * q4 + 4 * hi;
              *reinterpret_cast<i16x4 LDS_AS*>(lds + (hb * 32 + (lane & 31)) * OPITCH + dim * 2) = v;
            }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        lds_barrier();
        short* dst;
        int64_t row_stride;
        if (seg.direct) {
          dst = reinterpret_cast<short*>(a.out) + (int64_t)b * a.out_sb + (int64_t)head_base * a.out_sh;
          row_stride = a.out_sh;
        } else {
          // the partial is a convex combination of cache rows, so it fits the
          // input dtype; it is stored there (half the bytes of float32)
          dst = a.mid_o + ((int64_t)seg.slot * a.num_heads + head_base) * DV;
          row_stride = DV;
        }
        // wave-uniform; only the waves that own a head block hold staged rows
        int rows = __builtin_amdgcn_readfirstlane(wave < NHB ? min(32, a.num_heads - head_base) : 0);
        // computed per segment: 32 hoisted row conditions would crowd the SGPRs
        asm volatile("" : "+s"(rows));
        const char LDS_AS* obuf = lds + wave * 32 * OPITCH;
        // eight rows per batch: their reads are all issued before the first
        // store waits for its data
#pragma unroll
        for (int r0 = 0; r0 < 32; r0 += 8) {
          i16x8 row[8];
#pragma unroll
          for (int k = 0; k < 8; ++k) row[k] = *reinterpret_cast<const i16x8 LDS_AS*>(obuf + (r0 + k) * OPITCH + lane * 16);
#pragma unroll
          for (int k = 0; k < 8; ++k)
            if (r0 + k < rows) store_through(reinterpret_cast<i16x8*>(dst + (r0 + k) * row_stride + lane * 8), row[k]);
        }
        if (head_ok && hi == 0) {
          if (seg.direct) {
            if (a.lse) a.lse[(int64_t)b * a.num_heads + head] = has ? lse2 * kLn2 : -INFINITY;
          }
          else
            store_through_f32(a.mid_lse + (int64_t)seg.slot * a.num_heads + head, lse2);
        }
        // the next segment refills the rings
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        lds_barrier();
      }
    }

    if (b == b_first) phase_stamp(4);
    if (a.fused && !seg.direct) {
      // every wave's write-through partial row and lse stores have
      // completed before the arrival
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      lds_barrier();
      if (wave == 0 && lane == 0) {
        const int old = sys_add(a.m_count + (int64_t)b * gridDim.y + blockIdx.y, 1);
        int* r = s_pend[b == b_first ? 0 : 1];
        r[4] = old == r[2] - 1;  // this arrival completed the count
      }
    }

    remaining -= t_end - t_start + wr.seg_cost;  // the next sequence's start is charged here
    seg_global_off += nt_b + wr.seg_cost;
    ++b;
    t_start = 0;
  }

  if (a.fused) {
    const CoherentLoads ld{
        __builtin_amdgcn_make_buffer_rsrc(a.mid_o, 0, a.mid_o_bytes, kBufferWord3),
        __builtin_amdgcn_make_buffer_rsrc(a.mid_lse, 0, a.mid_o_bytes / 256, kBufferWord3)};
    fused_merge_tail<DT>(MergeView{a.mid_o, a.mid_lse, a.num_heads, a.out, a.out_sb, a.out_sh, a.lse}, ld,
                         a.m_count, a.m_done, a.m_flag, a.spin_limit, wave, s_pend, s_msg, kHeadsPerWave * NHB);
  }
}

// ---------------------------------------------------------------------------
// Stage 1 at 128 heads per workgroup: the head-owner loop
// ---------------------------------------------------------------------------
//
// Wave w owns heads 32w..32w+31 of the workgroup for the whole computation:
// S^T = K . Q^T (36 MFMAs per 32-token sub-tile), the online softmax of its
// heads, and O^T += V^T . P^T over all 512 value dims (16 accumulator blocks
// of 32 dims x 32 heads in AGPRs, 32 MFMAs per sub-tile). P^T is the score
// tile itself, rounded in place: the 32x32 accumulator holds, in lane l,
// head l%32 and tokens 8(r/4) + 4(l/32) + r%4 in register r, so registers
// 0-7 are the B operand of the value product's k-step over tokens 0-15 and
// registers 8-15 that of tokens 16-31, with k taken in that token order; the
// V^T operand reads (ds_read_b64_tr_b16, addressing as in
// mla_partial_kernel) deliver the same order. No wave reads another wave's
// probabilities, so the workgroup barrier of an iteration only hands ring
// entries back to the copies.
//
// Iteration i of a segment (sub-tiles i and i+1 in the ring, i+2 and i+3 in
// flight): one run of steps that first issues the S^T MFMAs of sub-tile i+1,
// one K read each, beside the softmax of sub-tile i (whose scores the
// previous iteration computed) and the copies of sub-tile i+3, then the 32
// value MFMAs of sub-tile i, two V^T reads each, with the probabilities
// straight from registers. The softmax VALU work thus runs under MFMAs whose
// operands do not depend on it. Two score tiles alternate (one is turned into
// probabilities while the other accumulates), and the loop body is written
// out for both. When the reference max of a head moves (the lazy rescale,
// rare), O^T is rescaled before the value MFMAs of the sub-tile.
//
// LDS: V ring (dims 0..511, 4 entries) and rope ring (dims 512..575, 3
// entries) in mla_partial_kernel's swizzled block layout, and the rope rows of
// Q (read as the Q^T operand of the rope k-chunks, whose registers the loop
// cannot spare); 156 KiB.
// 1: 128-head workgroups run the head-owner loop (0: mla_partial_kernel)
#ifndef TMLA_OWN_LOOP
#define TMLA_OWN_LOOP 1
#endif
#ifndef TMLA_OWN_READ_AHEAD
#define TMLA_OWN_READ_AHEAD 3
#endif
// softmax schedule inside the step run of an iteration: first exponential at
// this step, then one every TMLA_OWN_EXP_STRIDE steps
#ifndef TMLA_OWN_EXP_START
#define TMLA_OWN_EXP_START 4
#endif
#ifndef TMLA_OWN_EXP_STRIDE
#define TMLA_OWN_EXP_STRIDE 2
#endif
// steps of an iteration's run that issue the copies of sub-tile i+3: from
// step TMLA_OWN_COPY_FIRST, spread over TMLA_OWN_COPY_SPAN steps
#ifndef TMLA_OWN_COPY_FIRST
#define TMLA_OWN_COPY_FIRST 1
#endif
#ifndef TMLA_OWN_COPY_SPAN
#define TMLA_OWN_COPY_SPAN 32
#endif
// operand registers beyond the read-ahead (an MFMA queued behind the one
// before it may read its operands after the next fetch was issued)
#ifndef TMLA_OWN_EXTRA_BUF
#define TMLA_OWN_EXTRA_BUF 0
#endif
// 1: a scheduling barrier after every step of the run
#ifndef TMLA_OWN_SCHED_FENCE
#define TMLA_OWN_SCHED_FENCE 1
#endif
// S^T accumulated in this many chains (1 or 2) over alternate k-chunks
#ifndef TMLA_OWN_S_CHAINS
#define TMLA_OWN_S_CHAINS 2
#endif
// the next sub-tile's max this many value steps after its last S^T MFMA
#ifndef TMLA_OWN_MAX_LAG
#define TMLA_OWN_MAX_LAG 8
#endif

// S^T MFMAs of the head-owner loop: volatile asm, so they keep their places
// among the operand reads and waits and keep their accumulators in VGPRs
// (the value accumulators own every AGPR). The VALU reads of their results
// are placed a fixed number of steps later, past the result latency.
template <int DT>
__device__ __forceinline__ f32x16 own_mfma_first(const i16x8& a, const i16x8& b) {
  f32x16 d;
  if constexpr (DT == TMLA_BF16)
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "v"(b));
  else
    asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "v"(b));
  return d;
}
template <int DT>
__device__ __forceinline__ void own_mfma_acc(f32x16& d, const i16x8& a, const i16x8& b) {
  if constexpr (DT == TMLA_BF16)
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "v"(b));
  else
    asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "v"(b));
}

// LDS reads issued by step t of a run of NS S^T steps and NV value steps
// (the rope k-chunks 32..35 read Q^T from LDS beside K).
template <int NS, int NV>
constexpr int own_step_reads(int t) {
  return t < NS ? (t < 32 ? 1 : 2) : (t < NS + NV ? 2 : 0);
}

template <int DT, bool PAGED, bool PAGE_UNIFORM>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void mla_partial_own_kernel(PartialArgs a) {
  constexpr int DV = 512, DQK = 576;
  constexpr int NCB = DQK / 64;   // 128-byte column blocks per row
  constexpr int NVB = DV / 64;    // ... of which hold V dims
  constexpr int NRB = NCB - NVB;  // ... and rope dims
  constexpr int NKC = DQK / 16;   // k-chunks of QK^T
  constexpr int NDB = DV / 32;    // 32-dim blocks of PV (all of them per wave)
  constexpr int VSLOT = 4 * NVB * 1024;
  constexpr int RSLOT = 4 * NRB * 1024;
  constexpr int RING = 4;         // entries of both rings
  constexpr int RRING = RING - 1;  // rope entries: dead once S of their sub-tile is done
  constexpr int OFF_R = RING * VSLOT;
  constexpr int OFF_Q = OFF_R + RRING * RSLOT;  // Q rope rows of the workgroup (read as Q^T)
  constexpr int SMEM = OFF_Q + 4 * RSLOT;
  constexpr int NKQ = DV / 16;    // k-chunks whose Q^T operand stays in VGPRs
  constexpr int LOADS = NCB;      // DMA instructions per wave per sub-tile (row-group `wave`)
  constexpr int OPITCH = DV * 2 + 16;
  constexpr int PD = TMLA_OWN_READ_AHEAD;
  // operand registers of a step are refilled NOB steps after their fetch:
  // at least two steps after the MFMA that read them was issued
  constexpr int NOB = PD + 1 + TMLA_OWN_EXTRA_BUF;
  constexpr int E0 = TMLA_OWN_EXP_START, ES = TMLA_OWN_EXP_STRIDE;
  constexpr int MX = NKC + TMLA_OWN_MAX_LAG;  // step of the next sub-tile's max
  constexpr int SCH = TMLA_OWN_S_CHAINS;      // accumulation chains of S^T
  // the copies of sub-tile i+3: at steps CP0 + k * CPS / LOADS, k < LOADS
  constexpr int CP0 = TMLA_OWN_COPY_FIRST, CPS = TMLA_OWN_COPY_SPAN;
  static_assert(NRB == 1 && NKC == 36 && NDB == 16 && NKQ == 32, "512 latent + 64 rope dims");
  static_assert(128 * OPITCH <= SMEM, "output staging fits the rings");
  static_assert(SMEM <= 160 * 1024, "LDS");
  static_assert(PD >= 1 && PD <= 4, "read-ahead");
  static_assert(SCH == 1 || SCH == 2, "S^T chains");
  static_assert(CP0 >= 1 && CP0 + (LOADS - 1) * CPS / LOADS < NKC + 2 * NDB, "copy schedule");
  // the probabilities of tokens 0-15 (exponentials 0-7) are packed before the
  // first value step, those of tokens 16-31 before the value steps of k-step 1
  static_assert(E0 >= 1 && E0 + 7 * ES + 1 < NKC && E0 + 15 * ES + 1 < NKC + NDB, "softmax schedule");
  static_assert(MX >= NKC + 6 && MX + 5 <= NKC + 2 * NDB, "max after the S^T results are ready");

  __shared__ __attribute__((aligned(1024))) char smem[SMEM];
  char LDS_AS* const lds = (char LDS_AS*)(void LDS_AS*)smem;
  __shared__ int s_pend[2][5];
  __shared__ int s_msg[4];

  phase_stamp(0);
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nwg = gridDim.x;
  const int worker = worker_index(a);
  const int head_base = blockIdx.y * 128 + wave * kHeadsPerWave;
  const int lag_wave = __builtin_amdgcn_readfirstlane(causal_lag(a, head_base));
  const int pre_len = __builtin_amdgcn_readfirstlane((a.fused && worker < a.batch) ? a.seqlens[worker] : 1);
  if (a.fused && tid == 0) s_pend[0][0] = s_pend[1][0] = -1;

  // Q rows of sequence bq for this wave's heads into V ring entry `wave` and
  // rope entry `wave`, in the KV copies' swizzled layout (heads past
  // num_heads copy head 0's row).
  auto stage_q = [&](int bq) __attribute__((always_inline)) {
    const int ln = lane_id_fresh();
    const int r = ln >> 3;
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      const int hq = head_base + 8 * rg + r;
      const char* src = a.q + ((int64_t)bq * a.q_sb + (int64_t)(hq < a.num_heads ? hq : 0) * a.q_sh) * 2 +
                        ((ln & 7) ^ piece_swizzle(r, rg)) * 16;
      static_for<NCB>([&](auto CB) __attribute__((always_inline)) {
        constexpr int cb = decltype(CB)::value;
        char LDS_AS* dst = cb < NVB ? lds + wave * VSLOT + (rg * NVB + cb) * 1024
                                    : lds + OFF_Q + wave * RSLOT + (rg * NRB + cb - NVB) * 1024;
        lds_copy16<cb * 128>(src, dst);
      });
    }
  };

  // ---- work range -------------------------------------------------------
  WorkRange wr;
  if (!work_range(a, worker, wr)) {
    if (!a.fused) return;
  }
  const int b_first = wr.b_first, tile_lo = wr.tile_lo, tile_hi = wr.tile_hi;
  const int off_first = wr.off_first, n_first = wr.n_first;
  if (a.fused) {
    // empty sequences worker, worker + nwg, ...: out = 0, lse = -inf
    const int lane = lane_id_fresh();
    const int hb0 = blockIdx.y * 128;
    const int nh = min(128, a.num_heads - hb0);
    const MergeView mv{a.mid_o, a.mid_lse, a.num_heads, a.out, a.out_sb, a.out_sh, a.lse};
    for (int bb = worker; bb < a.batch; bb += nwg) {
      const int len = bb == worker ? pre_len : a.seqlens[bb];
      if (tiles_of(len) == 0)
        for (int h = hb0 + wave; h < hb0 + nh; h += 4) merge_zero(mv, bb, h, lane);
    }
  }
  if (tile_lo >= tile_hi) return;
  phase_stamp(1);

  int b = b_first;
  int t_start = tile_lo;
  int remaining = tile_hi - tile_lo;
  int seg_global_off = off_first;

  while (remaining > 0) {
    const int n_b = b == b_first ? n_first : a.seqlens[b];
    const int nt_b = tiles_of(n_b);
    if (nt_b == 0) {
      ++b;
      continue;
    }
    const int t_end = min(nt_b, t_start + remaining);
    const int lane = lane_id_fresh();
    const int head = head_base + (lane & 31);
    const bool head_ok = head < a.num_heads;
    const int hi = lane >> 5;
    // S^T A operand: token lane%32, piece 2*(kc%4) + hi of column block kc/4
    int k_off_v[4];
    int k_rope_delta;
    {
      const int rg = (lane & 31) >> 3, r = lane & 7;
      const int sw = piece_swizzle(r, rg);
#pragma unroll
      for (int j = 0; j < 4; ++j) k_off_v[j] = rg * NVB * 1024 + (r * 8 + ((2 * j + hi) ^ sw)) * 16;
      k_rope_delta = OFF_R - rg * (NVB - NRB) * 1024;
    }
    // V^T operand of dim block db (ds_read_b64_tr_b16): group g = lane/16,
    // L = lane%16; read e2 of k-step c covers token 16c + 8e2 + 4(g/2) + L/4,
    // dims 32db + 16(g%2) + 4(L%4); the column block db/2 and the k-step are
    // immediate offsets.
    int v_off[2][2];  // [db & 1][e2]
    {
      const int g = lane >> 4, L = lane & 15;
      const int r = 4 * (g >> 1) + (L >> 2);
#pragma unroll
      for (int dbp = 0; dbp < 2; ++dbp)
#pragma unroll
        for (int e2 = 0; e2 < 2; ++e2) {
          const int piece = 4 * dbp + 2 * (g & 1) + ((L & 3) >> 1);
          v_off[dbp][e2] = e2 * NVB * 1024 + (r * 8 + (piece ^ piece_swizzle(r, e2))) * 16 + 8 * (L & 1);
        }
    }
    const int dma_r = lane >> 3;

    Segment seg;
    seg.b = b;
    seg.t0 = t_start;
    seg.t1 = t_end;
    {
      const SegmentSlot ss = segment_slot(a, wr, worker, b, t_start, nt_b, seg_global_off);
      seg.slot = ss.slot;
      seg.direct = ss.direct;
      if (a.fused && !seg.direct && wave == 0 && lane == 0) {
        int* r = s_pend[b == b_first ? 0 : 1];
        r[0] = b;
        r[1] = ss.index;
        r[2] = ss.count;
        r[3] = ss.first_slot;
      }
    }

    f32x16 acc[NDB];  // O^T: dims 32db.. of this wave's 32 heads
#pragma unroll
    for (int d = 0; d < NDB; ++d) acc[d] = (f32x16)0.0f;
    float m_run = kNoMax;  // base-2 reference max of the lane's head
    float l_run = 0.0f;    // sum of p over this lane's half of the tokens
    i16x8 qop[NKQ];  // Q^T of the latent k-chunks (the rope ones are read from OFF_Q)

    const int st0 = 2 * seg.t0;
    const int st1 = min(2 * seg.t1, (n_b + kSubTokens - 1) / kSubTokens);
    const int nst = st1 - st0;

    const int32_t* bt_row = PAGED ? a.bt + (int64_t)b * a.bt_sb : a.bt;
    auto page_fetch = [&](int st) __attribute__((always_inline)) -> int {
      return s_load_i32(bt_row + page_slot_of<PAGE_UNIFORM>(a, st * kSubTokens));
    };
    auto page_ready = [&](int v) __attribute__((always_inline)) -> int {
      v = s_wait_i32(v);
      return v < 0 ? 0 : min(v, a.max_page);
    };
    // this lane's piece of row 8*wave + lane/8 of a sub-tile that lies in
    // one page (32 rows of one page: below 2^31 bytes, which the host checks)
    const uint32_t lane_row_off =
        (uint32_t)((wave * 8 + dma_r) * (uint32_t)a.kv_s1) + ((lane & 7) ^ piece_swizzle(dma_r, wave)) * 16;
    auto copy_src = [&](int st, int page) __attribute__((always_inline)) -> const char* {
      const int tok_base = st * kSubTokens;
      if (PAGED && PAGE_UNIFORM && tok_base + kSubTokens <= n_b) {
        const int in_page = tok_base & (a.page_size - 1);
        return a.kv + (int64_t)page * a.kv_s0 + (int64_t)in_page * a.kv_s1 + lane_row_off;
      }
      const int tok = tok_base + wave * 8 + dma_r;
      int pg = page;
      if (PAGED && !PAGE_UNIFORM) pg = load_page(a, b, page_slot_of(a, min(tok, n_b - 1)));
      return a.kv + row_offset<PAGED>(a, b, tok, n_b, pg) + ((lane & 7) ^ piece_swizzle(dma_r, wave)) * 16;
    };
    auto copy_one = [&](int k, auto CB, const char* src) __attribute__((always_inline)) {
      constexpr int cb = decltype(CB)::value;
      char LDS_AS* dst = cb < NVB ? lds + (k & 3) * VSLOT + (wave * NVB + cb) * 1024
                                  : lds + OFF_R + (k % RRING) * RSLOT + (wave * NRB + cb - NVB) * 1024;
      lds_copy16<cb * 128>(src, dst);
    };
    auto issue = [&](int st, int page) __attribute__((always_inline)) {
      const char* src = copy_src(st, page);
      static_for<NCB>([&](auto CB) __attribute__((always_inline)) { copy_one(st - st0, CB, src); });
    };

    // A run of NS S^T steps (k-chunks 0..NS-1 of the sub-tile in ring entry
    // ks, accumulating into sacc, or with two chains into sacc and sacc2, whose
    // sum is the score tile) followed by NV value steps g = 0..NV-1
    // (k-step c = g / 16, dim block db = g % 16) of the sub-tile in entry vs,
    // with the probabilities of k-step c packed in pk[c]. LDS operands are
    // read PD steps ahead; the wait of every other step counts exactly the
    // reads issued after those of the step pair. hook(j) runs after step j's
    // MFMA (softmax pieces, copies, the rescale check).
    auto run = [&](auto NSC, auto NVC, f32x16& sacc, f32x16& sacc2, const f32x4 (&pk)[2], int ks, int kr, int vs,
                   auto&& hook)
                   __attribute__((always_inline)) {
      constexpr int NS = decltype(NSC)::value, NV = decltype(NVC)::value, NT = NS + NV;
      const char LDS_AS* kst_v = lds + ks * VSLOT;
      const char LDS_AS* kvb[4] = {kst_v + k_off_v[0], kst_v + k_off_v[1], kst_v + k_off_v[2], kst_v + k_off_v[3]};
      const int rope_shift = kr * RSLOT - ks * VSLOT + k_rope_delta;
      const char LDS_AS* vst = lds + vs * VSLOT;
      const char LDS_AS* vbase[2][2] = {{vst + v_off[0][0], vst + v_off[0][1]}, {vst + v_off[1][0], vst + v_off[1][1]}};
      // Q rope rows sit at OFF_Q in the rope ring's layout: the K rope
      // address plus a uniform shift
      const int q_shift = OFF_Q + wave * RSLOT - OFF_R - kr * RSLOT;
      i16x8 kb[NOB], qb[NOB];
      i16x4 vl[NOB], vh[NOB];
      auto fetch = [&](auto T) __attribute__((always_inline)) {
        constexpr int t = decltype(T)::value;
        if constexpr (t < NS) {
          constexpr int kc = t, cb = kc >> 2;
          if constexpr (cb < NVB) {
            kb[t % (NOB)] = ds_read_b128<cb * 1024>(kvb[kc & 3]);
          } else {
            const char LDS_AS* kr = kvb[kc & 3] + rope_shift;
            kb[t % (NOB)] = ds_read_b128<(cb - NVB) * 1024>(kr);
            qb[t % (NOB)] = ds_read_b128<(cb - NVB) * 1024>(kr + q_shift);
          }
        } else if constexpr (t < NT) {
          constexpr int g = t - NS, c = g / NDB, db = g % NDB;
          constexpr int off = c * 2 * NVB * 1024 + (db >> 1) * 1024;
          vl[t % (NOB)] = ds_read_tr<off>(vbase[db & 1][0]);
          vh[t % (NOB)] = ds_read_tr<off>(vbase[db & 1][1]);
        }
      };
      static_for<(PD < NT ? PD : NT)>([&](auto T) __attribute__((always_inline)) { fetch(T); });
      static_for<NT>([&](auto J) __attribute__((always_inline)) {
        constexpr int j = decltype(J)::value;
        if constexpr (j + PD < NT) fetch(std::integral_constant<int, j + PD>{});
        constexpr int r = j % (NOB);
        if constexpr (j % 2 == 0) {
          // one wait for the operands of steps j and j + 1
          constexpr int j2 = j + 1 < NT ? j + 1 : j;
          constexpr int last = j + PD < NT - 1 ? j + PD : NT - 1;
          constexpr int after2 = [] {
            int n = 0;
            for (int t = j2 + 1; t <= last; ++t) n += own_step_reads<NS, NV>(t);
            return n;
          }();
          static_assert(after2 <= 15, "lgkmcnt range");
          lgkm_wait<after2>();
          constexpr int r2 = j2 % (NOB);
          if constexpr (j < NS && j < NKQ) asm volatile("" : "+v"(kb[r]));
          else if constexpr (j < NS) asm volatile("" : "+v"(kb[r]), "+v"(qb[r]));
          else asm volatile("" : "+v"(vl[r]), "+v"(vh[r]));
          if constexpr (j2 != j) {
            if constexpr (j2 < NS && j2 < NKQ) asm volatile("" : "+v"(kb[r2]));
            else if constexpr (j2 < NS) asm volatile("" : "+v"(kb[r2]), "+v"(qb[r2]));
            else asm volatile("" : "+v"(vl[r2]), "+v"(vh[r2]));
          }
        }
        if constexpr (j < NS) {
          // SCH = 2: even k-chunks into sacc, odd ones into sacc2, so that no
          // MFMA waits for the result of the one just before it
          f32x16& dst = (SCH == 2 && j % 2 == 1) ? sacc2 : sacc;
          const i16x8& qo = j < NKQ ? qop[j < NKQ ? j : 0] : qb[r];
          if constexpr (j < SCH)
            dst = own_mfma_first<DT>(kb[r], qo);
          else
            own_mfma_acc<DT>(dst, kb[r], qo);
        } else {
          constexpr int g = j - NS, c = g / NDB, db = g % NDB;
          const i16x4 lo = vl[r], h4 = vh[r];
          const i16x8 vop = {lo[0], lo[1], lo[2], lo[3], h4[0], h4[1], h4[2], h4[3]};
          // (the builtin: the compiler sees this MFMA and inserts the wait
          // states after the VALU writes of pk that it reads)
          mfma_agpr_acc<DT>(acc[db], vop, __builtin_bit_cast(i16x8, pk[c]));
        }
        hook(J);
        // the scheduler keeps each step's work in its step (the softmax
        // pieces and copies spread over the MFMAs as placed, not clustered)
        if constexpr (TMLA_OWN_SCHED_FENCE) __builtin_amdgcn_sched_barrier(0);
      });
    };

    // O^T columns (one head per lane) times the lane's factor, one block at
    // a time so the accumulators stay in AGPRs.
    auto rescale = [&](float alpha) __attribute__((always_inline)) {
      mfma_agpr_fence(acc[NDB - 1]);
#pragma unroll
      for (int d = 0; d < NDB; ++d) {
        f32x16 t = acc[d];
        pin_vgpr(t);
        t *= alpha;
        acc[d] = t;
        pin_agpr(acc[d]);
      }
    };

    // Online softmax, base 2, with the lazy rescale. Scores stay unscaled: p
    // = 2^(s * c - m) with c = softmax scale * log2 e, and the max is taken on
    // s (c > 0) or -s (c < 0). m_run is the reference max the probabilities
    // of the current sub-tile use. soft_max() looks at the next sub-tile's
    // scores once their MFMAs are done: masks tokens past the sequence (last
    // sub-tile only) and moves the reference max, for the whole wave, only
    // when a score exceeds it by 2^8 (the two token halves of a head then
    // agree through one lane swap), so p <= 2^8 and O^T rarely needs a
    // rescale; soft_apply() applies the move at the end of the iteration,
    // after the current sub-tile's value MFMAs.
    float m_next = kNoMax, a_next = 1.0f;
    float mx_part = 0.0f;  // running max of the scores being examined
    const float cabs = fabsf(a.qk_scale_log2);
    // piece 0: mask, then the max of registers 0-3; pieces 1-3: registers
    // 4k..4k+3; piece 4: the decision (one piece per step, beside the MFMAs).
    // (A negative softmax scale runs on negated Q^T and |c|, so the scores
    // are always maximised.)
    auto soft_max_piece = [&](f32x16& s, int st, auto K) __attribute__((always_inline)) {
      constexpr int k = decltype(K)::value;
      if constexpr (k == 0) {
        if ((st + 1) * kSubTokens > n_b - lag_wave) {  // tokens past the sequence (for some head)
          const int ln = lane_id_fresh();
          const int tok0 = st * kSubTokens + 4 * (ln >> 5);
          const int lim = n_b - causal_lag(a, head_base + (ln & 31));
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (tok0 + 8 * (r >> 2) + (r & 3) >= lim) s[r] = -INFINITY;
        }
        pin_f16(s);
      }
      if constexpr (k < 4) {
        const float m4 = fmaxf(fmaxf(s[4 * k], s[4 * k + 1]), fmaxf(s[4 * k + 2], s[4 * k + 3]));
        mx_part = k == 0 ? m4 : fmaxf(mx_part, m4);
        pin_f1(mx_part);
      } else {
        const float mx = mx_part * cabs;
        m_next = m_run;
        a_next = 1.0f;
        if (__builtin_amdgcn_ballot_w64(mx > m_run + kRescaleLog2) != 0) {
          float x = mx, y = mx;
          swap_rows32(x, y);
          m_next = fmaxf(m_run, fmaxf(x, y));
          if (m_run != kNoMax) a_next = fast_exp2(m_run - m_next);
        }
        pin_f2(m_next, a_next);
      }
    };
    auto soft_max = [&](f32x16& s, int st) __attribute__((always_inline)) {
      static_for<5>([&](auto K) __attribute__((always_inline)) { soft_max_piece(s, st, K); });
    };
    auto soft_apply = [&]() __attribute__((always_inline)) {
      if (__builtin_amdgcn_ballot_w64(a_next != 1.0f) != 0) rescale(a_next);
      l_run *= a_next;
      m_run = m_next;
    };
    // p of score r of the current sub-tile, summed into lsum
    auto soft_exp = [&](f32x16& s, float& lsum, int r) __attribute__((always_inline)) {
      s[r] = fast_exp2(fmaf(s[r], cabs, -m_run));  // masked: -inf -> 0
      lsum += s[r];
      pin_f1(lsum);  // summed here, beside the MFMAs, not all at the end
    };

    // ---- start-up: page ids, Q through LDS, sub-tiles 0 and 1 -------------
    int pro_page[RING] = {0, 0, 0, 0};
    if (PAGED && PAGE_UNIFORM) {
#pragma unroll
      for (int i = 0; i < RING; ++i) pro_page[i] = page_fetch(st0 + min(i, nst - 1));
    }
    stage_q(b);
    wait_vmcnt<0>();
#pragma unroll
    for (int kc = 0; kc < NKQ; ++kc)
      qop[kc] = *reinterpret_cast<const i16x8 LDS_AS*>(lds + wave * VSLOT + k_off_v[kc & 3] + (kc >> 2) * 1024);
    if (a.qk_scale_log2 < 0.0f) {
      // negative softmax scale: s * c = (-s) * |c|, with -s from Q^T negated
      // (a sign flip, exact) in registers and in this wave's Q rope rows
      const i16x8 sgn = (i16x8)(short)0x8000;
#pragma unroll
      for (int kc = 0; kc < NKQ; ++kc) qop[kc] ^= sgn;
      char LDS_AS* qr = lds + OFF_Q + wave * RSLOT + lane * 16;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        i16x8 v = *reinterpret_cast<const i16x8 LDS_AS*>(qr + 1024 * j);
        *reinterpret_cast<i16x8 LDS_AS*>(qr + 1024 * j) = v ^ sgn;
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    lds_barrier();  // every wave has its Q^T before the rings are refilled
    if (PAGED && PAGE_UNIFORM) {
#pragma unroll
      for (int i = 0; i < RING; ++i) pro_page[i] = page_ready(pro_page[i]);
    }
    issue(st0, pro_page[0]);  // nst >= 1
    if (nst > 1) {
      issue(st0 + 1, pro_page[1]);
      wait_vmcnt<LOADS>();
    } else {
      wait_vmcnt<0>();
    }
    int next_page = 0;
    if (b == b_first) phase_stamp(2);

    // ---- prologue: S(0), copies of sub-tile 2 ---------------------------
    // Copies past the segment's last sub-tile (here and in the last two
    // iterations with S) read the sequence's last row again into entries no
    // later step of the segment reads: one loop body serves every iteration
    // (a loop body instantiated with and without copies leaves the register
    // allocator no room beside Q^T and O^T).
    f32x16 sA, sB, sX;  // score tiles of alternate sub-tiles; the second chain's accumulator
    const char* csrc_n = nullptr;  // copy source (this lane's row) of the next iteration's sub-tile
    lds_barrier();  // every wave's copies of sub-tile 0 have landed
    {
      const char* csrc = nullptr;
      const f32x4 none[2] = {(f32x4)0.0f, (f32x4)0.0f};
      run(std::integral_constant<int, NKC>{}, std::integral_constant<int, 0>{}, sA, sX, none, 0, 0, 0,
          [&](auto J) __attribute__((always_inline)) {
            constexpr int j = decltype(J)::value;
            if constexpr (j == 0) csrc = copy_src(st0 + 2, pro_page[2]);
            static_for<LOADS>([&](auto K) __attribute__((always_inline)) {
              constexpr int k = decltype(K)::value;
              if constexpr (k * (NKC - 4) / LOADS + 1 == j) copy_one(2, std::integral_constant<int, k>{}, csrc);
            });
          });
      mfma_vgpr_fence(sA);
      csrc_n = copy_src(st0 + 3, pro_page[3]);  // iteration 0's copies
      if constexpr (SCH == 2) {
        mfma_vgpr_fence(sX);
        sA += sX;
      }
      soft_max(sA, st0);
      soft_apply();
    }

    // ---- iterations ---------------------------------------------------------
    // iteration i < nst - 1: the softmax of sc (sub-tile i) beside S(i+1) into
    // sn, the copies of sub-tile i+3, then PV(i) and the max of sub-tile i+1
    auto iteration = [&](const int i, f32x16& sc, f32x16& sn) __attribute__((always_inline)) {
      // own copies of sub-tile i+1 have landed (those of i+2 may fly)
      wait_vmcnt<LOADS>();
      // every wave's copies of sub-tile i+1 have landed and every wave is
      // done with the entries the copies of sub-tile i+3 refill
      lds_barrier();
      const bool stamped = TMLA_STAMPS && b == b_first && (i == kStampIter || i == kStampIter + 1);
      StampRec st_begin{}, st_mid{}, st_end{};
      if (stamped) st_begin = stamp_now();
      // the page id of sub-tile i+4: its load goes out before every counted
      // LDS read of the run
      if (PAGED && PAGE_UNIFORM) next_page = page_fetch(st0 + min(i + RING, nst - 1));
      const int ks = (i + 1) & 3, kr = (i + 1) % RRING, vs = i & 3;
      const char* const csrc = csrc_n;
      float lsum = 0.0f;
      f32x4 pk[2];  // probabilities of sub-tile i, two per register: tokens 0-15, 16-31
      run(std::integral_constant<int, NKC>{}, std::integral_constant<int, 2 * NDB>{}, sn, sX, pk, ks, kr, vs,
          [&](auto J) __attribute__((always_inline)) {
            constexpr int j = decltype(J)::value;
            if constexpr (j >= E0 && (j - E0) % ES == 0 && (j - E0) / ES < 16) {
              constexpr int r = (j - E0) / ES;
              soft_exp(sc, lsum, r);
              if constexpr (r % 2 == 1) pk[r / 8][(r / 2) % 4] = pack_pair<DT>(sc[r - 1], sc[r]);
            }
            static_for<LOADS>([&](auto K) __attribute__((always_inline)) {
              constexpr int k = decltype(K)::value;
              if constexpr (CP0 + k * CPS / LOADS == j) copy_one(i + 3, std::integral_constant<int, k>{}, csrc);
            });
            if constexpr (j == NKC - 1) {
              if (stamped) st_mid = stamp_now();
            }
            // the scores of sub-tile i+1: their last MFMA issued MX - NKC
            // steps (and as many MFMAs and operand reads) ago
            if constexpr (j == MX && SCH == 2) {
              pin_f16(sX);
              sn += sX;
            }
            if constexpr (j >= MX && j < MX + 5) soft_max_piece(sn, st0 + i + 1, std::integral_constant<int, j - MX>{});
          });
      l_run += lsum;
      soft_apply();
      // the copy source of the next iteration (sub-tile i+4), computed here
      // while the last value MFMAs run (every counted LDS read is done, and
      // the page id requested at the start has arrived)
      csrc_n = copy_src(st0 + i + 4, (PAGED && PAGE_UNIFORM) ? page_ready(next_page) : 0);
      if (stamped) {
        st_end = stamp_now();
        if (i == kStampIter) {
          stamp_store(5, st_begin);
          stamp_store(6, st_mid);
          stamp_store(7, st_end);
        } else {
          stamp_store(8, st_begin);
        }
      }
    };
    int it = 0;
    while (it + 1 < nst) {
      iteration(it, sA, sB);
      if (++it + 1 >= nst) {
        sA = sB;  // the last sub-tile's scores
        break;
      }
      iteration(it, sB, sA);
      ++it;
    }
    // last sub-tile of the segment: its softmax, then its value steps
    {
      // (every wave's copies of it have landed: the barrier of the last
      // iteration, or of the prologue, came after their waits)
      float lsum = 0.0f;
      f32x4 pk[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        soft_exp(sA, lsum, r);
        if (r % 2 == 1) pk[r / 8][(r / 2) % 4] = pack_pair<DT>(sA[r - 1], sA[r]);
      }
      asm volatile("s_nop 4" : "+v"(pk[0]), "+v"(pk[1]));  // VALU results read by the asm MFMAs below
      l_run += lsum;
      run(std::integral_constant<int, 0>{}, std::integral_constant<int, 2 * NDB>{}, sB, sX, pk, 0, 0, (nst - 1) & 3,
          [](auto) {});
    }
    mfma_agpr_fence(acc[NDB - 1]);
    wait_vmcnt<0>();
    lds_barrier();  // every wave is done with the rings
    if (b == b_first) phase_stamp(3);

    // ---- finalize: out = acc / l, lse2 = m + log2(l) ----------------------
    {
      const int ln = lane_id_fresh();
      const int hq = head_base + (ln & 31);
      const bool hq_ok = hq < a.num_heads;
      const int h2 = ln >> 5;
      float l_a = l_run, l_b = l_run;
      swap_rows32(l_a, l_b);
      const float l_tot = l_a + l_b;
      const bool has = l_tot > 0.0f;
      const float inv = has ? 1.0f / l_tot : 0.0f;
      const float lse2 = has ? m_run + fast_log2(l_tot) : -INFINITY;
      // rows of this wave's heads through its own part of the idle rings
      // (padded pitch: the lanes' 8-byte writes spread over all banks), so
      // that every global store writes one whole row
      // (one accumulator block at a time: moved to VGPRs, scaled, rounded
      // and written before the next block is read)
      char LDS_AS* obuf = lds + wave * 32 * OPITCH;
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        f32x16 t = acc[db];
        pin_vgpr(t);
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          i16x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = Elt<DT>::from_float(t[4 * q4 + e] * inv);
          const int dim = 32 * db + 8 * q4 + 4 * h2;
          *reinterpret_cast<i16x4 LDS_AS*>(obuf + (ln & 31) * OPITCH + dim * 2) = v;
        }
        asm volatile("" ::: "memory");
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      short* dst;
      int64_t row_stride;
      if (seg.direct) {
        dst = reinterpret_cast<short*>(a.out) + (int64_t)b * a.out_sb + (int64_t)head_base * a.out_sh;
        row_stride = a.out_sh;
      } else {
        dst = a.mid_o + ((int64_t)seg.slot * a.num_heads + head_base) * DV;
        row_stride = DV;
      }
      int rows = __builtin_amdgcn_readfirstlane(max(0, min(32, a.num_heads - head_base)));
      // computed per segment: 32 hoisted row conditions would crowd the SGPRs
      asm volatile("" : "+s"(rows));
#pragma unroll
      for (int r0 = 0; r0 < 32; r0 += 8) {
        i16x8 row[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) row[k] = *reinterpret_cast<const i16x8 LDS_AS*>(obuf + (r0 + k) * OPITCH + ln * 16);
#pragma unroll
        for (int k = 0; k < 8; ++k)
          if (r0 + k < rows) store_through(reinterpret_cast<i16x8*>(dst + (r0 + k) * row_stride + ln * 8), row[k]);
      }
      if (hq_ok && h2 == 0) {
        if (seg.direct) {
          if (a.lse) a.lse[(int64_t)b * a.num_heads + hq] = has ? lse2 * kLn2 : -INFINITY;
        }
        else
          store_through_f32(a.mid_lse + (int64_t)seg.slot * a.num_heads + hq, lse2);
      }
      // the next segment refills the rings
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      lds_barrier();
    }

    if (b == b_first) phase_stamp(4);
    if (a.fused && !seg.direct) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      lds_barrier();
      if (wave == 0 && lane == 0) {
        const int old = sys_add(a.m_count + (int64_t)b * gridDim.y + blockIdx.y, 1);
        int* r = s_pend[b == b_first ? 0 : 1];
        r[4] = old == r[2] - 1;
      }
    }

    remaining -= t_end - t_start + wr.seg_cost;  // the next sequence's start is charged here
    seg_global_off += nt_b + wr.seg_cost;
    ++b;
    t_start = 0;
  }

  if (a.fused) {
    const CoherentLoads ld{
        __builtin_amdgcn_make_buffer_rsrc(a.mid_o, 0, a.mid_o_bytes, kBufferWord3),
        __builtin_amdgcn_make_buffer_rsrc(a.mid_lse, 0, a.mid_o_bytes / 256, kBufferWord3)};
    fused_merge_tail<DT>(MergeView{a.mid_o, a.mid_lse, a.num_heads, a.out, a.out_sb, a.out_sh, a.lse}, ld,
                         a.m_count, a.m_done, a.m_flag, a.spin_limit, wave, s_pend, s_msg, 4 * kHeadsPerWave);
  }
}

// ---------------------------------------------------------------------------
// Stage 2: log-sum-exp merge (kernel.py:159-181). A workgroup merges 4 * HPW
// heads of sequence b: one head per wave (HPW = 1), or, for calls with many
// (sequence, head) pairs, four heads per wave (HPW = 4) so that every
// workgroup fits the compute units in one round and each wave has four
// heads' rows in flight. Both give the same bits.
// ---------------------------------------------------------------------------
template <int DT, int DV, int HPW>
__global__ __launch_bounds__(256) void mla_combine_kernel(CombineArgs a) {
  static_assert(DV % 256 == 0, "8 dims per lane");
  static_assert(HPW == 1 || HPW == 4, "one or four heads per wave");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b = blockIdx.x;
  const int h_lo = blockIdx.y * 4 * HPW;
  const int h_hi = min(h_lo + 4 * HPW, a.num_heads);
  __shared__ int s_red[3][4];

  // partial slots of sequence b
  const int n_b = a.seqlens[b];
  const int nt_b = tiles_of(n_b);
  int slot0 = 0, count = 0;
  if (a.num_splits > 0) {
    const int S = a.num_splits;
    if (nt_b > 0) {
      const int spt = (nt_b + S - 1) / S;
      count = (nt_b + spt - 1) / spt;
    }
    slot0 = b * S;
  } else {
    // tiles in all (the snapped form), and positions before b and in all on
    // the straddling form's line, where every non-empty sequence starts with
    // kSegCostTiles extra positions (work_range)
    int total = 0, vbefore = 0, vtotal = 0;
    for (int i = threadIdx.x; i < a.batch; i += 256) {
      const int nt = tiles_of(a.seqlens[i]);
      const int vt = nt > 0 ? nt + kSegCostTiles : 0;
      total += nt;
      vtotal += vt;
      if (i < b) vbefore += vt;
    }
    for (int d = 32; d >= 1; d >>= 1) {
      total += __shfl_xor(total, d);
      vbefore += __shfl_xor(vbefore, d);
      vtotal += __shfl_xor(vtotal, d);
    }
    if (lane == 0) {
      s_red[0][wave] = total;
      s_red[1][wave] = vbefore;
      s_red[2][wave] = vtotal;
    }
    __syncthreads();
    total = s_red[0][0] + s_red[0][1] + s_red[0][2] + s_red[0][3];
    vbefore = s_red[1][0] + s_red[1][1] + s_red[1][2] + s_red[1][3];
    vtotal = s_red[2][0] + s_red[2][1] + s_red[2][2] + s_red[2][3];
    if (nt_b > 0) {  // (then total > 0; uniform over the workgroup)
      const int chunk = (total + a.num_workers - 1) / a.num_workers;
      // the partial kernel's snapped ranges when the pieces fit the workers
      int pbefore = 0, ptotal = 0;
      for (int i = threadIdx.x; i < a.batch; i += 256) {
        const int np = (tiles_of(a.seqlens[i]) + chunk - 1) / chunk;
        ptotal += np;
        if (i < b) pbefore += np;
      }
      for (int d = 32; d >= 1; d >>= 1) {
        pbefore += __shfl_xor(pbefore, d);
        ptotal += __shfl_xor(ptotal, d);
      }
      __syncthreads();  // every wave has read s_red
      if (lane == 0) {
        s_red[0][wave] = pbefore;
        s_red[1][wave] = ptotal;
      }
      __syncthreads();
      pbefore = s_red[0][0] + s_red[0][1] + s_red[0][2] + s_red[0][3];
      ptotal = s_red[1][0] + s_red[1][1] + s_red[1][2] + s_red[1][3];
      if (ptotal <= a.num_workers) {
        count = (nt_b + chunk - 1) / chunk;
        slot0 = pbefore + b;
      } else {  // straddling: the workers whose ranges hold b's tiles
        const int vchunk = (vtotal + a.num_workers - 1) / a.num_workers;
        const int first = vbefore + kSegCostTiles;  // position of b's tile 0
        const int g1 = first / vchunk, g2 = (first + nt_b - 1) / vchunk;
        count = g2 - g1 + 1;
        slot0 = g1 + b;
      }
    }
  }
  if (count == 1) return;  // written by stage 1
  static_assert(DV == 512, "one row = 64 lanes x 8 elements");
  const MergeView mv{a.mid_o, a.mid_lse, a.num_heads, a.out, a.out_sb, a.out_sh, a.lse};
  const PlainLoads ld{a.mid_o, a.mid_lse};
  if (count == 0) {
    for (int h = h_lo + wave; h < h_hi; h += 4) merge_zero(mv, b, h, lane);
  } else if (count <= 8) {
    // HPW heads of one wave together: HPW * count rows in flight
    const int h = h_lo + HPW * wave;
    if (h < h_hi) merge_rows_at_once<DT, HPW, 8>(mv, ld, b, h, min(HPW, h_hi - h), slot0, count, lane);
  } else if (count <= 16) {
    constexpr int P = HPW == 4 ? 2 : 1;  // heads per pass
    for (int h = h_lo + P * wave; h < h_hi; h += 4 * P)
      merge_rows_at_once<DT, P, 16>(mv, ld, b, h, min(P, h_hi - h), slot0, count, lane);
  } else if (count <= 32) {  // e.g. a few long sequences cut over all workers: one round trip
    for (int h = h_lo + wave; h < h_hi; h += 4) merge_rows_at_once<DT, 1, 32>(mv, ld, b, h, 1, slot0, count, lane);
  } else {
    for (int h = h_lo + wave; h < h_hi; h += 4) merge_row_loop<DT, 32>(mv, ld, b, h, slot0, count, lane);
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

int hip_fail(hipError_t e, const char* where) {
  snprintf(g_err, sizeof(g_err), "%s: %s", where, hipGetErrorString(e));
  return TMLA_ERR_HIP;
}

constexpr int kDefaultSpinLimit = 1 << 14;  // polls (about 2^7 clocks each) before a share is handed over

// Compute units of the current device, read once per device (relaxed atomics:
// concurrent first calls store the same value).
int current_cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < 64) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (dev < 64) cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

// Calls of at most kG16Heads heads (virtual heads of a multi-token call) on a
// 16-bit cache run the 16-head-group kernel, as two launches.
bool uses_g16(int32_t num_heads) { return num_heads <= kG16Heads; }

// Scales of an fp8 cache: element strides per page (dense: per sequence)
// and per row.
struct Fp8Scales {
  const float* scale;
  int64_t s0, s1;
};

template <int DT, int NHB, bool PAGED, bool UNI, bool F8 = false>
hipError_t launch_partial_t(const PartialArgs& a, dim3 grid, hipStream_t stream) {
  hipLaunchKernelGGL((mla_partial_kernel<DT, 512, 64, NHB, PAGED, UNI, F8>), grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

template <int DT, int NHB>
hipError_t launch_partial_nw(const PartialArgs& a, dim3 grid, hipStream_t stream, bool paged, bool uni) {
  if (!paged) return launch_partial_t<DT, NHB, false, false>(a, grid, stream);
  if (uni) return launch_partial_t<DT, NHB, true, true>(a, grid, stream);
  return launch_partial_t<DT, NHB, true, false>(a, grid, stream);
}

// fp8 cache widened once per workgroup into the 16-bit ring (paged, pages
// of whole sub-tiles, one scale per page or per tensor)
template <int DT>
hipError_t launch_partial_ring8(const PartialArgs& a, dim3 grid, int nhb, hipStream_t stream) {
  if (nhb == 1) return launch_partial_t<DT, 1, true, true, true>(a, grid, stream);
  if (nhb == 2) return launch_partial_t<DT, 2, true, true, true>(a, grid, stream);
  return launch_partial_t<DT, 4, true, true, true>(a, grid, stream);
}

template <int DT, bool PAGED, bool UNI>
hipError_t launch_partial_own_t(const PartialArgs& a, dim3 grid, hipStream_t stream) {
  hipLaunchKernelGGL((mla_partial_own_kernel<DT, PAGED, UNI>), grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

template <int DT>
hipError_t launch_partial_dt(const PartialArgs& a, dim3 grid, int nhb, hipStream_t stream, bool paged, bool uni) {
  if (nhb == 1) return launch_partial_nw<DT, 1>(a, grid, stream, paged, uni);
  if (nhb == 2) return launch_partial_nw<DT, 2>(a, grid, stream, paged, uni);
  if constexpr (TMLA_OWN_LOOP) {
    // 128 heads per workgroup: the head-owner loop
    if (!paged) return launch_partial_own_t<DT, false, false>(a, grid, stream);
    if (uni) return launch_partial_own_t<DT, true, true>(a, grid, stream);
    return launch_partial_own_t<DT, true, false>(a, grid, stream);
  } else {
    return launch_partial_nw<DT, 4>(a, grid, stream, paged, uni);
  }
}

}  // namespace tmla

using namespace tmla;

extern "C" {

const char* tmla_last_error(void) { return g_err; }

int tmla_version(void) { return 300; }

size_t tmla_workspace_bytes(int32_t batch, int32_t num_heads, int32_t head_dim_v, int32_t num_splits,
                            int32_t num_workers) {
  return workspace_bytes(batch, num_heads, head_dim_v, num_splits, num_workers);
}

int32_t tmla_partition_segment_tiles(void) { return kSegCostTiles; }

int tmla_debug_stamps(void* host, size_t bytes) {
#if TMLA_STAMPS
  const size_t n = sizeof(g_stamps) < bytes ? sizeof(g_stamps) : bytes;
  hipError_t e = hipMemcpyFromSymbol(host, HIP_SYMBOL(g_stamps), n, 0, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpyFromSymbol(g_stamps)");
  return TMLA_OK;
#else
  (void)host;
  (void)bytes;
  return fail(TMLA_ERR_UNSUPPORTED, "phase stamps need a library built with TMLA_STAMPS=1 (build.py --stamps)");
#endif
}

int32_t tmla_device_cu_count(int32_t device) {
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return 0;
  return n;
}

}  // extern "C"

namespace tmla {

// mode 0: stage 1 only; 1: stage 1 with the fused merge when every
// workgroup fits on the device at once, else both stages; 2: both stages.
int decode_launch(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kv, int64_t kv_stride_0,
                  int64_t kv_stride_1, int64_t num_blocks, int32_t page_size, const int32_t* block_table,
                  int64_t bt_stride_b, int32_t bt_cols, const int32_t* seqlens, int32_t batch, int32_t num_heads,
                  int32_t head_dim_v, int32_t rope_dim, int32_t dtype, float softmax_scale, int32_t num_splits,
                  int32_t num_workers, void* out, int64_t out_stride_b, int64_t out_stride_h, float* lse,
                  void* workspace, size_t workspace_bytes_, void* stream, int mode, int32_t q_len = 1,
                  int32_t spin_limit = -1, const Fp8Scales* f8 = nullptr) {
  const Common c{batch, num_heads, head_dim_v, rope_dim, dtype, num_splits, num_workers};
  int rc = check_common(c, workspace, workspace_bytes_);
  if (rc != TMLA_OK) return rc;
  if (rope_dim != 64) return fail(TMLA_ERR_UNSUPPORTED, "rope_dim must be 64");
  if (batch == 0) return TMLA_OK;
  if (!q || !kv || !seqlens || !out) return fail(TMLA_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (page_size <= 0 || num_blocks <= 0) return fail(TMLA_ERR_INVALID_ARGUMENT, "page_size and num_blocks must be > 0");
  const bool paged = block_table != nullptr;
  if (paged && bt_cols <= 0) return fail(TMLA_ERR_INVALID_ARGUMENT, "block_table needs at least one column");
  if (!paged && page_size != 1) return fail(TMLA_ERR_INVALID_ARGUMENT, "dense cache requires page_size == 1");
  if (((uintptr_t)q | (uintptr_t)kv | (uintptr_t)out) & 15)
    return fail(TMLA_ERR_INVALID_ARGUMENT, "q, kv and out must be 16-byte aligned");
  if ((q_stride_b | q_stride_h | kv_stride_0 | kv_stride_1 | out_stride_b | out_stride_h) & 7)
    return fail(TMLA_ERR_INVALID_ARGUMENT, "strides must be multiples of 8 elements");
  if (f8) {
    if ((kv_stride_0 | kv_stride_1) & 15)
      return fail(TMLA_ERR_INVALID_ARGUMENT, "fp8 cache strides must be multiples of 16 elements");
    if (paged && page_size % 16 != 0)
      return fail(TMLA_ERR_UNSUPPORTED, "fp8 cache pages must hold a multiple of 16 tokens");
    if (!f8->scale || ((uintptr_t)f8->scale & 3))
      return fail(TMLA_ERR_INVALID_ARGUMENT, "kv_scale must be a 4-byte aligned float32 pointer");
  }
  if (kv_stride_1 <= 0 || kv_stride_1 > (1 << 25))
    return fail(TMLA_ERR_UNSUPPORTED, "kv token stride must be in (0, 2^25] elements");

  PartialArgs a{};
  a.q = static_cast<const char*>(q);
  a.q_sb = q_stride_b;
  a.q_sh = q_stride_h;
  a.kv = static_cast<const char*>(kv);
  const int kv_elt = f8 ? 1 : 2;  // bytes per cache element
  a.kv_s0 = kv_stride_0 * kv_elt;
  a.kv_s1 = kv_stride_1 * kv_elt;
  a.num_blocks = num_blocks;
  a.max_page = (int32_t)(num_blocks - 1 < INT32_MAX ? num_blocks - 1 : INT32_MAX);
  a.page_size = page_size;
  a.page_shift = (page_size & (page_size - 1)) == 0 ? __builtin_ctz((unsigned)page_size) : -1;
  a.bt = block_table;
  a.bt_sb = bt_stride_b;
  a.bt_cols = paged ? bt_cols : 1;
  a.seqlens = seqlens;
  a.batch = batch;
  a.num_heads = num_heads;
  if (q_len < 1 || num_heads % q_len != 0) return fail(TMLA_ERR_INVALID_ARGUMENT, "q_len must be >= 1");
  a.q_len = q_len;
  a.heads_per_token = num_heads / q_len;
  // A zero scale (every score 0) runs as the smallest normal float instead:
  // the probabilities then differ from 1 by far less than one ulp, and masked
  // tokens (score -inf) still get exactly 0.
  a.qk_scale_log2 = softmax_scale * kLog2e;
  if (a.qk_scale_log2 == 0.0f) a.qk_scale_log2 = 1.17549435e-38f;
  a.num_splits = num_splits;
  a.num_workers = num_workers;
  a.xcds = TMLA_XCDS;  // MI355X: 8 XCDs
  a.out = static_cast<char*>(out);
  a.out_sb = out_stride_b;
  a.out_sh = out_stride_h;
  a.lse = lse;
  char* ws = static_cast<char*>(workspace);
  const WsLayout wl = ws_layout(batch, num_heads, 512, num_splits, num_workers);
  a.mid_o = reinterpret_cast<short*>(ws + wl.o);
  a.mid_lse = reinterpret_cast<float*>(ws + wl.l);
  a.spin_limit = spin_limit >= 0 ? spin_limit : kDefaultSpinLimit;

  const int64_t cap_tokens = paged ? (int64_t)bt_cols * page_size : num_blocks;
  const size_t mid_o_bytes = wl.l - wl.o;  // partial rows, 256-byte aligned
  hipStream_t s = static_cast<hipStream_t>(stream);
  // one page per 32-token sub-tile (sub-tiles never straddle a page) and a
  // power-of-two page size: page slots and in-page rows by shifts and masks
  const bool uni = paged && (page_size % kSubTokens == 0) && a.page_shift >= 0;
  if (f8) {
    // fp8 cache, always two launches (no in-kernel merge). More than
    // kFp8GroupHeads heads with one scale per page (or per tensor) and pages
    // of whole sub-tiles: the 16-bit kernel with the cache widened once per
    // workgroup into its ring; otherwise groups of 16 heads, each streaming
    // and widening the cache on its own.
    a.kv_scale = f8->scale;
    a.sc_s0 = f8->s0;
    a.sc_s1 = f8->s1;
    hipError_t e;
    if (uni && f8->s1 == 0 && num_heads > kFp8GroupHeads) {
      const LaunchPlan plan = plan_launch(batch, num_heads, num_splits, num_workers, cap_tokens, mid_o_bytes,
                                          mode == 0 ? 0 : 2, current_cu_count());
      a.fused = 0;
      e = dtype == TMLA_BF16 ? launch_partial_ring8<TMLA_BF16>(a, dim3(plan.grid_x, plan.grid_y), plan.nhb, s)
                             : launch_partial_ring8<TMLA_FP16>(a, dim3(plan.grid_x, plan.grid_y), plan.nhb, s);
      if (e != hipSuccess) return hip_fail(e, "mla_partial_kernel (fp8 ring) launch");
    } else {
      const dim3 grid(worker_grid(batch, num_splits, num_workers, cap_tokens), ((int64_t)num_heads + 15) / 16);
      e = launch_partial_fp8(a, grid, dtype, paged, s);
    }
    if (e != hipSuccess) return hip_fail(e, "mla_partial_fp8_kernel launch");
    if (mode != 0)
      return tmla_mla_decode_combine(seqlens, batch, num_heads, head_dim_v, dtype, num_splits, num_workers, out,
                                     out_stride_b, out_stride_h, lse, workspace, workspace_bytes_, stream);
    return TMLA_OK;
  }
  const bool g16 = uses_g16(num_heads);  // few heads: the 16-head-group kernel
  const LaunchPlan plan =
      g16 ? plan_launch_g16(batch, num_heads, num_splits, num_workers, cap_tokens, mid_o_bytes, mode,
                            current_cu_count())
          : plan_launch(batch, num_heads, num_splits, num_workers, cap_tokens, mid_o_bytes, mode, current_cu_count());
  const int nhb = plan.nhb;
  const dim3 grid(plan.grid_x, plan.grid_y);
  a.mid_o_bytes = (int32_t)(mid_o_bytes < (size_t)INT32_MAX ? mid_o_bytes : 0);
  a.fused = plan.fused ? 1 : 0;
  // the single launch's counters and flags [batch | batch | slots][grid.y] at
  // the start of the counter block at the end of the caller's buffer
  // (check_common: it holds wl.total bytes, a multiple of 256, so the block
  // starts at or after wl.part_end)
  char* cnt = ws + ((workspace_bytes_ & ~(size_t)255) - wl.cnt_bytes);
  a.m_count = reinterpret_cast<int32_t*>(cnt);
  a.m_done = a.m_count + (int64_t)batch * grid.y;
  a.m_flag = a.m_done + (int64_t)batch * grid.y;
  hipError_t e = g16 ? launch_partial_g16(a, grid, dtype, paged, s)
                 : dtype == TMLA_BF16 ? launch_partial_dt<TMLA_BF16>(a, grid, nhb, s, paged, uni)
                                      : launch_partial_dt<TMLA_FP16>(a, grid, nhb, s, paged, uni);
  if (e != hipSuccess) return hip_fail(e, g16 ? "mla_partial_g16_kernel launch" : "mla_partial_kernel launch");
  if (mode != 0 && !a.fused)
    return tmla_mla_decode_combine(seqlens, batch, num_heads, head_dim_v, dtype, num_splits, num_workers, out,
                                   out_stride_b, out_stride_h, lse, workspace, workspace_bytes_, stream);
  return TMLA_OK;
}

// ---------------------------------------------------------------------------
// Built-in workspace of tmla_mla_decode_noalloc: a device array of fixed size
// that the code object carries, so that callers that may not allocate
// (code under HIP graph capture, serving loops, harnesses that forbid
// hipMalloc) can still run the two-kernel decode. Each device that loads the
// library holds its own copy until the process ends. Host code never passes
// the array's name to a kernel (on the host it is a stand-in, not a device
// address): its per-device address comes from hipGetSymbolAddress, once per
// device, with that device current.
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The address of `scratch` on the device `stream` belongs to (the current
// device for the null stream), which must be the current device.
int scratch_for_stream(void* stream, void** out) {
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  int dev = cur;
  if (stream != nullptr) {
    hipDevice_t sd = 0;
    e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &sd);
    if (e != hipSuccess) return hip_fail(e, "hipStreamGetDevice");
    dev = (int)sd;
  }
  if (dev != cur) return fail(TMLA_ERR_INVALID_ARGUMENT, "stream belongs to a device other than the current one");
  if (dev < 0 || dev >= kMaxDevices) return fail(TMLA_ERR_UNSUPPORTED, "device index beyond the scratch table");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return TMLA_OK;
}

}  // namespace tmla

extern "C" {

int tmla_mla_decode_partial(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kv,
                            int64_t kv_stride_0, int64_t kv_stride_1, int64_t num_blocks, int32_t page_size,
                            const int32_t* block_table, int64_t bt_stride_b, int32_t bt_cols,
                            const int32_t* seqlens, int32_t batch, int32_t num_heads, int32_t head_dim_v,
                            int32_t rope_dim, int32_t dtype, float softmax_scale, int32_t num_splits,
                            int32_t num_workers, void* out, int64_t out_stride_b, int64_t out_stride_h,
                            float* lse, void* workspace, size_t workspace_bytes_, void* stream) {
  return decode_launch(q, q_stride_b, q_stride_h, kv, kv_stride_0, kv_stride_1, num_blocks, page_size, block_table,
                       bt_stride_b, bt_cols, seqlens, batch, num_heads, head_dim_v, rope_dim, dtype, softmax_scale,
                       num_splits, num_workers, out, out_stride_b, out_stride_h, lse, workspace, workspace_bytes_,
                       stream, 0);
}

int tmla_mla_decode_combine(const int32_t* seqlens, int32_t batch, int32_t num_heads, int32_t head_dim_v,
                            int32_t dtype, int32_t num_splits, int32_t num_workers, void* out,
                            int64_t out_stride_b, int64_t out_stride_h, float* lse, const void* workspace,
                            size_t workspace_bytes_, void* stream) {
  const Common c{batch, num_heads, head_dim_v, 64, dtype, num_splits, num_workers};
  int rc = check_common(c, workspace, workspace_bytes_);
  if (rc != TMLA_OK) return rc;
  if (batch == 0) return TMLA_OK;
  if (!seqlens || !out) return fail(TMLA_ERR_INVALID_ARGUMENT, "null pointer argument");
  CombineArgs a{};
  a.seqlens = seqlens;
  a.batch = batch;
  a.num_heads = num_heads;
  a.num_splits = num_splits;
  a.num_workers = num_workers;
  a.out = static_cast<char*>(out);
  a.out_sb = out_stride_b;
  a.out_sh = out_stride_h;
  a.lse = lse;
  const char* ws = static_cast<const char*>(workspace);
  const WsLayout wl = ws_layout(batch, num_heads, 512, num_splits, num_workers);
  a.mid_o = reinterpret_cast<const short*>(ws + wl.o);
  a.mid_lse = reinterpret_cast<const float*>(ws + wl.l);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // four heads per wave once one head per wave would take more than
  // kCombineWideWgs workgroups
  const bool wide = (int64_t)batch * ((num_heads + 3) / 4) > kCombineWideWgs;
  const dim3 grid(batch, wide ? (num_heads + 15) / 16 : (num_heads + 3) / 4);
  if (dtype == TMLA_BF16) {
    if (wide)
      hipLaunchKernelGGL((mla_combine_kernel<TMLA_BF16, 512, 4>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((mla_combine_kernel<TMLA_BF16, 512, 1>), grid, dim3(256), 0, s, a);
  } else {
    if (wide)
      hipLaunchKernelGGL((mla_combine_kernel<TMLA_FP16, 512, 4>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((mla_combine_kernel<TMLA_FP16, 512, 1>), grid, dim3(256), 0, s, a);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "mla_combine_kernel launch");
  return TMLA_OK;
}

int tmla_mla_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kv, int64_t kv_stride_0,
                    int64_t kv_stride_1, int64_t num_blocks, int32_t page_size, const int32_t* block_table,
                    int64_t bt_stride_b, int32_t bt_cols, const int32_t* seqlens, int32_t batch,
                    int32_t num_heads, int32_t head_dim_v, int32_t rope_dim, int32_t dtype, float softmax_scale,
                    int32_t num_splits, int32_t num_workers, void* out, int64_t out_stride_b,
                    int64_t out_stride_h, float* lse, void* workspace, size_t workspace_bytes_, void* stream) {
  return decode_launch(q, q_stride_b, q_stride_h, kv, kv_stride_0, kv_stride_1, num_blocks, page_size, block_table,
                       bt_stride_b, bt_cols, seqlens, batch, num_heads, head_dim_v, rope_dim, dtype, softmax_scale,
                       num_splits, num_workers, out, out_stride_b, out_stride_h, lse, workspace, workspace_bytes_,
                       stream, 2);
}

int tmla_mla_decode_fused(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kv, int64_t kv_stride_0,
                          int64_t kv_stride_1, int64_t num_blocks, int32_t page_size, const int32_t* block_table,
                          int64_t bt_stride_b, int32_t bt_cols, const int32_t* seqlens, int32_t batch,
                          int32_t num_heads, int32_t head_dim_v, int32_t rope_dim, int32_t dtype, float softmax_scale,
                          int32_t num_splits, int32_t num_workers, void* out, int64_t out_stride_b,
                          int64_t out_stride_h, float* lse, void* workspace, size_t workspace_bytes_,
                          int32_t spin_limit, void* stream) {
  return decode_launch(q, q_stride_b, q_stride_h, kv, kv_stride_0, kv_stride_1, num_blocks, page_size, block_table,
                       bt_stride_b, bt_cols, seqlens, batch, num_heads, head_dim_v, rope_dim, dtype, softmax_scale,
                       num_splits, num_workers, out, out_stride_b, out_stride_h, lse, workspace, workspace_bytes_,
                       stream, 1, 1, spin_limit);
}

int tmla_mla_decode_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kv,
                            int64_t kv_stride_0, int64_t kv_stride_1, int64_t num_blocks, int32_t page_size,
                            const int32_t* block_table, int64_t bt_stride_b, int32_t bt_cols,
                            const int32_t* seqlens, int32_t batch, int32_t num_heads, int32_t head_dim_v,
                            int32_t rope_dim, int32_t dtype, float softmax_scale, int32_t num_splits,
                            int32_t num_workers, void* out, int64_t out_stride_b, int64_t out_stride_h,
                            float* lse, void* stream) {
  const size_t need = workspace_bytes(batch, num_heads, head_dim_v, num_splits, num_workers);
  if (need > kScratchBytes) {
    snprintf(g_err, sizeof(g_err),
             "the call needs %zu bytes of workspace, more than the %zu of the built-in scratch "
             "(use tmla_mla_decode with a caller-owned workspace)",
             need, kScratchBytes);
    return TMLA_ERR_WORKSPACE_TOO_SMALL;
  }
  void* ws = nullptr;
  const int rc = scratch_for_stream(stream, &ws);
  if (rc != TMLA_OK) return rc;
  return decode_launch(q, q_stride_b, q_stride_h, kv, kv_stride_0, kv_stride_1, num_blocks, page_size, block_table,
                       bt_stride_b, bt_cols, seqlens, batch, num_heads, head_dim_v, rope_dim, dtype, softmax_scale,
                       num_splits, num_workers, out, out_stride_b, out_stride_h, lse, ws, kScratchBytes, stream, 2);
}

size_t tmla_workspace_zero_bytes(int32_t batch, int32_t num_heads, int32_t head_dim_v, int32_t num_splits,
                                 int32_t num_workers) {
  if (batch < 0 || num_heads <= 0 || head_dim_v < 0) return 0;
  // the counter block plus the slack of rounding the buffer size down to 256
  return ws_layout(batch, num_heads, head_dim_v, num_splits, num_workers).cnt_bytes + 255;
}

int32_t tmla_mla_decode_fused_is_single(int32_t batch, int32_t num_heads, int32_t head_dim_v, int32_t num_splits,
                                        int32_t num_workers, int64_t capacity_tokens, int32_t device) {
  if (batch <= 0 || num_heads <= 0 || head_dim_v != 512 || num_splits < 0 ||
      (num_splits == 0 && num_workers <= 0))
    return 0;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return 0;
  const WsLayout wl = ws_layout(batch, num_heads, head_dim_v, num_splits, num_workers);
  const LaunchPlan p =
      uses_g16(num_heads)
          ? plan_launch_g16(batch, num_heads, num_splits, num_workers, capacity_tokens, wl.l - wl.o, 1, cus)
          : plan_launch(batch, num_heads, num_splits, num_workers, capacity_tokens, wl.l - wl.o, 1, cus);
  return p.fused ? 1 : 0;
}

int tmla_mla_decode_causal(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kv,
                           int64_t kv_stride_0, int64_t kv_stride_1, int64_t num_blocks, int32_t page_size,
                           const int32_t* block_table, int64_t bt_stride_b, int32_t bt_cols, const int32_t* seqlens,
                           int32_t batch, int32_t q_len, int32_t num_heads, int32_t head_dim_v, int32_t rope_dim,
                           int32_t dtype, float softmax_scale, int32_t num_splits, int32_t num_workers, void* out,
                           int64_t out_stride_b, int64_t out_stride_h, float* lse, void* workspace,
                           size_t workspace_bytes_, int32_t single_launch, void* stream) {
  if (q_len < 1 || num_heads <= 0 || (int64_t)q_len * num_heads > INT32_MAX)
    return fail(TMLA_ERR_INVALID_ARGUMENT, "q_len must be >= 1 and q_len * num_heads must fit int32");
  return decode_launch(q, q_stride_b, q_stride_h, kv, kv_stride_0, kv_stride_1, num_blocks, page_size, block_table,
                       bt_stride_b, bt_cols, seqlens, batch, q_len * num_heads, head_dim_v, rope_dim, dtype,
                       softmax_scale, num_splits, num_workers, out, out_stride_b, out_stride_h, lse, workspace,
                       workspace_bytes_, stream, single_launch ? 1 : 2, q_len);
}

int tmla_mla_decode_fp8(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kv, int64_t kv_stride_0,
                        int64_t kv_stride_1, int64_t num_blocks, int32_t page_size, const float* kv_scale,
                        int64_t scale_stride_0, int64_t scale_stride_1, const int32_t* block_table,
                        int64_t bt_stride_b, int32_t bt_cols, const int32_t* seqlens, int32_t batch, int32_t q_len,
                        int32_t num_heads, int32_t head_dim_v, int32_t rope_dim, int32_t dtype, float softmax_scale,
                        int32_t num_splits, int32_t num_workers, void* out, int64_t out_stride_b,
                        int64_t out_stride_h, float* lse, void* workspace, size_t workspace_bytes_, void* stream) {
  if (q_len < 1 || num_heads <= 0 || (int64_t)q_len * num_heads > INT32_MAX)
    return fail(TMLA_ERR_INVALID_ARGUMENT, "q_len must be >= 1 and q_len * num_heads must fit int32");
  const Fp8Scales f8{kv_scale, scale_stride_0, scale_stride_1};
  return decode_launch(q, q_stride_b, q_stride_h, kv, kv_stride_0, kv_stride_1, num_blocks, page_size, block_table,
                       bt_stride_b, bt_cols, seqlens, batch, q_len * num_heads, head_dim_v, rope_dim, dtype,
                       softmax_scale, num_splits, num_workers, out, out_stride_b, out_stride_h, lse, workspace,
                       workspace_bytes_, stream, 2, q_len, -1, &f8);
}

int tmla_mla_decode_fp8_partial(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kv,
                                int64_t kv_stride_0, int64_t kv_stride_1, int64_t num_blocks, int32_t page_size,
                                const float* kv_scale, int64_t scale_stride_0, int64_t scale_stride_1,
                                const int32_t* block_table, int64_t bt_stride_b, int32_t bt_cols,
                                const int32_t* seqlens, int32_t batch, int32_t num_heads, int32_t head_dim_v,
                                int32_t rope_dim, int32_t dtype, float softmax_scale, int32_t num_splits,
                                int32_t num_workers, void* out, int64_t out_stride_b, int64_t out_stride_h,
                                float* lse, void* workspace, size_t workspace_bytes_, void* stream) {
  const Fp8Scales f8{kv_scale, scale_stride_0, scale_stride_1};
  return decode_launch(q, q_stride_b, q_stride_h, kv, kv_stride_0, kv_stride_1, num_blocks, page_size, block_table,
                       bt_stride_b, bt_cols, seqlens, batch, num_heads, head_dim_v, rope_dim, dtype, softmax_scale,
                       num_splits, num_workers, out, out_stride_b, out_stride_h, lse, workspace, workspace_bytes_,
                       stream, 0, 1, -1, &f8);
}

}  // extern "C"
