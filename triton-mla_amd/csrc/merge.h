// The log-sum-exp merge of split partials: the stage-2 combine kernel
// (mla_decode.hip) and the single launch's in-kernel merge of the partial
// kernels (mla_decode.hip, mla_decode_g16.hip) use it.
#pragma once

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include "cdna.h"
#include "decode_common.h"

namespace tmla {

// ---------------------------------------------------------------------------
// Log-sum-exp merge of split partials (kernel.py:159-181):
//   m = max_j lse2_j (-inf -> 0), w_j = 2^(lse2_j - m),
//   out = sum_j w_j o_j / sum_j w_j, lse = (m + log2 sum_j w_j) ln 2.
// One wave per head row (64 lanes x 8 elements of 512).
// ---------------------------------------------------------------------------
struct MergeView {
  const short* mid_o;    // [slots, H, 512]
  const float* mid_lse;  // [slots, H]
  int32_t num_heads;
  char* out;
  int64_t out_sb, out_sh;
  float* lse;            // [batch, H], natural log
};

// Partial rows and lse values written by an earlier launch (stage 2).
struct PlainLoads {
  const short* mid_o;
  const float* mid_lse;
  __device__ __forceinline__ float lse(int64_t row) const { return mid_lse[row]; }
  __device__ __forceinline__ i16x8 rowv(int64_t row, int lane) const {
    return *reinterpret_cast<const i16x8*>(mid_o + row * 512 + lane * 8);
  }
};

// Written by other workgroups of the same launch (the fused merge): loads
// that bypass this CU's L1 and the L2 (system-coherent, sc0 sc1) see the
// write-through stores of the partials without any cache maintenance. Byte
// offsets are 32-bit (the host keeps the partials below 2 GiB).
// Buffer resource word 3 of gfx9-family raw buffers (32-bit data format).
constexpr int kBufferWord3 = 0x00020000;

struct CoherentLoads {
  __amdgpu_buffer_rsrc_t ro, rl;
  static constexpr int kSysCoherent = 1 | 16;  // sc0 | sc1
  __device__ __forceinline__ float lse(int64_t row) const {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rl, (int)row * 4, 0, kSysCoherent));
  }
  __device__ __forceinline__ i16x8 rowv(int64_t row, int lane) const {
    return __builtin_bit_cast(i16x8, __builtin_amdgcn_raw_buffer_load_b128(ro, (int)row * 1024 + lane * 16, 0,
                                                                           kSysCoherent));
  }
};

template <int DT>
__device__ __forceinline__ void merge_store(const MergeView& mv, int b, int head, const float (&acc)[8], float wsum,
                                            float m, int lane) {
  const float inv = wsum > 0.0f ? 1.0f / wsum : 1.0f;
  i16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = Elt<DT>::from_float(acc[e] * inv);
  short* orow = reinterpret_cast<short*>(mv.out) + (int64_t)b * mv.out_sb + (int64_t)head * mv.out_sh;
  *reinterpret_cast<i16x8*>(orow + lane * 8) = o;
  if (lane == 0 && mv.lse)
    mv.lse[(int64_t)b * mv.num_heads + head] = wsum > 0.0f ? (m + fast_log2(wsum)) * kLn2 : -INFINITY;
}

// Empty sequence: out = 0, lse = -inf (kernel.py:126-128, 178-181).
__device__ __forceinline__ void merge_zero(const MergeView& mv, int b, int head, int lane) {
  short* orow = reinterpret_cast<short*>(mv.out) + (int64_t)b * mv.out_sb + (int64_t)head * mv.out_sh;
  *reinterpret_cast<i16x8*>(orow + lane * 8) = (i16x8)0;
  if (lane == 0 && mv.lse) mv.lse[(int64_t)b * mv.num_heads + head] = -INFINITY;
}

// Heads [head, head + nh), nh <= NH, over slots [slot0, slot0 + count),
// count <= NR: every lse and row load is issued before the first use. Slots
// past `count` repeat the last one with weight 0; heads past `nh` repeat the
// last head and are not stored.
template <int DT, int NH, int NR, class LD>
__device__ __forceinline__ void merge_rows_at_once(const MergeView& mv, const LD& ld, int b, int head, int nh,
                                                   int slot0, int count, int lane) {
  float l[NH][NR];
  i16x8 v[NH][NR];
  // row indices in VGPRs: vector address arithmetic instead of one scalar
  // register pair per row
  int r0 = slot0 * mv.num_heads + head;
  pin_i1(r0);
#pragma unroll
  for (int i = 0; i < NH; ++i) {
    const int hh = min(i, nh - 1);
#pragma unroll
    for (int j = 0; j < NR; ++j) {
      const int64_t row = (int64_t)(r0 + min(j, count - 1) * mv.num_heads + hh);
      l[i][j] = ld.lse(row);
      v[i][j] = ld.rowv(row, lane);
    }
  }
#pragma unroll
  for (int i = 0; i < NH; ++i) {
    if (i >= nh) break;
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < NR; ++j)
      if (j < count) m = fmaxf(m, l[i][j]);
    if (m == -INFINITY) m = 0.0f;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0}, wsum = 0.0f;
#pragma unroll
    for (int j = 0; j < NR; ++j) {
      const float w = j < count ? fast_exp2(l[i][j] - m) : 0.0f;
      wsum += w;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += w * Elt<DT>::to_float(v[i][j][e]);
    }
    merge_store<DT>(mv, b, head + i, acc, wsum, m, lane);
  }
}

// Any count: the max over all slots first, then BATCH rows in flight per
// batch. The result does not depend on BATCH, and equals merge_rows_at_once
// over the same slots bit for bit (the same max, weights and order of sums).
template <int DT, int BATCH, class LD>
__device__ __forceinline__ void merge_row_loop(const MergeView& mv, const LD& ld, int b, int head, int slot0,
                                               int count, int lane) {
  float m = -INFINITY;
  for (int s = lane; s < count; s += 64) m = fmaxf(m, ld.lse((int64_t)(slot0 + s) * mv.num_heads + head));
  for (int d = 32; d >= 1; d >>= 1) m = fmaxf(m, __shfl_xor(m, d));
  if (m == -INFINITY) m = 0.0f;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0}, wsum = 0.0f;
  for (int s0 = 0; s0 < count; s0 += BATCH) {
    float w[BATCH];
    i16x8 v[BATCH];
#pragma unroll
    for (int j = 0; j < BATCH; ++j) {
      const int sj = s0 + j;
      const int64_t row = (int64_t)(slot0 + min(sj, count - 1)) * mv.num_heads + head;
      w[j] = sj < count ? fast_exp2(ld.lse(row) - m) : 0.0f;
      v[j] = ld.rowv(row, lane);
    }
#pragma unroll
    for (int j = 0; j < BATCH; ++j) {
      wsum += w[j];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += w[j] * Elt<DT>::to_float(v[j][e]);
    }
  }
  merge_store<DT>(mv, b, head, acc, wsum, m, lane);
}

// ---------------------------------------------------------------------------
// Fused merge (single launch): run by every workgroup of the partial kernel
// after its last segment.
//
// The c workers of a split sequence b (per head block of a workgroup) each
// store their partial, then add 1 to m_count[b]. Sibling k then merges share
// k of the workgroup's heads, heads [k*nh/c, (k+1)*nh/c), once m_count[b]
// reaches c. The wait is bounded (spin_limit polls): a worker that runs out
// hands its share over (m_flag 0 -> 1) and then reads m_count again with a
// read-modify-write; if all have arrived by then it takes the share back
// (1 -> 2) and merges it itself, else the worker whose arrival completed the
// count finds the flag at 1 and takes the share over (1 -> 2). Every share is
// merged exactly once and no worker waits without bound, whether or not the
// siblings are resident together. The worker that completes m_done[b]
// (shares merged) resets the sequence's counters and flags to zero, so the
// workspace is ready for the next launch.
//
// Coherence without cache maintenance: partial rows and lse values are
// stored write-through at system scope (sc0 sc1) and their stores have
// completed (vmcnt 0) before the arrival; counters and flags are system-scope
// atomics, performed at memory; merges read the partials with loads that
// bypass L1 and L2 (CoherentLoads). A release/acquire at agent scope would
// instead write back and invalidate the whole L2 of the XCD for every
// arrival and merge. Two atomics whose order matters are separated by a wait
// for the first one's completion.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void mem_wait_all() { asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory"); }

__device__ __forceinline__ int sys_load(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ int sys_add(int* p, int v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ bool sys_cas(int* p, int expect, int desired) {
  return __hip_atomic_compare_exchange_strong(p, &expect, desired, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void sys_store(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

template <int DT>
__device__ __forceinline__ void merge_share(const MergeView& mv, const CoherentLoads& ld, int b, int j, int c, int s0,
                                            int hb0, int nh, int wave, int lane) {
  const int h_lo = hb0 + (j * nh) / c, h_hi = hb0 + ((j + 1) * nh) / c;
  if (c <= 8) {
    for (int h = h_lo + 4 * wave; h < h_hi; h += 16)
      merge_rows_at_once<DT, 4, 8>(mv, ld, b, h, min(4, h_hi - h), s0, c, lane);
  } else if (c <= 16) {
    for (int h = h_lo + 2 * wave; h < h_hi; h += 8)
      merge_rows_at_once<DT, 2, 16>(mv, ld, b, h, min(2, h_hi - h), s0, c, lane);
  } else {
    for (int h = h_lo + wave; h < h_hi; h += 4) merge_row_loop<DT, 8>(mv, ld, b, h, s0, c, lane);
  }
}

template <int DT>
__device__ __forceinline__ void fused_merge_tail(const MergeView& mv, const CoherentLoads& ld, int32_t* m_count,
                                                 int32_t* m_done, int32_t* m_flag, int spin_limit, int wave,
                                                 int (*s_pend)[5], int* s_msg, int wg_heads) {
  const int lane = lane_id_fresh();
  const int gy = gridDim.y, y = blockIdx.y;
  const int hb0 = y * wg_heads;
  const int nh = min(wg_heads, mv.num_heads - hb0);
  mem_wait_all();
  lds_barrier();  // the merge records written by thread 0
  for (int p = 0; p < 2; ++p) {
    const int b = s_pend[p][0], k = s_pend[p][1], c = s_pend[p][2], s0 = s_pend[p][3];
    if (b < 0) continue;
    int* cnt = m_count + (int64_t)b * gy + y;
    int* done = m_done + (int64_t)b * gy + y;
    int* flag = m_flag + (int64_t)s0 * gy + y;  // sibling j: flag[j * gy]
    if (wave == 0) {
      const bool last = s_pend[p][4] != 0;
      int own = last ? 1 : 0;
      if (!last) {
        int v = 0;
        for (int it = 0;; ++it) {
          int x = 0;
          if (lane == 0) x = sys_load(cnt);
          v = __builtin_amdgcn_readfirstlane(x);
          if (v >= c || it >= spin_limit) break;
          __builtin_amdgcn_s_sleep(2);
        }
        if (v >= c) {
          own = 1;
        } else {
          int r = 0;
          if (lane == 0) {
            int* fk = flag + (int64_t)k * gy;
            sys_cas(fk, 0, 1);
            mem_wait_all();  // the hand-over is in place before the count is read again
            const int v2 = sys_add(cnt, 0);
            mem_wait_all();
            if (v2 >= c) r = sys_cas(fk, 1, 2) ? 1 : 0;
          }
          own = __builtin_amdgcn_readfirstlane(r);
        }
      }
      if (lane == 0) {
        s_msg[0] = own;
        s_msg[1] = last ? 1 : 0;
      }
    }
    mem_wait_all();
    lds_barrier();
    const int own = s_msg[0], last = s_msg[1];
    int merged = 0;
    if (own) {
      merge_share<DT>(mv, ld, b, k, c, s0, hb0, nh, wave, lane);
      merged = 1;
    }
    if (last) {
      // shares handed over by siblings that stopped waiting
      for (int j0 = 0; j0 < c; j0 += 64) {
        mem_wait_all();
        lds_barrier();  // every wave has read s_msg
        if (wave == 0) {
          const int j = j0 + lane;
          bool won = false;
          if (j < c && j != k) {
            int* fj = flag + (int64_t)j * gy;
            if (sys_load(fj) == 1) won = sys_cas(fj, 1, 2);
          }
          const uint64_t mask = __ballot(won);
          if (lane == 0) {
            s_msg[2] = (int)(uint32_t)mask;
            s_msg[3] = (int)(uint32_t)(mask >> 32);
          }
        }
        mem_wait_all();
        lds_barrier();
        uint64_t mask = (uint64_t)(uint32_t)s_msg[2] | ((uint64_t)(uint32_t)s_msg[3] << 32);
        while (mask != 0) {
          const int j = j0 + __builtin_ctzll(mask);
          mask &= mask - 1;
          merge_share<DT>(mv, ld, b, j, c, s0, hb0, nh, wave, lane);
          ++merged;
        }
      }
    }
    // the worker whose shares complete the count resets b's state
    if (wave == 0 && merged > 0) {
      int r = 0;
      if (lane == 0) r = sys_add(done, merged) + merged == c;
      if (__builtin_amdgcn_readfirstlane(r)) {
        for (int j = lane; j < c; j += 64) sys_store(flag + (int64_t)j * gy, 0);
        if (lane == 0) {
          sys_store(cnt, 0);
          sys_store(done, 0);
        }
      }
    }
    mem_wait_all();
    lds_barrier();  // s_msg is rewritten for the next record
  }
}

}  // namespace tmla
