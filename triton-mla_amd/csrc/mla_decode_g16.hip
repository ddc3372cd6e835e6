// MLA decode over a 16-bit (bf16 / fp16) latent cache for at most 16 query
// heads per workgroup: the split-KV stage-1 kernel for MI355X (gfx950) that
// mla_decode.hip's decode_launch runs for such calls. Stage 2 is
// mla_decode.hip's combine kernel: the partial slots, their base-2 lse and
// the direct outputs are exactly those of the other partial kernels.
//
// The reference computes this with its stage-1 kernel (src/triton_mla/
// kernel.py:43-138) for any head count; DeepSeek-V2-Lite's 16 heads leave
// half of a 32-head MFMA block idle, and one wave running S for the whole
// workgroup keeps the other three waiting, so a call with few heads runs here:
//
//  * one workgroup = one worker of the split-KV partition, 4 waves (one per
//    SIMD), heads head0 .. head0 + 15 (grid.y covers more heads in groups of
//    16, each group streaming the cache on its own);
//  * wave w owns token slice w (tokens 16w .. 16w + 15) of every 64-token
//    tile of the worker's range and streams it through its own 2-entry LDS
//    ring with LDS-DMA (global_load_lds: no VGPR staging); the waves never
//    wait for one another inside the tile loop. A ring entry holds the
//    slice's 16 rows (1152 bytes each) with 16-byte chunk (row r, column c)
//    at byte 256 c + 16 r;
//  * S^T = K . Q^T (16 tokens x 16 heads) with v_mfma_f32_16x16x32_{bf16,f16}:
//    the K operand of lane (g, r) = chunk (r, 4j + g), one ds_read_b128 per
//    MFMA (1 KiB contiguous per instruction); Q^T lives in VGPRs in the same
//    dimension order;
//  * online softmax in the base-2 domain with a lazy rescale (the reference
//    max moves only when a score exceeds it by 2^8). Lane (g, n) holds
//    tokens 4g .. 4g + 3 of head n, the B operand layout of
//    v_mfma_f32_16x16x16 with k = token: the probabilities feed the value
//    product straight from the score registers;
//  * O^T += V^T . P^T (dims x heads): V^T from ds_read_b64_tr_b16, whose 16
//    lanes of a group fetch four 8-byte pieces of four token rows each and
//    return one dimension of the four tokens per lane;
//  * at the end of a segment the four waves' running max, sum and O^T are
//    merged through LDS and written as the output row (+ lse) or as a
//    partial (+ base-2 lse).
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include "cdna.h"
#include "decode_common.h"
#include "group16.h"
#include "merge.h"
#include "triton_mla.h"

namespace tmla {

namespace g16 {

using namespace grp;

constexpr int kSlice = 16;               // tokens per wave per 64-token tile
constexpr int kHeads = 16;               // heads per workgroup: N of the MFMAs
constexpr int kRow = 1152;               // bytes per cache row (576 16-bit elements)
constexpr int kKv = kSlice * kRow;       // 18432 bytes per ring entry
constexpr int kLoads = kKv / 1024;       // LDS-DMA instructions per slice
constexpr int kStages = 2;               // ring entries per wave
constexpr int kRing = kStages * kKv;
constexpr int kStats = 4 * kRing;        // per-wave max and sum of every head
constexpr int kSmem = kStats + 2 * 4 * kHeads * 4;
constexpr int kOPitch = 512 * 4 + 16;    // merge staging: one fp32 row of a head, padded
constexpr int kChunks = 576 / 32;        // k-steps of S^T (32 dims each)
constexpr int kDimBlocks = 512 / 16;     // value steps (16 dims each)
static_assert(kKv % 1024 == 0 && kLoads < 64, "whole 1 KiB copies, vmcnt range");
static_assert(4 * kHeads * kOPitch <= kStats, "merge staging fits the rings");
static_assert(kSmem <= 160 * 1024, "LDS");

constexpr int KA = 6;  // K operand reads ahead of their MFMA
constexpr int VA = 8;  // V^T reads ahead of their MFMA
static_assert(KA <= kChunks && VA <= kDimBlocks && KA <= 16 && VA <= 16, "read-ahead within lgkmcnt");

// Element type of q, the cache and out: the two MFMAs, written as asm with
// the accumulator tied in place (S^T in VGPRs, O^T in AGPRs) so that no
// accumulator is ever copied between registers, and volatile so that they
// keep their places among the LDS reads and waits. The compiler cannot see
// the hazards of asm: the value MFMA carries the two wait states a VALU
// result (the probabilities) needs before an MFMA reads it, and mfma_fence
// waits out the MFMA result latency before VALU code reads S^T.
template <int DT>
struct Elt16;
template <>
struct Elt16<TMLA_BF16> {
  typedef bf16x8 v8;
  typedef bf16x4 v4;
  __device__ static __forceinline__ void mfma_qk_first(f32x4& d, const v8& k, const v8& q) {
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0" : "=&v"(d) : "v"(k), "v"(q));
  }
  __device__ static __forceinline__ void mfma_qk(f32x4& d, const v8& k, const v8& q) {
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(k), "v"(q));
  }
  __device__ static __forceinline__ void mfma_pv(f32x4& acc, const v4& v, const v4& p) {
    asm volatile("s_nop 1\n\tv_mfma_f32_16x16x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(v), "v"(p));
  }
  __device__ static __forceinline__ __bf16 round(float x) { return (__bf16)x; }
};
template <>
struct Elt16<TMLA_FP16> {
  typedef f16x8 v8;
  typedef f16x4 v4;
  __device__ static __forceinline__ void mfma_qk_first(f32x4& d, const v8& k, const v8& q) {
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, 0" : "=&v"(d) : "v"(k), "v"(q));
  }
  __device__ static __forceinline__ void mfma_qk(f32x4& d, const v8& k, const v8& q) {
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(d) : "v"(k), "v"(q));
  }
  __device__ static __forceinline__ void mfma_pv(f32x4& acc, const v4& v, const v4& p) {
    asm volatile("s_nop 1\n\tv_mfma_f32_16x16x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(v), "v"(p));
  }
  __device__ static __forceinline__ _Float16 round(float x) { return (_Float16)x; }
};

template <int N>
__device__ __forceinline__ void lgkm_tie16(i16x4& x) {
  static_assert(N >= 0 && N <= 15, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(x) : "i"(N));
}

}  // namespace g16

// PAGED: block table, else a dense [batch, capacity, 576] cache. UNI: pages
// of a multiple of 16 tokens (a slice lies in one page, whose id is a scalar
// load one slice ahead); otherwise each lane looks up its own row's page.
template <int DT, bool PAGED, bool UNI>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void mla_partial_g16_kernel(PartialArgs a) {
  using namespace g16;
  using E = Elt16<DT>;
  __shared__ __attribute__((aligned(1024))) char smem[kSmem];
  char LDS_AS* const lds = (char LDS_AS*)(void LDS_AS*)smem;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // slice of each tile
  const int worker = worker_index(a);
  const int head0 = blockIdx.y * kHeads;
  const int nh = min(kHeads, a.num_heads - head0);
  // single launch: this workgroup's merge records (first and last segment:
  // b, its index among b's workers, their count, b's first slot, whether its
  // arrival completed the count) and the tail's messages
  __shared__ int s_pend[2][5];
  __shared__ int s_msg[4];
  WorkRange wr;
  const bool has_range = work_range(a, worker, wr) && wr.tile_lo < wr.tile_hi;
  if (a.fused) {
    if (threadIdx.x == 0) s_pend[0][0] = s_pend[1][0] = -1;
    // empty sequences worker, worker + nwg, ...: out = 0, lse = -inf
    // (kernel.py:126-128, 178-181); the combine kernel does this otherwise
    const MergeView mv{a.mid_o, a.mid_lse, a.num_heads, a.out, a.out_sb, a.out_sh, a.lse};
    const int lane = lane_id_fresh();
    for (int bb = worker; bb < a.batch; bb += gridDim.x)
      if (tiles_of(a.seqlens[bb]) == 0)
        for (int h = head0 + wave; h < head0 + nh; h += 4) merge_zero(mv, bb, h, lane);
  }
  if (!has_range) return;  // (a workgroup without a range has no merge records)
  char LDS_AS* const ring = lds + wave * kRing;

  int b = wr.b_first;
  int t_start = wr.tile_lo;              // local tile index within b
  int remaining = wr.tile_hi - wr.tile_lo;
  int seg_global_off = wr.off_first;     // balanced mode: tile offset of b
  while (remaining > 0) {
    const int n_b = b == wr.b_first ? wr.n_first : a.seqlens[b];
    const int nt_b = tiles_of(n_b);
    if (nt_b == 0) {  // only possible in balanced mode between sequences
      ++b;
      continue;
    }
    const int t_end = min(nt_b, t_start + remaining);
    const SegmentSlot ss = segment_slot(a, wr, worker, b, t_start, nt_b, seg_global_off);
    if (a.fused && !ss.direct && threadIdx.x == 0) {
      int* rec = s_pend[b == wr.b_first ? 0 : 1];
      rec[0] = b;
      rec[1] = ss.index;
      rec[2] = ss.count;
      rec[3] = ss.first_slot;
    }

    const int lane = lane_id_fresh();
    const int g = lane >> 4, r = lane & 15;
    const int head = head0 + r;
    const bool head_ok = r < nh;
    // tokens [0, limit) are visible to this lane's head
    const int limit = n_b - causal_lag(a, head);

    // Q^T: operand j of lane (g, n) = dims 32j + 8g .. + 7 of head n
    typename E::v8 qop[kChunks];
    {
      const char* qrow = a.q + ((int64_t)b * a.q_sb + (int64_t)min(head, a.num_heads - 1) * a.q_sh) * 2 + g * 16;
#pragma unroll
      for (int j = 0; j < kChunks; ++j) {
        const i32x4 v = head_ok ? *reinterpret_cast<const i32x4*>(qrow + j * 64) : i32x4{0, 0, 0, 0};
        qop[j] = __builtin_bit_cast(typename E::v8, v);
      }
    }

    // this wave's slices: one per tile below t_end, the last one only when
    // its slice holds a token
    const int tiles_w = t_end - t_start;
    const int ns = tiles_w - (kTileTokens * (t_start + tiles_w - 1) + kSlice * wave >= n_b ? 1 : 0);
    auto slice_tok = [&](int k) __attribute__((always_inline)) { return kTileTokens * (t_start + k) + kSlice * wave; };
    const int32_t* bt_row = PAGED ? a.bt + (int64_t)b * a.bt_sb : a.bt;
    auto page_fetch = [&](int k) __attribute__((always_inline)) -> int {
      return PAGED && UNI ? s_load_i32(bt_row + page_slot_of(a, slice_tok(k))) : 0;
    };
    auto clamp_page = [&](int v) __attribute__((always_inline)) -> int { return v < 0 ? 0 : min(v, a.max_page); };
    // DMA lane role: row r (clamped to the sequence's last token), chunk
    // column g (+ 4j for copy j)
    auto issue = [&](int k, int page) __attribute__((always_inline)) {
      const int t0 = slice_tok(k);
      const int rr = min(r, n_b - 1 - t0);
      int64_t row;
      if constexpr (PAGED && UNI) {
        const int in_page = a.page_shift >= 0 ? (t0 & (a.page_size - 1)) : (t0 % a.page_size);
        row = (int64_t)page * a.kv_s0 + (int64_t)(in_page + rr) * a.kv_s1;
      } else if constexpr (PAGED) {
        const int t = t0 + rr;
        const int slot = page_slot_of(a, t);  // clamped to the table's last column
        const int in_page = min(t - slot * a.page_size, a.page_size - 1);
        row = (int64_t)load_page(a, b, slot) * a.kv_s0 + (int64_t)in_page * a.kv_s1;
      } else {
        const int t = min(t0 + rr, (int)(a.num_blocks - 1));
        row = (int64_t)b * a.kv_s0 + (int64_t)t * a.kv_s1;
      }
      const char* src = a.kv + row + g * 16;
      char LDS_AS* dst = ring + (k % kStages) * kKv;
      static_for<kLoads>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        lds_copy16<64 * j>(src, dst + 1024 * j);
      });
    };

    f32x4 o[kDimBlocks];
#pragma unroll
    for (int d = 0; d < kDimBlocks; ++d) {
      o[d] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      pin_acc(o[d]);
    }
    // base-2 reference max of the lane's head (kNoMax until it has seen a
    // token, so that p = 2^(x - m) of a masked score is 0 even then) and the
    // sum of p over the lane's tokens
    float m_ref = kNoMax;
    float l_run = 0.0f;
    // V^T reads (ds_read_b64_tr_b16): lane L of group g addresses token row
    // 4g + L/4 and dims 4(L%4) .. + 3 of a 16-dim block, i.e. chunk column
    // 2u + (L%4)/2 at byte 8(L%2) of the chunk, and receives dim L of the
    // block for tokens 4g .. 4g + 3
    const int tr_off = 256 * ((r & 3) >> 1) + 16 * (4 * g + (r >> 2)) + 8 * (r & 1);

    // Prologue: slice 0 in flight, page ids of slices 1 and 2 requested.
    // Page ids come from scalar loads without a wait; every wait for them is
    // an lgkmcnt(0) that names all ids still in flight, so none is read or
    // moved before it has arrived.
    int pg_a = 0, pg_b = 0;  // page ids of slices k + 1 and k + 2
    {
      int p0 = ns > 0 ? page_fetch(0) : 0;
      pg_a = ns > 1 ? page_fetch(1) : 0;
      pg_b = ns > 2 ? page_fetch(2) : 0;
      if (PAGED && UNI) asm volatile("s_waitcnt lgkmcnt(0)" : "+s"(p0), "+s"(pg_a), "+s"(pg_b));
      if (ns > 0) issue(0, clamp_page(p0));
    }
    // Q^T has arrived once the copies of slice 0 are the only loads in
    // flight; from here on the compiler sees it as plain registers
    if (ns > 0)
      wait_vmcnt<kLoads>();
    else
      wait_vmcnt<0>();
#pragma unroll
    for (int j = 0; j < kChunks; ++j) pin_v(qop[j]);

    for (int k = 0; k < ns; ++k) {
      // the copies of slice k + 1 go into the entry slice k - 1 has left
      const bool ahead = k + 1 < ns;
      if (ahead) {
        if (PAGED && UNI) asm volatile("s_waitcnt lgkmcnt(0)" : "+s"(pg_a), "+s"(pg_b));
        const int pcur = clamp_page(pg_a);
        pg_a = pg_b;
        issue(k + 1, pcur);
      }
      // slice k has landed once only the copies of slice k + 1 may remain
      if (ahead)
        wait_vmcnt<kLoads>();
      else
        wait_vmcnt<0>();
      const char LDS_AS* ent = ring + (k % kStages) * kKv;
      const int t0 = slice_tok(k);

      // ---- S^T = K . Q^T ----------------------------------------------------
      // K operands 0 .. KA - 1 first, then K operand j + KA after step j; the
      // wait of step j counts the K reads younger than operand j (an extra
      // scalar load in flight only makes a wait stricter: LDS reads complete
      // in order).
      const char LDS_AS* kp = ent + 16 * lane;
      const char LDS_AS* vp = ent + tr_off;
      i32x4 kr[kChunks];
      static_for<KA>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        kr[j] = ds_read_x4<1024 * j>(kp);
      });
      f32x4 s;
      static_for<kChunks>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        constexpr int younger = (KA - 1 < kChunks - 1 - j) ? KA - 1 : kChunks - 1 - j;
        lgkm_tie<younger>(kr[j]);
        const typename E::v8 kop = __builtin_bit_cast(typename E::v8, kr[j]);
        if constexpr (j == 0)
          E::mfma_qk_first(s, kop, qop[0]);
        else
          E::mfma_qk(s, kop, qop[j]);
        if constexpr (j + KA < kChunks) kr[j + KA] = ds_read_x4<1024 * (j + KA)>(kp);
        __builtin_amdgcn_sched_barrier(0);
      });
      // V^T reads 0 .. VA - 1 now, the rest one per value step
      i16x4 vr[kDimBlocks];
      static_for<VA>([&](auto uc) {
        constexpr int u = decltype(uc)::value;
        vr[u] = ds_read_tr<512 * u>(vp);
      });

      // ---- online softmax (base 2) ---------------------------------------
      mfma_fence(s);
      float x[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = t0 + 4 * g + i < limit ? s[i] * a.qk_scale_log2 : -INFINITY;
      const float mx = rows_max(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])));
      if (__ballot(mx > m_ref + kRescaleLog2) != 0) {
        const float m_new = mx > m_ref + kRescaleLog2 ? mx : m_ref;
        const float alpha = fast_exp2(m_ref - m_new);  // 0 from kNoMax, 1 where unchanged
        l_run *= alpha;
#pragma unroll
        for (int d = 0; d < kDimBlocks; ++d) scale_acc(o[d], alpha);
        m_ref = m_new;
      }
#pragma unroll
      for (int d = 0; d < kDimBlocks; ++d) pin_acc(o[d]);
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) p[i] = fast_exp2(x[i] - m_ref);
      l_run += (p[0] + p[1]) + (p[2] + p[3]);
      const typename E::v4 pb{E::round(p[0]), E::round(p[1]), E::round(p[2]), E::round(p[3])};
      // the page id of slice k + 3 is requested here, long before the wait
      // for it (top of iteration k + 2)
      if (k + 3 < ns) pg_b = page_fetch(k + 3);
      __builtin_amdgcn_sched_barrier(0);

      // ---- O^T += V^T . P^T ------------------------------------------------
      // V^T read u + VA is issued once read u has been awaited: the wait of
      // step u counts the VA - 1 reads after it (fewer at the end)
      static_for<kDimBlocks>([&](auto uc) {
        constexpr int u = decltype(uc)::value;
        constexpr int younger = (VA - 1 < kDimBlocks - 1 - u) ? VA - 1 : kDimBlocks - 1 - u;
        lgkm_tie16<younger>(vr[u]);
        if constexpr (u + VA < kDimBlocks) vr[u + VA] = ds_read_tr<512 * (u + VA)>(vp);
        E::mfma_pv(o[u], __builtin_bit_cast(typename E::v4, vr[u]), pb);
        __builtin_amdgcn_sched_barrier(0);
      });
#pragma unroll
      for (int j = 0; j < kChunks; ++j) pin_v(qop[j]);
    }

    // ---- merge the waves and store -------------------------------------------
    mfma_fence_a(o[kDimBlocks - 1]);  // the last value products have landed
    {
      const float l_tot = rows_sum(l_run);
      float LDS_AS* stats = reinterpret_cast<float LDS_AS*>(lds + kStats);  // [2][wave][head]
      if (g == 0) {
        stats[wave * kHeads + r] = m_ref;
        stats[4 * kHeads + wave * kHeads + r] = l_tot;
      }
      __syncthreads();  // every wave is past its loop: the rings are free
      float M = kNoMax;
#pragma unroll
      for (int w = 0; w < 4; ++w) M = fmaxf(M, stats[w * kHeads + r]);
      float L = 0.0f;
#pragma unroll
      for (int w = 0; w < 4; ++w) L += fast_exp2(stats[w * kHeads + r] - M) * stats[4 * kHeads + w * kHeads + r];
      const bool has = L > 0.0f;
      const float f = has ? fast_exp2(m_ref - M) / L : 0.0f;
      // staging region w holds wave w's normalised O^T share: row = head,
      // column = dim (lane (g, n) holds dims 16d + 4g .. + 3 of head n)
      char LDS_AS* stage = lds + wave * kHeads * kOPitch + r * kOPitch + 16 * g;
#pragma unroll
      for (int d = 0; d < kDimBlocks; ++d) *reinterpret_cast<f32x4 LDS_AS*>(stage + 64 * d) = o[d] * f;
      __syncthreads();
      // wave w writes heads 4w .. 4w + 3: lane l dims 8l .. 8l + 7
#pragma unroll
      for (int hh = 0; hh < 4; ++hh) {
        const int hr = 4 * wave + hh;
        f32x4 v0 = {0.0f, 0.0f, 0.0f, 0.0f}, v1 = v0;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const char LDS_AS* src = lds + (w * kHeads + hr) * kOPitch + 32 * lane;
          v0 += *reinterpret_cast<const f32x4 LDS_AS*>(src);
          v1 += *reinterpret_cast<const f32x4 LDS_AS*>(src + 16);
        }
        if (hr < nh) {
          i16x8 ov;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            ov[e] = __builtin_bit_cast(short, E::round(v0[e]));
            ov[4 + e] = __builtin_bit_cast(short, E::round(v1[e]));
          }
          short* dst = ss.direct ? reinterpret_cast<short*>(a.out) + (int64_t)b * a.out_sb + (int64_t)(head0 + hr) * a.out_sh
                                 : a.mid_o + ((int64_t)ss.slot * a.num_heads + head0 + hr) * 512;
          store_through(reinterpret_cast<i16x8*>(dst + 8 * lane), ov);
        }
      }
      if (wave == 0 && g == 0 && head_ok) {
        const float lse2 = has ? M + fast_log2(L) : -INFINITY;
        if (ss.direct) {
          if (a.lse) a.lse[(int64_t)b * a.num_heads + head] = has ? lse2 * kLn2 : -INFINITY;
        } else {
          store_through_f32(a.mid_lse + (int64_t)ss.slot * a.num_heads + head, lse2);
        }
      }
      __syncthreads();  // the staging is read before the next segment's copies land
    }
    if (a.fused && !ss.direct) {
      // every wave's write-through partial row and lse stores have completed
      // before the arrival
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (threadIdx.x == 0) {
        const int old = sys_add(a.m_count + (int64_t)b * gridDim.y + blockIdx.y, 1);
        int* rec = s_pend[b == wr.b_first ? 0 : 1];
        rec[4] = old == rec[2] - 1;  // this arrival completed the count
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
                         a.m_count, a.m_done, a.m_flag, a.spin_limit, wave, s_pend, s_msg, kHeads);
  }
}

template <int DT>
hipError_t launch_g16_dt(const PartialArgs& a, dim3 grid, bool paged, hipStream_t stream) {
  if (!paged)
    hipLaunchKernelGGL((mla_partial_g16_kernel<DT, false, false>), grid, dim3(256), 0, stream, a);
  else if (a.page_size % g16::kSlice == 0)
    hipLaunchKernelGGL((mla_partial_g16_kernel<DT, true, true>), grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((mla_partial_g16_kernel<DT, true, false>), grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_partial_g16(const PartialArgs& a, dim3 grid, int dtype, bool paged, hipStream_t stream) {
  return dtype == TMLA_BF16 ? launch_g16_dt<TMLA_BF16>(a, grid, paged, stream)
                            : launch_g16_dt<TMLA_FP16>(a, grid, paged, stream);
}

}  // namespace tmla
