// MLA decode over an fp8 latent cache (OCP e4m3, one byte per element, with
// float32 scales per page or per token): the split-KV stage-1 kernel for
// MI355X (gfx950). Stage 2 is mla_decode.hip's combine kernel: the partial
// slots, their base-2 lse and the direct outputs are exactly those of the
// bf16/fp16 partial kernel.
//
// No counterpart in the reference, which lists "no FP8 cache" among its
// limitations (README.md:32-33). The attention is the reference's
// (src/triton_mla/kernel.py:43-138) over the dequantised cache
//   k[t][d] = e4m3(byte[t][d]) * scale(t),
// scale(t) = kv_scale[page * sc_s0 + row_in_page * sc_s1] (sc_s1 = 0: one
// scale per page; sc_s0 = sc_s1 = 0: one per tensor).
//
// Design: one workgroup = one worker of the split-KV partition, 4 waves (one
// per SIMD), up to 16 query heads (grid.y covers more heads in groups of 16).
//  * Wave w owns token slice w (tokens 16w .. 16w + 15) of every 64-token tile
//    of the worker's range and streams it through its own 4-entry LDS ring
//    with LDS-DMA (global_load_lds: no VGPR staging); the waves never wait for
//    one another inside the tile loop. A ring entry holds the slice's 16 rows
//    (576 bytes each) with 16-byte chunk (row r, column c) at byte
//    256 c + 16 r, then the slice's 16 token scales.
//  * S^T = K . Q^T (tokens x heads) with v_mfma_f32_16x16x32_bf16: the K
//    operand of lane (g, r) = 16 bytes of row r, read with one ds_read_b128
//    (chunk column 4j + g: one contiguous KiB per instruction) and widened
//    exactly to bf16 (v_cvt_scalef32_pk_bf16_fp8, scale 1) for two MFMAs;
//    Q^T lives in VGPRs in the same dimension order.
//  * Scores x token scale x softmax scale x log2(e); online softmax in the
//    base-2 domain with a lazy rescale (the reference max moves only when a
//    score exceeds it by 2^8). Lane (g, n) holds tokens 4g .. 4g + 3 of head
//    n, which is exactly the B operand layout of v_mfma_f32_16x16x16 with
//    k = token: the probabilities (times the token scale, rounded to bf16)
//    feed the value product without leaving the registers.
//  * O^T += V^T . P^T (dims x heads): V^T from ds_read_b64_tr_b8, whose 16
//    lanes of a group fetch 8 byte rows and return one column each: rows
//    0-3 = tokens 4g .. 4g + 3 of dim block 2u, rows 4-7 the same tokens of
//    block 2u + 1, so one read feeds two MFMAs.
//  * At the end of a segment the four waves' running max, sum and O^T are
//    merged through LDS and written as the output row (+ lse) or as a
//    partial (+ base-2 lse), like the bf16 kernel.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include "cdna.h"
#include "decode_common.h"
#include "group16.h"
#include "triton_mla.h"

namespace tmla {

namespace f8 {

constexpr int kSlice = 16;               // tokens per wave per 64-token tile
constexpr int kHeads = 16;               // heads per workgroup: N of the MFMAs
constexpr int kRow = 576;                // bytes per cache row (512 latent + 64 rope dims)
constexpr int kKv = kSlice * kRow;       // 9216 bytes of rows per ring entry
constexpr int kEntry = kKv + 256;        // + token scales (64 lanes x 4 bytes, first 16 used)
constexpr int kOPitch = 512 * 4 + 16;    // merge staging: one fp32 row of a head, padded
constexpr int kLoads = kKv / 1024 + 1;   // LDS-DMA instructions per slice (rows, scales)

// Launch shape: NW waves (4: one per SIMD; 8: two per SIMD, so that one
// wave's MFMAs run under the other's VALU work), each with a ring of
// STAGES entries; K operand reads KA and V^T reads VA ahead of their use
// (fewer with two waves per SIMD, where registers are halved).
template <int NW>
struct F8Shape {
  static_assert(NW == 4 || NW == 8, "waves per workgroup");
  static constexpr int kStages = NW == 4 ? 4 : 2;
  static constexpr int kTileStride = NW / 4;  // tiles between a wave's slices
  static constexpr int KA = NW == 4 ? 9 : 3;
  static constexpr int VA = NW == 4 ? 16 : 6;
  static constexpr int kRing = kStages * kEntry;
  static constexpr int kStats = NW * kRing;  // per-wave max and sum of every head
  static constexpr int kSmem = kStats + 2 * NW * kHeads * 4;
  static_assert(4 * kHeads * kOPitch <= kStats, "merge staging fits the rings");
  static_assert(kSmem <= 160 * 1024, "LDS");
  static_assert((kStages - 1) * kLoads < 64, "vmcnt range");
};

using namespace grp;

// Element type of q and out: the widening of fp8 pairs (exact: every e4m3
// value is a bf16 and an fp16 value), the two MFMAs and the rounding of the
// probabilities.
//
// MFMA forms: written as asm with the accumulator tied in place (S^T in
// VGPRs, O^T in AGPRs), so that no accumulator is ever copied between
// registers, and volatile, so that they keep their places among the LDS
// reads and waits. The compiler cannot see the hazards of asm, so each MFMA
// carries the two wait states a VALU result needs before an MFMA reads it
// (its operands are widened by VALU just before), and mfma_fence waits out
// the MFMA result latency before VALU code reads an accumulator. Dependent
// MFMAs on one accumulator need no wait states.
template <int DT>
struct F8Elt;
template <>
struct F8Elt<TMLA_BF16> {
  typedef bf16x8 v8;
  typedef bf16x4 v4;
  template <bool HI>
  __device__ static __forceinline__ bf16x2 widen(int x) {
    return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(x, 1.0f, HI);
  }
  // (asm: see the note on MFMA forms below)
  __device__ static __forceinline__ void mfma_qk_first(f32x4& d, const v8& k, const v8& q) {
    asm volatile("s_nop 1\n\tv_mfma_f32_16x16x32_bf16 %0, %1, %2, 0" : "=&v"(d) : "v"(k), "v"(q));
  }
  __device__ static __forceinline__ void mfma_qk(f32x4& d, const v8& k, const v8& q) {
    asm volatile("s_nop 1\n\tv_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(k), "v"(q));
  }
  __device__ static __forceinline__ void mfma_pv(f32x4& acc, const v4& v, const v4& p) {
    asm volatile("s_nop 1\n\tv_mfma_f32_16x16x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(v), "v"(p));
  }
  __device__ static __forceinline__ __bf16 round(float x) { return (__bf16)x; }
};
template <>
struct F8Elt<TMLA_FP16> {
  typedef f16x8 v8;
  typedef f16x4 v4;
  template <bool HI>
  __device__ static __forceinline__ f16x2 widen(int x) {
    return __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x, 1.0f, HI);
  }
  __device__ static __forceinline__ void mfma_qk_first(f32x4& d, const v8& k, const v8& q) {
    asm volatile("s_nop 1\n\tv_mfma_f32_16x16x32_f16 %0, %1, %2, 0" : "=&v"(d) : "v"(k), "v"(q));
  }
  __device__ static __forceinline__ void mfma_qk(f32x4& d, const v8& k, const v8& q) {
    asm volatile("s_nop 1\n\tv_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(d) : "v"(k), "v"(q));
  }
  __device__ static __forceinline__ void mfma_pv(f32x4& acc, const v4& v, const v4& p) {
    asm volatile("s_nop 1\n\tv_mfma_f32_16x16x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(v), "v"(p));
  }
  __device__ static __forceinline__ _Float16 round(float x) { return (_Float16)x; }
};

// 8 fp8 bytes (two dwords) -> one 8-element K operand
template <int DT>
__device__ __forceinline__ typename F8Elt<DT>::v8 widen8(int x, int y) {
  using E = F8Elt<DT>;
  const auto a0 = E::template widen<false>(x), a1 = E::template widen<true>(x);
  const auto b0 = E::template widen<false>(y), b1 = E::template widen<true>(y);
  return typename E::v8{a0[0], a0[1], a1[0], a1[1], b0[0], b0[1], b1[0], b1[1]};
}
// 4 fp8 bytes -> one 4-element operand
template <int DT>
__device__ __forceinline__ typename F8Elt<DT>::v4 widen4(int x) {
  using E = F8Elt<DT>;
  const auto a = E::template widen<false>(x), b = E::template widen<true>(x);
  return typename E::v4{a[0], a[1], b[0], b[1]};
}

// vmcnt: the copies of up to `pending` younger slices may stay in flight
template <int MAXP>
__device__ __forceinline__ void wait_slices(int pending) {
  if (MAXP >= 3 && pending >= 3)
    wait_vmcnt<3 * kLoads>();
  else if (MAXP >= 2 && pending >= 2)
    wait_vmcnt<2 * kLoads>();
  else if (pending >= 1)
    wait_vmcnt<kLoads>();
  else
    wait_vmcnt<0>();
}

}  // namespace f8

// PAGED: block table (pages of a multiple of 16 tokens); else a dense
// [batch, capacity, 576] cache. NW: waves per workgroup (F8Shape).
template <int DT, bool PAGED, int NW>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * NW, 64 * NW), amdgpu_waves_per_eu(NW / 4, NW / 4)))
void mla_partial_fp8_kernel(PartialArgs a) {
  using namespace f8;
  using E = F8Elt<DT>;
  using SH = F8Shape<NW>;
  constexpr int kStages = SH::kStages;
  constexpr int LEAD = kStages - 1;  // slices in flight ahead of the one computed
  constexpr int KA = SH::KA, VA = SH::VA;
  __shared__ __attribute__((aligned(1024))) char smem[SH::kSmem];
  char LDS_AS* const lds = (char LDS_AS*)(void LDS_AS*)smem;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int sw = wave & 3;                   // slice of the tile: tokens 16 sw .. 16 sw + 15
  const int par = wave >> 2;                 // first tile of the wave (NW = 8: tile parity)
  const int worker = worker_index(a);
  WorkRange wr;
  if (!work_range(a, worker, wr) || wr.tile_lo >= wr.tile_hi) return;
  const int head0 = blockIdx.y * kHeads;
  const int nh = min(kHeads, a.num_heads - head0);
  char LDS_AS* const ring = lds + wave * SH::kRing;

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

    const int lane = lane_id_fresh();
    const int g = lane >> 4, r = lane & 15;
    const int head = head0 + r;
    const bool head_ok = r < nh;
    // tokens [0, limit) are visible to this lane's head
    const int limit = n_b - causal_lag(a, head);

    // Q^T: operand 2j + h of lane (g, n) = dims 64j + 16g + 8h .. + 7 of head n
    typename E::v8 qop[18];
    {
      const char* qrow = a.q + ((int64_t)b * a.q_sb + (int64_t)min(head, a.num_heads - 1) * a.q_sh) * 2 + g * 32;
#pragma unroll
      for (int j = 0; j < 9; ++j) {
        const i32x4 v0 = head_ok ? *reinterpret_cast<const i32x4*>(qrow + j * 128) : i32x4{0, 0, 0, 0};
        const i32x4 v1 = head_ok ? *reinterpret_cast<const i32x4*>(qrow + j * 128 + 16) : i32x4{0, 0, 0, 0};
        qop[2 * j] = __builtin_bit_cast(typename E::v8, v0);
        qop[2 * j + 1] = __builtin_bit_cast(typename E::v8, v1);
      }
    }

    // this wave's slices: tiles t_start + par, + NW / 4, ... below t_end, the
    // last one only when its slice holds a token
    constexpr int TS = SH::kTileStride;
    const int tiles_w = t_end - t_start - par > 0 ? (t_end - t_start - par + TS - 1) / TS : 0;
    const int ns = tiles_w - (tiles_w > 0 && kTileTokens * (t_start + par + TS * (tiles_w - 1)) + kSlice * sw >= n_b ? 1 : 0);
    auto slice_tok = [&](int k) __attribute__((always_inline)) {
      return kTileTokens * (t_start + par + TS * k) + kSlice * sw;
    };
    const int32_t* bt_row = PAGED ? a.bt + (int64_t)b * a.bt_sb : a.bt;
    auto page_fetch = [&](int k) __attribute__((always_inline)) -> int {
      return PAGED ? s_load_i32(bt_row + page_slot_of(a, slice_tok(k))) : 0;
    };
    auto clamp_page = [&](int v) __attribute__((always_inline)) -> int { return v < 0 ? 0 : min(v, a.max_page); };
    // DMA lane role: row r (clamped to the sequence's last token), chunk
    // column g (+ 4j for copy j)
    auto issue = [&](int k, int page) __attribute__((always_inline)) {
      const int t0 = slice_tok(k);
      const int rr = min(r, n_b - 1 - t0);
      int64_t row;
      int64_t sidx;
      if constexpr (PAGED) {
        const int in_page = a.page_shift >= 0 ? (t0 & (a.page_size - 1)) : (t0 % a.page_size);
        row = (int64_t)page * a.kv_s0 + (int64_t)(in_page + rr) * a.kv_s1;
        sidx = (int64_t)page * a.sc_s0 + (int64_t)(in_page + rr) * a.sc_s1;
      } else {
        const int t = min(t0 + rr, (int)(a.num_blocks - 1));
        row = (int64_t)b * a.kv_s0 + (int64_t)t * a.kv_s1;
        sidx = (int64_t)b * a.sc_s0 + (int64_t)t * a.sc_s1;
      }
      const char* src = a.kv + row + g * 16;
      char LDS_AS* dst = ring + (k % kStages) * kEntry;
      static_for<kKv / 1024>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        lds_copy16<64 * j>(src, dst + 1024 * j);
      });
      __builtin_amdgcn_global_load_lds(a.kv_scale + sidx, (void LDS_AS*)(dst + kKv), 4, 0, 0);
    };

    f32x4 o[32];
#pragma unroll
    for (int d = 0; d < 32; ++d) {
      o[d] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      pin_acc(o[d]);
    }
    // base-2 reference max of the lane's head (kNoMax until it has seen a
    // token, so that p = 2^(x - m) of a masked score is 0 even then) and the
    // sum of p over the lane's tokens
    float m_ref = kNoMax;
    float l_run = 0.0f;
    // V^T reads: lane i of group g fetches byte row j = i / 2, half i % 2 =
    // token 4g + j % 4 of chunk column 2u + j / 4
    const int tr_off = (((r >> 1) >> 2) * 16 + 4 * g + ((r >> 1) & 3)) * 16 + 8 * (r & 1);

    // Prologue: slices 0 .. LEAD - 1 in flight, page ids of slices LEAD and
    // LEAD + 1 requested. Page ids come from scalar loads without a wait;
    // every wait for them is an lgkmcnt(0) that names all ids still in
    // flight, so none is read or moved before it has arrived.
    int pg_a = 0, pg_b = 0;  // page ids of slices k + LEAD and k + LEAD + 1
    {
      int p[LEAD];
#pragma unroll
      for (int i = 0; i < LEAD; ++i) p[i] = ns > i ? page_fetch(i) : 0;
      pg_a = ns > LEAD ? page_fetch(LEAD) : 0;
      pg_b = ns > LEAD + 1 ? page_fetch(LEAD + 1) : 0;
      if (PAGED) {
        asm volatile("s_waitcnt lgkmcnt(0)" : "+s"(pg_a), "+s"(pg_b));
#pragma unroll
        for (int i = 0; i < LEAD; ++i) asm volatile("" : "+s"(p[i]));
      }
#pragma unroll
      for (int i = 0; i < LEAD; ++i)
        if (ns > i) issue(i, clamp_page(p[i]));
    }
    // Q^T has arrived once the copies of the first slices are the only loads
    // in flight; from here on the compiler sees it as plain registers (no
    // load wait of its own inside the loop)
    wait_slices<LEAD>(min(LEAD, ns));
#pragma unroll
    for (int j = 0; j < 18; ++j) pin_v(qop[j]);

    for (int k = 0; k < ns; ++k) {
      // the copies of slice k + LEAD go into the entry slice k - 1 has left
      if (k + LEAD < ns) {
        if (PAGED) asm volatile("s_waitcnt lgkmcnt(0)" : "+s"(pg_a), "+s"(pg_b));
        const int pcur = clamp_page(pg_a);
        pg_a = pg_b;
        issue(k + LEAD, pcur);
      }
      wait_slices<LEAD>(min(LEAD, ns - 1 - k));
      const char LDS_AS* ent = ring + (k % kStages) * kEntry;
      const int t0 = slice_tok(k);

      // ---- S^T = K . Q^T ----------------------------------------------------
      // LDS operations in program order: token scales, K operands 0 .. KA - 1,
      // then K operand j + KA after step j; the wait of step j counts the K
      // reads younger than operand j. Each operand is widened right after the
      // MFMA before it has issued (the scheduling barriers keep this order).
      f32x4 tsc = __builtin_bit_cast(f32x4, ds_read_x4<kKv>(ent + 16 * g));
      const char LDS_AS* kp = ent + 16 * lane;
      const char LDS_AS* vp = ent + tr_off;
      i32x4 kr[9];
      static_for<KA>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        kr[j] = ds_read_x4<1024 * j>(kp);
      });
      f32x4 s;
      static_for<9>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        constexpr int younger = (KA - 1 < 8 - j) ? KA - 1 : 8 - j;
        lgkm_tie<younger>(kr[j]);
        if constexpr (j == 0) pin_v(tsc);  // older than K operand 0: complete
        const typename E::v8 k0 = widen8<DT>(kr[j][0], kr[j][1]);
        if constexpr (j == 0)
          E::mfma_qk_first(s, k0, qop[0]);
        else
          E::mfma_qk(s, k0, qop[2 * j]);
        __builtin_amdgcn_sched_barrier(0);
        const typename E::v8 k1 = widen8<DT>(kr[j][2], kr[j][3]);
        E::mfma_qk(s, k1, qop[2 * j + 1]);
        if constexpr (j + KA < 9) kr[j + KA] = ds_read_x4<1024 * (j + KA)>(kp);
        __builtin_amdgcn_sched_barrier(0);
      });
      // V^T reads 0 .. VA - 1 now, the rest one per value step
      i32x2 vr[16];
      static_for<VA>([&](auto uc) {
        constexpr int u = decltype(uc)::value;
        vr[u] = ds_read_tr8<512 * u>(vp);
      });

      // ---- online softmax (base 2) ---------------------------------------
      mfma_fence(s);
      float x[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        x[i] = t0 + 4 * g + i < limit ? s[i] * (tsc[i] * a.qk_scale_log2) : -INFINITY;
      const float mx = rows_max(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])));
      if (__ballot(mx > m_ref + kRescaleLog2) != 0) {
        const float m_new = mx > m_ref + kRescaleLog2 ? mx : m_ref;
        const float alpha = fast_exp2(m_ref - m_new);  // 0 from kNoMax, 1 where unchanged
        l_run *= alpha;
#pragma unroll
        for (int d = 0; d < 32; ++d) scale_acc(o[d], alpha);
        m_ref = m_new;
      }
#pragma unroll
      for (int d = 0; d < 32; ++d) pin_acc(o[d]);
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) p[i] = fast_exp2(x[i] - m_ref);
      l_run += (p[0] + p[1]) + (p[2] + p[3]);
      const typename E::v4 pb{E::round(p[0] * tsc[0]), E::round(p[1] * tsc[1]), E::round(p[2] * tsc[2]),
                              E::round(p[3] * tsc[3])};
      // the page id of slice k + LEAD + 2 is requested here, long before the
      // wait for it (top of iteration k + 2)
      if (k + LEAD + 2 < ns) pg_b = page_fetch(k + LEAD + 2);
      __builtin_amdgcn_sched_barrier(0);

      // ---- O^T += V^T . P^T ------------------------------------------------
      // V^T read u + VA is issued once read u has been awaited: the wait of
      // step u counts the VA - 1 reads after it (fewer at the end)
      static_for<16>([&](auto uc) {
        constexpr int u = decltype(uc)::value;
        constexpr int younger = (VA - 1 < 15 - u) ? VA - 1 : 15 - u;
        lgkm_tie<younger>(vr[u]);
        if constexpr (u + VA < 16) vr[u + VA] = ds_read_tr8<512 * (u + VA)>(vp);
        E::mfma_pv(o[2 * u], widen4<DT>(vr[u][0]), pb);
        __builtin_amdgcn_sched_barrier(0);
        E::mfma_pv(o[2 * u + 1], widen4<DT>(vr[u][1]), pb);
        __builtin_amdgcn_sched_barrier(0);
      });
#pragma unroll
      for (int j = 0; j < 18; ++j) pin_v(qop[j]);
    }

    // ---- merge the waves and store -------------------------------------------
    mfma_fence_a(o[31]);  // the last value products have landed
    {
      const float l_tot = rows_sum(l_run);
      float LDS_AS* stats = reinterpret_cast<float LDS_AS*>(lds + SH::kStats);  // [2][wave][head]
      if (g == 0) {
        stats[wave * kHeads + r] = m_ref;
        stats[NW * kHeads + wave * kHeads + r] = l_tot;
      }
      __syncthreads();  // every wave is past its loop: the rings are free
      float M = kNoMax;
#pragma unroll
      for (int w = 0; w < NW; ++w) M = fmaxf(M, stats[w * kHeads + r]);
      float L = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) L += fast_exp2(stats[w * kHeads + r] - M) * stats[NW * kHeads + w * kHeads + r];
      const bool has = L > 0.0f;
      const float f = has ? fast_exp2(m_ref - M) / L : 0.0f;
      // staging region q of 4 holds one normalised O^T share: row = head,
      // column = dim; with eight waves, wave q + 4 first hands its share to
      // wave q through region q
      char LDS_AS* stage = lds + (wave & 3) * kHeads * kOPitch + r * kOPitch + 16 * g;
      if constexpr (NW == 8) {
        if (wave >= 4) {
#pragma unroll
          for (int d = 0; d < 32; ++d) *reinterpret_cast<f32x4 LDS_AS*>(stage + 64 * d) = o[d] * f;
        }
        __syncthreads();
        if (wave < 4) {
#pragma unroll
          for (int d = 0; d < 32; ++d) o[d] = o[d] * f + *reinterpret_cast<const f32x4 LDS_AS*>(stage + 64 * d);
        }
        __syncthreads();
        if (wave < 4) {
#pragma unroll
          for (int d = 0; d < 32; ++d) *reinterpret_cast<f32x4 LDS_AS*>(stage + 64 * d) = o[d];
        }
      } else {
#pragma unroll
        for (int d = 0; d < 32; ++d) *reinterpret_cast<f32x4 LDS_AS*>(stage + 64 * d) = o[d] * f;
      }
      __syncthreads();
      // wave w writes heads w * 16 / NW ..: lane l dims 8l .. 8l + 7
      constexpr int HPW = kHeads / NW;
#pragma unroll
      for (int hh = 0; hh < HPW; ++hh) {
        const int hr = HPW * wave + hh;
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
        }
        else
          store_through_f32(a.mid_lse + (int64_t)ss.slot * a.num_heads + head, lse2);
      }
      __syncthreads();  // the staging is read before the next segment's copies land
    }

    remaining -= t_end - t_start + wr.seg_cost;  // the next sequence's start is charged here
    seg_global_off += nt_b + wr.seg_cost;
    ++b;
    t_start = 0;
  }
}

// Waves per workgroup (build-time knob, F8Shape): 4 by default. The
// two-waves-per-SIMD form hides one wave's MFMAs under the other's VALU
// work, but its two-entry rings leave one slice in flight per wave, and on
// the 16-head ragged workload it measured 130.5 us against 114.4 us.
#ifndef TMLA_FP8_WAVES
#define TMLA_FP8_WAVES 4
#endif

template <int DT, bool PAGED>
hipError_t launch_fp8_t(const PartialArgs& a, dim3 grid, hipStream_t stream) {
  constexpr int NW = TMLA_FP8_WAVES;
  hipLaunchKernelGGL((mla_partial_fp8_kernel<DT, PAGED, NW>), grid, dim3(64 * NW), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_partial_fp8(const PartialArgs& a, dim3 grid, int dtype, bool paged, hipStream_t stream) {
  if (dtype == TMLA_BF16)
    return paged ? launch_fp8_t<TMLA_BF16, true>(a, grid, stream) : launch_fp8_t<TMLA_BF16, false>(a, grid, stream);
  return paged ? launch_fp8_t<TMLA_FP16, true>(a, grid, stream) : launch_fp8_t<TMLA_FP16, false>(a, grid, stream);
}

}  // namespace tmla
