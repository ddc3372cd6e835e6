// Pieces shared by the decode partial kernels (bf16/fp16 cache in
// mla_decode.hip, fp8 cache in mla_decode_fp8.hip): the launch arguments, the
// split-KV work partition (which worker owns which 64-token tiles, and where
// its result goes), page-table helpers and a few device utilities.
//
// Reference behaviour: the split ranges of src/triton_mla/kernel.py:83-86
// (uniform num_splits) and the stage-1 outputs of kernel.py:130-138.
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "cdna.h"
#include "host_plan.h"

namespace tmla {

constexpr float kRescaleLog2 = 8.0f;    // lazy rescale threshold (p <= 2^8)
constexpr float kNoMax = -__FLT_MAX__;  // running max of a head that has seen no token
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kLog2e = 1.4426950408889634f;

struct PartialArgs {
  const char* q;           // element pointer (bytes)
  int64_t q_sb, q_sh;      // element strides
  const char* kv;
  int64_t kv_s0, kv_s1;    // byte strides: block (dense: batch), token
  int64_t num_blocks;
  int32_t max_page;               // min(num_blocks - 1, INT32_MAX): page ids are clamped to it
  int32_t page_size, page_shift;  // page_shift = log2(page_size) or -1
  const int32_t* bt;
  int64_t bt_sb;
  int32_t bt_cols;
  const int32_t* seqlens;
  int32_t batch, num_heads;
  // Multi-token queries: head index v = t * heads_per_token + h for query
  // token t < q_len, which sees the first seqlen - (q_len - 1 - t) tokens
  // (q_len = 1: single-token decode, every head sees seqlen tokens).
  int32_t q_len, heads_per_token;
  float qk_scale_log2;
  int32_t num_splits, num_workers;
  int32_t xcds;            // workgroups are dealt round-robin over this many L2 domains
  char* out;
  int64_t out_sb, out_sh;  // element strides
  float* lse;
  short* mid_o;            // [slots, H, DV] normalised partials, input dtype
  float* mid_lse;          // [slots, H], base-2
  // In-kernel merge (fused): the workers of a split sequence each merge one
  // share of its heads once all of them have stored their partials.
  int32_t fused;
  int32_t spin_limit;      // polls before a waiting worker hands its share over
  int32_t* m_count;        // [batch, head blocks] partials stored
  int32_t* m_done;         // [batch, head blocks] shares merged
  int32_t* m_flag;         // [slots, head blocks] 0 owner merges, 1 handed over, 2 taken over
  int32_t mid_o_bytes;     // bytes of the partial rows (< 2^31 when fused)
  // fp8 cache only: dequantised row value = e4m3(byte) * kv_scale[page *
  // sc_s0 + row_in_page * sc_s1] (dense caches: sequence instead of page)
  const float* kv_scale;
  int64_t sc_s0, sc_s1;    // element strides
};

// ---------------------------------------------------------------------------
// small device helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ int tiles_of(int n) { return n > 0 ? (n + kTileTokens - 1) / kTileTokens : 0; }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// Keeps an int in a VGPR at this point (vector address arithmetic instead of
// one scalar register pair per use).
__device__ __forceinline__ void pin_i1(int& a) { asm volatile("" : "+v"(a)); }

// The lane id through an instruction the compiler cannot look through:
// offsets derived from it are recomputed where they are needed instead of
// being kept live across the whole kernel (where they would be spilled to
// scratch and reloaded, one memory round trip each, at start-up and in the
// finalize).
__device__ __forceinline__ int lane_id_fresh() {
  int v;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(v));
  return v;
}

// Tokens at the end of the sequence that query head `head` does not see:
// q_len - 1 - t for the head's query token t (0 for single-token decode).
__device__ __forceinline__ int causal_lag(const PartialArgs& a, int head) {
  return a.q_len <= 1 ? 0 : a.q_len - 1 - min(head, a.num_heads - 1) / a.heads_per_token;
}

// A uniform value the compiler must treat as new at this point: divisions by
// it are not hoisted out of the enclosing loop (their reciprocal would occupy
// a VGPR for the whole loop).
__device__ __forceinline__ int fresh_s(int x) {
  asm volatile("" : "+s"(x));
  return x;
}

// Scalar load of one int (uniform address) with no wait; s_wait_i32 waits
// for every outstanding LDS/scalar operation and ties the value to that point.
// Issued only where no LDS read that a later lgkmcnt count relies on is
// older than it, so the out-of-order scalar return cannot satisfy such a wait
// early.
__device__ __forceinline__ int s_load_i32(const int32_t* p) {
  int r;
  asm volatile("s_load_dword %0, %1, 0x0" : "=s"(r) : "s"(p));
  return r;
}
__device__ __forceinline__ float s_load_f32(const float* p) {
  return __builtin_bit_cast(float, s_load_i32(reinterpret_cast<const int32_t*>(p)));
}
__device__ __forceinline__ int s_wait_i32(int v) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+s"(v));
  return v;
}

// 16-byte store written through to memory (sc0 sc1: system-scope write-
// through), so a kernel that ends with many such stores leaves no dirty L2
// lines for the end-of-kernel write-back. The s_nop supplies the wait state
// the hardware needs before a VALU instruction may overwrite the data VGPRs
// of a store wider than 64 bits: the compiler inserts it for the stores it
// generates, but cannot see into this asm.
__device__ __forceinline__ void store_through(i16x8* p, i16x8 v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc0 sc1\n\ts_nop 1" : : "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store_through_f32(float* p, float v) {
  asm volatile("global_store_dword %0, %1, off sc0 sc1" : : "v"(p), "v"(v) : "memory");
}

// POW2: the page size is known to be a power of two (page_shift >= 0)
template <bool POW2 = false>
__device__ __forceinline__ int page_slot_of(const PartialArgs& a, int t) {
  const int s = (POW2 || a.page_shift >= 0) ? (t >> a.page_shift) : (t / a.page_size);
  return min(s, a.bt_cols - 1);
}

__device__ __forceinline__ int load_page(const PartialArgs& a, int b, int slot) {
  int p = a.bt[(int64_t)b * a.bt_sb + slot];
  p = p < 0 ? 0 : p;
  return min(p, a.max_page);
}

// ---------------------------------------------------------------------------
// Work partition
// ---------------------------------------------------------------------------

// Worker index of this workgroup: consecutive workers (the pieces of one
// sequence, which share its Q rows and write neighbouring partial slots) are
// placed on the same XCD, since the dispatcher deals workgroups round-robin
// over the XCDs and each XCD has its own L2.
__device__ __forceinline__ int worker_index(const PartialArgs& a) {
  const int nwg = gridDim.x;
  return (a.xcds > 1 && nwg % a.xcds == 0) ? (int)(blockIdx.x % a.xcds) * (nwg / a.xcds) + (int)(blockIdx.x / a.xcds)
                                           : (int)blockIdx.x;
}

// A worker's range: tiles [tile_lo, tile_hi) counted from the start of
// sequence b_first (whose length is n_first; in balanced mode the range may
// run on into the following sequences), off_first = the position of b_first's
// first tile on the partition's line, chunk = positions per worker
// (balanced), snapped = one piece of one sequence per worker (balanced),
// seg_cost = positions charged for each following sequence's start
// (straddling ranges; 0 otherwise).
struct WorkRange {
  int b_first, tile_lo, tile_hi, off_first, n_first, chunk, seg_cost;
  bool snapped;
};

// Returns false when the worker has no tiles (balanced mode only). Every
// wave computes the same range on its own (registers and cross-lane moves
// only, no LDS or barrier).
__device__ __forceinline__ bool work_range(const PartialArgs& a, int worker, WorkRange& w) {
  w.chunk = 0;
  w.seg_cost = 0;
  w.snapped = false;
  if (a.num_splits > 0) {
    // uniform: sequence b is cut into num_splits pieces of cdiv(tiles, S)
    // tiles (kernel.py:83-86); worker b * S + s takes piece s
    const int S = a.num_splits;
    const int b = worker / S, s = worker - b * S;
    w.n_first = a.seqlens[b];
    const int nt = tiles_of(w.n_first);
    const int spt = (nt + S - 1) / S;
    w.tile_lo = s * spt;
    w.tile_hi = min(w.tile_lo + spt, nt);
    w.b_first = b;
    w.off_first = 0;
    return true;
  }
  // Balanced: the T tiles of all sequences are shared by num_workers
  // workers, c = cdiv(T, num_workers) tiles each, as one piece of one
  // sequence per worker (snapped) or as ranges that run across sequences
  // (straddling). Lane l sums the tile counts of sequences
  // [l * per, (l + 1) * per), a wave-wide inclusive scan gives each lane the
  // tile offset where its sequences end.
  const int lane0 = lane_id_fresh();
  const int per = (a.batch + 63) >> 6;
  const int lo_b = min(lane0 * per, a.batch), hi_b = min(lo_b + per, a.batch);
  const int len0 = lo_b < hi_b ? a.seqlens[lo_b] : 0;
  int sum = tiles_of(len0), live = len0 > 0;
  for (int b = lo_b + 1; b < hi_b; ++b) {
    const int nt = tiles_of(a.seqlens[b]);
    sum += nt;
    live += nt > 0;
  }
  int incl = sum;
  int vsum = sum + kSegCostTiles * live, vincl = vsum;  // positions on the straddling line
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int v = __shfl_up(incl, d), vv = __shfl_up(vincl, d);
    if (lane0 >= d) {
      incl += v;
      vincl += vv;
    }
  }
  const int total = __builtin_amdgcn_readlane(incl, 63);
  const int chunk = (total + a.num_workers - 1) / a.num_workers;
  w.chunk = chunk;
  // Snapped ranges: when every sequence cut into pieces of at most c tiles
  // gives no more pieces than workers, worker w takes piece w instead (the
  // pieces of each sequence in order, piece j = tiles [j c, (j + 1) c)).
  // The longest range is still c tiles, and no worker pays a second
  // start-up and finalize for a range that straddles two sequences.
  int pcs = 0, pinc = 0;
  bool snapped = false;
  if (chunk > 0) {
    pcs = (tiles_of(len0) + chunk - 1) / chunk;  // len0 = 0 for a lane without sequences
    for (int b = lo_b + 1; b < hi_b; ++b) pcs += (tiles_of(a.seqlens[b]) + chunk - 1) / chunk;
    pinc = pcs;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int v = __shfl_up(pinc, d);
      if (lane0 >= d) pinc += v;
    }
    snapped = __builtin_amdgcn_readlane(pinc, 63) <= a.num_workers;
  }
  w.snapped = snapped;
  if (snapped && worker < __builtin_amdgcn_readlane(pinc, 63)) {
    // the one lane whose sequences hold piece `worker` finds which of them
    int poff = pinc - pcs, off = incl - sum, fb = lo_b, flen = len0;
    for (int b = lo_b; b < hi_b; ++b) {
      const int len = b == lo_b ? len0 : a.seqlens[b];
      const int nt = tiles_of(len);
      const int np = (nt + chunk - 1) / chunk;
      fb = b;
      flen = len;
      if (worker < poff + np) break;
      poff += np;
      off += nt;
    }
    const int src = __builtin_ctzll(__ballot(pcs > 0 && pinc - pcs <= worker && worker < pinc));
    w.b_first = __builtin_amdgcn_readlane(fb, src);
    w.off_first = __builtin_amdgcn_readlane(off, src);
    w.n_first = __builtin_amdgcn_readlane(flen, src);
    w.tile_lo = (worker - __builtin_amdgcn_readlane(poff, src)) * chunk;  // local to b_first
    w.tile_hi = min(w.tile_lo + chunk, tiles_of(w.n_first));
    return true;
  }
  // Straddling ranges: the sequences' tiles in order on a line where each
  // non-empty sequence starts with kSegCostTiles extra positions (what a
  // segment's start-up and finalize cost, in tiles), cut into num_workers
  // ranges of vc = cdiv(VT, num_workers) positions (VT = the line's length).
  // Tile j of sequence b sits at position voff_b + kSegCostTiles + j, so a
  // range that holds the starts of further sequences holds fewer tiles.
  const int vtotal = __builtin_amdgcn_readlane(vincl, 63);
  const int vchunk = (vtotal + a.num_workers - 1) / a.num_workers;
  const int vlo = worker * vchunk;
  if (snapped || vlo >= vtotal) {  // wave-uniform, and the same in every wave
    w.b_first = w.off_first = w.n_first = w.tile_lo = w.tile_hi = 0;
    return false;
  }
  w.chunk = vchunk;
  w.seg_cost = kSegCostTiles;
  // the one lane whose sequences hold position vlo finds which of them it is
  int voff = vincl - vsum, fb = lo_b, flen = len0;
  for (int b = lo_b; b < hi_b; ++b) {
    const int len = b == lo_b ? len0 : a.seqlens[b];
    const int nt = tiles_of(len);
    const int vt = nt > 0 ? nt + kSegCostTiles : 0;
    fb = b;
    flen = len;
    if (vlo < voff + vt) break;
    voff += vt;
  }
  const int src = __builtin_ctzll(__ballot(vsum > 0 && vincl - vsum <= vlo && vlo < vincl));
  w.b_first = __builtin_amdgcn_readlane(fb, src);
  w.off_first = __builtin_amdgcn_readlane(voff, src) + kSegCostTiles;  // position of b_first's tile 0
  w.n_first = __builtin_amdgcn_readlane(flen, src);
  // local to b_first; tile_hi may run past b_first, and is <= tile_lo when the
  // range holds no tile at all (only positions of b_first's start)
  w.tile_lo = max(vlo - w.off_first, 0);
  w.tile_hi = min(vlo + vchunk, vtotal) - w.off_first;
  return true;
}

// Where the result of one segment (tiles [t_start, ...) of sequence b, which
// has nt_b tiles and starts at global tile seg_global_off) goes: partial slot
// `slot`, or straight to out/lse when this worker covers the whole sequence
// (`direct`). `index` is the worker's position among the `count` workers of
// b, whose partials occupy slots first_slot, first_slot + 1, ...
struct SegmentSlot {
  int slot, index, count, first_slot;
  bool direct;
};

__device__ __forceinline__ SegmentSlot segment_slot(const PartialArgs& a, const WorkRange& w, int worker, int b,
                                                    int t_start, int nt_b, int seg_global_off) {
  SegmentSlot s;
  if (a.num_splits > 0) {
    const int S = a.num_splits;
    const int spt = (nt_b + S - 1) / S;
    s.count = (nt_b + spt - 1) / spt;
    s.index = t_start / spt;
    s.slot = b * S + s.index;
    s.first_slot = b * S;
  } else {
    const int ch = fresh_s(w.chunk);
    // the workers of b: g1..g2 (straddling ranges: seg_global_off = the
    // position of b's tile 0) or g1 = worker - j .. g1 + pieces - 1
    // (snapped: this is piece j = t_start / c of b)
    const int g1 = w.snapped ? worker - t_start / ch : seg_global_off / ch;
    const int g2 = w.snapped ? g1 + (nt_b + ch - 1) / ch - 1 : (seg_global_off + nt_b - 1) / ch;
    s.slot = worker + b;
    s.index = worker - g1;
    s.count = g2 - g1 + 1;
    s.first_slot = g1 + b;
  }
  s.direct = s.count == 1;
  return s;
}

// Stage 1 over an fp8 cache (mla_decode_fp8.hip): grid = (workers, head
// groups of 16); dtype is the element type of q and out.
hipError_t launch_partial_fp8(const PartialArgs& a, dim3 grid, int dtype, bool paged, hipStream_t stream);

// Stage 1 over a 16-bit cache with at most 16 heads per workgroup
// (mla_decode_g16.hip): grid = (workers, head groups of 16).
hipError_t launch_partial_g16(const PartialArgs& a, dim3 grid, int dtype, bool paged, hipStream_t stream);

}  // namespace tmla
