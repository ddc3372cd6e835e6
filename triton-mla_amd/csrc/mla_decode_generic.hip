// Decode for the head dims and element types that the matrix-core kernels
// are not built for: any power-of-two head_dim_v in [16, 1024] and rope_dim
// in [16, 256], bf16, fp16 or fp32. It runs the reference's two stages the
// reference's way (src/triton_mla/kernel.py:43-181): sequence b is cut into
// num_splits pieces of cdiv(seqlens[b], num_splits) tokens (kernel.py:84-86);
// a workgroup per (group of heads, piece, sequence) writes a float32
// partial and its base-2 log-sum-exp (kernel.py:88-138); a second kernel
// merges the pieces (kernel.py:141-181).
//
// Stage 1 (mla_generic_partial_kernel), 256 threads = 4 waves of 4 heads:
//   * Q of the 16 heads is staged once in LDS as float, times
//     softmax_scale * log2(e), so scores are base-2 exponents;
//   * per step, `tile` cache rows (a power of two <= 64, as many as the LDS
//     form holds) are copied into LDS with 16-byte loads, eight per thread
//     in flight (element loads when the cache rows are not 16-byte aligned),
//     rows past the piece zeroed;
//   * scores: lane l takes token l % tile and every (64 / tile)-th group of 8
//     dims from group l / tile on, accumulates the partial dot products of
//     its wave's 4 heads, and the lanes of a token add theirs (xor shuffles);
//   * online softmax per head, the wave's state held uniformly by its lanes:
//     m = max(m, tile max), alpha = exp2(m_old - m), l = l * alpha + sum p;
//     the accumulators are scaled by alpha; p rounded to the element type is
//     stored in LDS for the value product (kernel.py:118-124);
//   * values: lane l takes groups of 8 value dims (l % (dv / 8), and l + 64
//     at dv = 1024) and, when dv < 512, every (64 / (dv / 8))-th token of the
//     tile from l / (dv / 8) on; the lanes of one dim group add their sums at
//     the end;
//   * out = acc / l (or 0) and lse = m + log2(l) (or -inf) per head
//     (kernel.py:126-138).
// Stage 2 (mla_generic_combine_kernel), one wave per (sequence, head): the
// merge of kernel.py:163-181, w = exp2(lse_s - max) in split order.
//
// Stage 1 above is the vector-ALU form (float32 arithmetic, any accepted dims
// and types); bf16 / fp16 calls with head_dim_v <= 512, head_dim_v +
// rope_dim <= 576 and 16-byte aligned q and cache rows take the matrix-core
// form further down (mla_generic_mfma_kernel), which writes the same partial
// format. Neither uses LDS-DMA.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdio.h>

#include "cdna.h"
#include "host_plan.h"
#include "triton_mla.h"

namespace tmla {
namespace gen {

struct GenericArgs {
  const char* q;
  int64_t q_sb, q_sh;  // element strides
  const char* kv;
  int64_t kv_s0, kv_s1;  // element strides
  int64_t num_blocks;
  int32_t page_size;
  const int32_t* bt;  // NULL: dense cache
  int64_t bt_sb;
  int32_t bt_cols;
  const int32_t* seqlens;
  int32_t batch, heads, dv, dr, splits;
  int64_t capacity;  // tokens a sequence can hold
  float qk_scale;    // softmax_scale * log2(e)
  int32_t tile;      // tokens per LDS step
  int32_t pitch;     // LDS bytes per staged row
  int32_t vec;       // 1: cache rows start on 16-byte boundaries
  int32_t qvec;      // 1: q rows start on 16-byte boundaries
  float* mid_o;      // [batch, heads, splits, dv]
  float* mid_lse;    // [batch, heads, splits], base 2
  char* out;
  int64_t out_sb, out_sh;
  float* lse;  // [batch, heads] natural log, or NULL
};

template <int DT>
struct GElt;
template <>
struct GElt<TMLA_BF16> {
  static constexpr int ES = 2;
  __device__ static float ld(const char* p) { return Elt<TMLA_BF16>::to_float(*(const short*)p); }
  __device__ static void st(char* p, float x) { *(short*)p = Elt<TMLA_BF16>::from_float(x); }
  __device__ static float round(float x) { return Elt<TMLA_BF16>::to_float(Elt<TMLA_BF16>::from_float(x)); }
  // 8 elements from 16 bytes of LDS
  __device__ static void lds8(const char* p, float (&f)[8]) {
    const i16x8 v = *(const i16x8*)p;
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = Elt<TMLA_BF16>::to_float(v[e]);
  }
};
template <>
struct GElt<TMLA_FP16> {
  static constexpr int ES = 2;
  __device__ static float ld(const char* p) { return Elt<TMLA_FP16>::to_float(*(const short*)p); }
  __device__ static void st(char* p, float x) { *(short*)p = Elt<TMLA_FP16>::from_float(x); }
  __device__ static float round(float x) { return Elt<TMLA_FP16>::to_float(Elt<TMLA_FP16>::from_float(x)); }
  __device__ static void lds8(const char* p, float (&f)[8]) {
    const i16x8 v = *(const i16x8*)p;
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = Elt<TMLA_FP16>::to_float(v[e]);
  }
};
template <>
struct GElt<TMLA_FP32> {
  static constexpr int ES = 4;
  __device__ static float ld(const char* p) { return *(const float*)p; }
  __device__ static void st(char* p, float x) { *(float*)p = x; }
  __device__ static float round(float x) { return x; }
  __device__ static void lds8(const char* p, float (&f)[8]) {
    const f32x4 a = *(const f32x4*)p, b = *(const f32x4*)(p + 16);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f[e] = a[e];
      f[4 + e] = b[e];
    }
  }
};

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) x = fmaxf(x, __shfl_xor(x, off));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) x += __shfl_xor(x, off);
  return x;
}

// Start of cache row `tok` (< capacity) of sequence b: through the block
// table, slot and page id clamped into the table and the cache.
__device__ __forceinline__ const char* row_ptr(const GenericArgs& a, int b, int tok, int es) {
  if (a.bt == nullptr) return a.kv + ((int64_t)b * a.kv_s0 + (int64_t)tok * a.kv_s1) * es;
  const int slot = min(tok / a.page_size, a.bt_cols - 1);
  int64_t page = a.bt[(int64_t)b * a.bt_sb + slot];
  page = page < 0 ? 0 : (page >= a.num_blocks ? a.num_blocks - 1 : page);
  return a.kv + (page * a.kv_s0 + (int64_t)(tok % a.page_size) * a.kv_s1) * es;
}

// NGL: groups of 8 value dims per lane (2 at head_dim_v 1024, else 1);
// LDSB: the workgroup's LDS (kGenSmallLds or kGenLargeLds).
template <int DT, int NGL, int LDSB>
__global__ __launch_bounds__(256) void mla_generic_partial_kernel(GenericArgs a) {
  using E = GElt<DT>;
  constexpr int ES = E::ES;
  __shared__ __attribute__((aligned(16))) char smem[LDSB];
  const int hb = blockIdx.x, s = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int D = a.dv + a.dr;
  const int T = a.tile;
  float* qs = (float*)smem;             // [16 heads][D]
  float* ps = qs + kGenHeads * D;       // [4 waves][64 tokens][4 heads]
  char* kvs = (char*)(ps + 4 * 64 * 4);  // [T][pitch]

  // (lengths cut to the capacity, and far enough below 2^31 that n0 + tile
  // cannot wrap)
  const int n = (int)min(min((int64_t)max(a.seqlens[b], 0), a.capacity), (int64_t)INT32_MAX - 128);
  const int split_len = (int)(((int64_t)n + a.splits - 1) / a.splits);
  const int start = (int)min((int64_t)s * split_len, (int64_t)n);
  const int end = (int)min((int64_t)start + split_len, (int64_t)n);

  // Q: eight loads in flight per thread before their stores
  for (int i0 = tid; i0 < kGenHeads * D; i0 += 8 * 256) {
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int i = i0 + 256 * k;
      v[k] = 0.0f;
      if (i < kGenHeads * D) {
        const int h = i / D, d = i - h * D;
        const int hg = hb * kGenHeads + h;
        if (hg < a.heads) v[k] = E::ld(a.q + ((int64_t)b * a.q_sb + (int64_t)hg * a.q_sh + d) * ES);
      }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (i0 + 256 * k < kGenHeads * D) qs[i0 + 256 * k] = v[k] * a.qk_scale;
  }

  // scores: token t_qk, dim groups c_qk, c_qk + C, ... of 8
  const int C = 64 / T;
  const int t_qk = lane & (T - 1), c_qk = lane / T;
  const int NG = D / 8;
  // values: dim group dg (and dg + 64), tokens g_pv, g_pv + G, ...
  const int NDG = a.dv / 8;
  const int G = NDG >= 64 ? 1 : 64 / NDG;
  const int dg = NDG >= 64 ? lane : lane % NDG;
  const int g_pv = NDG >= 64 ? 0 : lane / NDG;
  const float* qw = qs + wave * 4 * D;
  float* pw = ps + wave * 64 * 4;

  float m_run[4], l_run[4], acc[4][8 * NGL];
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    m_run[h] = -INFINITY;
    l_run[h] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8 * NGL; ++j) acc[h][j] = 0.0f;
  }

  const int cpr = D * ES / 16;  // 16-byte chunks per row
  for (int n0 = start; n0 < end; n0 += T) {
    __syncthreads();  // Q staged; the previous step's rows and probabilities read
    // batches of 8 chunks per thread: their page ids, then their rows, are
    // in flight together (rows past the piece read its last row, zeroed after)
    for (int i0 = tid; i0 < T * cpr; i0 += 8 * 256) {
      const char* src[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int i = min(i0 + 256 * k, T * cpr - 1);
        const int t = i / cpr, ch = i - t * cpr;
        src[k] = row_ptr(a, b, min(n0 + t, end - 1), ES) + ch * 16;
      }
      f32x4 v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        if (a.vec) {
          v[k] = *(const f32x4*)src[k];
        } else {
          char* vb = (char*)&v[k];
#pragma unroll
          for (int e = 0; e < 16; e += ES) {
            if constexpr (ES == 2)
              *(short*)(vb + e) = *(const short*)(src[k] + e);
            else
              *(float*)(vb + e) = *(const float*)(src[k] + e);
          }
        }
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int i = i0 + 256 * k;
        if (i < T * cpr) {
          const int t = i / cpr, ch = i - t * cpr;
          *(f32x4*)(kvs + t * a.pitch + ch * 16) = n0 + t < end ? v[k] : (f32x4)0.0f;
        }
      }
    }
    __syncthreads();

    float sc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const char* krow = kvs + t_qk * a.pitch;
    for (int g = c_qk; g < NG; g += C) {
      float kf[8];
      E::lds8(krow + g * 8 * ES, kf);
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const f32x4 q0 = *(const f32x4*)(qw + h * D + g * 8), q1 = *(const f32x4*)(qw + h * D + g * 8 + 4);
        float x = sc[h];
#pragma unroll
        for (int e = 0; e < 4; ++e) x = fmaf(q0[e], kf[e], x);
#pragma unroll
        for (int e = 0; e < 4; ++e) x = fmaf(q1[e], kf[4 + e], x);
        sc[h] = x;
      }
    }
    for (int off = T; off < 64; off <<= 1) {
#pragma unroll
      for (int h = 0; h < 4; ++h) sc[h] += __shfl_xor(sc[h], off);
    }
    const bool valid = n0 + t_qk < end;
    float pr[4];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const float m_new = fmaxf(m_run[h], wave_max(valid ? sc[h] : -INFINITY));
      const float alpha = exp2f(m_run[h] - m_new);
      const float p = valid ? exp2f(sc[h] - m_new) : 0.0f;
      l_run[h] = l_run[h] * alpha + wave_sum(c_qk == 0 ? p : 0.0f);
      m_run[h] = m_new;
#pragma unroll
      for (int j = 0; j < 8 * NGL; ++j) acc[h][j] *= alpha;
      pr[h] = E::round(p);
    }
    if (c_qk == 0) *(f32x4*)(pw + t_qk * 4) = f32x4{pr[0], pr[1], pr[2], pr[3]};
    __syncthreads();

    for (int t = g_pv; t < T && n0 + t < end; t += G) {
      const f32x4 p4 = *(const f32x4*)(pw + t * 4);
      const char* vrow = kvs + t * a.pitch;
#pragma unroll
      for (int j = 0; j < NGL; ++j) {
        float vf[8];
        E::lds8(vrow + (dg + 64 * j) * 8 * ES, vf);
#pragma unroll
        for (int h = 0; h < 4; ++h)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[h][8 * j + e] = fmaf(p4[h], vf[e], acc[h][8 * j + e]);
      }
    }
  }

  for (int off = NDG; off < 64; off <<= 1) {
#pragma unroll
    for (int h = 0; h < 4; ++h)
#pragma unroll
      for (int j = 0; j < 8 * NGL; ++j) acc[h][j] += __shfl_xor(acc[h][j], off);
  }
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const int hg = hb * kGenHeads + wave * 4 + h;
    if (hg >= a.heads) continue;
    const bool has = l_run[h] > 0.0f;
    const float den = has ? l_run[h] : 1.0f;
    const int64_t row = ((int64_t)b * a.heads + hg) * a.splits + s;
    if (g_pv == 0) {
      float* dst = a.mid_o + row * a.dv;
#pragma unroll
      for (int j = 0; j < NGL; ++j) {
        f32x4 lo, hi;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          lo[e] = acc[h][8 * j + e] / den;
          hi[e] = acc[h][8 * j + 4 + e] / den;
        }
        *(f32x4*)(dst + (dg + 64 * j) * 8) = lo;
        *(f32x4*)(dst + (dg + 64 * j) * 8 + 4) = hi;
      }
    }
    if (lane == 0) a.mid_lse[row] = has ? m_run[h] + log2f(l_run[h]) : -INFINITY;
  }
}

// One wave per (sequence, head): lane l takes value dims l, l + 64, ...
template <int DT>
__global__ __launch_bounds__(64) void mla_generic_combine_kernel(GenericArgs a) {
  using E = GElt<DT>;
  constexpr int ES = E::ES;
  constexpr float kLn2 = 0.693147180559945309f;
  const int b = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
  const int64_t row = (int64_t)b * a.heads + h;
  const float* ml = a.mid_lse + row * a.splits;
  float m = -INFINITY;
  for (int s = lane; s < a.splits; s += 64) m = fmaxf(m, ml[s]);
  m = wave_max(m);
  if (m == -INFINITY) m = 0.0f;
  const float* mo = a.mid_o + row * a.splits * a.dv;
  float acc[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) acc[k] = 0.0f;
  float w_sum = 0.0f;
  // four splits' rows in flight at a time, merged in split order
  int s = 0;
  for (; s + 4 <= a.splits; s += 4) {
    float lv[4], x[4][16];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      lv[j] = ml[s + j];
      const float* src = mo + (int64_t)(s + j) * a.dv;
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const int d = lane + 64 * k;
        x[j][k] = d < a.dv ? src[d] : 0.0f;
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float w = exp2f(lv[j] - m);
#pragma unroll
      for (int k = 0; k < 16; ++k)
        if (lane + 64 * k < a.dv) acc[k] = fmaf(w, x[j][k], acc[k]);
      w_sum += w;
    }
  }
  for (; s < a.splits; ++s) {
    const float w = exp2f(ml[s] - m);
    const float* src = mo + (int64_t)s * a.dv;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int d = lane + 64 * k;
      if (d < a.dv) acc[k] = fmaf(w, src[d], acc[k]);
    }
    w_sum += w;
  }
  const float den = w_sum > 0.0f ? w_sum : 1.0f;
  char* o = a.out + ((int64_t)b * a.out_sb + (int64_t)h * a.out_sh) * ES;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int d = lane + 64 * k;
    if (d < a.dv) E::st(o + (int64_t)d * ES, acc[k] / den);
  }
  if (a.lse != nullptr && lane == 0) a.lse[row] = w_sum > 0.0f ? (m + log2f(w_sum)) * kLn2 : -INFINITY;
}


// ---------------------------------------------------------------------------
// Matrix-core form (bf16 / fp16, head_dim_v <= 512, D <= 576)
// ---------------------------------------------------------------------------
//
// The same algorithm and partial format on v_mfma_f32_16x16x32: a workgroup
// of 4 waves takes 64 heads (16 per wave) and steps over 32 tokens:
//   * the 32 cache rows are loaded into registers one step ahead (units of
//     4 rows x 16 bytes per lane) and written to LDS twice: as rows (the S
//     operand) and, for the value dims, transposed to [dim][token] (the PV
//     operand);
//   * S (16 heads x 16 tokens, two tiles) = Q . K^T over k-chunks of 32 dims:
//     lane l reads 8 consecutive dims 32c + 8(l/16) of head l%16 (Q) and of
//     token l%16 (K), the same k order for both operands; a last chunk of 16
//     dims gives its upper lane groups zeros. Result: lane l holds token
//     l%16, heads 4(l/16) + i;
//   * the online softmax per head reduces over the 16 lanes of a group;
//     probabilities rounded to the element type go through LDS to the layout
//     of the PV operand (head l%16, tokens 8(l/16)..+7);
//   * O (16 heads x 16 dims per tile) += P . V, dims 16n + l%16 from the
//     transposed values; lane l holds dim 16n + l%16 of heads 4(l/16) + i,
//     the heads of the softmax state it holds, so the rescale stays in-lane.
constexpr int kMP = kGenMP;  // bytes per row of the transposed values and probabilities

// Workgroup barrier after this wave's LDS accesses have completed, without
// waiting for its global loads (a __syncthreads would also wait for the
// next step's row loads, which are meant to fly across the barrier).
__device__ __forceinline__ void lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int DT>
__device__ __forceinline__ f32x4 mfma16(const i16x8& a, const i16x8& b, const f32x4& c) {
  if constexpr (DT == TMLA_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                    0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                   0, 0);
}

// Reductions over the 16 lanes of a DPP row (lanes 16r .. 16r + 15): row
// rotations by 8, 4, 2 and 1 leave every lane with the row's result.
template <int N>
__device__ __forceinline__ float row_ror(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x120 | N, 0xF, 0xF, false));
}
__device__ __forceinline__ float group16_max(float x) {
  x = fmaxf(x, row_ror<8>(x));
  x = fmaxf(x, row_ror<4>(x));
  x = fmaxf(x, row_ror<2>(x));
  return fmaxf(x, row_ror<1>(x));
}
__device__ __forceinline__ float group16_sum(float x) {
  x += row_ror<8>(x);
  x += row_ror<4>(x);
  x += row_ror<2>(x);
  return x + row_ror<1>(x);
}

// NDT: 16-dim output tiles (head_dim_v / 16)
template <int DT, int LDSB, int NDT>
__global__ __launch_bounds__(256) void mla_generic_mfma_kernel(GenericArgs a) {
  using E = GElt<DT>;
  constexpr int MT = kGenMfmaTokens;
  constexpr int kPreU = 3;  // units (4 rows x 16 bytes) per thread and step: 8 x 576 / 8 / 256 <= 3
  static_assert(NDT >= 1 && NDT <= 32, "head_dim_v <= 512");
  __shared__ __attribute__((aligned(16))) char smem[LDSB];
  const int hb = blockIdx.x, s = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int D = a.dv + a.dr, DV = a.dv;
  const int rp = 2 * D + kGenRowPad;  // bytes per staged row (and per Q row)
  char* const R = smem;                        // [32 tokens][rp]
  char* const VT = R + MT * rp;                // [DV][kMP]
  char* const Pw = VT + DV * kMP + wave * 16 * kMP;    // [16 heads][kMP] of this wave
  char* const Qw = VT + DV * kMP + 4 * 16 * kMP + wave * 16 * rp;  // [16 heads][rp] of this wave

  const int n = (int)min(min((int64_t)max(a.seqlens[b], 0), a.capacity), (int64_t)INT32_MAX - 128);
  const int split_len = (int)(((int64_t)n + a.splits - 1) / a.splits);
  const int start = (int)min((int64_t)s * split_len, (int64_t)n);
  const int end = (int)min((int64_t)start + split_len, (int64_t)n);

  // Q rows of the wave's 16 heads in 16-byte chunks, eight in flight per lane
  const int qn = 16 * (D / 8);
  for (int i0 = lane; i0 < qn; i0 += 8 * 64) {
    i16x8 v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int i = i0 + 64 * k;
      v[k] = (i16x8)0;
      if (i < qn) {
        const int r = i / (D / 8), ch = i - r * (D / 8);
        const int hg = hb * kGenMfmaHeads + wave * 16 + r;
        if (hg < a.heads) v[k] = *(const i16x8*)(a.q + ((int64_t)b * a.q_sb + (int64_t)hg * a.q_sh + ch * 8) * 2);
      }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int i = i0 + 64 * k;
      if (i < qn) {
        const int r = i / (D / 8), ch = i - r * (D / 8);
        *(i16x8*)(Qw + r * rp + ch * 16) = v[k];
      }
    }
  }

  const int g = lane >> 4, c16 = lane & 15;
  const int nkc = (D + 31) / 32;
  const bool half_last = (D & 31) != 0;
  const int cpr = D / 8;      // 16-byte chunks per row
  const int vcpr = DV / 8;    // ... of which hold value dims
  const int nun = (MT / 4) * cpr;  // units of 4 rows x one chunk

  f32x4 acc[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) acc[t] = (f32x4)0.0f;
  float m_run[4], l_run[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m_run[i] = -INFINITY;
    l_run[i] = 0.0f;
  }

  // unit u: rows 4(u % 8) .. +3, 16-byte column u / 8; the transposed
  // values take one 8-byte write (4 tokens) per value dim of the unit, and
  // the 8 lanes of one column fill 64 contiguous bytes of a transposed row
  // Straight-line loads (rows past the piece read its last row and are
  // zeroed afterwards), so all of a step's page ids, then all of its rows,
  // are in flight together. The form is used only for 16-byte aligned rows.
  f32x4 pre[4 * kPreU];
  auto fetch = [&](int n0) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < kPreU; ++k) {
      const int u = tid + 256 * k;
      if (u < nun) {
        const int t4 = u & 7, ch = u >> 3;
        const char* src[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) src[r] = row_ptr(a, b, min(n0 + 4 * t4 + r, end - 1), 2) + ch * 16;
#pragma unroll
        for (int r = 0; r < 4; ++r) pre[4 * k + r] = *(const f32x4*)src[r];
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (n0 + 4 * t4 + r >= end) pre[4 * k + r] = (f32x4)0.0f;
      }
    }
  };
  auto store = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < kPreU; ++k) {
      const int u = tid + 256 * k;
      if (u < nun) {
        const int t4 = u & 7, ch = u >> 3;
#pragma unroll
        for (int r = 0; r < 4; ++r) *(f32x4*)(R + (4 * t4 + r) * rp + ch * 16) = pre[4 * k + r];
        if (ch < vcpr) {
          const i16x8 v0 = __builtin_bit_cast(i16x8, pre[4 * k]), v1 = __builtin_bit_cast(i16x8, pre[4 * k + 1]);
          const i16x8 v2 = __builtin_bit_cast(i16x8, pre[4 * k + 2]), v3 = __builtin_bit_cast(i16x8, pre[4 * k + 3]);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const i16x4 col = {v0[e], v1[e], v2[e], v3[e]};
            *(i16x4*)(VT + (ch * 8 + e) * kMP + 8 * t4) = col;
          }
        }
      }
    }
  };

  if (start < end) fetch(start);
  for (int n0 = start; n0 < end; n0 += MT) {
    lds_sync();  // Q staged; the previous step's operands read
    store();
    lds_sync();
    if (n0 + MT < end) fetch(n0 + MT);  // in flight until the next store

    // S, the operands of chunk c + 1 read before the MFMAs of chunk c
    f32x4 s0 = (f32x4)0.0f, s1 = (f32x4)0.0f;
    auto operands = [&](int c, i16x8& qa, i16x8& k0, i16x8& k1) __attribute__((always_inline)) {
      qa = (i16x8)0;
      k0 = (i16x8)0;
      k1 = (i16x8)0;
      if (!(half_last && c == nkc - 1 && g >= 2)) {
        const int off = (32 * c + 8 * g) * 2;
        qa = *(const i16x8*)(Qw + c16 * rp + off);
        k0 = *(const i16x8*)(R + c16 * rp + off);
        k1 = *(const i16x8*)(R + (16 + c16) * rp + off);
      }
    };
    i16x8 qa, k0, k1;
    operands(0, qa, k0, k1);
    for (int c = 0; c < nkc; ++c) {
      i16x8 qn = qa, kn0 = k0, kn1 = k1;
      if (c + 1 < nkc) operands(c + 1, qn, kn0, kn1);
      s0 = mfma16<DT>(qa, k0, s0);
      s1 = mfma16<DT>(qa, k1, s1);
      qa = qn;
      k0 = kn0;
      k1 = kn1;
    }

    const bool v0 = n0 + c16 < end, v1 = n0 + 16 + c16 < end;
    float alpha[4];
    bool moved = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float x0 = v0 ? s0[i] * a.qk_scale : -INFINITY;
      const float x1 = v1 ? s1[i] * a.qk_scale : -INFINITY;
      const float m_new = fmaxf(m_run[i], group16_max(fmaxf(x0, x1)));
      alpha[i] = exp2f(m_run[i] - m_new);
      moved |= m_new != m_run[i];
      const float e0 = v0 ? exp2f(x0 - m_new) : 0.0f;
      const float e1 = v1 ? exp2f(x1 - m_new) : 0.0f;
      l_run[i] = l_run[i] * alpha[i] + group16_sum(e0 + e1);
      m_run[i] = m_new;
      *(short*)(Pw + (4 * g + i) * kMP + c16 * 2) = Elt<DT>::from_float(e0);
      *(short*)(Pw + (4 * g + i) * kMP + (16 + c16) * 2) = Elt<DT>::from_float(e1);
    }
    // a head whose max did not move has alpha = 1 exactly, so the rescale is
    // skipped when no head of the wave moved (the same bits)
    if (__any(moved)) {
#pragma unroll
      for (int t = 0; t < NDT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][i] *= alpha[i];
    }
    lds_sync();

    const i16x8 pa = *(const i16x8*)(Pw + c16 * kMP + 16 * g);
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
      const i16x8 vb = *(const i16x8*)(VT + (16 * t + c16) * kMP + 16 * g);
      acc[t] = mfma16<DT>(pa, vb, acc[t]);
    }
  }

#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int hg = hb * kGenMfmaHeads + wave * 16 + 4 * g + i;
    if (hg >= a.heads) continue;
    const bool has = l_run[i] > 0.0f;
    const float den = has ? l_run[i] : 1.0f;
    const int64_t row = ((int64_t)b * a.heads + hg) * a.splits + s;
    float* dst = a.mid_o + row * DV;
#pragma unroll
    for (int t = 0; t < NDT; ++t) dst[16 * t + c16] = acc[t][i] / den;
    if (c16 == 0) a.mid_lse[row] = has ? m_run[i] + log2f(l_run[i]) : -INFINITY;
  }
}

template <int DT, int NGL>
hipError_t launch_partial_t(const GenericArgs& a, int lds, dim3 grid, hipStream_t stream) {
  if (lds == kGenSmallLds)
    hipLaunchKernelGGL((mla_generic_partial_kernel<DT, NGL, kGenSmallLds>), grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((mla_generic_partial_kernel<DT, NGL, kGenLargeLds>), grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

template <int DT, int NDT>
hipError_t launch_mfma_ndt(const GenericArgs& a, int lds, dim3 grid, hipStream_t stream) {
  if (lds == kGenMfmaSmallLds)
    hipLaunchKernelGGL((mla_generic_mfma_kernel<DT, kGenMfmaSmallLds, NDT>), grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((mla_generic_mfma_kernel<DT, kGenMfmaLargeLds, NDT>), grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

template <int DT>
hipError_t launch_mfma_t(const GenericArgs& a, int lds, hipStream_t stream) {
  const dim3 grid((a.heads + kGenMfmaHeads - 1) / kGenMfmaHeads, a.splits, a.batch);
  switch (a.dv) {
    case 16: return launch_mfma_ndt<DT, 1>(a, lds, grid, stream);
    case 32: return launch_mfma_ndt<DT, 2>(a, lds, grid, stream);
    case 64: return launch_mfma_ndt<DT, 4>(a, lds, grid, stream);
    case 128: return launch_mfma_ndt<DT, 8>(a, lds, grid, stream);
    case 256: return launch_mfma_ndt<DT, 16>(a, lds, grid, stream);
    default: return launch_mfma_ndt<DT, 32>(a, lds, grid, stream);  // 512 (generic_mfma_form: dv <= 512)
  }
}

// lds: the vector-ALU form's LDS; mfma_lds: the matrix-core form's, or 0
// when that form does not apply.
template <int DT>
hipError_t launch_t(const GenericArgs& a, int lds, int mfma_lds, hipStream_t stream) {
  hipError_t e;
  if constexpr (DT != TMLA_FP32) {
    if (mfma_lds != 0) {
      e = launch_mfma_t<DT>(a, mfma_lds, stream);
      if (e != hipSuccess) return e;
      hipLaunchKernelGGL((mla_generic_combine_kernel<DT>), dim3(a.batch, a.heads), dim3(64), 0, stream, a);
      return hipGetLastError();
    }
  }
  const dim3 grid((a.heads + kGenHeads - 1) / kGenHeads, a.splits, a.batch);
  e = a.dv == 1024 ? launch_partial_t<DT, 2>(a, lds, grid, stream) : launch_partial_t<DT, 1>(a, lds, grid, stream);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((mla_generic_combine_kernel<DT>), dim3(a.batch, a.heads), dim3(64), 0, stream, a);
  return hipGetLastError();
}

}  // namespace gen

extern int hip_fail(hipError_t e, const char* where);

}  // namespace tmla

using namespace tmla;

extern "C" {

size_t tmla_generic_workspace_bytes(int32_t batch, int32_t num_heads, int32_t head_dim_v, int32_t num_splits) {
  return generic_workspace_bytes(batch, num_heads, head_dim_v, num_splits);
}

int32_t tmla_generic_heads_per_workgroup(int32_t head_dim_v, int32_t rope_dim, int32_t dtype) {
  if (dtype != TMLA_BF16 && dtype != TMLA_FP16 && dtype != TMLA_FP32) return 0;
  if (!pow2_between(head_dim_v, 16, 1024) || !pow2_between(rope_dim, 16, 256)) return 0;
  return generic_mfma_form(head_dim_v, rope_dim, dtype) != 0 ? kGenMfmaHeads : kGenHeads;
}

int tmla_mla_decode_generic(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kv,
                            int64_t kv_stride_0, int64_t kv_stride_1, int64_t num_blocks, int32_t page_size,
                            const int32_t* block_table, int64_t bt_stride_b, int32_t bt_cols,
                            const int32_t* seqlens, int32_t batch, int32_t num_heads, int32_t head_dim_v,
                            int32_t rope_dim, int32_t dtype, float softmax_scale, int32_t num_splits, void* out,
                            int64_t out_stride_b, int64_t out_stride_h, float* lse, void* workspace,
                            size_t workspace_bytes_, void* stream) {
  const bool paged = block_table != nullptr;
  const GenericCall c{batch, num_heads, head_dim_v, rope_dim, dtype, num_splits,
                      paged, page_size, bt_cols, num_blocks};
  const int rc = check_generic(c, workspace, workspace_bytes_);
  if (rc != TMLA_OK) return rc;
  if (batch == 0) return TMLA_OK;
  if (q == nullptr || kv == nullptr || seqlens == nullptr || out == nullptr)
    return fail(TMLA_ERR_INVALID_ARGUMENT, "q, kv, seqlens and out must not be NULL");
  if ((uintptr_t)workspace % 16 != 0) return fail(TMLA_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
  const int es = elem_bytes(dtype);
  const GenericPlan p = generic_plan(head_dim_v, rope_dim, dtype);
  gen::GenericArgs a;
  a.q = (const char*)q;
  a.q_sb = q_stride_b;
  a.q_sh = q_stride_h;
  a.kv = (const char*)kv;
  a.kv_s0 = kv_stride_0;
  a.kv_s1 = kv_stride_1;
  a.num_blocks = num_blocks;
  a.page_size = page_size;
  a.bt = block_table;
  a.bt_sb = bt_stride_b;
  a.bt_cols = bt_cols;
  a.seqlens = seqlens;
  a.batch = batch;
  a.heads = num_heads;
  a.dv = head_dim_v;
  a.dr = rope_dim;
  a.splits = num_splits;
  a.capacity = paged ? (int64_t)bt_cols * page_size : num_blocks;
  a.qk_scale = softmax_scale * 1.4426950408889634f;
  a.tile = p.tile;
  a.pitch = p.pitch;
  a.vec = ((uintptr_t)kv % 16 == 0 && (kv_stride_0 * es) % 16 == 0 && (kv_stride_1 * es) % 16 == 0) ? 1 : 0;
  a.qvec = ((uintptr_t)q % 16 == 0 && (q_stride_b * es) % 16 == 0 && (q_stride_h * es) % 16 == 0) ? 1 : 0;
  const int64_t rows = (int64_t)batch * num_heads * num_splits;
  a.mid_o = (float*)workspace;
  a.mid_lse = (float*)((char*)workspace + ((rows * head_dim_v * 4 + 255) & ~(int64_t)255));
  a.out = (char*)out;
  a.out_sb = out_stride_b;
  a.out_sh = out_stride_h;
  a.lse = lse;
  hipStream_t st = (hipStream_t)stream;
  // the matrix-core form reads q and the cache in 16-byte pieces only
  const int mfma_lds = a.vec && a.qvec ? generic_mfma_form(head_dim_v, rope_dim, dtype) : 0;
  const hipError_t e = dtype == TMLA_BF16   ? gen::launch_t<TMLA_BF16>(a, p.lds, mfma_lds, st)
                       : dtype == TMLA_FP16 ? gen::launch_t<TMLA_FP16>(a, p.lds, mfma_lds, st)
                                            : gen::launch_t<TMLA_FP32>(a, p.lds, mfma_lds, st);
  return e == hipSuccess ? TMLA_OK : hip_fail(e, "mla_generic kernels launch");
}

}  // extern "C"
