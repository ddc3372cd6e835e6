// MLA layer glue for MI355X (gfx950): the absorbed-projection steps on
// either side of mla_decode in the DeepSeek MLA decode layer, and their C ABI
// (include/triton_mla.h).
//
// Reference behaviour: src/triton_mla/model.py:74-124 (MLA._project's RoPE,
// MLA._append_kv, the W_UK and W_UV einsums of MLA.forward), apply_rope
// model.py:44-50, RMSNorm model.py:34-41. The dense projections (wq_a, wq_b,
// wkv_a, wo) of a decode step's few rows run in mla_project_kernel; larger
// batches stay library GEMMs.
//
//  * mla_absorb_q_kernel: q[b, h, :rank] = q_nope[b, h] . W_UK[h] and
//    q[b, h, rank:] = RoPE(q_pe[b, h]). W_UK[h] (the nope rows of wkv_b,
//    [nope, rank], rank contiguous) is contracted over its rows, so it is
//    copied into LDS with LDS-DMA in the swizzled 8-row x 128-byte block
//    layout of the decode kernel and read back transposed with
//    ds_read_b64_tr_b16 as the A operand of v_mfma_f32_32x32x16; q_nope^T is
//    the B operand, loaded from memory in the k order the transposed read
//    produces. Output tile O^T = W_UK^T . q_nope^T, 32 columns x 32 batch rows
//    per MFMA block, one block per wave.
//  * mla_absorb_out_kernel: o[b, h*vd + v] = o_lat[b, h] . W_UV[h][v] (the v
//    rows of wkv_b, [vd, rank], rank contiguous): both MFMA operands are
//    contiguous in the contraction index, so they are loaded straight from
//    memory; four waves split the contraction of each 32 x 32 block.
//  * mla_kv_append_kernel: RMSNorm of the latent, RoPE of the key, and the
//    new row written at position cache_seqlens[b] through the block table.
//  * mla_rms_norm_kernel: RMSNorm of rows (the query latent, model.py:34-41,
//    76), float32, rounded once.
//  * mla_project_kernel: the dense projections (wq_a, wq_b, wkv_a, wo;
//    nn.Linear, model.py:66-72) for a decode step's few rows,
//    y[M, N] = x[M, K] . W[N, K]^T: each weight row is read from HBM once,
//    16 rows per workgroup, the contraction split over the workgroup's
//    waves and summed through LDS in a fixed order.
#include <math.h>
#include <stdio.h>

#include "cdna.h"
#include "host_plan.h"
#include "triton_mla.h"

namespace tmla {

namespace layer {

constexpr int kNope = 128;   // qk_nope_head_dim the q kernel is built for
constexpr int kRope = 64;    // qk_rope_head_dim
constexpr int kColsWG = 128; // W_UK columns per workgroup (4 waves x 1 block of 32)
constexpr int kBTile = 32;   // batch rows per MFMA block (N of the 32x32x16 MFMA)
constexpr int kProjectMaxRows = 64;  // rows of x the projection kernel takes (4 blocks of 16)

struct AbsorbQArgs {
  const short* qp;       // [B, qp_sb]: head h at h*(nope+rope): q_nope then q_pe
  int64_t qp_sb;
  const short* w;        // wkv_b [H*(nope+vd), rank], row stride w_s0
  int64_t w_s0;
  const int32_t* pos;    // [B] rotary positions
  short* out;            // [B, H, rank + rope]
  int64_t out_sb, out_sh;
  int32_t batch, heads, rank, vd;
  float theta;
};

struct AbsorbOutArgs {
  const short* o;        // [B, H, rank]
  int64_t o_sb, o_sh;
  const short* w;        // wkv_b
  int64_t w_s0;
  short* out;            // [B, H*vd]
  int64_t out_sb;
  int32_t batch, heads, nope, rank, vd;
};

struct KvAppendArgs {
  const short* kvp;      // [B, kvp_sb]: latent (rank) then rope key
  int64_t kvp_sb;
  const short* norm_w;   // [rank] or null
  float eps, theta;
  const int32_t* pos;    // [B]
  int32_t* pos_next;     // [B] or null: pos + 1 (the sequence lengths after the step)
  char* cache;           // paged [num_blocks, page_size, rank+rope] or dense [B, capacity, rank+rope]
  int64_t s0, s1;        // byte strides
  int64_t num_blocks;    // pages (paged) or capacity (dense)
  int32_t page_size;
  const int32_t* bt;     // [B, bt_cols] or null (dense)
  int64_t bt_sb;
  int32_t bt_cols, batch, rank;
};

struct ProjectArgs {
  const short* x;        // [M, K], row stride x_s (elements)
  int64_t x_s;
  const short* w;        // [N, K] (nn.Linear weight), row stride w_s
  int64_t w_s;
  short* y;              // [M, N], row stride y_s
  int64_t y_s;
  float* ws;             // partial tiles of split contractions (KS > 1)
  int32_t* cnt;          // their arrival counters, one per column group
  int32_t m, n, k;
};

// RoPE of one rotation pair (x1 = element i, x2 = element i + dim/2) at
// position pos, in float32 like the reference's apply_rope: the frequency is
// theta ** (2i / dim) and the angle pos / frequency.
__device__ __forceinline__ void rope_pair(float x1, float x2, int pos, int i, int dim, float theta, float& y1,
                                          float& y2) {
  const float freq = powf(theta, (float)(2 * i) / (float)dim);
  const float ang = (float)pos / freq;
  const float c = cosf(ang), s = sinf(ang);
  // each product and sum rounded on its own (no fused multiply-add), as the
  // reference's separate float32 tensor operations round them
  y1 = __fsub_rn(__fmul_rn(x1, c), __fmul_rn(x2, s));
  y2 = __fadd_rn(__fmul_rn(x2, c), __fmul_rn(x1, s));
}

template <int DT>
__device__ __forceinline__ float ld(const short* p) {
  return Elt<DT>::to_float(*p);
}

// ---------------------------------------------------------------------------
// q side: grid (heads, rank / 128, cdiv(batch, 32)), 4 waves
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(256) void mla_absorb_q_kernel(AbsorbQArgs a) {
  constexpr int NCB = kColsWG / 64;       // 128-byte column blocks per W row in LDS
  constexpr int SUB = 32;                 // W rows per LDS sub-tile
  constexpr int SUBBYTES = SUB * kColsWG * 2;
  constexpr int NSUB = kNope / SUB;       // 4
  __shared__ __attribute__((aligned(1024))) char smem[NSUB * SUBBYTES];  // 32 KiB
  char LDS_AS* const lds = (char LDS_AS*)(void LDS_AS*)smem;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = blockIdx.x;
  const int col0 = blockIdx.y * kColsWG;
  const int b0 = blockIdx.z * kBTile;

  // W_UK[h] rows [32*wave, 32*wave + 32), columns [col0, col0 + 128) into
  // sub-tile `wave`: block (rg, cb) holds rows 8rg..8rg+7 x 128 bytes, piece p
  // of row r at slot r*8 + (p ^ piece_swizzle(r, rg)).
  {
    const int r = lane >> 3;
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      const int p = (lane & 7) ^ piece_swizzle(r, rg);
      const int64_t row = (int64_t)h * (kNope + a.vd) + SUB * wave + 8 * rg + r;
      const char* src = reinterpret_cast<const char*>(a.w + row * a.w_s0 + col0) + p * 16;
      char LDS_AS* dst = lds + wave * SUBBYTES + rg * NCB * 1024;
      static_for<NCB>([&](auto CB) __attribute__((always_inline)) {
        constexpr int cb = decltype(CB)::value;
        lds_copy16<cb * 128>(src, dst + cb * 1024);
      });
    }
  }

  // B operand q_nope^T (k = 16 rows of W per MFMA): lane (n = batch row
  // b0 + lane%32, hi = lane/32), element i is q_nope[d] with
  // d = 16*kk + 8*(i/4) + 4*hi + i%4 -- the k order of the transposed W read.
  const int bl = lane & 31, hi = lane >> 5;
  const bool brow_ok = b0 + bl < a.batch;
  const short* qrow = a.qp + (int64_t)(b0 + bl) * a.qp_sb + (int64_t)h * (kNope + kRope);
  i16x8 qop[kNope / 16];
#pragma unroll
  for (int kk = 0; kk < kNope / 16; ++kk) {
    i16x4 lo = (i16x4)0, hi4 = (i16x4)0;
    if (brow_ok) {
      lo = *reinterpret_cast<const i16x4*>(qrow + 16 * kk + 4 * hi);
      hi4 = *reinterpret_cast<const i16x4*>(qrow + 16 * kk + 8 + 4 * hi);
    }
    qop[kk] = (i16x8){lo[0], lo[1], lo[2], lo[3], hi4[0], hi4[1], hi4[2], hi4[3]};
  }
  wait_vmcnt<0>();
  lds_barrier();

  // A operand W_UK^T: this wave's 32-column block (half dbp = wave & 1 of
  // the 128-byte column block wave >> 1); the addressing is that of the
  // decode kernel's V^T operand with the row-group stride of this tile
  // (NCB KiB).
  const int g = lane >> 4, L = lane & 15;
  const int rr = 4 * (g >> 1) + (L >> 2);
  const char LDS_AS* base[2];
#pragma unroll
  for (int e2 = 0; e2 < 2; ++e2) {
    const int piece = 4 * (wave & 1) + 2 * (g & 1) + ((L & 3) >> 1);
    base[e2] = lds + e2 * NCB * 1024 + (wave >> 1) * 1024 + (rr * 8 + (piece ^ piece_swizzle(rr, e2))) * 16 +
               8 * (L & 1);
  }
  f32x16 acc = (f32x16)0.0f;
  static_for<kNope / 16>([&](auto KK) __attribute__((always_inline)) {
    constexpr int kk = decltype(KK)::value;
    constexpr int st = kk / 2, c2 = kk % 2;
    constexpr int off = st * SUBBYTES + c2 * 2 * NCB * 1024;
    i16x4 l0 = ds_read_tr<off>(base[0]), h0 = ds_read_tr<off>(base[1]);
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(l0), "+v"(h0));
    const i16x8 v0 = {l0[0], l0[1], l0[2], l0[3], h0[0], h0[1], h0[2], h0[3]};
    acc = Elt<DT>::mfma(v0, qop[kk], acc);
  });

  // D[m = column][n = batch row]: lane holds batch row b0 + lane%32 and
  // columns 8j + 4*hi + e of each block (e = 0..3): one 8-byte store each
  if (brow_ok) {
    short* orow = a.out + (int64_t)(b0 + bl) * a.out_sb + (int64_t)h * a.out_sh;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      i16x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = Elt<DT>::from_float(acc[4 * j + e]);
      const int c = col0 + 32 * wave + 8 * j + 4 * hi;
      *reinterpret_cast<i16x4*>(orow + c) = v;
    }
  }

  // RoPE of q_pe: rows x pairs of the batch tile, shared by the workgroups
  // of all column blocks (each rotation costs a power and a large-argument
  // sine and cosine: kept in one column block, they made its workgroups the
  // last to finish)
  {
    const int nthreads = 256 * gridDim.y;
    for (int idx = threadIdx.x + 256 * blockIdx.y; idx < kBTile * (kRope / 2); idx += nthreads) {
      const int b = b0 + idx / (kRope / 2), i = idx % (kRope / 2);
      if (b >= a.batch) break;
      const short* pe = a.qp + (int64_t)b * a.qp_sb + (int64_t)h * (kNope + kRope) + kNope;
      float y1, y2;
      rope_pair(ld<DT>(pe + i), ld<DT>(pe + i + kRope / 2), a.pos[b], i, kRope, a.theta, y1, y2);
      short* o = a.out + (int64_t)b * a.out_sb + (int64_t)h * a.out_sh + a.rank;
      o[i] = Elt<DT>::from_float(y1);
      o[i + kRope / 2] = Elt<DT>::from_float(y2);
    }
  }
}

// ---------------------------------------------------------------------------
// output side: grid (heads, vd / 32, cdiv(batch, 32)); the 4 waves of a
// workgroup split the contraction (rank) in four and their 32x32 partial
// products are summed through LDS
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(256) void mla_absorb_out_kernel(AbsorbOutArgs a) {
  __shared__ f32x16 part[3][64];  // waves 1..3: one 32x32 fp32 block each
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = blockIdx.x;
  const int vb = blockIdx.y;
  const int b0 = blockIdx.z * kBTile;
  const int l32 = lane & 31, hi = lane >> 5;
  const bool brow_ok = b0 + l32 < a.batch;
  const int kq = a.rank / 4;  // contraction quarter of this wave
  // A: W_UV row v = 32*vb + lane%32 (k = rank index, 8 per lane-half);
  // B: o_lat^T column b0 + lane%32
  const short* wrow =
      a.w + ((int64_t)h * (a.nope + a.vd) + a.nope + 32 * vb + l32) * a.w_s0 + wave * kq + 8 * hi;
  const short* orow = a.o + (int64_t)(b0 + l32) * a.o_sb + (int64_t)h * a.o_sh + wave * kq + 8 * hi;
  f32x16 acc = (f32x16)0.0f;
  constexpr int CH = 8;  // k steps per batch of loads (all loads of a batch in flight together)
  for (int k0 = 0; k0 < kq; k0 += 16 * CH) {
    i16x8 wa[CH], ob[CH];
#pragma unroll
    for (int t = 0; t < CH; ++t) {
      wa[t] = *reinterpret_cast<const i16x8*>(wrow + k0 + 16 * t);
      ob[t] = brow_ok ? *reinterpret_cast<const i16x8*>(orow + k0 + 16 * t) : (i16x8)0;
    }
#pragma unroll
    for (int t = 0; t < CH; ++t) acc = Elt<DT>::mfma(wa[t], ob[t], acc);
  }
  if (wave > 0) part[wave - 1][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  acc += part[0][lane] + part[1][lane] + part[2][lane];
  if (brow_ok) {
    short* dst = a.out + (int64_t)(b0 + l32) * a.out_sb + (int64_t)h * a.vd + 32 * vb + 4 * hi;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      i16x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = Elt<DT>::from_float(acc[4 * j + e]);
      *reinterpret_cast<i16x4*>(dst + 8 * j) = v;
    }
  }
}

// ---------------------------------------------------------------------------
// cache append: one wave per sequence, grid cdiv(batch, 4)
// ---------------------------------------------------------------------------
template <int DT>
__device__ __forceinline__ void kv_append_row(const KvAppendArgs& a, int b, int lane) {
  const int pos = a.pos[b];
  if (a.pos_next && lane == 0) a.pos_next[b] = pos + 1;
  // destination row; rows outside the table or the cache are not written
  char* dst = nullptr;
  if (pos >= 0) {
    if (a.bt) {
      const int slot = pos / a.page_size;
      if (slot < a.bt_cols) {
        const int page = a.bt[(int64_t)b * a.bt_sb + slot];
        if (page >= 0 && page < a.num_blocks) dst = a.cache + (int64_t)page * a.s0 + (int64_t)(pos % a.page_size) * a.s1;
      }
    } else if (pos < a.num_blocks) {
      dst = a.cache + (int64_t)b * a.s0 + (int64_t)pos * a.s1;
    }
  }
  if (dst == nullptr) return;  // wave-uniform
  short* out = reinterpret_cast<short*>(dst);
  const short* x = a.kvp + (int64_t)b * a.kvp_sb;

  // RMSNorm over the latent in float32, rounded once:
  // y = x * rsqrt(mean(x^2) + eps) * weight
  const int per = a.rank / 64;  // elements per lane (8 for rank 512)
  float v[16];
  float ss = 0.0f;
  for (int e = 0; e < per; ++e) {
    v[e] = ld<DT>(x + lane * per + e);
    ss += v[e] * v[e];
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) ss += __shfl_xor(ss, d);
  const float rstd = rsqrtf(ss / (float)a.rank + a.eps);
  for (int e = 0; e < per; ++e) {
    float y = v[e] * rstd;
    if (a.norm_w) y = y * ld<DT>(a.norm_w + lane * per + e);
    out[lane * per + e] = Elt<DT>::from_float(y);
  }
  // RoPE of the shared key: lanes 0..31, one rotation pair each
  if (lane < kRope / 2) {
    float y1, y2;
    rope_pair(ld<DT>(x + a.rank + lane), ld<DT>(x + a.rank + lane + kRope / 2), pos, lane, kRope, a.theta, y1, y2);
    out[a.rank + lane] = Elt<DT>::from_float(y1);
    out[a.rank + lane + kRope / 2] = Elt<DT>::from_float(y2);
  }
}

template <int DT>
__global__ __launch_bounds__(256) void mla_kv_append_kernel(KvAppendArgs a) {
  const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (b < a.batch) kv_append_row<DT>(a, b, threadIdx.x & 63);  // wave-uniform
}

// ---------------------------------------------------------------------------
// RMSNorm of rows (the query latent): grid (cdiv(rows, 4)), one wave per row
// ---------------------------------------------------------------------------
struct RmsNormArgs {
  const short* x;
  int64_t x_s;
  const short* w;        // [dim] or null (weight 1)
  short* y;
  int64_t y_s;
  float eps;
  int32_t rows, dim;
};

// y = x * rsqrt(mean(x^2) + eps) * weight in float32, rounded once (the
// arithmetic of the latent's norm in mla_kv_append_kernel). Lane l owns the
// 8-element chunks l, l + 64, ...; the row is read twice (the second pass
// from cache).
template <int DT>
__device__ __forceinline__ void rms_norm_row(const RmsNormArgs& a, int row, int lane) {
  const short* x = a.x + (int64_t)row * a.x_s;
  const int chunks = a.dim / 8;
  float ss = 0.0f;
  for (int j = lane; j < chunks; j += 64) {
    const i16x8 v = *reinterpret_cast<const i16x8*>(x + 8 * j);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float f = Elt<DT>::to_float(v[e]);
      ss += f * f;
    }
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) ss += __shfl_xor(ss, d);
  const float rstd = rsqrtf(ss / (float)a.dim + a.eps);
  short* y = a.y + (int64_t)row * a.y_s;
  for (int j = lane; j < chunks; j += 64) {
    const i16x8 v = *reinterpret_cast<const i16x8*>(x + 8 * j);
    i16x8 w8 = (i16x8)0;
    if (a.w) w8 = *reinterpret_cast<const i16x8*>(a.w + 8 * j);
    i16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float f = Elt<DT>::to_float(v[e]) * rstd;
      if (a.w) f = f * Elt<DT>::to_float(w8[e]);
      o[e] = Elt<DT>::from_float(f);
    }
    *reinterpret_cast<i16x8*>(y + 8 * j) = o;
  }
}

template <int DT>
__global__ __launch_bounds__(256) void mla_rms_norm_kernel(RmsNormArgs a) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row < a.rows) rms_norm_row<DT>(a, row, threadIdx.x & 63);  // wave-uniform
}

// The query latent's RMSNorm and the cache append of one step in one launch
// (they read different rows of the same GEMM output and do not depend on each
// other): workgroups [0, cdiv(rows, 4)) normalise query rows, the rest append
// one sequence per wave, with the same per-row code as the two kernels above.
template <int DT>
__global__ __launch_bounds__(256) void mla_norm_append_kernel(RmsNormArgs r, KvAppendArgs k) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nq = (r.rows + 3) / 4;
  if ((int)blockIdx.x < nq) {
    const int row = blockIdx.x * 4 + wave;
    if (row < r.rows) rms_norm_row<DT>(r, row, lane);
  } else {
    const int b = (blockIdx.x - nq) * 4 + wave;
    if (b < k.batch) kv_append_row<DT>(k, b, lane);
  }
}

// ---------------------------------------------------------------------------
// dense projection: grid (N / (16 CB), KS), 4 waves; y rows in MB blocks of 16
// ---------------------------------------------------------------------------
template <int DT>
__device__ __forceinline__ f32x4 mfma16(i16x8 a, i16x8 b, f32x4 c) {
  if constexpr (DT == TMLA_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
}

// Partial tiles are exchanged between the workgroups of one column group
// through memory within the launch: written through to memory (sc0 sc1),
// counted with a system-scope atomic, read back with loads that bypass the
// caches (sc0 sc1), so no cache maintenance is needed between workgroups on
// different XCDs.
__device__ __forceinline__ void store_through16(void* p, f32x4 v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc0 sc1\n\ts_nop 1" : : "v"(p), "v"(v) : "memory");
}
constexpr int kBufferWord3 = 0x00020000;  // raw buffer resource word 3 (32-bit data format)
constexpr int kSysCoherent = 1 | 16;      // sc0 | sc1

// Workgroup = output columns [16 CB * blockIdx.x, +16 CB) over chunks (64
// contraction elements, 128 bytes of a weight row) [ks * C / KS,
// (ks + 1) * C / KS) of the C = K / 64, ks = blockIdx.y; its 4 waves split
// that range evenly. Each wave streams its chunks of the group's weight rows
// into its own LDS slots with LDS-DMA (8 rows x 128 bytes per copy: whole
// cache lines, one chunk ahead of its MFMAs), so no barrier is needed, and
// reads them back as MFMA operands. v_mfma_f32_16x16x32: A = x rows (lane:
// row lane % 16), B = W rows (lane: column lane % 16), D lane: column
// lane % 16, rows 4 * (lane / 16) .. +4; k-step s of a chunk gives lane
// group q = lane / 16 the elements 8 * (4 s + q) .. +8 of the chunk (the
// same for x and W). The 16-byte piece p of row r of an 8-row block sits at
// p ^ r, which keeps both the copies (one row per 8 lanes) and the operand
// reads (16 rows, one piece each) free of bank conflicts. x costs MB KiB per
// k-step from L2 against CB KiB of weights. The waves' tiles are summed in
// LDS in wave order; with KS > 1 each workgroup stores its tile to the
// workspace and the last of the column group's KS workgroups to arrive sums
// the KS tiles in ks order, writes y and resets the group's counter, so the
// result does not depend on arrival order.
template <int DT, int MB, int CB>
__global__ __launch_bounds__(256) void mla_project_kernel(ProjectArgs a) {
  constexpr int NW = 4;
  constexpr int NT = MB * CB;             // 16 x 16 tiles per workgroup
  constexpr int SLOT = CB * 2 * 1024;     // one chunk of the group's rows: CB x 2 blocks of 8 rows x 128 B
  constexpr int WAVE_LDS = 2 * SLOT;      // two slots per wave
  static_assert(NW * WAVE_LDS >= NW * NT * 1024, "tile sums fit the staging area");
  __shared__ __attribute__((aligned(1024))) char smem[NW * WAVE_LDS];
  __shared__ int s_last;
  char LDS_AS* const lds = (char LDS_AS*)(void LDS_AS*)smem;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n0 = blockIdx.x * 16 * CB;
  const int C = a.k / 64, KS = gridDim.y, ks = blockIdx.y;
  const int r0 = ks * C / KS, r1 = (ks + 1) * C / KS;
  const int c0 = r0 + wave * (r1 - r0) / NW, c1 = r0 + (wave + 1) * (r1 - r0) / NW;
  const int c = lane & 15, q = lane >> 4;
  char LDS_AS* const mine = lds + wave * WAVE_LDS;
  // copies: lane -> row 8 h + lane / 8 of column block cb, piece (lane % 8) ^ (lane / 8)
  const int dr = lane >> 3, dp = (lane & 7) ^ dr;
  const char* wsrc[CB][2];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      wsrc[cb][h] = reinterpret_cast<const char*>(a.w + (int64_t)(n0 + 16 * cb + 8 * h + dr) * a.w_s) + dp * 16;
  auto issue = [&](int ch, int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        lds_copy16<0>(wsrc[cb][h] + (int64_t)ch * 128, mine + slot * SLOT + (cb * 2 + h) * 1024);
  };
  // operand reads: row c of column block cb = block 2 cb + c / 8, row c % 8, piece (4 s + q) ^ (c % 8)
  const int rd0 = (c >> 3) * 1024 + (c & 7) * 128;
  const short* xp[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int row = min(mb * 16 + c, a.m - 1);  // rows past M repeat the last (never stored)
    xp[mb] = a.x + (int64_t)row * a.x_s + q * 8;
  }
  f32x4 acc[MB][CB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) acc[mb][cb] = (f32x4)0.0f;
  if (c0 < c1) issue(c0, 0);
  for (int ch = c0; ch < c1; ++ch) {
    const int slot = (ch - c0) & 1;
    i16x8 xv[2][MB];
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        xv[st][mb] = *reinterpret_cast<const i16x8*>(xp[mb] + (int64_t)ch * 64 + 32 * st);
    if (ch + 1 < c1) {
      issue(ch + 1, slot ^ 1);  // the next chunk in flight while this one is used
      wait_vmcnt<2 * CB>();     // this chunk's copies and x loads have landed
    } else {
      wait_vmcnt<0>();
    }
    asm volatile("" ::: "memory");  // the operand reads below stay after the wait
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const int off = rd0 + (((4 * st + q) ^ (c & 7)) << 4);
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const i16x8 wv = *reinterpret_cast<const i16x8 LDS_AS*>(mine + slot * SLOT + cb * 2048 + off);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[mb][cb] = mfma16<DT>(xv[st][mb], wv, acc[mb][cb]);
      }
    }
  }
  __syncthreads();  // every wave is done with its staging slots
  f32x4 LDS_AS* red = (f32x4 LDS_AS*)lds;  // [NW][NT][64]
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) red[(wave * NT + mb * CB + cb) * 64 + lane] = acc[mb][cb];
  __syncthreads();

  // tile entry e = (mb * CB + cb) * 64 + lane holds rows mb * 16 + 4 * (lane / 16) .. +4 of column
  // n0 + 16 * cb + lane % 16
  auto sum_waves = [&](int e) __attribute__((always_inline)) {
    f32x4 v = red[e];
#pragma unroll
    for (int w = 1; w < NW; ++w) v += red[w * NT * 64 + e];
    return v;
  };
  auto store_y = [&](int e, f32x4 v) __attribute__((always_inline)) {
    const int t = e >> 6, l = e & 63, mb = t / CB, cb = t % CB;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = mb * 16 + 4 * (l >> 4) + r;
      if (row < a.m) a.y[(int64_t)row * a.y_s + n0 + 16 * cb + (l & 15)] = Elt<DT>::from_float(v[r]);
    }
  };
  if (KS == 1) {
    for (int e = tid; e < NT * 64; e += 256) store_y(e, sum_waves(e));
    return;
  }
  float* part = a.ws + ((int64_t)blockIdx.x * KS) * NT * 256;  // [KS][NT * 64] f32x4 of this column group
  for (int e = tid; e < NT * 64; e += 256) store_through16(part + ((int64_t)ks * NT * 64 + e) * 4, sum_waves(e));
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's stores are complete
  __syncthreads();
  if (tid == 0) {
    // the tiles were written through to memory and their stores completed
    // before this arrival; the last workgroup reads them past its caches
    const int old = __hip_atomic_fetch_add(a.cnt + blockIdx.x, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    s_last = old == KS - 1;
  }
  __syncthreads();
  if (!s_last) return;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(part, 0, KS * NT * 64 * 16, kBufferWord3);
  for (int e = tid; e < NT * 64; e += 256) {
    f32x4 v = (f32x4)0.0f;
    for (int j = 0; j < KS; ++j)
      v += __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (j * NT * 64 + e) * 16, 0,
                                                                           kSysCoherent));
    store_y(e, v);
  }
  if (tid == 0) __hip_atomic_store(a.cnt + blockIdx.x, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Launch shape of a projection: 64 columns per workgroup when N allows (x
// read once per 4 weight tiles), and the contraction split over KS
// workgroups so that about kProjectTargetWGs workgroups cover the chip,
// with at least one 64-element chunk per wave.
#ifndef TMLA_PROJECT_TARGET_WGS
#define TMLA_PROJECT_TARGET_WGS 512
#endif
constexpr int kProjectTargetWGs = TMLA_PROJECT_TARGET_WGS;  // two resident per compute unit
// The workspace starts with a fixed block of arrival counters (one per
// column group, at most kProjectCounterBytes / 4 groups), the partial tiles
// follow: whatever the shapes of the calls that share a workspace, no call's
// tiles overlap any call's counters, and every call leaves its counters at
// zero.
constexpr size_t kProjectCounterBytes = 64 * 1024;
struct ProjectPlan {
  int cb, ks, groups;
  size_t part_bytes, cnt_bytes;
};
ProjectPlan project_plan(int32_t m, int32_t n, int32_t k) {
  ProjectPlan p;
  p.cb = n % 64 == 0 ? 4 : 1;
  p.groups = n / (16 * p.cb);
  const int chunks = k / 64;
  int ks = kProjectTargetWGs / p.groups;  // one round of resident workgroups
  ks = min(ks, chunks / 4);  // at least one chunk per wave
  p.ks = max(ks, 1);
  const int mb = (m + 15) / 16;
  p.part_bytes = p.ks > 1 ? (size_t)p.groups * p.ks * mb * p.cb * 64 * 16 : 0;
  p.cnt_bytes = p.ks > 1 ? kProjectCounterBytes : 0;
  return p;
}

template <int DT, int MB>
hipError_t launch_project(const ProjectArgs& a, const ProjectPlan& p, hipStream_t s) {
  const dim3 grid(p.groups, p.ks);
  if (p.cb == 4)
    hipLaunchKernelGGL((mla_project_kernel<DT, MB, 4>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((mla_project_kernel<DT, MB, 1>), grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int DT>
hipError_t launch_project_dt(const ProjectArgs& a, const ProjectPlan& p, hipStream_t s) {
  switch ((a.m + 15) / 16) {
    case 1: return launch_project<DT, 1>(a, p, s);
    case 2: return launch_project<DT, 2>(a, p, s);
    case 3: return launch_project<DT, 3>(a, p, s);
    default: return launch_project<DT, 4>(a, p, s);
  }
}

}  // namespace layer

extern int hip_fail(hipError_t e, const char* where);

}  // namespace tmla

using namespace tmla;
using namespace tmla::layer;

extern "C" {

int tmla_mla_absorb_q(const void* q_proj, int64_t q_proj_stride_b, const void* wkv_b, int64_t wkv_b_stride_0,
                      const int32_t* positions, int32_t batch, int32_t num_heads, int32_t qk_nope_dim,
                      int32_t qk_rope_dim, int32_t kv_lora_rank, int32_t v_head_dim, float rope_theta,
                      int32_t dtype, void* q_out, int64_t q_out_stride_b, int64_t q_out_stride_h, void* stream) {
  if (batch < 0 || num_heads <= 0) return fail(TMLA_ERR_INVALID_ARGUMENT, "batch must be >= 0 and num_heads > 0");
  if (dtype != TMLA_BF16 && dtype != TMLA_FP16) return fail(TMLA_ERR_INVALID_ARGUMENT, "dtype must be TMLA_BF16 or TMLA_FP16");
  if (qk_nope_dim != kNope || qk_rope_dim != kRope || kv_lora_rank <= 0 || kv_lora_rank % kColsWG != 0 || v_head_dim <= 0)
    return fail(TMLA_ERR_UNSUPPORTED, "absorb_q is built for qk_nope_dim 128, qk_rope_dim 64, kv_lora_rank a multiple of 128");
  if (batch == 0) return TMLA_OK;
  if (!q_proj || !wkv_b || !positions || !q_out) return fail(TMLA_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (((uintptr_t)q_proj | (uintptr_t)wkv_b | (uintptr_t)q_out) & 15)
    return fail(TMLA_ERR_INVALID_ARGUMENT, "q_proj, wkv_b and q_out must be 16-byte aligned");
  if ((q_proj_stride_b | wkv_b_stride_0 | q_out_stride_b | q_out_stride_h) & 7)
    return fail(TMLA_ERR_INVALID_ARGUMENT, "strides must be multiples of 8 elements");
  AbsorbQArgs a{};
  a.qp = static_cast<const short*>(q_proj);
  a.qp_sb = q_proj_stride_b;
  a.w = static_cast<const short*>(wkv_b);
  a.w_s0 = wkv_b_stride_0;
  a.pos = positions;
  a.out = static_cast<short*>(q_out);
  a.out_sb = q_out_stride_b;
  a.out_sh = q_out_stride_h;
  a.batch = batch;
  a.heads = num_heads;
  a.rank = kv_lora_rank;
  a.vd = v_head_dim;
  a.theta = rope_theta;
  dim3 grid(num_heads, kv_lora_rank / kColsWG, (batch + kBTile - 1) / kBTile);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == TMLA_BF16)
    hipLaunchKernelGGL(mla_absorb_q_kernel<TMLA_BF16>, grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(mla_absorb_q_kernel<TMLA_FP16>, grid, dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? TMLA_OK : hip_fail(e, "mla_absorb_q_kernel launch");
}

int tmla_mla_absorb_out(const void* o_latent, int64_t o_stride_b, int64_t o_stride_h, const void* wkv_b,
                        int64_t wkv_b_stride_0, int32_t batch, int32_t num_heads, int32_t qk_nope_dim,
                        int32_t kv_lora_rank, int32_t v_head_dim, int32_t dtype, void* out, int64_t out_stride_b,
                        void* stream) {
  if (batch < 0 || num_heads <= 0) return fail(TMLA_ERR_INVALID_ARGUMENT, "batch must be >= 0 and num_heads > 0");
  if (dtype != TMLA_BF16 && dtype != TMLA_FP16) return fail(TMLA_ERR_INVALID_ARGUMENT, "dtype must be TMLA_BF16 or TMLA_FP16");
  if (v_head_dim <= 0 || v_head_dim % 32 != 0 || kv_lora_rank <= 0 || kv_lora_rank % 512 != 0 || qk_nope_dim < 0)
    return fail(TMLA_ERR_UNSUPPORTED, "absorb_out is built for v_head_dim a multiple of 32 and kv_lora_rank a multiple of 512");
  if (batch == 0) return TMLA_OK;
  if (!o_latent || !wkv_b || !out) return fail(TMLA_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (((uintptr_t)o_latent | (uintptr_t)wkv_b | (uintptr_t)out) & 15)
    return fail(TMLA_ERR_INVALID_ARGUMENT, "o_latent, wkv_b and out must be 16-byte aligned");
  if ((o_stride_b | o_stride_h | wkv_b_stride_0 | out_stride_b) & 7)
    return fail(TMLA_ERR_INVALID_ARGUMENT, "strides must be multiples of 8 elements");
  AbsorbOutArgs a{};
  a.o = static_cast<const short*>(o_latent);
  a.o_sb = o_stride_b;
  a.o_sh = o_stride_h;
  a.w = static_cast<const short*>(wkv_b);
  a.w_s0 = wkv_b_stride_0;
  a.out = static_cast<short*>(out);
  a.out_sb = out_stride_b;
  a.batch = batch;
  a.heads = num_heads;
  a.nope = qk_nope_dim;
  a.rank = kv_lora_rank;
  a.vd = v_head_dim;
  dim3 grid(num_heads, v_head_dim / 32, (batch + kBTile - 1) / kBTile);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == TMLA_BF16)
    hipLaunchKernelGGL(mla_absorb_out_kernel<TMLA_BF16>, grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(mla_absorb_out_kernel<TMLA_FP16>, grid, dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? TMLA_OK : hip_fail(e, "mla_absorb_out_kernel launch");
}

}  // extern "C"

namespace {

// Checks the arguments of a cache append and fills its kernel arguments;
// TMLA_OK with batch 0 means nothing to do.
int kv_append_args(const void* kv_proj, int64_t kv_proj_stride_b, const void* norm_weight, float eps,
                   float rope_theta, const int32_t* positions, int32_t batch, int32_t kv_lora_rank, int32_t rope_dim,
                   int32_t dtype, void* kv_cache, int64_t kv_stride_0, int64_t kv_stride_1, int64_t num_blocks,
                   int32_t page_size, const int32_t* block_table, int64_t bt_stride_b, int32_t bt_cols,
                   KvAppendArgs& a) {
  a = KvAppendArgs{};
  if (batch < 0) return fail(TMLA_ERR_INVALID_ARGUMENT, "batch must be >= 0");
  if (dtype != TMLA_BF16 && dtype != TMLA_FP16) return fail(TMLA_ERR_INVALID_ARGUMENT, "dtype must be TMLA_BF16 or TMLA_FP16");
  if (rope_dim != kRope || kv_lora_rank <= 0 || kv_lora_rank % 64 != 0 || kv_lora_rank > 1024)
    return fail(TMLA_ERR_UNSUPPORTED, "kv_append is built for rope_dim 64 and kv_lora_rank a multiple of 64 up to 1024");
  if (batch == 0) return TMLA_OK;
  if (!kv_proj || !positions || !kv_cache) return fail(TMLA_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (num_blocks <= 0 || page_size <= 0) return fail(TMLA_ERR_INVALID_ARGUMENT, "num_blocks and page_size must be > 0");
  if (block_table && bt_cols <= 0) return fail(TMLA_ERR_INVALID_ARGUMENT, "block_table needs at least one column");
  if (!block_table && page_size != 1) return fail(TMLA_ERR_INVALID_ARGUMENT, "dense cache requires page_size == 1");
  a.kvp = static_cast<const short*>(kv_proj);
  a.kvp_sb = kv_proj_stride_b;
  a.norm_w = static_cast<const short*>(norm_weight);
  a.eps = eps;
  a.theta = rope_theta;
  a.pos = positions;
  a.cache = static_cast<char*>(kv_cache);
  a.s0 = kv_stride_0 * 2;
  a.s1 = kv_stride_1 * 2;
  a.num_blocks = num_blocks;
  a.page_size = page_size;
  a.bt = block_table;
  a.bt_sb = bt_stride_b;
  a.bt_cols = bt_cols;
  a.batch = batch;
  a.rank = kv_lora_rank;
  return TMLA_OK;
}

// Checks the arguments of a row RMSNorm and fills its kernel arguments; TMLA_OK
// with rows 0 means nothing to do.
int rms_norm_args(const void* x, int64_t x_stride, const void* weight, float eps, int32_t rows, int32_t dim,
                  int32_t dtype, void* y, int64_t y_stride, RmsNormArgs& a) {
  a = RmsNormArgs{};
  if (rows < 0 || dim <= 0) return fail(TMLA_ERR_INVALID_ARGUMENT, "rows must be >= 0 and dim > 0");
  if (dtype != TMLA_BF16 && dtype != TMLA_FP16) return fail(TMLA_ERR_INVALID_ARGUMENT, "dtype must be TMLA_BF16 or TMLA_FP16");
  if (dim % 8 != 0) return fail(TMLA_ERR_UNSUPPORTED, "rms_norm is built for dim a multiple of 8");
  if (rows == 0) return TMLA_OK;
  if (!x || !y) return fail(TMLA_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (((uintptr_t)x | (uintptr_t)y | (uintptr_t)weight) & 15)
    return fail(TMLA_ERR_INVALID_ARGUMENT, "x, weight and y must be 16-byte aligned");
  if ((x_stride | y_stride) & 7 || x_stride < dim || y_stride < dim)
    return fail(TMLA_ERR_INVALID_ARGUMENT, "row strides must be multiples of 8 elements and >= dim");
  a.x = static_cast<const short*>(x);
  a.x_s = x_stride;
  a.w = static_cast<const short*>(weight);
  a.y = static_cast<short*>(y);
  a.y_s = y_stride;
  a.eps = eps;
  a.rows = rows;
  a.dim = dim;
  return TMLA_OK;
}

}  // namespace

extern "C" {

int tmla_mla_kv_append(const void* kv_proj, int64_t kv_proj_stride_b, const void* norm_weight, float eps,
                       float rope_theta, const int32_t* positions, int32_t batch, int32_t kv_lora_rank,
                       int32_t rope_dim, int32_t dtype, void* kv_cache, int64_t kv_stride_0, int64_t kv_stride_1,
                       int64_t num_blocks, int32_t page_size, const int32_t* block_table, int64_t bt_stride_b,
                       int32_t bt_cols, void* stream) {
  KvAppendArgs a;
  const int rc = kv_append_args(kv_proj, kv_proj_stride_b, norm_weight, eps, rope_theta, positions, batch,
                                kv_lora_rank, rope_dim, dtype, kv_cache, kv_stride_0, kv_stride_1, num_blocks,
                                page_size, block_table, bt_stride_b, bt_cols, a);
  if (rc != TMLA_OK || batch == 0) return rc;
  dim3 grid((batch + 3) / 4);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == TMLA_BF16)
    hipLaunchKernelGGL(mla_kv_append_kernel<TMLA_BF16>, grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(mla_kv_append_kernel<TMLA_FP16>, grid, dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? TMLA_OK : hip_fail(e, "mla_kv_append_kernel launch");
}

int tmla_mla_rms_norm(const void* x, int64_t x_stride, const void* weight, float eps, int32_t rows, int32_t dim,
                      int32_t dtype, void* y, int64_t y_stride, void* stream) {
  RmsNormArgs a;
  const int rc = rms_norm_args(x, x_stride, weight, eps, rows, dim, dtype, y, y_stride, a);
  if (rc != TMLA_OK || rows == 0) return rc;
  dim3 grid((rows + 3) / 4);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == TMLA_BF16)
    hipLaunchKernelGGL(mla_rms_norm_kernel<TMLA_BF16>, grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(mla_rms_norm_kernel<TMLA_FP16>, grid, dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? TMLA_OK : hip_fail(e, "mla_rms_norm_kernel launch");
}

int tmla_mla_norm_append(const void* q_lat, int64_t q_lat_stride, const void* q_norm_weight, float q_eps,
                         int32_t q_dim, void* q_out, int64_t q_out_stride, const void* kv_proj,
                         int64_t kv_proj_stride_b, const void* kv_norm_weight, float kv_eps, float rope_theta,
                         const int32_t* positions, int32_t* next_positions, int32_t batch, int32_t kv_lora_rank,
                         int32_t rope_dim, int32_t dtype, void* kv_cache, int64_t kv_stride_0, int64_t kv_stride_1,
                         int64_t num_blocks, int32_t page_size, const int32_t* block_table, int64_t bt_stride_b,
                         int32_t bt_cols, void* stream) {
  RmsNormArgs r;
  KvAppendArgs k;
  int rc = rms_norm_args(q_lat, q_lat_stride, q_norm_weight, q_eps, batch, q_dim, dtype, q_out, q_out_stride, r);
  if (rc != TMLA_OK) return rc;
  rc = kv_append_args(kv_proj, kv_proj_stride_b, kv_norm_weight, kv_eps, rope_theta, positions, batch, kv_lora_rank,
                      rope_dim, dtype, kv_cache, kv_stride_0, kv_stride_1, num_blocks, page_size, block_table,
                      bt_stride_b, bt_cols, k);
  if (rc != TMLA_OK || batch == 0) return rc;
  if (!next_positions) return fail(TMLA_ERR_INVALID_ARGUMENT, "null pointer argument");
  k.pos_next = next_positions;
  dim3 grid(2 * ((batch + 3) / 4));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == TMLA_BF16)
    hipLaunchKernelGGL(mla_norm_append_kernel<TMLA_BF16>, grid, dim3(256), 0, s, r, k);
  else
    hipLaunchKernelGGL(mla_norm_append_kernel<TMLA_FP16>, grid, dim3(256), 0, s, r, k);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? TMLA_OK : hip_fail(e, "mla_norm_append_kernel launch");
}

size_t tmla_mla_project_workspace_bytes(int32_t m, int32_t n, int32_t k) {
  if (m <= 0 || m > kProjectMaxRows || n <= 0 || n % 16 != 0 || k <= 0 || k % 64 != 0) return 0;
  const ProjectPlan p = project_plan(m, n, k);
  return p.part_bytes + p.cnt_bytes;
}

int tmla_mla_project(const void* x, int64_t x_stride, const void* w, int64_t w_stride, int32_t m, int32_t n,
                     int32_t k, int32_t dtype, void* y, int64_t y_stride, void* workspace, size_t workspace_bytes,
                     void* stream) {
  if (m < 0 || n <= 0 || k <= 0) return fail(TMLA_ERR_INVALID_ARGUMENT, "m must be >= 0, n and k > 0");
  if (dtype != TMLA_BF16 && dtype != TMLA_FP16) return fail(TMLA_ERR_INVALID_ARGUMENT, "dtype must be TMLA_BF16 or TMLA_FP16");
  if (m > kProjectMaxRows || n % 16 != 0 || k % 64 != 0)
    return fail(TMLA_ERR_UNSUPPORTED, "project is built for m <= 64, n a multiple of 16 and k a multiple of 64");
  if (m == 0) return TMLA_OK;
  if (!x || !w || !y) return fail(TMLA_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (((uintptr_t)x | (uintptr_t)w) & 15 || (uintptr_t)y & 1)
    return fail(TMLA_ERR_INVALID_ARGUMENT, "x and w must be 16-byte aligned, y 2-byte aligned");
  if ((x_stride | w_stride) & 7 || x_stride < k || w_stride < k || y_stride < n)
    return fail(TMLA_ERR_INVALID_ARGUMENT, "x and w row strides must be multiples of 8 elements and >= k, y's >= n");
  const ProjectPlan p = project_plan(m, n, k);
  if (p.ks > 1 && (size_t)p.groups * 4 > kProjectCounterBytes)
    return fail(TMLA_ERR_UNSUPPORTED, "project splits the contraction of at most 16384 column groups");
  const size_t need = p.part_bytes + p.cnt_bytes;
  if (need > 0 && (workspace == nullptr || workspace_bytes < need || ((uintptr_t)workspace & 255)))
    return fail(TMLA_ERR_WORKSPACE_TOO_SMALL,
                "workspace is missing, smaller than tmla_mla_project_workspace_bytes() or not 256-byte aligned");
  ProjectArgs a{};
  a.x = static_cast<const short*>(x);
  a.x_s = x_stride;
  a.w = static_cast<const short*>(w);
  a.w_s = w_stride;
  a.y = static_cast<short*>(y);
  a.y_s = y_stride;
  a.m = m;
  a.n = n;
  a.k = k;
  if (need > 0) {
    a.cnt = static_cast<int32_t*>(workspace);
    a.ws = reinterpret_cast<float*>(static_cast<char*>(workspace) + kProjectCounterBytes);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = dtype == TMLA_BF16 ? launch_project_dt<TMLA_BF16>(a, p, s) : launch_project_dt<TMLA_FP16>(a, p, s);
  return e == hipSuccess ? TMLA_OK : hip_fail(e, "mla_project_kernel launch");
}

}  // extern "C"
