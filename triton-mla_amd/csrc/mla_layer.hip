// MLA layer glue for MI355X (gfx950): the absorbed-projection steps on
// either side of mla_decode in the DeepSeek MLA decode layer, and their C ABI
// (include/triton_mla.h).
//
// Reference behaviour: src/triton_mla/model.py:74-124 (MLA._project's RoPE,
// MLA._append_kv, the W_UK and W_UV einsums of MLA.forward), apply_rope
// model.py:44-50, RMSNorm model.py:34-41. The dense projections (wq_a, wq_b,
// wkv_a, wo) stay library GEMMs.
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
#include <math.h>
#include <stdio.h>

#include "cdna.h"
#include "triton_mla.h"

namespace tmla {

namespace layer {

constexpr int kNope = 128;   // qk_nope_head_dim the q kernel is built for
constexpr int kRope = 64;    // qk_rope_head_dim
constexpr int kColsWG = 128; // W_UK columns per workgroup (4 waves x 1 block of 32)
constexpr int kBTile = 32;   // batch rows per MFMA block (N of the 32x32x16 MFMA)

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
  char* cache;           // paged [num_blocks, page_size, rank+rope] or dense [B, capacity, rank+rope]
  int64_t s0, s1;        // byte strides
  int64_t num_blocks;    // pages (paged) or capacity (dense)
  int32_t page_size;
  const int32_t* bt;     // [B, bt_cols] or null (dense)
  int64_t bt_sb;
  int32_t bt_cols, batch, rank;
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

  // RoPE of q_pe: the first column block of every batch tile; rows x pairs
  // over the 256 threads
  if (blockIdx.y == 0) {
    for (int idx = threadIdx.x; idx < kBTile * (kRope / 2); idx += 256) {
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
__global__ __launch_bounds__(256) void mla_kv_append_kernel(KvAppendArgs a) {
  const int lane = threadIdx.x & 63;
  const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (b >= a.batch) return;
  const int pos = a.pos[b];
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

}  // namespace layer

extern int fail(int code, const char* msg);
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

int tmla_mla_kv_append(const void* kv_proj, int64_t kv_proj_stride_b, const void* norm_weight, float eps,
                       float rope_theta, const int32_t* positions, int32_t batch, int32_t kv_lora_rank,
                       int32_t rope_dim, int32_t dtype, void* kv_cache, int64_t kv_stride_0, int64_t kv_stride_1,
                       int64_t num_blocks, int32_t page_size, const int32_t* block_table, int64_t bt_stride_b,
                       int32_t bt_cols, void* stream) {
  if (batch < 0) return fail(TMLA_ERR_INVALID_ARGUMENT, "batch must be >= 0");
  if (dtype != TMLA_BF16 && dtype != TMLA_FP16) return fail(TMLA_ERR_INVALID_ARGUMENT, "dtype must be TMLA_BF16 or TMLA_FP16");
  if (rope_dim != kRope || kv_lora_rank <= 0 || kv_lora_rank % 64 != 0 || kv_lora_rank > 1024)
    return fail(TMLA_ERR_UNSUPPORTED, "kv_append is built for rope_dim 64 and kv_lora_rank a multiple of 64 up to 1024");
  if (batch == 0) return TMLA_OK;
  if (!kv_proj || !positions || !kv_cache) return fail(TMLA_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (num_blocks <= 0 || page_size <= 0) return fail(TMLA_ERR_INVALID_ARGUMENT, "num_blocks and page_size must be > 0");
  if (block_table && bt_cols <= 0) return fail(TMLA_ERR_INVALID_ARGUMENT, "block_table needs at least one column");
  if (!block_table && page_size != 1) return fail(TMLA_ERR_INVALID_ARGUMENT, "dense cache requires page_size == 1");
  KvAppendArgs a{};
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
  dim3 grid((batch + 3) / 4);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == TMLA_BF16)
    hipLaunchKernelGGL(mla_kv_append_kernel<TMLA_BF16>, grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(mla_kv_append_kernel<TMLA_FP16>, grid, dim3(256), 0, s, a);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? TMLA_OK : hip_fail(e, "mla_kv_append_kernel launch");
}

}  // extern "C"
