// Host-side planning of a decode call: argument checks, the workspace
// layout and the launch shape. Plain C++ with no HIP dependency, so that
// the same code is also compiled for the CPU with the address and
// undefined-behaviour sanitizers (tests/plan_sanitize.cpp).
//
// All size arithmetic is done in 64 bits and checked: a call whose
// workspace would not fit in 2^62 bytes is rejected (workspace_bytes
// returns 0 for it), so no size can wrap around to a small value.
#pragma once

#include <stddef.h>
#include <stdint.h>
#include <stdio.h>

#include "triton_mla.h"

namespace tmla {

constexpr int kTileTokens = 64;                   // planning unit (one page at page_size 64)
// Balanced partition with straddling ranges: tiles charged for the start of
// each sequence in a worker's range (its segment's start-up and finalize)
#ifndef TMLA_SEG_COST_TILES
#define TMLA_SEG_COST_TILES 2
#endif
constexpr int kSegCostTiles = TMLA_SEG_COST_TILES;
constexpr size_t kFusedCounterBytes = 256 * 1024;  // the single launch's counter block
constexpr int64_t kMaxWorkspaceBytes = (int64_t)1 << 62;

inline thread_local char g_err[512] = "no error";

inline int fail(int code, const char* msg) {
  snprintf(g_err, sizeof(g_err), "%s", msg);
  return code;
}

// Workgroups per worker along the heads (32, 64 or 128 heads each).
inline int64_t head_blocks(int32_t heads) {
  const int64_t per = heads <= 32 ? 32 : heads <= 64 ? 64 : 128;
  return ((int64_t)heads + per - 1) / per;
}

// Partial slots of a call: batch * num_splits (uniform) or num_workers +
// batch (balanced).
inline int64_t partial_slots(int32_t batch, int32_t splits, int32_t workers) {
  return splits > 0 ? (int64_t)batch * splits : (int64_t)workers + batch;
}

// Workspace of a call: partial rows [slots, H, dv] (input dtype) at offset 0,
// their base-2 lse [slots, H] (float) after them, and the fused merge's int32
// counters m_count and m_done [batch, head blocks] and flags m_flag [slots,
// head blocks] at the start of a block of fixed size (kFusedCounterBytes)
// anchored at the END of the caller's buffer (its size rounded down to 256
// bytes). Every call reserves the whole block, so no call's partials reach
// it, whatever the shapes of the calls that share the buffer: the block is
// zero-filled once, and every single launch leaves its counters at zero
// again. A call whose counters exceed the block runs as two kernels.
struct WsLayout {
  size_t o, l, part_end;  // byte offsets: partial rows, lse, end of both
  size_t cnt_bytes;       // counter block (a multiple of 256)
  size_t total;           // part_end + cnt_bytes: the bytes the call needs; 0 if too large
};

inline WsLayout ws_layout(int32_t batch, int32_t heads, int32_t dv, int32_t splits, int32_t workers) {
  WsLayout w{0, 0, 0, kFusedCounterBytes, 0};
  const int64_t slots = partial_slots(batch, splits, workers);
  if (slots < 0 || heads < 0 || dv < 0) return w;
  // rows = slots * heads, each dv * 2 bytes, all below 2^62
  if (heads > 0 && slots > kMaxWorkspaceBytes / heads) return w;
  const int64_t rows = slots * heads;
  if (rows > 0 && (int64_t)dv * 2 > kMaxWorkspaceBytes / rows) return w;
  const int64_t o_bytes = rows * dv * 2, l_bytes = rows * 4;
  auto al = [](int64_t x) { return (x + 255) & ~(int64_t)255; };
  const int64_t total = al(o_bytes) + al(l_bytes) + (int64_t)kFusedCounterBytes;
  if (total > kMaxWorkspaceBytes) return w;
  w.o = 0;
  w.l = (size_t)al(o_bytes);
  w.part_end = w.l + (size_t)al(l_bytes);
  w.total = w.part_end + w.cnt_bytes;
  return w;
}

// 0 for invalid or too large arguments
inline size_t workspace_bytes(int32_t batch, int32_t heads, int32_t dv, int32_t splits, int32_t workers) {
  if (batch < 0 || heads <= 0 || dv < 0) return 0;
  return ws_layout(batch, heads, dv, splits, workers).total;
}

// Bytes of the fused merge's counters and flags of a call whose grid has gy
// workgroups along the heads.
inline int64_t fused_counter_bytes(int32_t batch, int64_t gy, int32_t splits, int32_t workers) {
  return (2 * (int64_t)batch + partial_slots(batch, splits, workers)) * gy * 4;
}

// Workgroups along the workers: all of them for uniform splits; for the
// balanced partition no more than the 64-token tiles the call can hold
// (block-table width or dense capacity: capacity_tokens per sequence), since
// workers past them never get a range. At least 1, at most INT32_MAX.
inline int64_t worker_grid(int32_t batch, int32_t num_splits, int32_t num_workers, int64_t capacity_tokens) {
  if (num_splits > 0) {
    const int64_t w = (int64_t)batch * num_splits;
    return w < 1 ? 1 : (w > INT32_MAX ? INT32_MAX : w);
  }
  const int64_t cap = capacity_tokens > 0 ? capacity_tokens : 0;
  const int64_t tiles_per_seq = cap / kTileTokens + (cap % kTileTokens != 0);
  // batch * tiles_per_seq, saturated
  const int64_t tile_bound =
      batch > 0 && tiles_per_seq > INT64_MAX / batch ? INT64_MAX : (int64_t)(batch > 0 ? batch : 0) * tiles_per_seq;
  const int64_t w = tile_bound < num_workers ? tile_bound : num_workers;
  return w < 1 ? 1 : w;
}

// Launch shape of a decode call: blocks of 32 heads per workgroup (1, 2 or 4)
// and the grid, and whether the single launch merges in-kernel.
struct LaunchPlan {
  int nhb;
  int64_t grid_x, grid_y;
  bool fused;
};

// capacity_tokens: tokens the block table (or dense cache) can hold per
// sequence; mode as in decode_launch (1: the single launch if it fits);
// cus: compute units of the device.
inline LaunchPlan plan_launch(int32_t batch, int32_t num_heads, int32_t num_splits, int32_t num_workers,
                              int64_t capacity_tokens, size_t mid_o_bytes, int mode, int cus) {
  LaunchPlan p;
  p.nhb = num_heads <= 32 ? 1 : num_heads <= 64 ? 2 : 4;
  // When the busy workgroups would leave compute units idle, fewer heads per
  // workgroup (more, shorter workgroups: less Q to load, less MFMA work per
  // sub-tile, smaller partial rows) use them. (Halving keeps grid.x * grid.y
  // within the compute units, so it never takes a call off the single launch.)
  const int64_t heads = num_heads > 0 ? num_heads : 1;
  p.grid_x = worker_grid(batch, num_splits, num_workers, capacity_tokens);
  while (p.nhb > 1 && p.grid_x * ((heads + 16 * p.nhb - 1) / (16 * p.nhb)) <= cus) p.nhb /= 2;
  const int64_t heads_per_wg = 32 * p.nhb;
  p.grid_y = (heads + heads_per_wg - 1) / heads_per_wg;
  // The fused merge: one workgroup per compute unit at most (the kernel's LDS
  // use admits one), so that siblings normally run side by side; its
  // counters (per sequence and per slot, for each workgroup along the heads)
  // fit the workspace's counter block.
  p.fused = mode == 1 && p.grid_x * p.grid_y <= cus && mid_o_bytes < (size_t)INT32_MAX &&
            fused_counter_bytes(batch, p.grid_y, num_splits, num_workers) <= (int64_t)kFusedCounterBytes;
  return p;
}

// Launch shape of a call that runs the 16-head-group kernel (workgroups of
// 16 heads along grid.y); the single launch under the conditions of
// plan_launch.
inline LaunchPlan plan_launch_g16(int32_t batch, int32_t num_heads, int32_t num_splits, int32_t num_workers,
                                  int64_t capacity_tokens, size_t mid_o_bytes, int mode, int cus) {
  LaunchPlan p;
  p.nhb = 0;
  p.grid_x = worker_grid(batch, num_splits, num_workers, capacity_tokens);
  p.grid_y = ((int64_t)(num_heads > 0 ? num_heads : 1) + 15) / 16;
  p.fused = mode == 1 && p.grid_x * p.grid_y <= cus && mid_o_bytes < (size_t)INT32_MAX &&
            fused_counter_bytes(batch, p.grid_y, num_splits, num_workers) <= (int64_t)kFusedCounterBytes;
  return p;
}

struct Common {
  int32_t batch, heads, dv, dr, dtype, splits, workers;
};

inline int check_common(const Common& c, const void* workspace, size_t ws_bytes) {
  if (c.batch < 0 || c.heads <= 0) return fail(TMLA_ERR_INVALID_ARGUMENT, "batch must be >= 0 and num_heads > 0");
  if (c.dtype != TMLA_BF16 && c.dtype != TMLA_FP16) return fail(TMLA_ERR_INVALID_ARGUMENT, "dtype must be TMLA_BF16 or TMLA_FP16");
  if (c.splits < 0) return fail(TMLA_ERR_INVALID_ARGUMENT, "num_splits must be >= 0");
  if (c.splits == 0 && c.workers <= 0) return fail(TMLA_ERR_INVALID_ARGUMENT, "num_workers must be > 0 when num_splits == 0");
  if (c.splits > 0 && (int64_t)c.batch * c.splits > INT32_MAX) return fail(TMLA_ERR_INVALID_ARGUMENT, "batch * num_splits overflows");
  if (c.dv != 512) return fail(TMLA_ERR_UNSUPPORTED, "head_dim_v must be 512");
  const size_t need = workspace_bytes(c.batch, c.heads, c.dv, c.splits, c.workers);
  if (need == 0) return fail(TMLA_ERR_INVALID_ARGUMENT, "the call's workspace would exceed 2^62 bytes");
  if (workspace == nullptr || ws_bytes < need)
    return fail(TMLA_ERR_WORKSPACE_TOO_SMALL, "workspace is missing or smaller than tmla_workspace_bytes()");
  return TMLA_OK;
}

// ---------------------------------------------------------------------------
// The generic decode: head dims and element types outside the specialised
// kernels (any power-of-two head_dim_v in [16, 1024] and rope_dim in
// [16, 256]; bf16, fp16 or fp32), with the reference's uniform splits and
// float32 partials [batch, heads, splits, dv] plus their base-2 lse
// [batch, heads, splits].
// ---------------------------------------------------------------------------
constexpr int kGenHeads = 16;                   // heads per workgroup (4 per wave)
constexpr int kGenSmallLds = 64 * 1024;         // two workgroups per compute unit
constexpr int kGenLargeLds = 152 * 1024;        // one
constexpr int kGenProbBytes = 4 * 64 * 4 * 4;   // probabilities: [waves][tokens][4 heads] float
constexpr int kGenMaxSplits = 65535;            // grid.y of the partial kernel
constexpr int kGenMaxBatchHeads = 65535;        // grid.z of the partial kernel, grid.y of the merge

inline bool pow2_between(int64_t x, int64_t lo, int64_t hi) { return x >= lo && x <= hi && (x & (x - 1)) == 0; }
inline int elem_bytes(int32_t dtype) { return dtype == TMLA_FP32 ? 4 : 2; }

struct GenericPlan {
  int lds;    // LDS bytes of the kernel form (kGenSmallLds or kGenLargeLds)
  int tile;   // tokens staged per step: a power of two in [1, 64]
  int pitch;  // LDS bytes per staged row: the row plus 16 bytes of padding
};

// LDS of a workgroup: Q of its heads in float (64 * D bytes), the
// probabilities, and `tile` rows. The small form when it holds at least 16
// rows. Valid for dims accepted by check_generic (D <= 1280: the large form
// holds at least 8 fp32 rows beside Q).
inline GenericPlan generic_plan(int32_t dv, int32_t dr, int32_t dtype) {
  const int64_t d = (int64_t)dv + dr;
  GenericPlan p;
  p.pitch = (int)(d * elem_bytes(dtype) + 16);
  auto tile_in = [&](int lds) {
    const int64_t room = lds - 64 * d - kGenProbBytes;
    int t = 64;
    while (t > 0 && (int64_t)t * p.pitch > room) t >>= 1;
    return t;
  };
  const int small = tile_in(kGenSmallLds);
  if (small >= 16) {
    p.lds = kGenSmallLds;
    p.tile = small;
  } else {
    p.lds = kGenLargeLds;
    p.tile = tile_in(kGenLargeLds);
  }
  return p;
}

// The matrix-core form of the generic decode (bf16 / fp16, head_dim_v <= 512,
// D = head_dim_v + rope_dim <= 576): workgroups of 4 waves x 16 heads over
// 32-token steps. LDS: the rows (32 x (2D + 16) bytes), the value dims
// transposed ([dv][32 tokens], 80-byte rows), the probabilities (4 waves x
// 16 heads x 80 bytes) and Q (64 heads x (2D + 16) bytes) (the 16-byte
// paddings are kGenRowPad and kGenMP - 64). 0 when the form
// does not apply; else the LDS form (kGenMfmaSmallLds: two workgroups per
// compute unit, or kGenMfmaLargeLds).
constexpr int kGenMfmaTokens = 32;
constexpr int kGenMfmaHeads = 64;
// padding bytes of the staged rows and of the transposed rows (bank spread)
#ifndef TMLA_GEN_ROW_PAD
#define TMLA_GEN_ROW_PAD 16
#endif
#ifndef TMLA_GEN_MP_PAD
#define TMLA_GEN_MP_PAD 16
#endif
constexpr int kGenRowPad = TMLA_GEN_ROW_PAD;
constexpr int kGenMP = 2 * kGenMfmaTokens + TMLA_GEN_MP_PAD;
constexpr int kGenMfmaSmallLds = 78 * 1024;
constexpr int kGenMfmaLargeLds = 156 * 1024;

inline int64_t generic_mfma_lds_need(int32_t dv, int32_t dr) {
  const int64_t d = (int64_t)dv + dr;
  return kGenMfmaTokens * (2 * d + kGenRowPad) + (int64_t)dv * kGenMP + 4 * 16 * kGenMP +
         kGenMfmaHeads * (2 * d + kGenRowPad);
}

inline int generic_mfma_form(int32_t dv, int32_t dr, int32_t dtype) {
  if (dtype != TMLA_BF16 && dtype != TMLA_FP16) return 0;
  if (dv > 512 || (int64_t)dv + dr > 576) return 0;
  const int64_t need = generic_mfma_lds_need(dv, dr);
  return need <= kGenMfmaSmallLds ? kGenMfmaSmallLds : (need <= kGenMfmaLargeLds ? kGenMfmaLargeLds : 0);
}

// Workspace of a generic call: the float32 partial rows, then their lse
// values (both 256-byte aligned); 0 for invalid or too large arguments.
inline size_t generic_workspace_bytes(int32_t batch, int32_t heads, int32_t dv, int32_t splits) {
  if (batch < 0 || heads <= 0 || dv <= 0 || splits <= 0) return 0;
  int64_t rows = (int64_t)batch * heads;  // below 2^62
  if (rows > 0 && splits > kMaxWorkspaceBytes / rows) return 0;
  rows *= splits;
  if (rows > 0 && ((int64_t)dv + 1) * 4 > kMaxWorkspaceBytes / rows) return 0;
  auto al = [](int64_t x) { return (x + 255) & ~(int64_t)255; };
  const int64_t total = al(rows * dv * 4) + al(rows * 4) + 256;
  return total > kMaxWorkspaceBytes ? 0 : (size_t)total;
}

struct GenericCall {
  int32_t batch, heads, dv, dr, dtype, splits;
  bool paged;
  int32_t page_size, bt_cols;
  int64_t num_blocks;
};

inline int check_generic(const GenericCall& c, const void* workspace, size_t ws_bytes) {
  if (c.batch < 0 || c.heads <= 0) return fail(TMLA_ERR_INVALID_ARGUMENT, "batch must be >= 0 and num_heads > 0");
  if (c.dtype != TMLA_BF16 && c.dtype != TMLA_FP16 && c.dtype != TMLA_FP32)
    return fail(TMLA_ERR_INVALID_ARGUMENT, "dtype must be TMLA_BF16, TMLA_FP16 or TMLA_FP32");
  if (!pow2_between(c.dv, 16, 1024) || !pow2_between(c.dr, 16, 256))
    return fail(TMLA_ERR_UNSUPPORTED,
                "head_dim_v must be a power of two in [16, 1024] and rope_dim a power of two in [16, 256]");
  if (c.splits < 1 || c.splits > kGenMaxSplits) return fail(TMLA_ERR_INVALID_ARGUMENT, "num_splits must be in [1, 65535]");
  if (c.batch > kGenMaxBatchHeads || c.heads > kGenMaxBatchHeads)
    return fail(TMLA_ERR_UNSUPPORTED, "batch and num_heads must be at most 65535");
  if (c.paged && (c.page_size < 1 || c.bt_cols < 1 || c.num_blocks < 1))
    return fail(TMLA_ERR_INVALID_ARGUMENT, "a paged cache needs page_size, bt_cols and num_blocks >= 1");
  if (!c.paged && (c.page_size != 1 || c.num_blocks < 0))
    return fail(TMLA_ERR_INVALID_ARGUMENT, "a dense cache needs page_size 1 and num_blocks (its capacity) >= 0");
  const size_t need = generic_workspace_bytes(c.batch, c.heads, c.dv, c.splits);
  if (need == 0) return fail(TMLA_ERR_INVALID_ARGUMENT, "the call's workspace would exceed 2^62 bytes");
  if (workspace == nullptr || ws_bytes < need)
    return fail(TMLA_ERR_WORKSPACE_TOO_SMALL, "workspace is missing or smaller than tmla_generic_workspace_bytes()");
  return TMLA_OK;
}

}  // namespace tmla
