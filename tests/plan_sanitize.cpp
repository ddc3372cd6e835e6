// CPU harness of the host-side planning code (triton-mla_amd/csrc/host_plan.h),
// built by tests/test_plan_sanitize.py with the address and undefined-behaviour
// sanitizers (any signed overflow, out-of-range shift or bad access aborts).
// It sweeps extreme batch, head, split, worker and capacity values through
// check_common, ws_layout, worker_grid, plan_launch and plan_launch_g16, and the
// generic decode's check_generic, generic_plan and generic_workspace_bytes, and checks
// the invariants the kernels rely on. Prints "ok <cases>" on success.
#include <stdio.h>
#include <stdlib.h>

#include "host_plan.h"

using namespace tmla;

static int failures = 0;
#define EXPECT(cond, ...)                                    \
  do {                                                       \
    if (!(cond)) {                                           \
      if (failures++ < 20) {                                 \
        fprintf(stderr, "FAIL %s: ", #cond);                 \
        fprintf(stderr, __VA_ARGS__);                        \
        fprintf(stderr, "\n");                               \
      }                                                      \
    }                                                        \
  } while (0)

int main() {
  const int32_t I32 = INT32_MAX;
  const int32_t batches[] = {0, 1, 7, 64, 65535, 1 << 20, I32 - 1, I32};
  const int32_t heads[] = {1, 16, 17, 32, 33, 64, 65, 128, 129, 4096, 1 << 20, I32 - 31, I32};
  const int32_t splits[] = {0, 1, 3, 64, 1 << 16, I32};
  const int32_t workers[] = {0, 1, 256, 1 << 20, I32};
  const int64_t caps[] = {0, 1, 63, 64, 8192, (int64_t)1 << 31, INT64_MAX / 2, INT64_MAX};
  const int cus_list[] = {1, 256, 1024};
  long cases = 0;
  char dummy;
  for (int32_t b : batches)
    for (int32_t h : heads)
      for (int32_t s : splits)
        for (int32_t w : workers) {
          const Common c{b, h, 512, 64, TMLA_BF16, s, w};
          const size_t need = workspace_bytes(b, h, 512, s, w);
          // a workspace of the size asked for is accepted; one byte less is not
          const int rc = check_common(c, &dummy, need);
          const bool valid_shape = b >= 0 && h > 0 && !(s == 0 && w <= 0) && !(s > 0 && (int64_t)b * s > I32);
          if (valid_shape && need > 0) {
            EXPECT(rc == TMLA_OK, "b=%d h=%d s=%d w=%d need=%zu rc=%d", b, h, s, w, need, rc);
            EXPECT(check_common(c, &dummy, need - 1) == TMLA_ERR_WORKSPACE_TOO_SMALL, "b=%d h=%d", b, h);
            const WsLayout l = ws_layout(b, h, 512, s, w);
            const int64_t slots = partial_slots(b, s, w);
            // partial rows and lse values fit below the counter block, 256-byte aligned
            EXPECT(l.l >= (size_t)(slots * h) * 1024 && l.l % 256 == 0, "layout o b=%d h=%d", b, h);
            EXPECT(l.part_end >= l.l + (size_t)(slots * h) * 4 && l.part_end % 256 == 0, "layout l b=%d h=%d", b, h);
            EXPECT(l.total == l.part_end + kFusedCounterBytes && l.total == need, "total b=%d h=%d", b, h);
            EXPECT((int64_t)need <= kMaxWorkspaceBytes, "bound");
          } else if (valid_shape) {
            // too large: rejected, never a wrapped small size
            EXPECT(rc == TMLA_ERR_INVALID_ARGUMENT, "oversize b=%d h=%d s=%d w=%d rc=%d", b, h, s, w, rc);
          } else {
            EXPECT(rc != TMLA_OK, "invalid accepted b=%d h=%d s=%d w=%d", b, h, s, w);
          }
          if (!valid_shape) continue;
          for (int64_t cap : caps)
            for (int cus : cus_list)
              for (int mode = 0; mode <= 2; ++mode) {
                ++cases;
                const LaunchPlan p = plan_launch(b, h, s, w, cap, need, mode, cus);
                EXPECT(p.nhb == 1 || p.nhb == 2 || p.nhb == 4, "nhb");
                EXPECT(p.grid_x >= 1 && p.grid_x <= I32, "grid_x %lld", (long long)p.grid_x);
                EXPECT(p.grid_y >= 1 && p.grid_y * 32 * p.nhb >= h && (p.grid_y - 1) * 32 * p.nhb < h, "grid_y");
                if (s > 0) EXPECT(p.grid_x == ((int64_t)b * s < 1 ? 1 : (int64_t)b * s), "uniform grid");
                else EXPECT(p.grid_x <= w, "balanced grid within the workers");
                if (p.fused) {
                  EXPECT(mode == 1 && p.grid_x * p.grid_y <= cus, "fused fits the CUs");
                  EXPECT(fused_counter_bytes(b, p.grid_y, s, w) <= (int64_t)kFusedCounterBytes, "counters fit");
                }
                EXPECT(head_blocks(h) >= 1, "head blocks");
                // the 16-head-group kernel's plan: 16 heads per workgroup
                const LaunchPlan g = plan_launch_g16(b, h, s, w, cap, need, mode, cus);
                EXPECT(g.grid_x == p.grid_x, "g16 grid_x");
                EXPECT(g.grid_y >= 1 && g.grid_y * 16 >= h && (g.grid_y - 1) * 16 < h, "g16 grid_y");
                if (g.fused) {
                  EXPECT(mode == 1 && g.grid_x * g.grid_y <= cus, "g16 fused fits the CUs");
                  EXPECT(fused_counter_bytes(b, g.grid_y, s, w) <= (int64_t)kFusedCounterBytes, "g16 counters fit");
                }
              }
        }
  // the generic decode: dims, element types, shapes, workspaces
  const int32_t gdims[] = {0, 8, 16, 24, 32, 64, 128, 256, 512, 1024, 2048, -16};
  const int32_t gsplits[] = {-1, 0, 1, 7, 64, 65535, 65536, I32};
  const int32_t gbatches[] = {0, 1, 65535, 65536, I32};
  const int32_t gheads[] = {0, 1, 17, 65535, 65536, I32};
  for (int32_t dv : gdims)
    for (int32_t dr : gdims)
      for (int dt = 0; dt <= 3; ++dt) {
        const bool dims_ok = dv >= 16 && dv <= 1024 && dr >= 16 && dr <= 256 && (dv & (dv - 1)) == 0 &&
                             (dr & (dr - 1)) == 0;
        if (dims_ok && dt <= 2) {
          const GenericPlan gp = generic_plan(dv, dr, dt);
          const int64_t d = (int64_t)dv + dr;
          EXPECT(gp.lds == kGenSmallLds || gp.lds == kGenLargeLds, "lds form");
          EXPECT(gp.tile >= 8 && gp.tile <= 64 && (gp.tile & (gp.tile - 1)) == 0, "tile %d dv=%d dr=%d", gp.tile, dv, dr);
          EXPECT(64 * d + kGenProbBytes + (int64_t)gp.tile * gp.pitch <= gp.lds, "LDS fits dv=%d dr=%d", dv, dr);
          EXPECT(gp.pitch % 16 == 0 && gp.pitch == d * elem_bytes(dt) + 16, "pitch");
          EXPECT(gp.lds <= 160 * 1024 && (gp.lds != kGenSmallLds || gp.tile >= 16), "the small form holds 16 rows");
          // the matrix-core form: bf16 / fp16 at dv <= 512 and D <= 576 only, inside its LDS form, and
          // at most 9 16-byte chunks per thread and step (32 rows of D / 8 chunks over 256 threads)
          const int mf = generic_mfma_form(dv, dr, dt);
          const bool mf_ok = dt != TMLA_FP32 && dv <= 512 && d <= 576;
          EXPECT((mf != 0) == mf_ok, "mfma form applies dv=%d dr=%d dt=%d", dv, dr, dt);
          if (mf) {
            EXPECT(generic_mfma_lds_need(dv, dr) <= mf && mf <= 160 * 1024, "mfma LDS dv=%d dr=%d", dv, dr);
            EXPECT(kGenMfmaTokens * (d / 8) <= 9 * 256, "mfma chunks per thread");
            EXPECT(mf == kGenMfmaLargeLds || 2 * kGenMfmaSmallLds <= 160 * 1024, "two small forms per CU");
          }
        }
        for (int32_t b : gbatches)
          for (int32_t h : gheads)
            for (int32_t s : gsplits)
              for (int paged = 0; paged <= 1; ++paged) {
                ++cases;
                const GenericCall c{b, h, dv, dr, dt, s, paged != 0, paged ? 64 : 1, 16, 1024};
                const size_t need = generic_workspace_bytes(b, h, dv, s);
                const bool valid = b >= 0 && b <= 65535 && h > 0 && h <= 65535 && dims_ok && dt <= 2 && s >= 1 &&
                                   s <= 65535;
                const int rc = check_generic(c, &dummy, need);
                if (valid) {
                  EXPECT(need > 0 && rc == TMLA_OK, "generic b=%d h=%d dv=%d dr=%d s=%d rc=%d", b, h, dv, dr, s, rc);
                  const int64_t rows = (int64_t)b * h * s;
                  EXPECT((int64_t)need >= rows * ((int64_t)dv + 1) * 4 && need % 256 == 0, "generic need");
                  EXPECT(check_generic(c, &dummy, need - 1) == TMLA_ERR_WORKSPACE_TOO_SMALL, "generic ws-1");
                  EXPECT(check_generic(c, nullptr, need) == TMLA_ERR_WORKSPACE_TOO_SMALL, "generic null ws");
                } else {
                  EXPECT(rc != TMLA_OK, "generic invalid accepted b=%d h=%d dv=%d dr=%d dt=%d s=%d", b, h, dv, dr, dt, s);
                }
              }
      }
  if (failures) {
    fprintf(stderr, "%d failures\n", failures);
    return 1;
  }
  printf("ok %ld\n", cases);
  return 0;
}
