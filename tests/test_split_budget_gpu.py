"""Elementwise error budget of the split partials, which the kernels store in
the input dtype (bf16) where the reference keeps float32 (`mid_o`,
src/triton_mla/kernel.py:268).

For one output element, with exact per-split partials o_s (each a softmax-
weighted mean of the split's value rows) and merge weights w_s >= 0:

    out = sum_s w_s o_s / sum_s w_s,
    stored partial o_s (1 + d_s), |d_s| <= 2^-9 (bf16, round to nearest)

so storing the partials in bf16 adds at most 2^-9 * max_s |o_s| to the
element. The other terms of the budget, present with or without splits, are:
the probabilities rounded to bf16 before the value product (as the
reference's stage 1 does, kernel.py:123): at most 2^-9 * A with
A = sum_t p_t |v_t| / sum_t p_t; float32 scores and accumulation (a few
2^-24 relative on the scores, which are O(10) here, so below 2^-14 * A); and
the final rounding of out to bf16 (half an ulp). The test states

    |out_gpu - out_exact| <= ulp(out_exact) / 2 * (1 + 2^-7)
                             + 2^-9 * max_s |o_s|   (split runs only)
                             + (2^-9 + 2^-12) * A

and checks it elementwise against a float64 computation of o_s, A and the
exact output (itself checked against the C oracle), for an 8-way uniform
split and for the unsplit run (where the partial term is absent).
"""

import numpy as np
import pytest
import torch

import oracle
from conftest import bits

pytestmark = pytest.mark.gpu


def exact_terms(inp, splits):
    """float64: exact out, A = sum p|v| / sum p, and max_s |o_s| per element."""
    kv = oracle.half_to_float(bits(inp.kv_cache), "bf16")
    q = oracle.half_to_float(bits(inp.q), "bf16")
    bt = inp.block_table.numpy()
    outs, amags, pmax = [], [], []
    for b in range(inp.batch):
        n = int(inp.seqlens[b])
        rows = kv[bt[b]].reshape(-1, kv.shape[-1])[:n]  # [n, 576]
        s = (q[b] @ rows.T) * inp.softmax_scale  # [H, n]
        e = np.exp(s - s.max(axis=1, keepdims=True))
        v = rows[:, :512]
        outs.append((e @ v) / e.sum(axis=1, keepdims=True))
        amags.append((e @ np.abs(v)) / e.sum(axis=1, keepdims=True))
        tiles = -(-n // 64)
        spt = -(-tiles // splits)
        m = np.zeros((q.shape[1], 512))
        for t0 in range(0, tiles, spt):
            lo, hi = t0 * 64, min((t0 + spt) * 64, n)
            es = e[:, lo:hi]
            m = np.maximum(m, np.abs((es @ v[lo:hi]) / es.sum(axis=1, keepdims=True)))
        pmax.append(m)
    return np.stack(outs), np.stack(amags), np.stack(pmax)


@pytest.mark.parametrize("splits", [8, 1])
def test_split_partial_budget(gpu, splits):
    from triton_mla import mla_decode, workloads

    inp = workloads.uniform(4, 128, 8192, seed=3)
    g = inp.to(gpu)
    out = mla_decode(g.q, g.kv_cache, g.seqlens, g.block_table, softmax_scale=inp.softmax_scale,
                     num_splits=splits).float().cpu().numpy().astype(np.float64)
    exact, amag, pmax = exact_terms(inp, splits)
    # the float64 restatement above is the C oracle's result (which it
    # returns rounded to float32)
    ref, _ = oracle.mla_decode_ref(bits(inp.q), bits(inp.kv_cache), inp.seqlens.numpy(), inp.block_table.numpy(),
                                   512, inp.softmax_scale)
    np.testing.assert_allclose(exact, ref, rtol=2.0 ** -23, atol=1e-30)

    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(exact), 2.0 ** -126))) - 7)
    bound = 0.5 * ulp * (1 + 2.0 ** -7) + (2.0 ** -9 + 2.0 ** -12) * amag
    if splits > 1:
        bound += 2.0 ** -9 * pmax
    ratio = np.abs(out - exact) / bound
    print(f"splits={splits}: max err / budget {ratio.max():.3f}, mean {ratio.mean():.3f}, "
          f"max |err| {np.abs(out - exact).max():.2e}", flush=True)
    assert ratio.max() <= 1.0
