"""Parity at the measured workloads, at their full sizes.

Each decode workload (triton_mla.workloads: uniform B=1 and B=8 at 1K, the
B=32 8K headline, ragged B=64 1K..32K at 128 and 16 heads; seeded draws as in
the reference bench, src/triton_mla/bench.py:20-27) runs through mla_decode
with the balanced default and with the reference's split count, and is
compared with the float64 CPU oracle on every sequence: out atol = rtol =
1e-2, lse atol = rtol = 1e-3. Two size-independent bit-exact properties run
at full size too: moving pages to other physical slots (same logical cache)
changes no output bit, and a query aimed at one cached row returns that row
bit for bit wherever it sits (the gather through the block table). The MLA
layer at DeepSeek-V3 dims (B=16, 16K context) is checked against the oracle's
float64 restatement of the absorbed decode step.
"""

import numpy as np
import pytest
import torch

import oracle
from conftest import bits

pytestmark = pytest.mark.gpu

OUT_TOL = dict(atol=1e-2, rtol=1e-2)
LSE_TOL = dict(atol=1e-3, rtol=1e-3)
NAMES = ["b1_h128_ctx1k", "b8_h128_ctx1k", "b32_h128_ctx8k", "ragged_b64_h128_ctx1k-32k",
         "ragged_b64_h16_ctx1k-32k"]


def workload(name):
    from triton_mla.bench import WORKLOADS

    return WORKLOADS[name]()


_oracle_cache = {}


def oracle_result(name):
    if name not in _oracle_cache:
        inp = workload(name)
        ref = oracle.mla_decode_ref(bits(inp.q), bits(inp.kv_cache), inp.seqlens.numpy(),
                                    inp.block_table.numpy(), 512, inp.softmax_scale, dtype="bf16")
        _oracle_cache[name] = (inp, ref)
    return _oracle_cache[name]


@pytest.mark.parametrize("name", NAMES)
def test_workload_matches_oracle(gpu, name):
    from triton_mla import get_num_splits, mla_decode

    inp, (ref_out, ref_lse) = oracle_result(name)
    g = inp.to(gpu)
    ref_splits = get_num_splits(inp.batch, inp.heads, int(inp.seqlens.max()),
                                torch.cuda.get_device_properties(gpu).multi_processor_count)
    print(f"{name}: B={inp.batch} H={inp.heads} tokens={int(inp.seqlens.sum())} ref_splits={ref_splits}",
          flush=True)
    for splits in (None, ref_splits):
        out, lse = mla_decode(g.q, g.kv_cache, g.seqlens, g.block_table, softmax_scale=inp.softmax_scale,
                              num_splits=splits, return_lse=True)
        torch.testing.assert_close(out.float().cpu(), torch.from_numpy(ref_out), **OUT_TOL)
        torch.testing.assert_close(lse.cpu(), torch.from_numpy(ref_lse), **LSE_TOL)


@pytest.mark.parametrize("name", ["b32_h128_ctx8k", "ragged_b64_h16_ctx1k-32k"])
def test_page_placement_is_invisible(gpu, name):
    """The same logical cache with its pages moved to other physical slots
    gives bit-identical results (nothing depends on where a page lives)."""
    from triton_mla import mla_decode

    inp = workload(name).to(gpu)
    num_pages = inp.kv_cache.shape[0]
    gen = torch.Generator().manual_seed(1)
    move = torch.randperm(num_pages, generator=gen).to(gpu)  # old slot p -> new slot move[p]
    kv2 = torch.empty_like(inp.kv_cache)
    kv2[move.long()] = inp.kv_cache
    bt2 = move[inp.block_table.long()].to(torch.int32)
    a = mla_decode(inp.q, inp.kv_cache, inp.seqlens, inp.block_table, softmax_scale=inp.softmax_scale,
                   return_lse=True)
    b = mla_decode(inp.q, kv2, inp.seqlens, bt2, softmax_scale=inp.softmax_scale, return_lse=True)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


@pytest.mark.parametrize("name", ["b32_h128_ctx8k", "ragged_b64_h128_ctx1k-32k"])
def test_spike_query_returns_the_cached_row_bit_exact(gpu, name):
    """q = 4 * K[t] for a chosen token t of each sequence: its score beats
    every other by far more than fp32 exp2 can resolve, so its probability is
    exactly 1, every other exactly 0, and out must equal the latent row of t
    (found through the block table) bit for bit."""
    from triton_mla import mla_decode
    from triton_mla.reference import gather_kv

    inp = workload(name)
    gen = torch.Generator().manual_seed(2)
    lens = inp.seqlens.long()
    targets = (torch.rand(inp.batch, generator=gen) * lens).long().clamp(max=lens - 1)
    targets[0] = lens[0] - 1  # the last token of a sequence
    if inp.batch > 1:
        targets[1] = 63  # last row of the first page
    kv_rows = gather_kv(inp.kv_cache, inp.seqlens, inp.block_table)  # [B, S_max, 576]
    rows = kv_rows[torch.arange(inp.batch), targets]  # [B, 576]
    q = (4.0 * rows.float())[:, None, :].expand(-1, inp.heads, -1).to(inp.q.dtype).contiguous()
    g = inp.to(gpu)
    out = mla_decode(q.to(gpu), g.kv_cache, g.seqlens, g.block_table, softmax_scale=inp.softmax_scale)
    expect = rows[:, None, :512].expand(-1, inp.heads, -1)
    assert torch.equal(out.cpu(), expect), "gathered row differs from the cached row"


def _layer_weights(model):
    return {name.replace(".weight", ""): p.detach().float().cpu().numpy().astype(np.float64)
            for name, p in model.named_parameters()}


def test_mla_layer_deepseek_v3_dims(gpu):
    """MLA.forward at DeepSeek-V3 dims, B=16, 16K cached tokens (seeded N(0, 0.02)
    weights, N(0, 1) cache and hidden states) against the oracle's float64
    absorbed step: projections, RoPE, RMSNorm, cache append, attention (C
    oracle) and W_UV / wo.

    Three elementwise checks:
      * the latent decode at this shape (16 sequences x 16,385 tokens, 128
        heads: the snapped split of 17 workers per sequence) on the oracle's
        own query and cache: out within atol = rtol = 1e-2, lse within 1e-3;
      * the appended cache rows: atol = rtol = 1e-2 (the GPU's projections
        round to bf16 before the norm and the rotation);
      * the layer output: within half a bf16 ulp plus 2^-7 * sum_i |o_i w_ji|
        (the wo product of the oracle's W_UV output o with the weights: a
        relative error of 2^-7 in every o_i, about four bf16 roundings of the
        chain of bf16 GEMMs before it), and within the reference's own layer
        tolerance atol = rtol = 3e-2 (tests/test_model.py:34-35)."""
    from triton_mla import MLA, MLAConfig, mla_decode

    cfg = MLAConfig()
    batch, ctx, page = 16, 16384, 64
    gen = torch.Generator().manual_seed(0)
    model = MLA(cfg)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if "norm" not in name:
                p.copy_(torch.randn(p.shape, generator=gen) * 0.02)
    model = model.to(torch.bfloat16)
    x = torch.randn(batch, cfg.hidden_size, generator=gen).to(torch.bfloat16)
    pages = -(-(ctx + 1) // page)  # 257: the append at position 16384 opens a page
    kv_cache = torch.randn(batch * pages, page, cfg.kv_cache_dim, generator=gen).to(torch.bfloat16)
    bt = torch.randperm(batch * pages, generator=gen).view(batch, pages).to(torch.int32)
    seqlens = torch.full((batch,), ctx, dtype=torch.int32)

    gm, gcache = model.to(gpu), kv_cache.to(gpu)
    with torch.no_grad():
        out, new_lens = gm(x.to(gpu), gcache, seqlens.to(gpu), bt.to(gpu))
    assert torch.equal(new_lens.cpu(), seqlens + 1)

    # oracle: float64 step on the same (bf16-valued) weights and inputs
    w = _layer_weights(model)
    ocfg = {"num_heads": cfg.num_heads, "qk_nope_head_dim": cfg.qk_nope_head_dim,
            "qk_rope_head_dim": cfg.qk_rope_head_dim, "v_head_dim": cfg.v_head_dim,
            "kv_lora_rank": cfg.kv_lora_rank, "rms_norm_eps": cfg.rms_norm_eps, "rope_theta": cfg.rope_theta}
    xf = x.float().numpy().astype(np.float64)
    q_nope, q_pe, c_kv, k_pe = oracle.layer_project(w, ocfg, xf, seqlens.numpy())
    entries = np.concatenate([c_kv, k_pe], axis=-1)
    cache_bits = bits(kv_cache).copy()
    pos = seqlens.numpy()
    page_ids = bt.numpy()[np.arange(batch), pos // page]
    cache_bits[page_ids, pos % page] = oracle.float_to_half(entries, "bf16")
    q_abs = oracle.float_to_half(oracle.layer_absorbed_query(w, ocfg, q_nope, q_pe), "bf16")
    scale = (cfg.qk_head_dim) ** -0.5
    o_lat, lse_lat = oracle.mla_decode_ref(q_abs, cache_bits, pos + 1, bt.numpy(), cfg.kv_lora_rank, scale,
                                           dtype="bf16")
    ref = oracle.layer_output(w, ocfg, o_lat)

    # 1. the decode inside the layer, on the oracle's own query and cache
    def from_bits(b):
        return torch.from_numpy(b.view(np.int16)).view(torch.bfloat16)

    o_gpu, lse_gpu = mla_decode(from_bits(q_abs).to(gpu), from_bits(cache_bits).to(gpu),
                                torch.from_numpy(pos + 1).to(gpu), bt.to(gpu), head_dim_v=cfg.kv_lora_rank,
                                softmax_scale=scale, return_lse=True)
    torch.testing.assert_close(o_gpu.float().cpu(), torch.from_numpy(o_lat).float(), atol=1e-2, rtol=1e-2)
    torch.testing.assert_close(lse_gpu.cpu(), torch.from_numpy(lse_lat).float(), atol=1e-3, rtol=1e-3)

    # 2. the appended rows
    appended = gcache[torch.from_numpy(page_ids).long().to(gpu), torch.from_numpy(pos % page).long().to(gpu)]
    torch.testing.assert_close(appended.float().cpu(), torch.from_numpy(entries).float(), atol=1e-2, rtol=1e-2)

    # 3. the layer output
    o_v = np.einsum("bhc,hdc->bhd", o_lat, w["wkv_b"].reshape(cfg.num_heads, -1, cfg.kv_lora_rank)
                    [:, cfg.qk_nope_head_dim:]).reshape(batch, -1)
    gemm_mag = np.abs(o_v) @ np.abs(w["wo"]).T  # sum_i |o_i w_ji|
    got = out.float().cpu().numpy().astype(np.float64)
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -126))) - 7)
    ratio = np.abs(got - ref) / (0.5 * ulp + 2.0 ** -7 * gemm_mag)
    print(f"layer output: max err / bound {ratio.max():.3f}", flush=True)
    assert ratio.max() <= 1.0
    torch.testing.assert_close(out.float().cpu(), torch.from_numpy(ref).float(), atol=3e-2, rtol=3e-2)
