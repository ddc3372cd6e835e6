"""MLA layer on the GPU: the absorbed decode step (HIP mla_decode inside)
against the non-absorbed one, as the reference's layer test does
(tests/test_model.py:8-35: hidden 256, 16 heads, q_lora_rank 128, weights
N(0, 0.05) with unit norm weights, seqlens [0, 5, max_len/2], page size 16,
dense and paged caches, bf16 atol = rtol = 3e-2), plus the same step
against the float64 oracle restatement of the layer."""

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def _model(cfg, gen):
    from triton_mla import MLA

    model = MLA(cfg)
    with torch.no_grad():
        for p in model.parameters():
            p.copy_(torch.randn(p.shape, generator=gen) * 0.05)
        model.q_norm.weight.fill_(1.0)
        model.kv_norm.weight.fill_(1.0)
    return model


@pytest.mark.parametrize("paged", [False, True])
def test_absorbed_decode_matches_naive(gpu, paged):
    from triton_mla import MLAConfig

    gen = torch.Generator().manual_seed(0)
    cfg = MLAConfig(hidden_size=256, num_heads=16, q_lora_rank=128)
    model = _model(cfg, gen).to(gpu, torch.bfloat16)
    batch, max_len, page_size = 3, 256, 16
    seqlens = torch.tensor([0, 5, max_len // 2], dtype=torch.int32, device=gpu)
    if paged:
        blocks = max_len // page_size
        block_table = torch.randperm(batch * blocks, generator=gen).view(batch, blocks).int().to(gpu)
        kv_cache = torch.randn(batch * blocks, page_size, cfg.kv_cache_dim, generator=gen).to(gpu, torch.bfloat16)
    else:
        block_table = None
        kv_cache = torch.randn(batch, max_len, cfg.kv_cache_dim, generator=gen).to(gpu, torch.bfloat16)
    x = torch.randn(batch, cfg.hidden_size, generator=gen).to(gpu, torch.bfloat16)
    cache_a, cache_b = kv_cache.clone(), kv_cache.clone()
    with torch.no_grad():
        out, new_lens = model(x, cache_a, seqlens, block_table)
        ref, _ = model.forward_naive(x, cache_b, seqlens, block_table)
    assert torch.equal(new_lens, seqlens + 1)
    # both paths append the same row: the HIP append (forward) and the torch
    # one (forward_naive) round float32 results once, so they agree to one
    # bf16 ulp; every other cache row is untouched by both
    spacing = torch.exp2(torch.floor(torch.log2(cache_b.float().abs().clamp_min(2.0 ** -126))) - 7)
    assert bool(((cache_a.float() - cache_b.float()).abs() <= spacing).all())
    torch.testing.assert_close(out.float(), ref.float(), atol=3e-2, rtol=3e-2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_other_dims_and_fp32_layer_matches_naive(gpu, dtype):
    """A layer outside the HIP glue's dims (latent 256, rope 32, nope 64, value
    64) and the reference test's fp32 layer (tests/test_model.py:34: atol 1e-4
    in fp32): the torch glue around the generic decode against the
    non-absorbed step."""
    from triton_mla import MLAConfig

    gen = torch.Generator().manual_seed(4)
    cfgs = [MLAConfig(hidden_size=256, num_heads=16, q_lora_rank=128, kv_lora_rank=256, qk_nope_head_dim=64,
                      qk_rope_head_dim=32, v_head_dim=64)]
    if dtype == torch.float32:
        cfgs.append(MLAConfig(hidden_size=256, num_heads=16, q_lora_rank=128))
    for cfg in cfgs:
        model = _model(cfg, gen).to(gpu, dtype)
        batch, max_len, page_size = 3, 256, 16
        seqlens = torch.tensor([0, 5, max_len // 2], dtype=torch.int32, device=gpu)
        blocks = max_len // page_size
        block_table = torch.randperm(batch * blocks, generator=gen).view(batch, blocks).int().to(gpu)
        kv_cache = torch.randn(batch * blocks, page_size, cfg.kv_cache_dim, generator=gen).to(gpu, dtype)
        x = torch.randn(batch, cfg.hidden_size, generator=gen).to(gpu, dtype)
        cache_a, cache_b = kv_cache.clone(), kv_cache.clone()
        with torch.no_grad():
            out, new_lens = model(x, cache_a, seqlens, block_table)
            ref, _ = model.forward_naive(x, cache_b, seqlens, block_table)
        assert torch.equal(new_lens, seqlens + 1)
        tol = 1e-4 if dtype == torch.float32 else 3e-2
        torch.testing.assert_close(out.float(), ref.float(), atol=tol, rtol=tol)


def test_absorbed_decode_matches_layer_oracle(gpu):
    from triton_mla import MLAConfig

    gen = torch.Generator().manual_seed(3)
    cfg = MLAConfig(hidden_size=256, num_heads=16, q_lora_rank=128)
    model = _model(cfg, gen)
    w = {n.replace(".weight", ""): p.detach().to(torch.bfloat16).double().numpy() for n, p in model.named_parameters()}
    model = model.to(gpu, torch.bfloat16)
    batch, page_size, blocks = 3, 16, 16
    lens = torch.tensor([0, 37, 200], dtype=torch.int32)
    block_table = torch.randperm(batch * blocks, generator=gen).view(batch, blocks).int()
    kv_cache = torch.randn(batch * blocks, page_size, cfg.kv_cache_dim, generator=gen).to(torch.bfloat16)
    x = torch.randn(batch, cfg.hidden_size, generator=gen).to(torch.bfloat16)
    with torch.no_grad():
        out, _ = model(x.to(gpu), kv_cache.to(gpu), lens.to(gpu), block_table.to(gpu))

    ocfg = {"num_heads": cfg.num_heads, "qk_nope_head_dim": cfg.qk_nope_head_dim,
            "qk_rope_head_dim": cfg.qk_rope_head_dim, "v_head_dim": cfg.v_head_dim,
            "kv_lora_rank": cfg.kv_lora_rank, "rms_norm_eps": cfg.rms_norm_eps, "rope_theta": cfg.rope_theta}
    dense = kv_cache[block_table.long()].reshape(batch, blocks * page_size, -1).double().numpy()
    toks = [dense[b, : int(lens[b])] for b in range(batch)]
    ref, _ = oracle.layer_forward_naive(w, ocfg, x.double().numpy(), toks, lens.numpy())
    err = np.linalg.norm(out.float().cpu().numpy() - ref) / np.linalg.norm(ref)
    assert err < 3e-2, err
