"""Host-side behaviour of the drop-in API that needs no GPU: the reference's
input assertions (src/triton_mla/kernel.py:235-245), the loud refusal to run
anywhere but on a HIP device, and the torch API functions kept for
compatibility (checked against the oracle)."""

import numpy as np
import pytest
import torch

import oracle
from conftest import bits

D = 576


def _inputs(batch=2, heads=16, n=40, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(0)
    q = torch.randn(batch, heads, D, generator=g).to(dtype)
    kv = torch.randn(batch, n, D, generator=g).to(dtype)
    return q, kv, torch.tensor([n, n // 2], dtype=torch.int32)[:batch]


def test_reference_assertions():
    from triton_mla import mla_decode

    q, kv, lens = _inputs()
    with pytest.raises(AssertionError):
        mla_decode(q[0], kv, lens)  # q must be 3-D
    with pytest.raises(AssertionError):
        mla_decode(q, kv[..., :500], lens)  # D mismatch
    with pytest.raises(AssertionError):
        mla_decode(q, kv, lens, head_dim_v=500)  # not a power of two
    with pytest.raises(AssertionError):
        mla_decode(q, kv.to(torch.float16), lens)  # dtype mismatch
    with pytest.raises(AssertionError):
        mla_decode(q, kv.unsqueeze(2).expand(2, 40, 2, D), lens)  # 4-D with 2 kv heads
    with pytest.raises(AssertionError):
        mla_decode(q.transpose(1, 2).contiguous().transpose(1, 2), kv, lens)  # last dim not contiguous


def test_cpu_tensors_are_refused_loudly():
    from triton_mla import mla_decode

    q, kv, lens = _inputs()
    with pytest.raises(RuntimeError, match="GPU only"):
        mla_decode(q, kv, lens)


def test_other_dims_and_fp32_take_the_generic_path():
    """head_dim_v / rope_dim other than 512 / 64, or fp32 inputs, go to the
    generic decode: the reference's assertions first, then its limits, then the
    same loud refusal of CPU tensors."""
    from triton_mla import mla_decode

    g = torch.Generator().manual_seed(0)
    q = torch.randn(2, 4, 160, generator=g)
    kv = torch.randn(2, 40, 160, generator=g)
    lens = torch.tensor([40, 3], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="GPU only"):
        mla_decode(q, kv, lens, head_dim_v=128)  # fp32, 128 + 32
    with pytest.raises(RuntimeError, match="GPU only"):
        mla_decode(q.to(torch.bfloat16), kv.to(torch.bfloat16), lens, head_dim_v=128)
    qf, kvf = torch.randn(2, 4, D, generator=g), torch.randn(2, 40, D, generator=g)
    with pytest.raises(RuntimeError, match="GPU only"):
        mla_decode(qf, kvf, lens)  # fp32 at 512 + 64
    with pytest.raises(AssertionError):
        mla_decode(q, kv, lens, head_dim_v=100)  # not a power of two
    with pytest.raises(AssertionError):
        mla_decode(q, kv.to(torch.float16), lens, head_dim_v=128)  # dtype mismatch
    with pytest.raises(NotImplementedError, match="rope_dim"):
        mla_decode(q[..., :136].contiguous(), kv[..., :136].contiguous(), lens, head_dim_v=128)  # rope 8
    with pytest.raises(NotImplementedError, match="head_dim_v"):
        mla_decode(torch.randn(2, 4, 2112), torch.randn(2, 40, 2112), lens, head_dim_v=2048)
    with pytest.raises(NotImplementedError, match="fp32"):
        mla_decode(q.double(), kv.double(), lens, head_dim_v=128)
    with pytest.raises(NotImplementedError, match="multi-token"):
        mla_decode(q.unsqueeze(1), kv, lens, head_dim_v=128)


def test_make_inputs_takes_the_reference_dims():
    """make_inputs keeps the reference's arguments (bench.py:20: ..., device,
    d_latent=512, d_rope=64) and draws the default dims exactly as before."""
    import inspect

    from triton_mla import bench, workloads

    params = list(inspect.signature(bench.make_inputs).parameters)
    assert params[:8] == ["batch", "seqlen", "num_heads", "page_size", "dtype", "device", "d_latent", "d_rope"]
    a = bench.make_inputs(2, 100, 4, 64, torch.float32, "cpu", 128, 32)
    assert a.q.shape == (2, 4, 160) and a.kv_cache.shape == (4, 64, 160) and a.head_dim_v == 128
    assert a.softmax_scale == 160 ** -0.5
    b = bench.make_inputs(2, 100, 4, 64, torch.bfloat16, "cpu")
    c = workloads.uniform(2, 4, 100)
    assert torch.equal(b.q, c.q) and torch.equal(b.kv_cache, c.kv_cache) and b.softmax_scale == 192 ** -0.5


def test_generic_default_splits():
    """One vector-ALU workgroup (16 heads) or about four matrix-core
    workgroups (64 heads) per compute unit, pieces of >= 256 tokens."""
    from triton_mla.kernel import _generic_splits

    assert _generic_splits(32, 128, 8192, 256) == 1  # 256 workgroup groups already
    assert _generic_splits(64, 16, 16384, 256) == 4
    assert _generic_splits(1, 16, 1000, 256) == 4  # capped by the length: cdiv(1000, 256)
    assert _generic_splits(1, 16, 0, 256) == 1
    assert _generic_splits(4096, 128, 1 << 20, 256) == 1
    assert _generic_splits(1, 1, 1 << 30, 1 << 20) == 65535
    assert _generic_splits(32, 128, 8192, 256, heads_per_wg=64) == 16  # 64 workgroup groups


def test_torch_reference_functions_match_oracle():
    """The package's mla_decode_ref / mla_decode_torch / gather_kv (torch API,
    reference.py:6-44) against the float64 oracle on the CPU."""
    from triton_mla import mla_decode_ref, mla_decode_torch
    from triton_mla.reference import gather_kv

    g = torch.Generator().manual_seed(1)
    lens = torch.tensor([0, 1, 37, 100], dtype=torch.int32)
    q = torch.randn(4, 16, D, generator=g)
    kv = torch.randn(4, 100, D, generator=g)
    out, lse = mla_decode_ref(q, kv, lens, softmax_scale=0.1)
    qb, kvb = q.to(torch.bfloat16), kv.to(torch.bfloat16)
    ref_out, ref_lse = oracle.mla_decode_ref(bits(qb), bits(kvb), lens.numpy(), None, 512, 0.1)
    out_b, lse_b = mla_decode_ref(qb.float(), kvb.float(), lens, softmax_scale=0.1)
    torch.testing.assert_close(out_b, torch.from_numpy(ref_out), atol=1e-5, rtol=1e-5)
    valid = lens > 0
    torch.testing.assert_close(lse_b[valid], torch.from_numpy(ref_lse)[valid], atol=1e-5, rtol=1e-5)
    assert out.shape == (4, 16, 512) and torch.all(torch.isneginf(lse[0]))
    tor = mla_decode_torch(qb.float(), kvb.float(), lens, softmax_scale=0.1)
    torch.testing.assert_close(tor[1:], torch.from_numpy(ref_out)[1:], atol=1e-5, rtol=1e-5)
    # paged gather
    bt = torch.randperm(8, generator=g).view(2, 4).int()
    cache = torch.randn(8, 16, D, generator=g).to(torch.bfloat16)
    got = gather_kv(cache, lens[:2], bt)
    assert np.array_equal(bits(got), oracle.gather_kv(bits(cache), lens[:2].numpy(), bt.numpy()))


def _partition_by_simulation(seqlens, workers, start=2):
    """Brute force over the workers: the tiles each one takes (a snapped
    piece, or a range of a line holding, per non-empty sequence, ``start``
    positions that belong to no tile and then its tiles) and the sequences
    they touch; returns the largest worker count of one sequence."""
    tile = 64
    tiles = [-(-n // tile) if n > 0 else 0 for n in seqlens]
    total = sum(tiles)
    if total == 0:
        return 0
    c = -(-total // workers)
    owners = [set() for _ in seqlens]
    if sum(-(-t // c) for t in tiles) <= workers:
        w = 0
        for b, t in enumerate(tiles):
            for _ in range(-(-t // c)):
                owners[b].add(w)
                w += 1
    else:
        line = []  # the sequence of each position, None for a start position
        for b, t in enumerate(tiles):
            if t:
                line += [None] * start + [b] * t
        v = -(-len(line) // workers)
        for w in range(workers):
            for b in line[w * v:(w + 1) * v]:
                if b is not None:
                    owners[b].add(w)
    return max(len(o) for o in owners)


@pytest.mark.parametrize("seqlens,workers,expect", [
    ([8192] * 32, 256, 8),          # headline: snapped, 8 pieces of 16 tiles
    ([1024], 256, 16),               # one sequence over 16 workers
    ([16385] * 4, 64, 16),           # snapped (64 pieces == 64 workers)
    ([16385] * 4, 63, None),         # straddling ranges
    ([0, 1, 65, 300, 4097, 2000], 19, None),
    ([0, 0], 256, 0),
])
def test_balanced_pieces_matches_the_partition(seqlens, workers, expect):
    """The integer split count triton-mla-bench writes for the balanced
    partition equals a brute-force walk of the workers' ranges."""
    from triton_mla.kernel import balanced_pieces

    got = balanced_pieces(seqlens, workers)
    assert got == _partition_by_simulation(seqlens, workers)
    if expect is not None:
        assert got == expect
    g = np.random.default_rng(0)
    for _ in range(200):
        lens = g.integers(0, 5000, size=int(g.integers(1, 40))).tolist()
        w = int(g.integers(1, 300))
        for start in (0, 2, 5):
            assert balanced_pieces(lens, w, start) == _partition_by_simulation(lens, w, start)


@pytest.mark.parametrize("made_in_inference", [False, True])
def test_down_projection_in_inference_mode(made_in_inference):
    """The step's first GEMM x . [wq_a; wkv_a]^T under torch.inference_mode:
    parameters made inside it keep no version counter (two GEMMs), parameters
    made outside it keep the joint weight, refreshed after an in-place change."""
    import torch.nn.functional as F
    from triton_mla.model import MLA, MLAConfig

    cfg = MLAConfig(hidden_size=128, num_heads=4, q_lora_rank=64)
    torch.manual_seed(0)
    if made_in_inference:
        with torch.inference_mode():
            layer = MLA(cfg)
    else:
        layer = MLA(cfg)
    x = torch.randn(3, cfg.hidden_size)
    with torch.inference_mode():
        for step in range(2):
            q_lat, kv = layer._down_proj(x)
            torch.testing.assert_close(q_lat, F.linear(x, layer.wq_a.weight), rtol=1e-5, atol=1e-5)
            torch.testing.assert_close(kv, F.linear(x, layer.wkv_a.weight), rtol=1e-5, atol=1e-5)
            layer.wkv_a.weight.mul_(-2.0)  # in place: the next call must see it
    # the joint weight kept from inference mode works with autograd on afterwards
    if not made_in_inference:
        xg = x.clone().requires_grad_(True)
        q_lat, kv = layer._down_proj(xg)
        (q_lat.sum() + kv.sum()).backward()
        assert xg.grad is not None
