"""fp8 (OCP E4M3) latent cache: the HIP decode against the float64 oracle.

The fp8 cache has no counterpart in the reference (README.md:32-33 lists "no
FP8 cache"); the expected result is the reference's attention over the
dequantised cache, e4m3(byte) * scale, computed by the pinned oracle
(oracle.mla_decode_fp8_ref; pins in tests/test_fp8_oracle.py).

Caches are seeded randn bf16 caches quantised with
triton_mla.quantize_kv_fp8 (scale = max|x| / 448 per page, per token or per
tensor). The kernels widen the codes exactly, apply the row scale to the
float32 scores and to the probabilities before rounding those to the input
dtype, and accumulate in float32, so every output element obeys the same
budget as the 16-bit path (derivation in test_split_budget_gpu.py):

    |out - exact| <= ulp(exact)/2 * (1 + 2^-7) + (2^-9 + 2^-12) * A
                     + 2^-9 * V          (only when a sequence is split)

with A = sum_t p_t |v_t| / sum_t p_t and V = max_t |v_t| (a bound of every
partial, which is a convex combination of value rows). For fp16 inputs the
probability term uses 2^-11 in place of 2^-9. lse: within 1e-5 relative +
1e-5 absolute of the oracle.
"""

import zlib

import numpy as np
import pytest
import torch

import oracle
from conftest import bits

pytestmark = pytest.mark.gpu


def _make(batch, heads, lens, page=64, granularity="page", dense=False, dtype=torch.bfloat16, seed=0,
          q_len=1):
    from triton_mla import quantize_kv_fp8

    g = torch.Generator().manual_seed(seed)
    lens = torch.tensor(lens, dtype=torch.int32)
    if dense:
        cap = int(lens.max())
        kv = torch.randn(batch, max(cap, 1), 576, generator=g).to(torch.bfloat16)
        bt = None
    else:
        per = [max(-(-int(n) // page), 1) for n in lens]
        kv = torch.randn(sum(per), page, 576, generator=g).to(torch.bfloat16)
        perm = torch.randperm(sum(per), generator=g).to(torch.int32)
        bt = torch.zeros(batch, max(per), dtype=torch.int32)
        s = 0
        for b, n in enumerate(per):
            bt[b, :n] = perm[s:s + n]
            s += n
    codes, scale = quantize_kv_fp8(kv, granularity)
    shape = (batch, q_len, heads, 576) if q_len > 1 else (batch, heads, 576)
    q = torch.randn(*shape, generator=g).to(dtype)
    return q, codes, scale, lens, bt


def _oracle(q, codes, scale, lens, bt, softmax_scale, dtype="bf16"):
    return oracle.mla_decode_fp8_ref(bits(q), codes.view(torch.uint8).numpy(), scale.numpy(), lens.numpy(),
                                     None if bt is None else bt.numpy(), 512, softmax_scale, dtype=dtype)


def _amag(q, codes, scale, lens, bt, softmax_scale, dtype="bf16"):
    """float64 A = sum p|v| / sum p and V = max |v| per (b, h, dim)."""
    from triton_mla import dequantize_kv_fp8

    vals = dequantize_kv_fp8(codes, scale).double().numpy()
    qf = oracle.half_to_float(bits(q), dtype)
    A = np.zeros(qf.shape[:2] + (512,))
    V = np.zeros_like(A)
    for b in range(qf.shape[0]):
        n = int(lens[b])
        if n == 0:
            continue
        rows = (vals[bt[b].numpy()].reshape(-1, 576) if bt is not None else vals[b])[:n]
        s = qf[b] @ rows.T * softmax_scale
        e = np.exp(s - s.max(axis=1, keepdims=True))
        A[b] = (e @ np.abs(rows[:, :512])) / e.sum(axis=1, keepdims=True)
        V[b] = np.abs(rows[:, :512]).max(axis=0)
    return A, V


def _check(out, lse, ref, q, codes, scale, lens, bt, softmax_scale, split, dtype="bf16"):
    ref_out, ref_lse = ref
    out = out.float().cpu().numpy().astype(np.float64)
    lse = lse.float().cpu().numpy()
    A, V = _amag(q, codes, scale, lens, bt, softmax_scale, dtype)
    exact = ref_out.astype(np.float64)
    mant = 7 if dtype == "bf16" else 10
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(exact), 2.0 ** -126))) - mant)
    prob = 2.0 ** -9 if dtype == "bf16" else 2.0 ** -11
    bound = 0.5 * ulp * (1 + 2.0 ** -7) + (prob + 2.0 ** -12) * A + (2.0 ** -9 * V if split else 0.0)
    empty = (lens.numpy() == 0)
    ratio = np.abs(out - exact) / np.maximum(bound, 1e-30)
    ratio[empty] = 0
    print(f"max err / budget {ratio.max():.3f}", flush=True)
    assert ratio.max() <= 1.0
    assert np.all(out[empty] == 0) and np.all(np.isneginf(lse[empty]))
    np.testing.assert_allclose(lse[~empty], ref_lse[~empty], rtol=1e-5, atol=1e-5)


CASES = {
    # name: (batch, heads, lens, page, granularity, dense, dtype, num_splits)
    "h16_ragged_page64_page_scale": (6, 16, [1, 15, 16, 17, 1000, 4103], 64, "page", False, torch.bfloat16, None),
    "h16_page16_token_scale_splits4": (3, 16, [64, 500, 2049], 16, "token", False, torch.bfloat16, 4),
    "h16_page48_nonpow2": (3, 16, [47, 48, 999], 48, "page", False, torch.bfloat16, None),
    "h128_page64": (2, 128, [777, 2048], 64, "page", False, torch.bfloat16, None),
    "h3_dense_tensor_scale": (2, 3, [100, 37], 1, "tensor", True, torch.bfloat16, None),
    "h1_page32_unsplit": (2, 1, [300, 64], 32, "page", False, torch.bfloat16, 1),
    "h20_two_head_groups": (2, 20, [129, 3000], 64, "token", False, torch.bfloat16, 2),
    "h16_fp16_q": (2, 16, [513, 90], 64, "page", False, torch.float16, None),
    "empty_and_short": (3, 16, [0, 50, 0], 64, "page", False, torch.bfloat16, None),
    # more than 16 heads, one scale per page or per tensor, pages of whole
    # 32-token sub-tiles: the cache widened once per workgroup into the
    # 16-bit kernel's ring (1, 2 and 4 head blocks per workgroup)
    "ring_h128_ragged_page64": (6, 128, [1, 15, 16, 17, 1000, 4103], 64, "page", False, torch.bfloat16, None),
    "ring_h64_page32_tensor_scale": (3, 64, [31, 32, 2500], 32, "tensor", False, torch.bfloat16, None),
    "ring_h32_page128_splits3": (4, 32, [128, 129, 700, 3000], 128, "page", False, torch.bfloat16, 3),
    "ring_h128_fp16_q_unsplit": (2, 128, [300, 64], 64, "page", False, torch.float16, 1),
    "ring_h48_partial_head_block": (2, 48, [900, 33], 64, "page", False, torch.bfloat16, None),
    "ring_h128_many_workers": (16, 128, [4096] * 16, 64, "page", False, torch.bfloat16, None),
    # empty sequences on the ring path (out = 0, lse = -inf), balanced and split
    "ring_h128_empty_and_short": (3, 128, [0, 50, 0], 64, "page", False, torch.bfloat16, None),
    "ring_h64_empty_splits4": (4, 64, [0, 1, 0, 1300], 32, "tensor", False, torch.bfloat16, 4),
    # dense fp8 caches wider than 16 heads (one scale per sequence / tensor)
    "dense_h128_page_scale": (3, 128, [0, 700, 2100], 1, "page", True, torch.bfloat16, None),
    "dense_h32_tensor_scale_splits2": (2, 32, [333, 64], 1, "tensor", True, torch.float16, 2),
}


@pytest.mark.parametrize("name", list(CASES))
def test_fp8_decode_matches_oracle(gpu, name):
    from triton_mla import mla_decode

    batch, heads, lens, page, gran, dense, dtype, splits = CASES[name]
    print(f"case {name}", flush=True)
    q, codes, scale, lens_t, bt = _make(batch, heads, lens, page, gran, dense, dtype, seed=zlib.crc32(name.encode()) % 1000)
    sm = 576 ** -0.5
    dt = "bf16" if dtype == torch.bfloat16 else "fp16"
    ref = _oracle(q, codes, scale, lens_t, bt, sm, dt)
    out, lse = mla_decode(q.to(gpu), codes.to(gpu), lens_t.to(gpu), None if bt is None else bt.to(gpu),
                          softmax_scale=sm, num_splits=splits, return_lse=True, kv_scale=scale.to(gpu))
    torch.cuda.synchronize()
    _check(out, lse, ref, q, codes, scale, lens_t, bt, sm, split=splits != 1, dtype=dt)


def test_fp8_causal_two_query_tokens(gpu):
    from triton_mla import mla_decode

    q, codes, scale, lens, bt = _make(3, 16, [1, 200, 1500], 64, "page", q_len=2, seed=11)
    sm = 576 ** -0.5
    ref_out, ref_lse = _oracle(q, codes, scale, lens, bt, sm)
    out, lse = mla_decode(q.to(gpu), codes.to(gpu), lens.to(gpu), bt.to(gpu), softmax_scale=sm, return_lse=True,
                          kv_scale=scale.to(gpu))
    torch.cuda.synchronize()
    # token 0 of the first sequence sees no token at all
    assert torch.all(out[0, 0].cpu() == 0) and torch.all(torch.isneginf(lse[0, 0].cpu()))
    for t in range(2):
        n_t = torch.clamp(lens - (1 - t), min=0)
        _check(out[:, t], lse[:, t], (ref_out[:, t], ref_lse[:, t]), q[:, t].contiguous(), codes, scale, n_t, bt,
               sm, split=True)


def test_fp8_partial_plus_combine_equals_one_call(gpu):
    from triton_mla.kernel import DecodeLaunch

    q, codes, scale, lens, bt = _make(4, 16, [100, 2000, 64, 5000], 64, "page", seed=5)
    g = [x.to(gpu) for x in (q, codes, lens, bt)]
    a = DecodeLaunch(*g, 512, None, None, kv_scale=scale.to(gpu))
    out1 = a.run()[0].clone()
    a.out.zero_()
    a.partial()
    a.combine()
    torch.cuda.synchronize()
    assert torch.equal(out1, a.out)


def test_fp8_matches_bf16_kernel_on_exact_cache(gpu):
    """Power-of-two page scales make every dequantised value a bf16 value:
    the fp8 and bf16 kernels then decode the same cache, and both must meet
    the budget around the same oracle result."""
    from triton_mla import dequantize_kv_fp8, mla_decode

    q, codes, amax_scale, lens, bt = _make(4, 16, [33, 700, 4096, 64], 64, "page", seed=9)
    # the quantiser's scales rounded down to powers of two: cache values of
    # the size the codes were made for
    scale = 2.0 ** torch.floor(torch.log2(amax_scale))
    kv16 = dequantize_kv_fp8(codes, scale).to(torch.bfloat16)
    assert torch.equal(kv16.float(), dequantize_kv_fp8(codes, scale))
    sm = 576 ** -0.5
    ref = _oracle(q, codes, scale, lens, bt, sm)
    o8, l8 = mla_decode(q.to(gpu), codes.to(gpu), lens.to(gpu), bt.to(gpu), softmax_scale=sm, return_lse=True,
                        kv_scale=scale.to(gpu))
    o16, l16 = mla_decode(q.to(gpu), kv16.to(gpu), lens.to(gpu), bt.to(gpu), softmax_scale=sm, return_lse=True)
    torch.cuda.synchronize()
    _check(o8, l8, ref, q, codes, scale, lens, bt, sm, split=True)
    _check(o16, l16, ref, q, codes, scale, lens, bt, sm, split=True)


def test_fp8_full_size_h16_ragged(gpu):
    """The 16-head ragged workload (B=64, lengths 1K..32K, page 64) with a
    per-page-scaled fp8 cache, every sequence against the oracle."""
    from triton_mla import mla_decode, quantize_kv_fp8, workloads

    inp = workloads.ragged_b64_h16()
    codes, scale = quantize_kv_fp8(inp.kv_cache, "page")
    print(f"B={inp.batch} H={inp.heads} tokens={int(inp.seqlens.sum())}", flush=True)
    ref = _oracle(inp.q, codes, scale, inp.seqlens, inp.block_table, inp.softmax_scale)
    out, lse = mla_decode(inp.q.to(gpu), codes.to(gpu), inp.seqlens.to(gpu), inp.block_table.to(gpu),
                          softmax_scale=inp.softmax_scale, return_lse=True, kv_scale=scale.to(gpu))
    torch.cuda.synchronize()
    np.testing.assert_allclose(out.float().cpu().numpy(), ref[0], atol=1e-2, rtol=1e-2)
    np.testing.assert_allclose(lse.cpu().numpy(), ref[1], atol=1e-5, rtol=1e-5)


def test_fp8_ring_matches_bf16_kernel_on_exact_cache(gpu):
    """128 heads (the widened ring): with power-of-two page scales the fp8
    and bf16 decodes see the same cache values; both meet the budget around
    the same oracle result."""
    from triton_mla import dequantize_kv_fp8, mla_decode

    q, codes, amax_scale, lens, bt = _make(3, 128, [64, 1000, 2049], 64, "page", seed=21)
    scale = 2.0 ** torch.floor(torch.log2(amax_scale))
    kv16 = dequantize_kv_fp8(codes, scale).to(torch.bfloat16)
    sm = 576 ** -0.5
    ref = _oracle(q, codes, scale, lens, bt, sm)
    o8, l8 = mla_decode(q.to(gpu), codes.to(gpu), lens.to(gpu), bt.to(gpu), softmax_scale=sm, return_lse=True,
                        kv_scale=scale.to(gpu))
    o16, l16 = mla_decode(q.to(gpu), kv16.to(gpu), lens.to(gpu), bt.to(gpu), softmax_scale=sm, return_lse=True)
    torch.cuda.synchronize()
    _check(o8, l8, ref, q, codes, scale, lens, bt, sm, split=True)
    _check(o16, l16, ref, q, codes, scale, lens, bt, sm, split=True)


def test_fp8_ring_full_size_h128(gpu):
    """The 32-sequence, 8K-token, 128-head workload with a per-page-scaled fp8
    cache (the widened ring); the first four sequences against the oracle
    (every output is checked for finiteness)."""
    from triton_mla import mla_decode, quantize_kv_fp8, workloads

    inp = workloads.b32_h128_8k()
    codes, scale = quantize_kv_fp8(inp.kv_cache, "page")
    print(f"B={inp.batch} H={inp.heads} tokens={int(inp.seqlens.sum())}", flush=True)
    out, lse = mla_decode(inp.q.to(gpu), codes.to(gpu), inp.seqlens.to(gpu), inp.block_table.to(gpu),
                          softmax_scale=inp.softmax_scale, return_lse=True, kv_scale=scale.to(gpu))
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all() and torch.isfinite(lse).all()
    n = 4
    ref = _oracle(inp.q[:n], codes, scale, inp.seqlens[:n], inp.block_table[:n], inp.softmax_scale)
    _check(out[:n], lse[:n], ref, inp.q[:n], codes, scale, inp.seqlens[:n], inp.block_table[:n], inp.softmax_scale,
           split=True)


def test_fp8_argument_errors(gpu):
    from triton_mla import mla_decode

    q, codes, scale, lens, bt = _make(2, 16, [40, 20], 64, "page", seed=3)
    with pytest.raises(ValueError, match="kv_scale"):
        mla_decode(q.to(gpu), codes.to(gpu), lens.to(gpu), bt.to(gpu))
    q8, c8, s8, l8, b8 = _make(2, 16, [40, 20], 8, "page", seed=3)
    with pytest.raises(NotImplementedError, match="multiple of 16"):
        mla_decode(q8.to(gpu), c8.to(gpu), l8.to(gpu), b8.to(gpu), kv_scale=s8.to(gpu))
    with pytest.raises(AssertionError):
        mla_decode(q.to(gpu), codes.to(gpu), lens.to(gpu), bt.to(gpu), kv_scale=scale[:1].repeat(3).to(gpu))
