"""Pins of the oracle's fp8 (OCP E4M3) functions: the code table, the
round-to-nearest-even encoder and the decode over a dequantised cache.

The fp8 cache has no counterpart in the reference (README.md:32-33 lists
"no FP8 cache"), so there are no reference vectors; each function is pinned
by closed forms, by an independent implementation (torch's
float8_e4m3fn conversions on the CPU) and, for the decode, by reduction to
the already-pinned 16-bit oracle.
"""

import numpy as np
import pytest
import torch

import oracle
from conftest import bits


def test_e4m3_closed_forms():
    v = oracle.e4m3_to_float(np.arange(256))
    assert v[0x00] == 0.0 and not np.signbit(v[0x00])
    assert v[0x80] == 0.0 and np.signbit(v[0x80])
    assert v[0x38] == 1.0          # exponent field 7 = bias
    assert v[0x3F] == 1.875        # 1 + 7/8
    assert v[0x40] == 2.0
    assert v[0x7E] == 448.0        # largest finite
    assert v[0xFE] == -448.0
    assert v[0x01] == 2.0 ** -9    # smallest subnormal
    assert v[0x07] == 7 * 2.0 ** -9
    assert v[0x08] == 2.0 ** -6    # smallest normal
    assert np.isnan(v[0x7F]) and np.isnan(v[0xFF])
    assert np.isnan(v).sum() == 2
    # sign symmetry and strict monotonicity of the non-negative codes
    np.testing.assert_array_equal(v[0x80:0xFF], -v[0x00:0x7F])
    assert np.all(np.diff(v[0x00:0x7F]) > 0)


def test_e4m3_table_matches_torch():
    codes = torch.arange(256, dtype=torch.uint8)
    ref = codes.view(torch.float8_e4m3fn).double().numpy()
    v = oracle.e4m3_to_float(np.arange(256))
    np.testing.assert_array_equal(np.nan_to_num(v, nan=7.0), np.nan_to_num(ref, nan=7.0))


def test_e4m3_encode_round_trip_and_ties():
    codes = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], dtype=np.uint8)
    np.testing.assert_array_equal(oracle.float_to_e4m3(oracle.e4m3_to_float(codes)), codes)
    # halfway cases go to the even mantissa
    assert oracle.float_to_e4m3(np.array([1.0625]))[0] == 0x38     # 1 | 1.125 -> 1
    assert oracle.float_to_e4m3(np.array([1.1875]))[0] == 0x3A     # 1.125 | 1.25 -> 1.25
    assert oracle.float_to_e4m3(np.array([2.0 ** -10]))[0] == 0x00  # 0 | 2^-9 -> 0
    assert oracle.float_to_e4m3(np.array([3 * 2.0 ** -10]))[0] == 0x02
    assert oracle.float_to_e4m3(np.array([464.0]))[0] == 0x7E       # 448 | (480) -> 448
    assert oracle.float_to_e4m3(np.array([464.5]))[0] == 0x7F       # overflow: NaN
    assert oracle.float_to_e4m3(np.array([-1000.0]))[0] == 0xFF


def test_e4m3_encode_matches_torch_rounding():
    rng = np.random.default_rng(7)
    x = np.concatenate([rng.standard_normal(20000) * 10.0 ** rng.uniform(-3, 2.6, 20000),
                        rng.uniform(-464, 464, 5000)]).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(oracle.float_to_e4m3(x.astype(np.float64)), ref)


def _fp8_case(seed, batch, heads, lens, page=64, cap_pages=None, exact_pow2=False, per_token=False):
    """Random fp8 cache (finite codes) with page scales and a block table."""
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, dtype=np.int32)
    pages_per = int(cap_pages or -(-int(lens.max()) // page))
    nblk = batch * pages_per
    codes = rng.integers(0, 256, size=(nblk, page, 576), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x38  # no NaN codes
    # keep magnitudes moderate so exp() stays informative: exponent field <= 9
    codes = np.where(((codes >> 3) & 15) > 9, codes & 0x87 | (9 << 3), codes).astype(np.uint8)
    if exact_pow2:
        scale = (2.0 ** rng.integers(-6, -2, size=nblk)).astype(np.float32)
    elif per_token:
        scale = rng.uniform(0.002, 0.05, size=(nblk, page)).astype(np.float32)
    else:
        scale = rng.uniform(0.002, 0.05, size=nblk).astype(np.float32)
    bt = rng.permutation(nblk).astype(np.int32).reshape(batch, pages_per)
    q = torch.randn(batch, heads, 576, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16)
    return bits(q), codes, scale, lens, bt


def _dequant(codes, scale, bt, lens):
    vals = oracle.e4m3_to_float(codes)
    if scale.ndim == 1:
        vals = vals * scale[:, None, None].astype(np.float64)
    else:
        vals = vals * scale[:, :, None].astype(np.float64)
    return vals


def test_fp8_decode_reduces_to_bf16_oracle():
    # power-of-two page scales: every dequantised value is exactly a bf16
    # value, so the two oracles see identical float64 inputs
    qb, codes, scale, lens, bt = _fp8_case(1, 3, 5, [1, 100, 257], exact_pow2=True)
    vals = _dequant(codes, scale, bt, lens)
    kv16 = oracle.float_to_half(vals.astype(np.float32), "bf16")
    np.testing.assert_array_equal(oracle.half_to_float(kv16, "bf16"), vals)
    o8, l8 = oracle.mla_decode_fp8_ref(qb, codes, scale, lens, bt, softmax_scale=0.07)
    o16, l16 = oracle.mla_decode_ref(qb, kv16, lens, bt, softmax_scale=0.07)
    np.testing.assert_array_equal(o8, o16)
    np.testing.assert_array_equal(l8, l16)


@pytest.mark.parametrize("per_token", [False, True])
def test_fp8_decode_matches_numpy_softmax(per_token):
    from scipy.special import logsumexp

    qb, codes, scale, lens, bt = _fp8_case(2, 2, 3, [70, 129], page=16, per_token=per_token)
    out, lse = oracle.mla_decode_fp8_ref(qb, codes, scale, lens, bt, softmax_scale=0.05)
    vals = _dequant(codes, scale, bt, lens)
    q = oracle.half_to_float(qb, "bf16")
    for b in range(2):
        rows = vals[bt[b]].reshape(-1, 576)[: lens[b]]
        s = q[b] @ rows.T * 0.05
        p = np.exp(s - logsumexp(s, axis=1, keepdims=True))
        np.testing.assert_allclose(out[b], p @ rows[:, :512], rtol=1e-6, atol=1e-12)
        np.testing.assert_allclose(lse[b], logsumexp(s, axis=1), rtol=1e-6)


def test_fp8_per_page_equals_repeated_per_token():
    qb, codes, scale, lens, bt = _fp8_case(3, 2, 4, [33, 90], page=16)
    tok = np.repeat(scale[:, None], 16, axis=1)
    a = oracle.mla_decode_fp8_ref(qb, codes, scale, lens, bt)
    b = oracle.mla_decode_fp8_ref(qb, codes, tok, lens, bt)
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1], b[1])


def test_fp8_empty_sequence():
    qb, codes, scale, lens, bt = _fp8_case(4, 2, 2, [0, 20], page=16)
    out, lse = oracle.mla_decode_fp8_ref(qb, codes, scale, lens, bt)
    assert np.all(out[0] == 0) and np.all(np.isneginf(lse[0]))
    assert np.all(np.isfinite(lse[1]))


def test_fp8_single_scale_any_shape():
    # one scale: a [1] array and a 0-d array both mean the whole cache
    qb, codes, scale, lens, bt = _fp8_case(5, 3, 2, [10, 40, 25], page=16)
    one = np.float32(0.013)
    a = oracle.mla_decode_fp8_ref(qb, codes, np.array([one]), lens, bt)
    b = oracle.mla_decode_fp8_ref(qb, codes, np.array(one), lens, bt)
    c = oracle.mla_decode_fp8_ref(qb, codes, np.full(codes.shape[0], one), lens, bt)
    for x in (b, c):
        np.testing.assert_array_equal(a[0], x[0])
        np.testing.assert_array_equal(a[1], x[1])
