"""Pins for the CPU oracle (oracle/mla_oracle.c, oracle/oracle.py).

Each oracle function is checked against something that does not restate its
own formula: the reference's published known-answer table, closed forms,
scipy's independent softmax/logsumexp, brute force in pure Python on tiny
inputs, invariances (token order, paging, splitting), and torch's own
rounding. The last group plants mistakes into a copy of the algorithm and
shows the same checks reject it.
"""

import json
import math
import os

import numpy as np
import pytest
import torch
from scipy.special import logsumexp, softmax

import oracle

HERE = os.path.dirname(os.path.abspath(__file__))
D = 576
DV = 512


def rand_bits(rng, shape, dtype="bf16", scale=1.0):
    return oracle.float_to_half(rng.standard_normal(shape) * scale, dtype)


def as_f64(bits, dtype="bf16"):
    return oracle.half_to_float(bits, dtype)


# ---------------------------------------------------------------------------
# get_num_splits: the reference's own results table (golden vectors)
# ---------------------------------------------------------------------------

def test_num_splits_known_answers():
    table = json.load(open(os.path.join(HERE, "golden", "num_splits_h100.json")))
    rows = [r for r in table["rows"] if r["source"] == "results/bench_h100.csv"]
    assert len(rows) == 16
    for r in rows:
        assert oracle.get_num_splits(r["batch"], r["heads"], r["seqlen"], table["num_sms"]) == r["num_splits"], r


def test_num_splits_edges():
    assert oracle.get_num_splits(1, 128, 0, 132) == 1  # max_seqlen 0
    assert oracle.get_num_splits(0, 128, 100000, 132) == 64  # empty batch: target = num_sms, capped at 64
    assert oracle.get_num_splits(0, 128, 4096, 132) == 32  # ... and by cdiv(4096, 128)
    for b in (1, 3, 17, 200):
        for s in (1, 100, 5000, 100000):
            v = oracle.get_num_splits(b, 128, s, 256)
            assert 1 <= v <= 64 and v & (v - 1) == 0


def test_package_num_splits_matches_oracle():
    from triton_mla import get_num_splits

    for b in (1, 2, 8, 32, 64, 128):
        for h in (16, 20, 64, 128):
            for s in (0, 1, 1024, 8192, 32768):
                for sms in (132, 256, 304):
                    assert get_num_splits(b, h, s, sms) == oracle.get_num_splits(b, h, s, sms)


# ---------------------------------------------------------------------------
# 16-bit rounding helpers against torch / numpy
# ---------------------------------------------------------------------------

def test_rounding_matches_torch_and_numpy():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(10000) * 10 ** rng.uniform(-8, 6, 10000),
                        [0.0, -0.0, 1e-40, 65504.0, 70000.0, -3e38]]).astype(np.float32)
    bf = oracle.float_to_half(x, "bf16")
    ref_bf = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bf, ref_bf)
    fp = oracle.float_to_half(x, "fp16")
    with np.errstate(over="ignore"):
        assert np.array_equal(fp, x.astype(np.float16).view(np.uint16))
    assert np.array_equal(as_f64(bf), ref_bf.astype(np.uint32).__lshift__(16).view(np.float32).astype(np.float64))


# ---------------------------------------------------------------------------
# gather_kv
# ---------------------------------------------------------------------------

def test_gather_kv_bit_exact():
    rng = np.random.default_rng(1)
    kv = rng.integers(0, 65535, size=(9, 16, D), dtype=np.uint16)
    bt = rng.permutation(9)[:8].reshape(2, 4).astype(np.int32)
    out = oracle.gather_kv(kv, np.array([50, 64], np.int32), bt)
    assert np.array_equal(out, kv[bt].reshape(2, 64, D))  # numpy fancy indexing
    dense = rng.integers(0, 65535, size=(2, 30, D), dtype=np.uint16)
    assert np.array_equal(oracle.gather_kv(dense, np.array([3, 30], np.int32)), dense)


# ---------------------------------------------------------------------------
# mla_decode_ref
# ---------------------------------------------------------------------------

def decode_checks(decode):
    """Closed forms and library cross-checks; `decode(q, kv, seqlens, bt, scale)`
    returns (out, lse) like oracle.mla_decode_ref. Raises AssertionError on failure."""
    rng = np.random.default_rng(2)
    # (1) one token: softmax weight 1 -> out is the latent row, lse the score
    q = rand_bits(rng, (3, 8, D))
    kv = rand_bits(rng, (3, 5, D))
    out, lse = decode(q, kv, np.array([1, 1, 1], np.int32), None, 0.1)
    k = as_f64(kv)
    qf = as_f64(q)
    assert np.array_equal(oracle.float_to_half(out, "bf16"), np.broadcast_to(kv[:, None, 0, :DV], out.shape))
    np.testing.assert_allclose(lse, (qf * k[:, None, 0, :]).sum(-1) * 0.1, rtol=1e-6, atol=1e-6)
    # (2) zero query: uniform weights -> mean of the latent rows, lse = log n
    n = np.array([4, 5, 1], np.int32)
    out, lse = decode(np.zeros_like(q), kv, n, None, 0.3)
    for b in range(3):
        np.testing.assert_allclose(out[b], np.broadcast_to(k[b, : n[b], :DV].mean(0), out[b].shape), rtol=1e-6, atol=1e-6)
        np.testing.assert_allclose(lse[b], math.log(n[b]), rtol=1e-6, atol=1e-6)
    # (3) random inputs against scipy's softmax / logsumexp
    q = rand_bits(rng, (2, 6, D))
    kv = rand_bits(rng, (2, 37, D))
    n = np.array([37, 20], np.int32)
    out, lse = decode(q, kv, n, None, 192 ** -0.5)
    k = as_f64(kv)
    qf = as_f64(q)
    for b in range(2):
        s = qf[b] @ k[b, : n[b]].T * 192 ** -0.5
        np.testing.assert_allclose(out[b], softmax(s, -1) @ k[b, : n[b], :DV], rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(lse[b], logsumexp(s, -1), rtol=1e-6, atol=1e-6)
    # (4) empty sequence: out 0, lse -inf
    out, lse = decode(q, kv, np.array([0, 3], np.int32), None, 1.0)
    assert np.all(out[0] == 0) and np.all(np.isneginf(lse[0]))
    return True


def test_decode_ref_pins():
    assert decode_checks(lambda q, kv, n, bt, s: oracle.mla_decode_ref(q, kv, n, bt, DV, s))


def test_decode_ref_brute_force_tiny():
    """Pure-Python loops (math.exp, no numpy reductions) on a tiny case."""
    rng = np.random.default_rng(3)
    q = rand_bits(rng, (1, 2, D))
    kv = rand_bits(rng, (1, 3, D))
    out, lse = oracle.mla_decode_ref(q, kv, np.array([3], np.int32), None, DV, 0.05)
    qf, k = as_f64(q).tolist(), as_f64(kv).tolist()
    for h in range(2):
        s = [sum(a * b for a, b in zip(qf[0][h], k[0][t])) * 0.05 for t in range(3)]
        z = sum(math.exp(x) for x in s)
        assert abs(lse[0, h] - math.log(z)) < 1e-5
        for c in (0, 17, 511):
            v = sum(math.exp(s[t]) / z * k[0][t][c] for t in range(3))
            assert abs(out[0, h, c] - v) < 1e-5


def test_decode_ref_paging_and_token_order_invariance():
    rng = np.random.default_rng(4)
    page, batch, pages = 16, 2, 5
    q = rand_bits(rng, (batch, 4, D))
    dense = rand_bits(rng, (batch, page * pages, D))
    n = np.array([70, 33], np.int32)
    perm = rng.permutation(batch * pages).astype(np.int32)
    bt = perm.reshape(batch, pages)
    paged = np.empty((batch * pages, page, D), np.uint16)
    paged[bt] = dense.reshape(batch, pages, page, D)
    a = oracle.mla_decode_ref(q, dense, n, None, DV, 0.07)
    b = oracle.mla_decode_ref(q, paged, n, bt, DV, 0.07)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    # reversing the valid tokens of each sequence changes nothing but rounding
    rev = dense.copy()
    for i in range(batch):
        rev[i, : n[i]] = dense[i, : n[i]][::-1]
    c = oracle.mla_decode_ref(q, rev, n, None, DV, 0.07)
    np.testing.assert_allclose(a[0], c[0], rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(a[1], c[1], rtol=1e-6, atol=1e-7)


def test_causal_ref_matches_masked_softmax():
    """Multi-token causal oracle against an explicit [T, N] visibility mask and
    scipy's softmax/logsumexp over the whole score matrix (a different
    computation from the per-token truncation the oracle uses), including a
    sequence shorter than q_len (query tokens that see nothing: out 0, lse -inf)."""
    rng = np.random.default_rng(11)
    T, H, page = 3, 4, 8
    n = np.array([13, 2, 8], np.int32)
    B = len(n)
    pages = 2
    q = rand_bits(rng, (B, T, H, D))
    kv = rand_bits(rng, (B * pages, page, D))
    bt = rng.permutation(B * pages).astype(np.int32).reshape(B, pages)
    out, lse = oracle.mla_decode_ref_causal(q, kv, n, bt, DV, 0.06)
    qf, kf = as_f64(q), as_f64(kv)
    for b in range(B):
        toks = kf[bt[b]].reshape(pages * page, D)[: n[b]]
        s = np.einsum("thd,nd->thn", qf[b], toks) * 0.06
        # token t (the (n - T + t)-th cached token) sees positions j <= n - T + t
        vis = np.arange(n[b])[None, :] <= (n[b] - T + np.arange(T))[:, None]
        for t in range(T):
            if not vis[t].any():
                assert np.all(out[b, t] == 0) and np.all(np.isneginf(lse[b, t]))
                continue
            st = np.where(vis[t][None, :], s[t], -np.inf)
            np.testing.assert_allclose(lse[b, t], logsumexp(st, axis=-1), rtol=1e-6, atol=1e-6)
            np.testing.assert_allclose(out[b, t], softmax(st, axis=-1) @ toks[:, :DV], rtol=1e-5, atol=1e-6)
    # one query token is the single-token oracle
    o1, l1 = oracle.mla_decode_ref_causal(q[:, :1], kv, n, bt, DV, 0.06)
    r1 = oracle.mla_decode_ref(q[:, 0], kv, n, bt, DV, 0.06)
    assert np.array_equal(o1[:, 0], r1[0]) and np.array_equal(l1[:, 0], r1[1])


def test_split_merge_matches_direct():
    """The fused kernel's split/merge algebra equals direct attention for any split count."""
    rng = np.random.default_rng(5)
    q = rand_bits(rng, (1, 3, D))
    kv = rand_bits(rng, (1, 200, D), scale=2.0)
    for n in (1, 7, 200):
        out, lse = oracle.mla_decode_ref(q, kv, np.array([n], np.int32), None, DV, 0.1)
        for splits in (1, 2, 3, 8, 64):
            for h in range(3):
                o2, l2 = oracle.split_merge(q[0, h], kv, 0, n, None, DV, 0.1, splits)
                np.testing.assert_allclose(o2, out[0, h], rtol=1e-5, atol=1e-6)
                assert abs(l2 - lse[0, h]) < 1e-5


def test_fp16_inputs():
    rng = np.random.default_rng(6)
    q = rand_bits(rng, (1, 4, D), "fp16")
    kv = rand_bits(rng, (1, 9, D), "fp16")
    out, lse = oracle.mla_decode_ref(q, kv, np.array([9], np.int32), None, DV, 0.1, dtype="fp16")
    qf, k = as_f64(q, "fp16"), as_f64(kv, "fp16")
    s = qf[0] @ k[0].T * 0.1
    np.testing.assert_allclose(out[0], softmax(s, -1) @ k[0, :, :DV], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(lse[0], logsumexp(s, -1), rtol=1e-6, atol=1e-6)


# ---------------------------------------------------------------------------
# other head dims and float32 elements (what the generic decode is checked by)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dv,dr", [(16, 16), (128, 32), (1024, 256)])
def test_decode_ref_other_dims_fp32(dv, dr):
    """float32 elements at other dims: scipy's softmax/logsumexp, the
    one-token closed form and an empty sequence."""
    rng = np.random.default_rng(dv + dr)
    d = dv + dr
    q = rng.standard_normal((2, 5, d)).astype(np.float32)
    kv = rng.standard_normal((2, 23, d)).astype(np.float32)
    out, lse = oracle.mla_decode_ref(q, kv, np.array([23, 0], np.int32), None, dv, 0.07, dtype="fp32")
    s = q[0].astype(np.float64) @ kv[0].astype(np.float64).T * 0.07
    np.testing.assert_allclose(out[0], softmax(s, -1) @ kv[0, :, :dv].astype(np.float64), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(lse[0], logsumexp(s, -1), rtol=1e-6, atol=1e-6)
    assert np.all(out[1] == 0) and np.all(np.isneginf(lse[1]))
    out1, lse1 = oracle.mla_decode_ref(q, kv, np.array([1, 1], np.int32), None, dv, 0.07, dtype="fp32")
    assert np.array_equal(out1, np.broadcast_to(kv[:, None, 0, :dv], out1.shape))
    sc = (q.astype(np.float64) * kv[:, None, 0, :].astype(np.float64)).sum(-1) * 0.07
    np.testing.assert_allclose(lse1, sc, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("paged", [False, True])
def test_decode_ref_fp32_equals_bf16_on_shared_values(paged):
    """bf16 values handed over as float32 give the bf16 oracle's results bit
    for bit, dense and through a block table (the element loader is the only
    difference between the two)."""
    rng = np.random.default_rng(11)
    dv, d = 128, 160
    q = rand_bits(rng, (3, 4, d))
    kv = rand_bits(rng, (3, 32, d))
    n = np.array([30, 17, 0], np.int32)
    bt = None
    if paged:
        kv = kv.reshape(3 * 4, 8, d)[rng.permutation(12)]
        bt = rng.permutation(12).astype(np.int32).reshape(3, 4)
    a = oracle.mla_decode_ref(q, kv, n, bt, dv, 0.1, dtype="bf16")
    b = oracle.mla_decode_ref(as_f64(q).astype(np.float32), as_f64(kv).astype(np.float32), n, bt, dv, 0.1,
                              dtype="fp32")
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


# ---------------------------------------------------------------------------
# planted mistakes: the checks above must reject a wrong algorithm
# ---------------------------------------------------------------------------

def _numpy_decode(mistake):
    def decode(q, kv, n, bt, scale):
        qf, k = as_f64(q), as_f64(kv)
        B, H = qf.shape[:2]
        out = np.zeros((B, H, DV), np.float32)
        lse = np.full((B, H), -np.inf, np.float32)
        for b in range(B):
            if n[b] == 0:
                continue
            kb = k[b, : n[b]]
            if mistake == "drop_rope":
                s = qf[b, :, :DV] @ kb[:, :DV].T * scale
            elif mistake == "wrong_scale":
                s = qf[b] @ kb.T * scale * 1.01
            elif mistake == "value_from_rope_end":
                s = qf[b] @ kb.T * scale
            elif mistake == "off_by_one_token":
                kb = k[b, : max(n[b] - 1, 1)]
                s = qf[b] @ kb.T * scale
            else:
                s = qf[b] @ kb.T * scale
            p = softmax(s, -1)
            vals = kb[:, D - DV:] if mistake == "value_from_rope_end" else kb[:, :DV]
            out[b] = p @ vals
            lse[b] = logsumexp(s, -1)
        return out, lse
    return decode


def test_checks_accept_a_correct_restatement():
    assert decode_checks(_numpy_decode(None))


@pytest.mark.parametrize("mistake", ["drop_rope", "wrong_scale", "value_from_rope_end", "off_by_one_token"])
def test_checks_reject_planted_mistakes(mistake):
    with pytest.raises(AssertionError):
        decode_checks(_numpy_decode(mistake))


# ---------------------------------------------------------------------------
# MLA layer restatement
# ---------------------------------------------------------------------------

def small_layer(rng, hidden=64, heads=4, q_rank=32, rank=512, dn=128, dr=64, dv=128):
    cfg = dict(hidden_size=hidden, num_heads=heads, q_lora_rank=q_rank, kv_lora_rank=rank,
               qk_nope_head_dim=dn, qk_rope_head_dim=dr, v_head_dim=dv, rope_theta=10000.0, rms_norm_eps=1e-6)
    w = {
        "wq_a": rng.standard_normal((q_rank, hidden)) * 0.05,
        "q_norm": 1 + 0.1 * rng.standard_normal(q_rank),
        "wq_b": rng.standard_normal((heads * (dn + dr), q_rank)) * 0.05,
        "wkv_a": rng.standard_normal((rank + dr, hidden)) * 0.05,
        "kv_norm": 1 + 0.1 * rng.standard_normal(rank),
        "wkv_b": rng.standard_normal((heads * (dn + dv), rank)) * 0.05,
        "wo": rng.standard_normal((hidden, heads * dv)) * 0.05,
    }
    return cfg, w


def test_rope_and_norm_closed_forms():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((3, 64))
    np.testing.assert_allclose(oracle.apply_rope(x, np.zeros(3), 10000.0), x, atol=0)  # position 0
    y = oracle.apply_rope(x, np.array([1, 17, 4000]), 10000.0)
    pair = lambda a: a[:, :32] ** 2 + a[:, 32:] ** 2  # rotation preserves each (i, i+32) pair norm
    np.testing.assert_allclose(pair(y), pair(x), rtol=1e-12)
    # first frequency is 1 rad per position: (x0, x32) rotated by p radians
    p = 17.0
    np.testing.assert_allclose(y[1, 0], x[1, 0] * math.cos(p) - x[1, 32] * math.sin(p), rtol=1e-12)
    r = oracle.rms_norm(x, np.ones(64), 0.0)
    np.testing.assert_allclose(np.sqrt((r ** 2).mean(-1)), 1.0, rtol=1e-12)


def test_layer_absorption_identity():
    """forward_naive == absorbed query -> latent attention -> W_UV -> wo (float64)."""
    rng = np.random.default_rng(8)
    cfg, w = small_layer(rng)
    B = 3
    lens = [0, 5, 19]
    x = rng.standard_normal((B, cfg["hidden_size"]))
    toks = [rng.standard_normal((n, 576)) for n in lens]
    naive, entries = oracle.layer_forward_naive(w, cfg, x, toks, lens)
    q_nope, q_pe, _, _ = oracle.layer_project(w, cfg, x, np.array(lens))
    q_abs = oracle.layer_absorbed_query(w, cfg, q_nope, q_pe)
    scale = 192 ** -0.5
    o_lat = np.zeros((B, cfg["num_heads"], 512))
    for b in range(B):
        rows = np.concatenate([toks[b], entries[b:b + 1]], 0)
        s = q_abs[b] @ rows.T * scale
        o_lat[b] = softmax(s, -1) @ rows[:, :512]
    absorbed = oracle.layer_output(w, cfg, o_lat)
    np.testing.assert_allclose(absorbed, naive, rtol=1e-10, atol=1e-12)


def test_package_forward_naive_matches_layer_oracle():
    """The package's torch MLA.forward_naive (CPU, float32) against the float64 restatement."""
    from triton_mla import MLA, MLAConfig

    torch.manual_seed(0)
    cfg = MLAConfig(hidden_size=64, num_heads=4, q_lora_rank=32)
    model = MLA(cfg).double()
    for p in model.parameters():
        p.data.normal_(0, 0.05)
    w = {k: v.detach().numpy() for k, v in {
        "wq_a": model.wq_a.weight, "q_norm": model.q_norm.weight, "wq_b": model.wq_b.weight,
        "wkv_a": model.wkv_a.weight, "kv_norm": model.kv_norm.weight, "wkv_b": model.wkv_b.weight,
        "wo": model.wo.weight}.items()}
    ocfg = dict(hidden_size=64, num_heads=4, q_lora_rank=32, kv_lora_rank=512, qk_nope_head_dim=128,
                qk_rope_head_dim=64, v_head_dim=128, rope_theta=10000.0, rms_norm_eps=1e-6)
    B, page, blocks = 3, 16, 3
    lens = torch.tensor([0, 5, 24], dtype=torch.int32)
    bt = torch.randperm(B * blocks).view(B, blocks).int()
    cache = torch.randn(B * blocks, page, 576, dtype=torch.float64)
    x = torch.randn(B, 64, dtype=torch.float64)
    toks = [cache[bt[b].long()].reshape(-1, 576)[: int(lens[b])].numpy() for b in range(B)]
    ref, _ = oracle.layer_forward_naive(w, ocfg, x.numpy(), toks, lens.numpy())
    with torch.no_grad():
        out, new_lens = model.forward_naive(x, cache, lens, bt)
    assert torch.equal(new_lens, lens + 1)
    # the layer keeps the reference's float32 RoPE (model.py:44-50): fp32-level agreement
    np.testing.assert_allclose(out.numpy(), ref, rtol=1e-4, atol=1e-6)
