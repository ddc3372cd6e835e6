"""The public mla_decode call on repeated shapes.

A shape seen before launches from its kept constant arguments (no
re-validation, no library queries); the result must be bit-identical to a
fresh DecodeLaunch of the same inputs on every call, for new data, for the
FlashMLA 4-D cache layout, on a second stream, and when an unaligned q sends
the call back through the full path. Checked against the oracle once (out
atol = rtol = 1e-2, lse 1e-3), the rest bit-exact.
"""

import pytest
import torch

import triton_mla
from triton_mla import kernel as K
from test_kernel_gpu import SCALE, check, run_oracle

pytestmark = pytest.mark.gpu


def _inputs(seed, batch=3, heads=20, pages=36, page=64, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, heads, 576, generator=g).to(dtype)
    kv = torch.randn(pages, page, 576, generator=g).to(dtype)
    bt = torch.randperm(pages, generator=g)[: batch * (pages // batch)].view(batch, -1).int()
    seqlens = torch.tensor([1, 200, 700][:batch], dtype=torch.int32)
    return q, kv, seqlens, bt


def _fresh(q, kv, seqlens, bt, splits=None):
    return K.DecodeLaunch(q, kv, seqlens, bt, 512, SCALE, splits).run(False)


@pytest.mark.parametrize("splits", [None, 4])
def test_repeated_shape_matches_a_fresh_launch(splits):
    dev = torch.device("cuda:0")
    for seed in range(3):  # the first call learns the shape, the others reuse it
        q, kv, seqlens, bt = (t.to(dev) for t in _inputs(seed))
        out, lse = triton_mla.mla_decode(q, kv, seqlens, bt, softmax_scale=SCALE, num_splits=splits,
                                         return_lse=True)
        ref_out, ref_lse = _fresh(q, kv, seqlens, bt, splits)
        torch.cuda.synchronize()
        assert torch.equal(out, ref_out) and torch.equal(lse, ref_lse), f"seed {seed}"
        if seed == 0:
            r_out, r_lse = run_oracle(q, kv, seqlens, bt, SCALE, q.dtype)
            check(out, lse, r_out, r_lse, seqlens)
    assert any(s for s in K._SHAPES.values()), "the repeated shape did not take the kept-argument path"


def test_four_dim_cache_second_stream_and_unaligned_q():
    dev = torch.device("cuda:0")
    q, kv, seqlens, bt = (t.to(dev) for t in _inputs(7, dtype=torch.float16))
    ref_out, ref_lse = _fresh(q, kv, seqlens, bt)
    kv4 = kv.unsqueeze(2)
    for _ in range(2):
        out = triton_mla.mla_decode(q, kv4, seqlens, bt, softmax_scale=SCALE)
        torch.cuda.synchronize()
        assert torch.equal(out, ref_out)
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        out, lse = triton_mla.mla_decode(q, kv4, seqlens, bt, softmax_scale=SCALE, return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(out, ref_out) and torch.equal(lse, ref_lse)
    # q at an 8-byte offset: the call copies it (full path) and still agrees
    buf = torch.empty(q.numel() + 4, dtype=q.dtype, device=dev)
    q_off = buf[4:].view_as(q)
    q_off.copy_(q)
    assert q_off.data_ptr() % 16 != 0
    out = triton_mla.mla_decode(q_off, kv, seqlens, bt, softmax_scale=SCALE)
    torch.cuda.synchronize()
    assert torch.equal(out, ref_out)


def test_graph_capture_and_threads_share_no_workspace():
    """A captured public call takes its workspace from the graph's memory:
    replays reproduce the eager bits with eager calls of another shape on the
    same stream between them. Two Python threads calling on one stream get
    the bits of calls made one at a time."""
    import threading

    dev = torch.device("cuda:0")
    a = [t.to(dev) for t in _inputs(11)]
    b = [t.to(dev) for t in _inputs(12, batch=2, heads=128)]
    ref_a, ref_b = _fresh(*a)[0], _fresh(*b)[0]
    triton_mla.mla_decode(*a, softmax_scale=SCALE)  # learn the shape eagerly first
    cap = torch.cuda.Stream(dev)
    cap.wait_stream(torch.cuda.current_stream(dev))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cap):
        g_out = triton_mla.mla_decode(*a, softmax_scale=SCALE)
    for rep in range(3):
        g_out.zero_()
        with torch.cuda.stream(cap):
            graph.replay()
            eager = triton_mla.mla_decode(*b, softmax_scale=SCALE)
        torch.cuda.synchronize()
        assert torch.equal(g_out, ref_a), f"replay {rep}"
        assert torch.equal(eager, ref_b), f"eager call after replay {rep}"

    results, errors = {}, []

    def worker(i, args):
        try:
            results[i] = [triton_mla.mla_decode(*args, softmax_scale=SCALE) for _ in range(20)]
        except Exception as e:  # pragma: no cover - reported below
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(i, a if i % 2 == 0 else b)) for i in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for i, outs in results.items():
        ref = ref_a if i % 2 == 0 else ref_b
        assert all(torch.equal(o, ref) for o in outs), f"thread {i}"
