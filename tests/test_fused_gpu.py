"""The single-launch decode (tmla_mla_decode_fused: the log-sum-exp merge of
the split partials done inside the partial kernel) against the two-kernel
form (tmla_mla_decode_partial + tmla_mla_decode_combine, the reference's two
launches, src/triton_mla/kernel.py:276-320) on the same inputs.

Both forms merge the same stored partials with the same code in the same
order, so out and lse must agree bit for bit; the two-kernel form itself is
checked against the oracle in test_kernel_gpu.py and test_configs_gpu.py, and
here the headline case is also checked against the oracle directly.

Covered: balanced partitions with 1, 8, 16 and more than 16 workers per
sequence; workers whose range straddles two split sequences (both of their
merge records in use); the uniform split; empty sequences (out = 0,
lse = -inf, cleared by the single launch itself); 3, 16, 24, 64, 128 and 200
heads (the 16-head-group kernel up to 16 heads; one or two head blocks per
worker above); fp16; repeated calls on one workspace
(the merge counters return to zero); one workspace shared by calls of
different sizes; the hand-over path (spin limit 0: every worker that does not
complete the count gives its share to the one that does); and HIP-graph
replays.
"""

import pytest
import torch

import oracle
from conftest import bits, dtype_name

pytestmark = pytest.mark.gpu


def launch(inp, gpu, num_splits=None, num_workers=None):
    from triton_mla.kernel import DecodeLaunch

    d = inp.to(gpu)
    return DecodeLaunch(d.q, d.kv_cache, d.seqlens, d.block_table, 512, d.softmax_scale, num_splits, num_workers)


def two_stage(call):
    call.out.fill_(1.0)
    call.lse.fill_(1.0)
    call.partial()
    call.combine()
    torch.cuda.synchronize()
    return call.out.clone(), call.lse.clone()


def single(call, spin_limit=-1):
    call.out.fill_(1.0)  # every element must be written by the launch
    call.lse.fill_(1.0)
    call.run(single_launch=True, spin_limit=spin_limit)
    torch.cuda.synchronize()
    return call.out.clone(), call.lse.clone()


def assert_same(a, b, what):
    (oa, la), (ob, lb) = a, b
    assert torch.equal(oa.view(torch.int16), ob.view(torch.int16)), f"{what}: out differs"
    assert torch.equal(la.view(torch.int32), lb.view(torch.int32)), f"{what}: lse differs"


def case(name):
    from triton_mla import workloads

    if name == "b32_h128_8k":
        return workloads.b32_h128_8k()
    if name == "b1_h128_1k":
        return workloads.b1_h128_1k()
    if name == "ragged_h128":  # empty, 1-token and long sequences
        inp = workloads.ragged(12, 128, 0, 6000, seed=5)
        inp.seqlens[[2, 7]] = torch.tensor([0, 1], dtype=torch.int32)
        return inp
    if name == "ragged_h24":
        return workloads.ragged(40, 24, 0, 3000, seed=6)
    if name == "ragged_h16":  # the 16-head-group kernel; empty and 1-token sequences
        inp = workloads.ragged(40, 16, 0, 3000, seed=9)
        inp.seqlens[[3, 11]] = torch.tensor([0, 1], dtype=torch.int32)
        return inp
    if name == "ragged_h3":  # one partly used 16-head group
        inp = workloads.ragged(20, 3, 0, 5000, seed=10)
        inp.seqlens[5] = 0
        return inp
    if name == "ragged_h64_fp16":
        return workloads.ragged(9, 64, 1, 5000, dtype=torch.float16, seed=7)
    if name == "ragged_h200":
        return workloads.ragged(6, 200, 0, 4000, seed=8)
    raise KeyError(name)


# (case, num_splits, num_workers): workers per split sequence from 1 to > 16;
# 7 and 24 workers give ranges that straddle sequence ends
CASES = [
    ("b32_h128_8k", None, None),      # 8 workers per sequence
    ("b1_h128_1k", None, None),       # 16 workers per sequence
    ("ragged_h128", None, None),      # up to ~90 workers per sequence, one-tile chunks
    ("ragged_h128", None, 7),         # straddling ranges
    ("ragged_h128", 4, None),         # uniform split
    ("ragged_h24", None, 24),
    ("ragged_h16", None, None),
    ("ragged_h16", None, 24),         # straddling ranges
    ("ragged_h16", 4, None),          # uniform split
    ("ragged_h3", None, None),
    ("ragged_h64_fp16", None, None),
    ("ragged_h64_fp16", 3, None),
    ("ragged_h200", None, 100),       # two head blocks per worker
]


@pytest.mark.parametrize("name,splits,workers", CASES)
def test_single_launch_equals_two_kernels(gpu, name, splits, workers):
    inp = case(name)
    call = launch(inp, gpu, splits, workers)
    assert call.fused, "the case must take the single-launch path"
    ref = two_stage(call)
    for rep in range(3):  # the same workspace again: the counters were reset
        assert_same(single(call), ref, f"{name} splits={splits} workers={workers} call {rep}")
    call.run()  # tmla_mla_decode: the two kernels
    torch.cuda.synchronize()
    assert_same((call.out.clone(), call.lse.clone()), ref, f"{name} tmla_mla_decode")
    empty = inp.seqlens == 0
    if bool(empty.any()):
        out, lse = single(call)
        assert torch.all(out[empty.to(gpu)] == 0) and torch.all(torch.isneginf(lse[empty.to(gpu)]))


@pytest.mark.parametrize("name,splits,workers", [CASES[0], CASES[2], CASES[3], CASES[5], CASES[6], CASES[7]])
def test_hand_over_path(gpu, name, splits, workers):
    """Spin limit 0 (a per-call argument): a worker that does not complete
    its sequence's count hands its share over at once; the worker that
    completes the count merges it. Same bits as the two-kernel form, and the
    counters still reset (the next call with the default limit agrees)."""
    call = launch(case(name), gpu, splits, workers)
    ref = two_stage(call)
    assert_same(single(call, spin_limit=0), ref, f"{name} hand-over")
    assert_same(single(call, spin_limit=0), ref, f"{name} hand-over, second call")
    assert_same(single(call), ref, f"{name} after hand-over")


def fused_on(lib, call, workspace, stream):
    """tmla_mla_decode_fused with call's arguments on another workspace."""
    from triton_mla import _native

    args = call._partial_args[:-2] + (workspace.data_ptr(), workspace.numel())
    _native.check(lib.tmla_mla_decode_fused(*args, -1, stream), "tmla_mla_decode_fused")


def test_workspace_reuse_across_sizes(gpu):
    """One workspace sized for the largest call serves smaller and larger
    calls in any order: the merge counters sit at the end of the buffer, so
    no call's partial rows overwrite another call's counters. The buffer is
    filled with garbage except the counter suffix (tmla_workspace_zero_bytes)."""
    from triton_mla import _native, workloads

    lib = _native.load()
    big = launch(workloads.b32_h128_8k(), gpu)
    small = launch(workloads.b8_h128_1k(), gpu)
    mid = launch(case("ragged_h128"), gpu)
    calls = {"big": big, "small": small, "mid": mid}
    for name, c in calls.items():
        assert c.fused, f"{name} must take the single-launch path"
        assert c.ws_bytes <= big.ws_bytes
    refs = {name: two_stage(c) for name, c in calls.items()}
    ws = torch.full((big.ws_bytes,), 0x5A, dtype=torch.uint8, device=gpu)
    z = min(lib.tmla_workspace_zero_bytes(big.batch, big.num_heads, 512, big.splits, big.workers), big.ws_bytes)
    ws[big.ws_bytes - z:].zero_()
    stream = torch.cuda.current_stream(gpu).cuda_stream
    for name in ["big", "small", "big", "mid", "small", "mid", "big"]:
        c = calls[name]
        c.out.fill_(1.0)
        c.lse.fill_(1.0)
        fused_on(lib, c, ws, stream)
        torch.cuda.synchronize()
        assert_same((c.out.clone(), c.lse.clone()), refs[name], f"{name} on the shared workspace")


def test_workspace_reuse_across_shapes(gpu):
    """Calls of other shapes on one workspace: a 24-head call with more
    sequences has a larger counter set but a smaller workspace than the
    128-head headline call that sized the buffer; its counters stay clear of
    the headline call's partials (the counter block is the same fixed size for
    every call), so both keep the two-kernel bits in any order."""
    from triton_mla import _native, workloads

    lib = _native.load()
    big = launch(workloads.b32_h128_8k(), gpu)
    wide = launch(workloads.ragged(64, 24, 1024, 32768), gpu)
    calls = {"big": big, "wide": wide}
    for name, c in calls.items():
        assert c.fused, f"{name} must take the single-launch path"
    assert wide.ws_bytes <= big.ws_bytes
    refs = {name: two_stage(c) for name, c in calls.items()}
    ws = torch.full((big.ws_bytes,), 0x5A, dtype=torch.uint8, device=gpu)
    z = min(lib.tmla_workspace_zero_bytes(big.batch, big.num_heads, 512, big.splits, big.workers), big.ws_bytes)
    assert z == lib.tmla_workspace_zero_bytes(wide.batch, wide.num_heads, 512, wide.splits, wide.workers)
    ws[big.ws_bytes - z:].zero_()
    stream = torch.cuda.current_stream(gpu).cuda_stream
    for name in ["big", "wide", "big", "wide"]:
        c = calls[name]
        c.out.fill_(1.0)
        c.lse.fill_(1.0)
        fused_on(lib, c, ws, stream)
        torch.cuda.synchronize()
        assert_same((c.out.clone(), c.lse.clone()), refs[name], f"{name} on the shared workspace")


def test_fuse_decision_matches_launch(gpu):
    """DecodeLaunch.fused comes from the library's own plan: a call it
    reports as single-launch needs no combine kernel (stage 2 after it would
    be redundant), and a grid larger than the device is reported as two-stage."""
    from triton_mla import workloads

    assert launch(workloads.b32_h128_8k(), gpu).fused
    assert launch(workloads.b1_h128_1k(), gpu).fused
    # 64 sequences x 128 heads with 512 uniform splits cannot be resident at once
    assert not launch(workloads.uniform(64, 128, 2048), gpu, num_splits=8).fused


def test_headline_against_oracle(gpu):
    """B=32, H=128, 8K context through the single launch, checked against the
    float64 oracle on the first two sequences (atol = rtol = 1e-2)."""
    inp = case("b32_h128_8k")
    call = launch(inp, gpu)
    out, lse = single(call)
    n = 2
    ref_out, ref_lse = oracle.mla_decode_ref(bits(inp.q[:n]), bits(inp.kv_cache), inp.seqlens[:n].numpy(),
                                             inp.block_table[:n].numpy(), 512, inp.softmax_scale,
                                             dtype=dtype_name(inp.q.dtype))
    torch.testing.assert_close(out[:n].float().cpu(), torch.from_numpy(ref_out), atol=1e-2, rtol=1e-2)
    torch.testing.assert_close(lse[:n].cpu(), torch.from_numpy(ref_lse), atol=1e-3, rtol=1e-3)


def test_graph_replays(gpu):
    """The single launch captured in a HIP graph: every replay (with eager
    work and synchronisation in between) reproduces the eager result."""
    call = launch(case("ragged_h128"), gpu)
    eager = single(call)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call.run(single_launch=True)
    for rep in range(4):
        call.out.fill_(1.0)
        call.lse.fill_(1.0)
        graph.replay()
        torch.cuda.synchronize()
        assert_same((call.out.clone(), call.lse.clone()), eager, f"graph replay {rep}")
        torch.randn(1024, device=gpu).sum().item()  # eager work between replays
