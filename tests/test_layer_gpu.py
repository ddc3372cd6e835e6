"""HIP glue of the absorbed MLA decode step (triton_mla.layer_ops) against the
float64 oracle restatement of the reference layer (oracle/oracle.py:
rms_norm, apply_rope, the W_UK / W_UV einsums; src/triton_mla/model.py:34-50,
74-124).

The kernels compute in float32 from bf16 inputs and round once to bf16, as
the reference's float32 torch steps do. Each output element must lie within
half a bf16 ulp of the float64 value plus the float32 error bound of its
computation (n * 2^-24 * sum |a_i b_i| for an n-term dot product; the float32
angle error (|angle| + 2) * 2^-22 times |x1| + |x2| for a rotation), and at
least 99.9% of the elements must equal the correctly rounded bf16 of the
float64 value. The cache append must leave every other cache row untouched,
bit for bit; RoPE is also compared with the reference's torch apply_rope run
on the GPU in float32 (within one bf16 ulp plus twice the float32 bound).
"""

import numpy as np
import pytest
import torch

import oracle
from conftest import bits

pytestmark = pytest.mark.gpu

ROPE_THETA = 10000.0


def ulp_bf16(x):
    """Spacing of bf16 numbers around |x| (float64)."""
    ax = np.maximum(np.abs(x), 2.0 ** -126)
    return 2.0 ** (np.floor(np.log2(ax)) - 7)


def assert_matches(got_bits, ref64, f32_bound, what, min_exact=0.999):
    """|got - ref| <= ulp/2 + f32_bound elementwise; most elements correctly rounded."""
    got = oracle.half_to_float(got_bits, "bf16")
    err = np.abs(got - ref64)
    bound = 0.5 * ulp_bf16(ref64) + f32_bound
    worst = float(np.max(err / bound))
    exact = float(np.mean(got_bits == oracle.float_to_half(ref64, "bf16")))
    print(f"{what}: max err / bound {worst:.3f}, correctly rounded {exact:.5f}", flush=True)
    assert worst <= 1.0, f"{what}: error above the float32 + rounding bound ({worst})"
    assert exact >= min_exact, f"{what}: only {exact:.4f} of the elements correctly rounded"


def dot_bound(n, abs_products_sum):
    """Float32 accumulation error bound of an n-term sum of products."""
    return n * 2.0 ** -24 * abs_products_sum


def rope_bound(x, positions, theta):
    """Float32 error of a rotation: the angle pos / theta^(2i/d) carries a
    relative error of a few 2^-24, times |x1| + |x2|."""
    d = x.shape[-1]
    freq = theta ** (np.arange(0, d, 2) / d)
    ang = np.asarray(positions, dtype=np.float64)[..., None] / freq
    mag = np.abs(x[..., : d // 2]) + np.abs(x[..., d // 2:])
    b = mag * (np.abs(ang) + 2.0) * 2.0 ** -22
    return np.concatenate([b, b], axis=-1)


def f64(t):
    return t.float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("layout", ["paged16", "paged64", "dense"])
def test_kv_append_matches_oracle(gpu, layout):
    from triton_mla import layer_ops

    gen = torch.Generator().manual_seed(11)
    rank, rope, eps = 512, 64, 1e-6
    positions = torch.tensor([0, 15, 16, 63, 64, 200, 511], dtype=torch.int32)
    batch = positions.shape[0]
    kv_proj = torch.randn(batch, rank + rope, generator=gen).to(torch.bfloat16)
    weight = (1.0 + 0.3 * torch.randn(rank, generator=gen)).to(torch.bfloat16)
    if layout == "dense":
        cache = torch.randn(batch, 512, rank + rope, generator=gen).to(torch.bfloat16)
        bt = None
    else:
        page = 16 if layout == "paged16" else 64
        pages = 512 // page
        cache = torch.randn(batch * pages, page, rank + rope, generator=gen).to(torch.bfloat16)
        bt = torch.randperm(batch * pages, generator=gen).view(batch, pages).int()
    before = cache.clone()
    gcache = cache.to(gpu)
    layer_ops.kv_append(kv_proj.to(gpu), weight.to(gpu), eps, ROPE_THETA, positions.to(gpu), gcache,
                        None if bt is None else bt.to(gpu), rank, rope)
    torch.cuda.synchronize(gpu)
    after = gcache.cpu()

    pos = positions.long()
    if bt is None:
        rows = (torch.arange(batch), pos)
    else:
        page = cache.shape[1]
        rows = (bt[torch.arange(batch), pos // page].long(), pos % page)
    got = bits(after[rows])
    x = f64(kv_proj)
    ref = np.concatenate([oracle.rms_norm(x[:, :rank], f64(weight), eps),
                          oracle.apply_rope(x[:, rank:], positions.numpy(), ROPE_THETA)], axis=-1)
    w = f64(weight)
    norm_bound = (rank + 8) * 2.0 ** -24 * np.abs(ref[:, :rank])  # mean of squares, rsqrt, two products
    bound = np.concatenate([norm_bound, rope_bound(x[:, rank:], positions.numpy(), ROPE_THETA)], axis=-1)
    assert_matches(got, ref, bound, f"appended rows ({layout})")
    mask = torch.ones(after.shape[:2], dtype=torch.bool)
    mask[rows] = False
    assert np.array_equal(bits(after[mask]), bits(before[mask])), "rows other than the appended ones changed"


@pytest.mark.parametrize("batch,heads", [(1, 16), (16, 128), (33, 16)])
def test_absorb_q_matches_oracle(gpu, batch, heads):
    from triton_mla import layer_ops

    gen = torch.Generator().manual_seed(12 + batch)
    nope, rope, rank, vd = 128, 64, 512, 128
    q_proj = torch.randn(batch, heads * (nope + rope), generator=gen).to(torch.bfloat16)
    wkv_b = (0.05 * torch.randn(heads * (nope + vd), rank, generator=gen)).to(torch.bfloat16)
    positions = torch.randint(0, 20000, (batch,), generator=gen, dtype=torch.int32)
    out = layer_ops.absorb_q(q_proj.to(gpu), wkv_b.to(gpu), positions.to(gpu), heads, nope, rope, rank, vd,
                             ROPE_THETA)
    torch.cuda.synchronize(gpu)
    assert out.shape == (batch, heads, rank + rope)
    q = f64(q_proj).reshape(batch, heads, nope + rope)
    w = {"wkv_b": f64(wkv_b)}
    cfg = {"num_heads": heads, "qk_nope_head_dim": nope, "v_head_dim": vd, "kv_lora_rank": rank}
    q_pe = oracle.apply_rope(q[..., nope:], positions.numpy()[:, None], ROPE_THETA)
    ref = oracle.layer_absorbed_query(w, cfg, q[..., :nope], q_pe)
    got = bits(out.cpu())
    w_uk = f64(wkv_b).reshape(heads, nope + vd, rank)[:, :nope]
    abs_sum = np.einsum("bhd,hdc->bhc", np.abs(q[..., :nope]), np.abs(w_uk))
    assert_matches(got[..., :rank], ref[..., :rank], dot_bound(nope, abs_sum), f"q_nope . W_UK (B={batch}, H={heads})")
    # positions up to 20000: the float32 angle (as in the reference's float32
    # apply_rope) moves about 2% of the results off the float64 rounding
    assert_matches(got[..., rank:], ref[..., rank:], rope_bound(q[..., nope:], positions.numpy()[:, None], ROPE_THETA),
                   f"RoPE(q_pe) (B={batch}, H={heads})", min_exact=0.95)
    # the reference's own float32 rotation on the GPU
    from triton_mla.model import apply_rope

    q_pe_dev = q_proj.to(gpu).view(batch, heads, nope + rope)[..., nope:]
    torch_rope = apply_rope(q_pe_dev, positions.to(gpu)[:, None], ROPE_THETA).float().cpu()
    # two float32 evaluations: each within rope_bound of float64
    tol = ulp_bf16(torch_rope.numpy().astype(np.float64)) + 2 * rope_bound(q[..., nope:], positions.numpy()[:, None],
                                                                           ROPE_THETA)
    diff = (out[..., rank:].float().cpu() - torch_rope).abs().numpy()
    assert bool((diff <= tol).all()), f"RoPE differs from torch's float32 rotation by {float(np.max(diff / tol))} x tol"


@pytest.mark.parametrize("batch,heads", [(1, 16), (16, 128), (40, 16)])
def test_absorb_out_matches_oracle(gpu, batch, heads):
    from triton_mla import layer_ops

    gen = torch.Generator().manual_seed(13 + batch)
    nope, rank, vd = 128, 512, 128
    o_lat = torch.randn(batch, heads, rank, generator=gen).to(torch.bfloat16)
    wkv_b = (0.05 * torch.randn(heads * (nope + vd), rank, generator=gen)).to(torch.bfloat16)
    out = layer_ops.absorb_out(o_lat.to(gpu), wkv_b.to(gpu), heads, nope, rank, vd)
    torch.cuda.synchronize(gpu)
    assert out.shape == (batch, heads * vd)
    w_uv = f64(wkv_b).reshape(heads, nope + vd, rank)[:, nope:]
    ref = np.einsum("bhc,hdc->bhd", f64(o_lat), w_uv).reshape(batch, heads * vd)
    abs_sum = np.einsum("bhc,hdc->bhd", np.abs(f64(o_lat)), np.abs(w_uv)).reshape(batch, heads * vd)
    assert_matches(bits(out.cpu()), ref, dot_bound(rank, abs_sum), f"o . W_UV (B={batch}, H={heads})")


@pytest.mark.parametrize("layout", ["paged64", "dense"])
@pytest.mark.parametrize("batch", [1, 7, 16])
def test_norm_append_equals_the_two_calls(gpu, layout, batch):
    """tmla_mla_norm_append (the query latent's RMSNorm and the cache append in
    one launch) gives the bits of tmla_mla_rms_norm and tmla_mla_kv_append
    run separately, leaves the same cache, and returns positions + 1 (a
    position past the block table included: its row is not written, its
    length still advances)."""
    from triton_mla import layer_ops

    gen = torch.Generator().manual_seed(batch * 7 + len(layout))
    rank, rope, qd = 512, 64, 1536
    positions = torch.randint(0, 500, (batch,), generator=gen, dtype=torch.int32)
    positions[-1] = 511 if layout == "dense" else 512  # paged: one past the table's last row
    q_lat = (2.0 * torch.randn(batch, qd, generator=gen)).to(torch.bfloat16)
    q_w = (1.0 + 0.3 * torch.randn(qd, generator=gen)).to(torch.bfloat16)
    kv_proj = torch.randn(batch, rank + rope, generator=gen).to(torch.bfloat16)
    kv_w = (1.0 + 0.3 * torch.randn(rank, generator=gen)).to(torch.bfloat16)
    if layout == "dense":
        cache = torch.randn(batch, 512, rank + rope, generator=gen).to(torch.bfloat16)
        bt = None
    else:
        cache = torch.randn(batch * 8, 64, rank + rope, generator=gen).to(torch.bfloat16)
        bt = torch.randperm(batch * 8, generator=gen).view(batch, 8).int().to(gpu)
    c1, c2 = cache.to(gpu), cache.to(gpu)
    pos = positions.to(gpu)
    y1 = layer_ops.rms_norm(q_lat.to(gpu), q_w.to(gpu), 1e-6)
    layer_ops.kv_append(kv_proj.to(gpu), kv_w.to(gpu), 1e-6, ROPE_THETA, pos, c1, bt, rank, rope)
    y2, nxt = layer_ops.norm_append(q_lat.to(gpu), q_w.to(gpu), 1e-6, kv_proj.to(gpu), kv_w.to(gpu), 1e-6,
                                    ROPE_THETA, pos, c2, bt, rank, rope)
    torch.cuda.synchronize(gpu)
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))
    assert torch.equal(c1.view(torch.int16), c2.view(torch.int16))
    assert nxt.dtype == torch.int32 and torch.equal(nxt.cpu(), positions + 1)
    if batch > 1 or layout == "dense":  # (batch 1 paged: the only position lies past the table)
        assert not torch.equal(c2.cpu().view(torch.int16), cache.view(torch.int16))  # rows were appended


@pytest.mark.parametrize("rows,dim,strided", [(16, 1536, True), (3, 512, False), (9, 4104, False)])
def test_rms_norm_matches_oracle(gpu, rows, dim, strided):
    """RMSNorm of rows (tmla_mla_rms_norm) against the float64 oracle's
    rms_norm: within half a bf16 ulp plus the float32 error of the sum of
    squares, the rsqrt and two products ((dim + 8) * 2^-24 relative)."""
    from triton_mla import layer_ops

    gen = torch.Generator().manual_seed(rows * 31 + dim)
    width = dim + (64 if strided else 0)
    xbuf = (2.0 * torch.randn(rows, width, generator=gen)).to(torch.bfloat16)
    w = (1.0 + 0.3 * torch.randn(dim, generator=gen)).to(torch.bfloat16)
    xg = xbuf.to(gpu)[:, :dim]
    y = layer_ops.rms_norm(xg, w.to(gpu), 1e-6)
    torch.cuda.synchronize(gpu)
    ref = oracle.rms_norm(f64(xbuf[:, :dim]), f64(w), 1e-6)
    assert_matches(bits(y.cpu()), ref, np.abs(ref) * (dim + 8) * 2.0 ** -24, f"rms_norm ({rows}x{dim})")


# (m, n, k): the four DeepSeek-V3 projections of a 16-row step (wq_a, wq_b,
# wkv_a, wo), then row counts of 1 to 64 (one to four 16-row blocks, partial
# blocks), 16-column groups (n not a multiple of 64), contractions of one
# 64-element chunk, fewer chunks than waves, and chunk counts that split
# unevenly over waves and workgroups
PROJECT_SHAPES = [(16, 1536, 7168), (16, 24576, 1536), (16, 576, 7168), (16, 7168, 16384),
                  (1, 64, 128), (5, 48, 1024), (33, 32, 320), (64, 16, 64), (17, 80, 4032),
                  (48, 112, 2112), (2, 4096, 64 * 37)]


@pytest.mark.parametrize("m,n,k", PROJECT_SHAPES)
def test_project_matches_oracle(gpu, m, n, k):
    """y = x . W^T (tmla_mla_project) against the float64 product: within half a
    bf16 ulp plus the float32 bound of a k-term dot product, elementwise;
    at least 99% correctly rounded (a float32 sum lands on the other side of
    a rounding boundary for about 2^-8 of the elements at k = 16K)."""
    from triton_mla import layer_ops

    gen = torch.Generator().manual_seed(m * 7919 + n * 31 + k)
    x = torch.randn(m, k, generator=gen).to(torch.bfloat16)
    w = (0.02 * torch.randn(n, k, generator=gen)).to(torch.bfloat16)
    xg, wg = x.to(gpu), w.to(gpu)
    assert layer_ops.project_fits(xg, wg)
    y = layer_ops.project(xg, wg)
    again = [layer_ops.project(xg, wg) for _ in range(5)]
    torch.cuda.synchronize(gpu)
    assert y.shape == (m, n) and y.dtype == torch.bfloat16
    for i, y2 in enumerate(again):
        assert np.array_equal(bits(y.cpu()), bits(y2.cpu())), f"call {i + 1} differs from the first"
    ref = f64(x) @ f64(w).T
    abs_sum = np.abs(f64(x)) @ np.abs(f64(w)).T
    assert_matches(bits(y.cpu()), ref, dot_bound(k, abs_sum), f"x . W^T ({m}x{n}x{k})", min_exact=0.99)


def test_project_workspace_shared_across_shapes(gpu):
    """Calls of different shapes in turn on one workspace, zero-filled once:
    a narrow weight (many split-contraction tiles, few counters) and a wide
    one (fewer tiles, more counters) give the bits of a call on a fresh
    workspace, every time."""
    from triton_mla import _native

    lib = _native.load()
    gen = torch.Generator().manual_seed(5)
    shapes = [(16, 1536, 7168), (16, 7168, 16384), (3, 576, 7168)]
    data = []
    for m, n, k in shapes:
        x = torch.randn(m, k, generator=gen).to(torch.bfloat16).to(gpu)
        w = (0.02 * torch.randn(n, k, generator=gen)).to(torch.bfloat16).to(gpu)
        data.append((x, w))
    need = max(lib.tmla_mla_project_workspace_bytes(m, n, k) for m, n, k in shapes)
    shared = torch.zeros(need, dtype=torch.uint8, device=gpu)
    stream = torch.cuda.current_stream(gpu).cuda_stream

    def call(i, ws):
        x, w = data[i]
        m, n, k = shapes[i]
        y = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
        with torch.cuda.device(gpu):
            _native.check(lib.tmla_mla_project(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), m, n, k,
                                               _native.DTYPE_CODE[torch.bfloat16], y.data_ptr(), y.stride(0),
                                               ws.data_ptr(), ws.numel(), stream), "tmla_mla_project")
        return y

    fresh = []
    for i in range(len(shapes)):
        ws = torch.zeros(max(lib.tmla_mla_project_workspace_bytes(*shapes[i]), 256), dtype=torch.uint8, device=gpu)
        fresh.append(call(i, ws))
        torch.cuda.synchronize(gpu)
    for rep in range(3):
        for i in (0, 1, 2, 1, 0):
            y = call(i, shared)
            torch.cuda.synchronize(gpu)
            assert torch.equal(y, fresh[i]), f"shape {shapes[i]} differs on the shared workspace (round {rep})"


def test_project_on_two_streams_and_in_a_graph(gpu):
    """layer_ops.project keeps a workspace per (device, stream): split
    contractions of different shapes running at once on two streams give the
    bits of the same calls run one at a time, a larger call on one stream
    replaces only that stream's workspace, and a graph captured on a stream
    with no workspace yet (its own counters cleared inside the graph)
    reproduces the eager bits on every replay, eager calls between them."""
    from triton_mla import layer_ops

    gen = torch.Generator().manual_seed(21)
    shapes = [(16, 1536, 7168), (8, 2048, 4096)]
    data = []
    for m, n, k in shapes:
        x = torch.randn(m, k, generator=gen).to(torch.bfloat16).to(gpu)
        w = (0.02 * torch.randn(n, k, generator=gen)).to(torch.bfloat16).to(gpu)
        data.append((x, w))
    serial = [layer_ops.project(x, w) for x, w in data]
    torch.cuda.synchronize(gpu)
    streams = [torch.cuda.Stream(gpu), torch.cuda.Stream(gpu)]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream(gpu))
    outs = [[], []]
    for rep in range(8):
        for i, s in enumerate(streams):
            with torch.cuda.stream(s):
                outs[i].append(layer_ops.project(*data[i]))
    torch.cuda.synchronize(gpu)
    for i in range(2):
        for rep, y in enumerate(outs[i]):
            assert torch.equal(y, serial[i]), f"stream {i}, call {rep} differs from the serial result"
    keys = {k for k in layer_ops._project_ws if k[0] == gpu.index or k[0] == torch.cuda.current_device()}
    assert {(torch.cuda.current_device(), s.cuda_stream) for s in streams} <= keys

    cap = torch.cuda.Stream(gpu)
    layer_ops._project_ws.pop((torch.cuda.current_device(), cap.cuda_stream), None)  # pooled streams recur
    graph = torch.cuda.CUDAGraph()
    cap.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.graph(graph, stream=cap):
        g_out = [layer_ops.project(x, w) for x, w in data]
    assert (torch.cuda.current_device(), cap.cuda_stream) not in layer_ops._project_ws
    for rep in range(3):
        for y in g_out:
            y.zero_()
        graph.replay()
        torch.cuda.synchronize(gpu)
        for i in range(2):
            assert torch.equal(g_out[i], serial[i]), f"replay {rep}, shape {shapes[i]} differs"
        eager = layer_ops.project(*data[rep % 2])  # eager work between replays
        torch.cuda.synchronize(gpu)
        assert torch.equal(eager, serial[rep % 2])


def test_project_fp16_and_strided_rows(gpu):
    """fp16 operands, and x / y rows inside wider buffers (row strides larger
    than the row): same product, other rows of the output buffer untouched."""
    from triton_mla import layer_ops, _native

    gen = torch.Generator().manual_seed(99)
    m, n, k = 9, 64, 640
    xbuf = torch.randn(m, k + 64, generator=gen).to(torch.float16)
    w = (0.05 * torch.randn(n, k, generator=gen)).to(torch.float16)
    xg, wg = xbuf.to(gpu)[:, :k], w.to(gpu)
    assert xg.stride(0) == k + 64 and layer_ops.project_fits(xg, wg)
    ybuf = torch.full((m, n + 16), 7.0, dtype=torch.float16, device=gpu)
    lib = _native.load()
    need = lib.tmla_mla_project_workspace_bytes(m, n, k)
    ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=gpu)
    with torch.cuda.device(gpu):
        _native.check(lib.tmla_mla_project(xg.data_ptr(), xg.stride(0), wg.data_ptr(), wg.stride(0), m, n, k,
                                           _native.DTYPE_CODE[torch.float16], ybuf.data_ptr(), ybuf.stride(0),
                                           ws.data_ptr(), ws.numel(), torch.cuda.current_stream(gpu).cuda_stream),
                      "tmla_mla_project")
    torch.cuda.synchronize(gpu)
    got = ybuf[:, :n].double().cpu().numpy()
    ref = f64(xbuf[:, :k]) @ f64(w).T
    abs_sum = np.abs(f64(xbuf[:, :k])) @ np.abs(f64(w)).T
    fp16_half_ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -14))) - 11)
    assert np.all(np.abs(got - ref) <= fp16_half_ulp + dot_bound(k, abs_sum)), "fp16 product off"
    assert bool((ybuf[:, n:] == 7.0).all()), "columns past n written"


def test_hip_glue_matches_torch_glue(gpu):
    """The absorbed step with the HIP glue and with the reference's torch glue
    (same mla_decode inside) on the same inputs: the appended rows agree to
    one bf16 ulp and the layer outputs to the bf16 GEMM tolerance."""
    from triton_mla import MLA, MLAConfig

    gen = torch.Generator().manual_seed(14)
    cfg = MLAConfig(hidden_size=512, num_heads=32, q_lora_rank=256)
    model = MLA(cfg)
    with torch.no_grad():
        for p in model.parameters():
            p.copy_(torch.randn(p.shape, generator=gen) * 0.05)
        model.kv_norm.weight.copy_(1.0 + 0.2 * torch.randn(cfg.kv_lora_rank, generator=gen))
    model = model.to(gpu, torch.bfloat16)
    batch, page, pages = 5, 64, 8
    seqlens = torch.tensor([0, 1, 63, 64, 300], dtype=torch.int32, device=gpu)
    bt = torch.randperm(batch * pages, generator=gen).view(batch, pages).int().to(gpu)
    cache = torch.randn(batch * pages, page, cfg.kv_cache_dim, generator=gen).to(gpu, torch.bfloat16)
    x = torch.randn(batch, cfg.hidden_size, generator=gen).to(gpu, torch.bfloat16)
    ca, cb = cache.clone(), cache.clone()
    with torch.no_grad():
        out_hip, lens_hip = model(x, ca, seqlens, bt)
        out_torch, lens_torch = model.forward_torch_glue(x, cb, seqlens, bt)
    assert torch.equal(lens_hip, lens_torch)
    diff = (ca.float() - cb.float()).abs()
    ulp = torch.from_numpy(ulp_bf16(cb.float().cpu().numpy().astype(np.float64))).to(gpu)
    assert bool((diff <= ulp).all()), "appended rows differ by more than one bf16 ulp"
    torch.testing.assert_close(out_hip.float(), out_torch.float(), atol=3e-2, rtol=3e-2)


def test_layer_step_graph_replays(gpu):
    """MLA.forward captured in a graph (the serving form of the decode step:
    no host work between its kernels) replays to the eager step's bits, three
    times, with eager steps in between."""
    from triton_mla import MLA, MLAConfig
    from triton_mla.bench import capture_layer_step

    gen = torch.Generator().manual_seed(21)
    cfg = MLAConfig(hidden_size=512, num_heads=32, q_lora_rank=256)
    model = MLA(cfg)
    with torch.no_grad():
        for p in model.parameters():
            p.copy_(torch.randn(p.shape, generator=gen) * 0.05)
    model = model.to(gpu, torch.bfloat16)
    batch, page, pages = 4, 64, 6
    seqlens = torch.tensor([5, 64, 200, 321], dtype=torch.int32, device=gpu)
    bt = torch.randperm(batch * pages, generator=gen).view(batch, pages).int().to(gpu)
    cache = torch.randn(batch * pages, page, cfg.kv_cache_dim, generator=gen).to(gpu, torch.bfloat16)
    x = torch.randn(batch, cfg.hidden_size, generator=gen).to(gpu, torch.bfloat16)
    with torch.no_grad():
        eager, _ = model(x, cache, seqlens, bt)
        eager = eager.clone()
        graph, out = capture_layer_step(model, x, cache, seqlens, bt, gpu)
        for _ in range(3):
            graph.replay()
            torch.cuda.synchronize(gpu)
            assert torch.equal(out, eager), "graph replay differs from the eager step"
            again, _ = model(x, cache, seqlens, bt)  # eager work between replays
            torch.cuda.synchronize(gpu)
            assert torch.equal(again, eager)
