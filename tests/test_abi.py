"""The C-ABI library: it loads, exports every entry point include/triton_mla.h
declares, and rejects bad arguments before touching a device (no GPU needed)."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "triton_mla.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tmla_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from triton_mla import _native

    if not os.path.exists(_native.LIB_PATH):
        pytest.fail(f"HIP library not built: {_native.LIB_PATH} (run __graft_entry__.build())")
    return _native.load()


def test_header_declares_the_entry_points():
    names = declared_functions()
    assert {"tmla_mla_decode", "tmla_mla_decode_partial", "tmla_mla_decode_combine",
            "tmla_workspace_bytes", "tmla_last_error", "tmla_version", "tmla_device_cu_count"} <= set(names)


def test_library_exports_every_declared_symbol(lib):
    from triton_mla import _native

    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in triton_mla.h but not exported"
        assert name in _native.SIGNATURES, f"{name} has no ctypes signature"


def _al(x):
    return (x + 255) // 256 * 256


COUNTER_BLOCK = 256 * 1024  # the single launch's counter block, the same for every call


def _counter_ints(batch, slots, heads):
    # the single launch's int32 counters: 2 per (sequence, workgroup along the
    # heads) and 1 per (slot, workgroup); at most, workgroups of 32 heads
    gy = -(-heads // 32)
    return (2 * batch + slots) * gy


def test_workspace_arithmetic(lib):
    # uniform: batch * splits slots; balanced: workers + batch slots (16-bit
    # partial + float32 lse, each region 256-byte aligned), then the fixed
    # counter block that the kernels place at the buffer's end
    def expect(batch, slots, heads, dv=512):
        assert _counter_ints(batch, slots, heads) * 4 <= COUNTER_BLOCK
        return _al(slots * heads * dv * 2) + _al(slots * heads * 4) + COUNTER_BLOCK

    assert lib.tmla_workspace_bytes(32, 128, 512, 8, 0) == expect(32, 256, 128)
    assert lib.tmla_workspace_bytes(32, 128, 512, 0, 256) == expect(32, 288, 128)
    assert lib.tmla_workspace_bytes(3, 20, 512, 1, 0) == expect(3, 3, 20)
    assert lib.tmla_workspace_bytes(4, 256, 512, 2, 0) == expect(4, 8, 256)
    assert lib.tmla_version() >= 200


def test_workspace_zero_suffix(lib):
    # the suffix to clear before the first single launch: the counter block
    # plus the slack of rounding the buffer size down to 256 bytes, the same
    # for every call (so calls of any shape can share a buffer)
    for batch, heads, splits, workers in [(32, 128, 0, 256), (8, 128, 0, 256), (3, 20, 1, 0), (4, 256, 2, 0)]:
        z = lib.tmla_workspace_zero_bytes(batch, heads, 512, splits, workers)
        assert z == COUNTER_BLOCK + 255
        assert z < lib.tmla_workspace_bytes(batch, heads, 512, splits, workers)
    # a smaller call's counters fit inside a larger call's suffix
    assert lib.tmla_workspace_zero_bytes(8, 128, 512, 0, 256) <= lib.tmla_workspace_zero_bytes(32, 128, 512, 0, 256)
    assert lib.tmla_mla_decode_fused_is_single(0, 128, 512, 0, 256, 8192, 0) == 0  # empty batch: nothing fuses
    # invalid arguments never fuse
    assert lib.tmla_mla_decode_fused_is_single(4, 16, 512, -1, 256, 8192, 0) == 0
    assert lib.tmla_mla_decode_fused_is_single(4, 1, 256, 2, 0, 8192, 0) == 0


def _partial(lib, **kw):
    args = dict(q=None, qsb=576 * 128, qsh=576, kv=None, kv0=64 * 576, kv1=576, nblocks=4, page=64,
                bt=None, btsb=1, btcols=1, seqlens=None, batch=2, heads=128, dv=512, dr=64, dtype=0,
                scale=0.1, splits=1, workers=0, out=None, osb=128 * 512, osh=512, lse=None, ws=None,
                wsb=0, stream=None)
    args.update(kw)
    return lib.tmla_mla_decode_partial(*args.values())


def test_invalid_arguments_rejected_on_host(lib):
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: validation fails first
    ws = lib.tmla_workspace_bytes(2, 128, 512, 1, 0)
    assert _partial(lib, dtype=7, ws=fake, wsb=ws) == 1
    assert b"dtype" in lib.tmla_last_error()
    assert _partial(lib, dv=256, ws=fake, wsb=ws) == 2  # unsupported head_dim_v
    assert _partial(lib, ws=None, wsb=0) == 3  # workspace missing
    assert _partial(lib, ws=fake, wsb=ws - 1) == 3  # workspace too small
    assert _partial(lib, splits=0, workers=0, ws=fake, wsb=ws) == 1  # balanced needs workers
    assert _partial(lib, heads=0, ws=fake, wsb=ws) == 1
    # null tensors are caught before any launch
    assert _partial(lib, ws=fake, wsb=ws) == 1
    assert b"null" in lib.tmla_last_error()


def _generic(lib, **kw):
    args = dict(q=None, qsb=160 * 16, qsh=160, kv=None, kv0=64 * 160, kv1=160, nblocks=64, page=1,
                bt=None, btsb=1, btcols=1, seqlens=None, batch=2, heads=16, dv=128, dr=32, dtype=2,
                scale=0.1, splits=2, out=None, osb=16 * 128, osh=128, lse=None, ws=None, wsb=0, stream=None)
    args.update(kw)
    return lib.tmla_mla_decode_generic(*args.values())


def test_generic_workspace_and_rejections(lib):
    # float32 partial rows [batch, heads, splits, dv], then their lse values,
    # each 256-byte aligned, plus 256 bytes (so an empty batch needs a buffer too)
    assert lib.tmla_generic_workspace_bytes(2, 16, 128, 2) == _al(64 * 128 * 4) + _al(64 * 4) + 256
    assert lib.tmla_generic_workspace_bytes(3, 5, 16, 7) == _al(105 * 16 * 4) + _al(105 * 4) + 256
    assert lib.tmla_generic_workspace_bytes(0, 5, 16, 7) == 256
    assert lib.tmla_generic_workspace_bytes(2, 16, 128, 0) == 0
    assert lib.tmla_generic_workspace_bytes(2, 0, 128, 1) == 0
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: validation fails first
    ws = lib.tmla_generic_workspace_bytes(2, 16, 128, 2)
    assert _generic(lib, dtype=3, ws=fake, wsb=ws) == 1
    assert b"dtype" in lib.tmla_last_error()
    for dv, dr in [(96, 32), (2048, 64), (128, 8), (128, 512), (8, 16), (128, 0)]:
        assert _generic(lib, dv=dv, dr=dr, ws=fake, wsb=ws) == 2, (dv, dr)
    assert _generic(lib, splits=0, ws=fake, wsb=ws) == 1
    assert _generic(lib, splits=65536, ws=fake, wsb=1 << 40) == 1
    assert _generic(lib, batch=65536, ws=fake, wsb=1 << 40) == 2
    assert _generic(lib, heads=0, ws=fake, wsb=ws) == 1
    assert _generic(lib, ws=fake, wsb=ws - 1) == 3
    assert _generic(lib, ws=None, wsb=0) == 3
    assert _generic(lib, page=64, ws=fake, wsb=ws) == 1  # a dense cache has page_size 1
    assert _generic(lib, bt=fake, page=0, ws=fake, wsb=ws) == 1  # a paged one at least 1
    assert _generic(lib, bt=fake, page=16, nblocks=0, ws=fake, wsb=ws) == 1
    assert _generic(lib, batch=0, ws=fake, wsb=256) == 0  # nothing to do
    # null tensors are caught before any launch
    assert _generic(lib, ws=fake, wsb=ws) == 1
    assert b"NULL" in lib.tmla_last_error()
    # heads per workgroup: the matrix-core form (bf16 / fp16, dv <= 512, D <= 576) or the vector-ALU one
    assert lib.tmla_generic_heads_per_workgroup(512, 64, 0) == 64
    assert lib.tmla_generic_heads_per_workgroup(256, 32, 1) == 64
    assert lib.tmla_generic_heads_per_workgroup(512, 128, 0) == 16
    assert lib.tmla_generic_heads_per_workgroup(1024, 64, 1) == 16
    assert lib.tmla_generic_heads_per_workgroup(128, 32, 2) == 16
    assert lib.tmla_generic_heads_per_workgroup(96, 32, 0) == 0
    assert lib.tmla_generic_heads_per_workgroup(128, 32, 3) == 0
    # the matrix-core entry points keep refusing float32
    assert _partial(lib, dtype=2, ws=fake, wsb=lib.tmla_workspace_bytes(2, 128, 512, 1, 0)) == 1


def test_fast_module_carries_the_plan(lib):
    """The CPython entry of the kept-shape call (csrc/fastcall.c) packs the
    constant arguments once and passes them with the call's pointers to the
    same library instance (its error text is the library's)."""
    from triton_mla import _native

    fast = _native.fast_module()
    assert fast is not None, "build the library with triton-mla_amd/build.py (it builds the module too)"
    fake = 1 << 20  # never dereferenced: validation fails first
    ws = lib.tmla_workspace_bytes(2, 128, 512, 1, 0)

    def plan(dtype=0, dv=512, ws_bytes=ws, splits=1):
        return fast.plan(576 * 128, 576, 64 * 576, 576, 4, 64, 1, 1, 2, 128, dv, 64, dtype, 0.1, splits, 0,
                         128 * 512, 512, ws_bytes)

    assert fast.decode(plan(dtype=7), fake, fake, None, fake, fake, None, fake, 0) == 1
    assert b"dtype" in lib.tmla_last_error()
    assert fast.decode(plan(dv=256), fake, fake, None, fake, fake, None, fake, 0) == 2
    assert fast.decode(plan(ws_bytes=ws - 1), fake, fake, None, fake, fake, None, fake, 0) == 3
    assert fast.decode(plan(splits=0), fake, fake, None, fake, fake, None, fake, 0) == 1  # balanced needs workers
    assert fast.decode(plan(), None, fake, None, fake, fake, None, fake, 0) == 1  # a null q is refused
    with pytest.raises(TypeError):
        fast.decode(plan(), fake)
    with pytest.raises(ValueError):
        fast.decode(object(), fake, fake, None, fake, fake, None, fake, 0)


def test_layer_glue_arguments_rejected_on_host(lib):
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: validation fails first
    # tmla_mla_absorb_q(q_proj, q_sb, wkv_b, w_s0, positions, batch, heads, nope, rope, rank, vd, theta,
    #                   dtype, q_out, qo_sb, qo_sh, stream)
    q = [fake, 128 * 192, fake, 512, fake, 2, 128, 128, 64, 512, 128, 1e4, 0, fake, 128 * 576, 576, None]
    args = list(q); args[12] = 5
    assert lib.tmla_mla_absorb_q(*args) == 1 and b"dtype" in lib.tmla_last_error()
    args = list(q); args[7] = 96
    assert lib.tmla_mla_absorb_q(*args) == 2  # qk_nope_dim other than 128
    args = list(q); args[9] = 320
    assert lib.tmla_mla_absorb_q(*args) == 2  # rank not a multiple of 128
    args = list(q); args[0] = None
    assert lib.tmla_mla_absorb_q(*args) == 1 and b"null" in lib.tmla_last_error()
    args = list(q); args[1] = 128 * 192 + 3
    assert lib.tmla_mla_absorb_q(*args) == 1  # stride not a multiple of 8 elements
    args = list(q); args[5] = 0
    assert lib.tmla_mla_absorb_q(*args) == 0  # empty batch: nothing to do
    # tmla_mla_absorb_out(o, o_sb, o_sh, wkv_b, w_s0, batch, heads, nope, rank, vd, dtype, out, out_sb, stream)
    o = [fake, 128 * 512, 512, fake, 512, 2, 128, 128, 512, 128, 0, fake, 128 * 128, None]
    args = list(o); args[9] = 48
    assert lib.tmla_mla_absorb_out(*args) == 2  # v_head_dim not a multiple of 32
    args = list(o); args[11] = None
    assert lib.tmla_mla_absorb_out(*args) == 1
    # tmla_mla_kv_append(kv_proj, sb, norm_w, eps, theta, positions, batch, rank, rope, dtype, cache, s0, s1,
    #                    num_blocks, page_size, bt, bt_sb, bt_cols, stream)
    k = [fake, 576, None, 1e-6, 1e4, fake, 2, 512, 64, 0, fake, 64 * 576, 576, 4, 64, fake, 4, 4, None]
    args = list(k); args[8] = 32
    assert lib.tmla_mla_kv_append(*args) == 2  # rope_dim other than 64
    args = list(k); args[15] = None  # dense cache needs page_size 1
    assert lib.tmla_mla_kv_append(*args) == 1 and b"page_size" in lib.tmla_last_error()
    args = list(k); args[13] = 0
    assert lib.tmla_mla_kv_append(*args) == 1
    # tmla_mla_norm_append(q_lat, q_s, q_w, q_eps, q_dim, q_out, qo_s, kv_proj, sb, kv_w, kv_eps, theta,
    #                      positions, next_positions, batch, rank, rope, dtype, cache, s0, s1, num_blocks,
    #                      page_size, bt, bt_sb, bt_cols, stream)
    na = [fake, 1536, fake, 1e-6, 1536, fake, 1536, fake, 576, None, 1e-6, 1e4, fake, fake, 2, 512, 64, 0,
          fake, 64 * 576, 576, 4, 64, fake, 4, 4, None]
    args = list(na); args[4] = 1540; args[1] = 1544; args[6] = 1544
    assert lib.tmla_mla_norm_append(*args) == 2  # q_dim not a multiple of 8
    args = list(na); args[16] = 32
    assert lib.tmla_mla_norm_append(*args) == 2  # rope_dim other than 64
    args = list(na); args[13] = None
    assert lib.tmla_mla_norm_append(*args) == 1 and b"null" in lib.tmla_last_error()
    args = list(na); args[5] = None
    assert lib.tmla_mla_norm_append(*args) == 1 and b"null" in lib.tmla_last_error()
    args = list(na); args[23] = None  # dense cache needs page_size 1
    assert lib.tmla_mla_norm_append(*args) == 1 and b"page_size" in lib.tmla_last_error()
    args = list(na); args[17] = 3
    assert lib.tmla_mla_norm_append(*args) == 1 and b"dtype" in lib.tmla_last_error()
    args = list(na); args[14] = 0
    assert lib.tmla_mla_norm_append(*args) == 0  # empty batch: nothing to do
    # tmla_mla_rms_norm(x, x_s, w, eps, rows, dim, dtype, y, y_s, stream)
    rn = [fake, 1536, fake, 1e-6, 16, 1536, 0, fake, 1536, None]
    args = list(rn); args[5] = 1540; args[1] = 1544; args[8] = 1544
    assert lib.tmla_mla_rms_norm(*args) == 2  # dim not a multiple of 8
    args = list(rn); args[7] = None
    assert lib.tmla_mla_rms_norm(*args) == 1 and b"null" in lib.tmla_last_error()
    args = list(rn); args[2] = ctypes.c_void_p((1 << 20) + 4)
    assert lib.tmla_mla_rms_norm(*args) == 1 and b"aligned" in lib.tmla_last_error()
    args = list(rn); args[1] = 1532
    assert lib.tmla_mla_rms_norm(*args) == 1  # row stride below dim
    args = list(rn); args[4] = 0
    assert lib.tmla_mla_rms_norm(*args) == 0  # no rows: nothing to do
    # tmla_mla_project(x, x_s, w, w_s, m, n, k, dtype, y, y_s, workspace, workspace_bytes, stream)
    need = lib.tmla_mla_project_workspace_bytes(16, 1536, 7168)
    assert need > 0 and lib.tmla_mla_project_workspace_bytes(65, 1536, 7168) == 0
    pr = [fake, 7168, fake, 7168, 16, 1536, 7168, 0, fake, 1536, fake, need, None]
    args = list(pr); args[4] = 65
    assert lib.tmla_mla_project(*args) == 2  # more than 64 rows
    args = list(pr); args[5] = 1544
    assert lib.tmla_mla_project(*args) == 2  # n not a multiple of 16
    args = list(pr); args[6] = 7144; args[1] = 7144; args[3] = 7144
    assert lib.tmla_mla_project(*args) == 2  # k not a multiple of 64 (nor of 32)
    args = list(pr); args[7] = 7
    assert lib.tmla_mla_project(*args) == 1 and b"dtype" in lib.tmla_last_error()
    args = list(pr); args[2] = None
    assert lib.tmla_mla_project(*args) == 1 and b"null" in lib.tmla_last_error()
    args = list(pr); args[0] = ctypes.c_void_p((1 << 20) + 8)
    assert lib.tmla_mla_project(*args) == 1 and b"aligned" in lib.tmla_last_error()
    args = list(pr); args[1] = 7164
    assert lib.tmla_mla_project(*args) == 1  # row stride not a multiple of 8 (and < k)
    args = list(pr); args[11] = need - 256
    assert lib.tmla_mla_project(*args) == 3  # workspace too small
    args = list(pr); args[10] = None
    assert lib.tmla_mla_project(*args) == 3  # workspace missing
    args = list(pr); args[4] = 0
    assert lib.tmla_mla_project(*args) == 0  # no rows: nothing to do


def test_noalloc_rejects_calls_beyond_the_scratch(lib):
    # no device is touched: the workspace the call would need is checked first
    fake = ctypes.c_void_p(1 << 20)
    need = lib.tmla_workspace_bytes(64, 512, 512, 0, 256)
    assert need > 64 << 20
    rc = lib.tmla_mla_decode_noalloc(fake, 512 * 576, 576, fake, 64 * 576, 576, 8, 64, fake, 1, 1, fake, 64, 512,
                                     512, 64, 0, 0.1, 0, 256, fake, 512 * 512, 512, fake, None)
    assert rc == 3 and b"built-in scratch" in lib.tmla_last_error()


def test_partition_constant_matches_the_host_restatement(lib):
    # the balanced partition's start charge, as the library reports it, is
    # the one triton_mla.kernel.balanced_pieces assumes
    from triton_mla.kernel import SEGMENT_START_TILES

    assert lib.tmla_partition_segment_tiles() == SEGMENT_START_TILES
