"""Host side of weight-absorbed MLA decode on MI355X (gfx950).

``mla_decode`` keeps the signature, defaults, validation and return values of
the reference wrapper (src/triton_mla/kernel.py:204-323). The device work is
done by the HIP kernels in triton-mla_amd/csrc/mla_decode.hip, called through
the C ABI in include/triton_mla.h:

  * ``tmla_mla_decode_partial`` -- split-KV partial attention (replaces the
    reference's stage-1 launch, kernel.py:276-302);
  * ``tmla_mla_decode_combine`` -- log-sum-exp merge (replaces the stage-2
    launch, kernel.py:303-320);
  * ``tmla_mla_decode_fp8`` / ``_fp8_partial`` -- the same decode over an
    fp8 (E4M3) latent cache with per-page, per-token or per-tensor scales
    (no reference counterpart: its README.md:32-33 lists "no FP8 cache").

Tensors stay on the GPU; there is no CPU or eager fallback. With
``num_splits=None`` the token-balanced work partition is computed on the
device from ``cache_seqlens``, so no call synchronises with the host.
"""

from __future__ import annotations

import torch

from . import _native

_DTYPES = (torch.bfloat16, torch.float16)
_FP8_CACHE = (torch.float8_e4m3fn, torch.uint8)  # E4M3 codes (uint8: the raw bytes)
_SUPPORTED_DIMS = {(512, 64)}  # (head_dim_v, rope_dim) with compiled kernels


def _next_power_of_2(n: int) -> int:
    return 1 if n <= 1 else 1 << (n - 1).bit_length()


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


_CU_COUNT = {}  # device index -> compute units


def _num_sms(device) -> int:
    """Compute units of ``device`` (kernel.py:184-187; 132 off-GPU as there)."""
    device = torch.device(device)
    if device.type == "cuda":
        idx = device.index if device.index is not None else torch.cuda.current_device()
        n = _CU_COUNT.get(idx)
        if n is None:
            n = _CU_COUNT[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
        return n
    return 132


def get_num_splits(batch, num_heads, max_seqlen, num_sms, min_tokens_per_split=128):
    """Uniform split count of the reference heuristic (kernel.py:190-201).

    Largest power of two <= min(num_sms // (batch * cdiv(num_heads, 64)),
    cdiv(max_seqlen, min_tokens_per_split), 64), at least 1. Kept bit-for-bit
    because callers pass its result as ``num_splits``. ``mla_decode`` with
    ``num_splits=None`` does not use it: it balances tiles over all compute
    units on the device instead.
    """
    head_groups = _cdiv(num_heads, 64)
    target = num_sms // max(batch * head_groups, 1)
    max_by_len = _cdiv(max_seqlen, min_tokens_per_split)
    splits = max(min(target, max_by_len, 64), 1)
    return 1 << (splits.bit_length() - 1)


# Positions the balanced partition's straddling ranges charge for the start
# of each non-empty sequence (csrc/host_plan.h kSegCostTiles; the library
# reports its value through tmla_partition_segment_tiles).
SEGMENT_START_TILES = 2


def balanced_pieces(seqlens, num_workers: int, segment_tiles: int = SEGMENT_START_TILES) -> int:
    """Largest number of workers the balanced partition (``num_splits=None``)
    gives one sequence of ``seqlens`` (host integers), i.e. its split count.

    Host restatement of the device planner (csrc/decode_common.h work_range /
    segment_slot): with T = sum cdiv(n, 64) tiles and c = cdiv(T,
    num_workers), when the sequences cut into pieces of at most c tiles make
    no more pieces than workers, each sequence has cdiv(tiles, c) pieces
    ("snapped"). Otherwise the tiles lie in order on a line where each
    non-empty sequence starts with ``segment_tiles`` extra positions, cut into
    ranges of v = cdiv(line length, num_workers) positions: a sequence whose
    first tile is at position p is covered by the workers
    p // v .. (p + tiles - 1) // v. 0 when every sequence is empty.
    """
    tiles = [_cdiv(int(n), 64) if int(n) > 0 else 0 for n in seqlens]
    total = sum(tiles)
    if total == 0 or num_workers <= 0:
        return 0
    c = _cdiv(total, num_workers)
    if sum(_cdiv(t, c) for t in tiles) <= num_workers:
        return max(_cdiv(t, c) for t in tiles)
    line = [t + segment_tiles if t else 0 for t in tiles]
    v = _cdiv(sum(line), num_workers)
    best, off = 0, 0
    for t, span in zip(tiles, line):
        if t:
            p = off + segment_tiles
            best = max(best, (p + t - 1) // v - p // v + 1)
        off += span
    return best


# The form mla_decode runs when single_launch is None: False = the two
# kernels of the reference's scheme (partial, then combine), True = the single
# launch (the merge inside the partial kernel, same bits) whenever its
# workgroups fit on the device at once.
DEFAULT_SINGLE_LAUNCH = False


# (device, shape, ...) -> (workspace bytes, counter bytes to clear, single launch)
_PLANS = {}


class _OnDevice:
    """torch.cuda.device(idx) only when idx is not already current (entering
    the context costs more than the launch it guards)."""

    __slots__ = ("idx", "ctx")

    def __init__(self, idx):
        self.idx = idx
        self.ctx = None

    def __enter__(self):
        if torch.cuda.current_device() != self.idx:
            self.ctx = torch.cuda.device(self.idx)
            self.ctx.__enter__()

    def __exit__(self, *exc):
        if self.ctx is not None:
            self.ctx.__exit__(*exc)


def _aligned(t: torch.Tensor, elems: int = 8) -> bool:
    return t.data_ptr() % 16 == 0 and all(s % elems == 0 for s in t.stride()[:-1])


def _scale_layout(kv_scale, lead: int, rows: int, device):
    """float32 scale tensor of an fp8 cache and its (page, row) element strides.

    lead = pages (paged cache) or sequences (dense), rows = rows per page
    (or capacity). Accepted: one scale (a float or a one-element tensor),
    [lead] (per page / sequence) or [lead, rows] (per token).
    """
    if not torch.is_tensor(kv_scale):
        kv_scale = torch.tensor([float(kv_scale)])
    kv_scale = kv_scale.to(device=device, dtype=torch.float32)
    if kv_scale.numel() == 1:
        return kv_scale.reshape(1).contiguous(), 0, 0
    if kv_scale.dim() == 1:
        assert kv_scale.shape[0] == lead, f"kv_scale of shape [{lead}] (per page) expected"
        return kv_scale, kv_scale.stride(0), 0
    assert kv_scale.dim() == 2 and tuple(kv_scale.shape) == (lead, rows), \
        f"kv_scale of shape [{lead}, {rows}] (per token) expected"
    return kv_scale, kv_scale.stride(0), kv_scale.stride(1)


class DecodeLaunch:
    """Validated arguments of one ``mla_decode`` call, launchable stage by stage.

    ``mla_decode`` builds one and runs both stages; benchmarks use it to time
    the partial and combine kernels separately on the same stream.
    """

    def __init__(self, q, kv_cache, cache_seqlens, block_table=None, head_dim_v=512,
                 softmax_scale=None, num_splits=None, num_workers=None, kv_scale=None):
        # validation mirrors kernel.py:235-245
        if kv_cache.dim() == 4:
            assert kv_cache.shape[2] == 1, "MLA uses a single shared latent KV head"
            kv_cache = kv_cache.squeeze(2)
        # Multi-token queries [batch, q_len, num_heads, D] (an extension: the
        # reference takes one query token, kernel.py:238): query token t sees
        # the first cache_seqlens - (q_len - 1 - t) tokens. Token and head
        # dims are packed into one "virtual head" dim t * num_heads + h.
        q_len = 1
        multi_token = q.dim() == 4
        if multi_token:
            q_len = q.shape[1]
            assert q_len >= 1, "q must hold at least one query token"
            if q.stride(1) != q.shape[2] * q.stride(2):
                q = q.contiguous()
            q = q.reshape(q.shape[0], q_len * q.shape[2], q.shape[3])
        assert q.dim() == 3 and kv_cache.dim() == 3
        batch, num_heads, d_qk = q.shape
        num_heads //= q_len  # heads per query token
        d_rope = d_qk - head_dim_v
        assert kv_cache.shape[-1] == d_qk
        assert q.stride(-1) == 1 and kv_cache.stride(-1) == 1
        assert _next_power_of_2(head_dim_v) == head_dim_v
        assert _next_power_of_2(d_rope) == d_rope
        fp8 = kv_cache.dtype in _FP8_CACHE
        if fp8:
            if kv_scale is None:
                raise ValueError("an fp8 kv_cache needs kv_scale (its dequantisation scales)")
            kv_cache = kv_cache.view(torch.uint8)
        else:
            assert kv_scale is None, "kv_scale applies to an fp8 (float8_e4m3fn) kv_cache only"
            assert q.dtype == kv_cache.dtype

        if q.device.type != "cuda" or kv_cache.device != q.device:
            raise RuntimeError("triton_mla.mla_decode runs on the GPU only: q and kv_cache must be "
                               "on the same HIP device")
        if q.dtype not in _DTYPES:
            raise NotImplementedError(f"mla_decode supports bf16 and fp16 inputs, got {q.dtype}")
        if (head_dim_v, d_rope) not in _SUPPORTED_DIMS:
            raise NotImplementedError(
                f"mla_decode kernels are built for head_dim_v=512, rope_dim=64; got {head_dim_v}, {d_rope}")
        if num_splits is not None:
            num_splits = int(num_splits)
            assert num_splits >= 1, "num_splits must be >= 1"

        if softmax_scale is None:
            softmax_scale = d_qk ** -0.5  # kernel.py:247-248
        device = q.device
        cache_seqlens = cache_seqlens.to(device=device, dtype=torch.int32).contiguous()
        assert cache_seqlens.shape == (batch,), "cache_seqlens must be [batch]"

        if block_table is not None:
            block_table = block_table.to(device=device, dtype=torch.int32)
            if block_table.stride(-1) != 1:
                block_table = block_table.contiguous()
            assert block_table.dim() == 2 and block_table.shape[0] == batch
            page_size, num_blocks = kv_cache.shape[1], kv_cache.shape[0]
            bt_args = (block_table.data_ptr(), block_table.stride(0), block_table.shape[1])
        else:
            assert kv_cache.shape[0] == batch  # kernel.py:258
            page_size, num_blocks = 1, kv_cache.shape[1]
            bt_args = (None, 0, 1)

        self.device = device
        self.batch, self.num_heads, self.head_dim_v, self.d_rope = batch, num_heads, head_dim_v, d_rope
        self.q_len = q_len
        shape = (batch, q_len, num_heads) if multi_token else (batch, num_heads)
        self.out = torch.empty(*shape, head_dim_v, dtype=q.dtype, device=device)
        self.lse = torch.empty(*shape, dtype=torch.float32, device=device)
        vheads = q_len * num_heads  # rows of q / out per sequence
        self.fused = False
        self.fp8 = fp8
        if batch == 0:
            return
        if num_blocks == 0:
            raise ValueError("kv_cache holds no tokens")
        if fp8 and block_table is not None and page_size % 16 != 0:
            raise NotImplementedError("an fp8 kv_cache needs pages of a multiple of 16 tokens")
        # a fresh copy (contiguous() keeps a contiguous view at its unaligned
        # address)
        if not _aligned(q):
            q = q.clone(memory_format=torch.contiguous_format)
        if not _aligned(kv_cache, 16 if fp8 else 8):
            kv_cache = kv_cache.clone(memory_format=torch.contiguous_format)
        scale_args = ()
        if fp8:
            lead = kv_cache.shape[0]
            kv_scale, sc0, sc1 = _scale_layout(kv_scale, lead, kv_cache.shape[1], device)
            scale_args = (kv_scale.data_ptr(), sc0, sc1)
        # keep every tensor whose address is handed to the kernels alive
        self._keep = (q, kv_cache, cache_seqlens, block_table, kv_scale)
        self.lib = _native.load()
        self.splits = num_splits if num_splits is not None else 0
        # balanced partition: one worker per compute unit unless asked otherwise
        self.workers = 0 if num_splits is not None else int(num_workers or _num_sms(device))
        dev_idx = device.index if device.index is not None else torch.cuda.current_device()
        self._dev_idx = dev_idx
        # The library's answers for this shape (workspace size, the counter
        # block the single launch needs cleared, whether it runs as one
        # launch) depend on the shape and device only: asked once per shape.
        # run(single_launch=True) merges inside the partial kernel when all of
        # its workgroups fit on the device at once, one per CU.
        capacity = (block_table.shape[1] * page_size) if block_table is not None else num_blocks
        key = (dev_idx, batch, vheads, head_dim_v, self.splits, self.workers, capacity, fp8, id(self.lib))
        plan = _PLANS.get(key)
        if plan is None:
            ws = self.lib.tmla_workspace_bytes(batch, vheads, head_dim_v, self.splits, self.workers)
            zero = min(self.lib.tmla_workspace_zero_bytes(batch, vheads, head_dim_v, self.splits, self.workers), ws)
            fused = not fp8 and bool(self.lib.tmla_mla_decode_fused_is_single(
                batch, vheads, head_dim_v, self.splits, self.workers, capacity, dev_idx))
            if len(_PLANS) > 4096:
                _PLANS.clear()
            plan = _PLANS[key] = (ws, zero, fused)
        self.ws_bytes, self._zero_bytes, self.fused = plan
        # Uninitialised like the reference's buffers (kernel.py:268-271): the
        # two-kernel form writes every byte it reads. Only the single launch's
        # merge counters (a small block at the end) must start at zero; they
        # are cleared before the first single launch and every launch leaves
        # them at zero again.
        self.workspace = torch.empty(max(self.ws_bytes, 1), dtype=torch.uint8, device=device)
        self._counters_clear = False
        out_sh = self.out.stride(-2)  # one output row per (query token, head)
        self._partial_args = (
            q.data_ptr(), q.stride(0), q.stride(1),
            kv_cache.data_ptr(), kv_cache.stride(0), kv_cache.stride(1), num_blocks, page_size,
            *bt_args, cache_seqlens.data_ptr(), batch, num_heads, head_dim_v, d_rope,
            _native.DTYPE_CODE[q.dtype], float(softmax_scale), self.splits, self.workers,
            self.out.data_ptr(), self.out.stride(0), out_sh, self.lse.data_ptr(),
            self.workspace.data_ptr(), self.ws_bytes)
        if q_len > 1:  # the same arguments with q_len before num_heads
            a = self._partial_args
            self._causal_args = a[:13] + (q_len,) + a[13:]
        if fp8:  # the scale pointer and strides after page_size (and q_len)
            a = self._partial_args
            self._fp8_partial_args = a[:8] + scale_args + a[8:]
            self._fp8_args = a[:8] + scale_args + a[8:13] + (q_len,) + a[13:]
        self._combine_args = (
            cache_seqlens.data_ptr(), batch, num_heads, head_dim_v, _native.DTYPE_CODE[q.dtype],
            self.splits, self.workers, self.out.data_ptr(), self.out.stride(0), self.out.stride(1),
            self.lse.data_ptr(), self.workspace.data_ptr(), self.ws_bytes)

    def _stream(self):
        return torch.cuda.current_stream(self.device).cuda_stream

    def partial(self):
        """Stage 1 on the current stream (tmla_mla_decode_partial)."""
        if self.q_len > 1:
            raise NotImplementedError("multi-token queries run both stages at once (run())")
        if self.batch:
            with _OnDevice(self._dev_idx):
                if self.fp8:
                    _native.check(self.lib.tmla_mla_decode_fp8_partial(*self._fp8_partial_args, self._stream()),
                                  "tmla_mla_decode_fp8_partial")
                else:
                    _native.check(self.lib.tmla_mla_decode_partial(*self._partial_args, self._stream()),
                                  "tmla_mla_decode_partial")

    def combine(self):
        """Stage 2 on the current stream (tmla_mla_decode_combine)."""
        if self.q_len > 1:
            raise NotImplementedError("multi-token queries run both stages at once (run())")
        if self.batch:
            with _OnDevice(self._dev_idx):
                _native.check(self.lib.tmla_mla_decode_combine(*self._combine_args, self._stream()),
                              "tmla_mla_decode_combine")

    def _clear_counters(self):
        if not self._counters_clear:
            if self._zero_bytes > 0:
                self.workspace[self.ws_bytes - self._zero_bytes:self.ws_bytes].zero_()
            self._counters_clear = True

    def run(self, single_launch=False, spin_limit=-1):
        """Both stages (tmla_mla_decode), or the single-launch form
        (tmla_mla_decode_fused) when single_launch is set. spin_limit: polls
        a worker of the in-kernel merge waits for its siblings before it hands
        its share over (< 0: the library's default). An fp8 cache always
        runs the two kernels."""
        if self.batch and self.fp8:
            with _OnDevice(self._dev_idx):
                _native.check(self.lib.tmla_mla_decode_fp8(*self._fp8_args, self._stream()), "tmla_mla_decode_fp8")
        elif self.batch and self.q_len > 1:
            with _OnDevice(self._dev_idx):
                if single_launch:
                    self._clear_counters()
                _native.check(self.lib.tmla_mla_decode_causal(*self._causal_args, int(bool(single_launch)),
                                                              self._stream()), "tmla_mla_decode_causal")
        elif self.batch:
            with _OnDevice(self._dev_idx):
                if single_launch:
                    self._clear_counters()
                    _native.check(self.lib.tmla_mla_decode_fused(*self._partial_args, int(spin_limit),
                                                                 self._stream()), "tmla_mla_decode_fused")
                else:
                    _native.check(self.lib.tmla_mla_decode(*self._partial_args, self._stream()),
                                  "tmla_mla_decode")
        return self.out, self.lse


def mla_decode(
    q: torch.Tensor,
    kv_cache: torch.Tensor,
    cache_seqlens: torch.Tensor,
    block_table: torch.Tensor = None,
    head_dim_v: int = 512,
    softmax_scale: float = None,
    num_splits: int = None,
    return_lse: bool = False,
    single_launch: bool = None,
    kv_scale=None,
):
    """Weight-absorbed MLA decode attention over a shared latent KV cache.

    Args:
        q: [batch, num_heads, head_dim_v + rope_dim]; the first head_dim_v dims
            are the W_UK-absorbed nope query, the rest the RoPE query. An
            extension beyond the reference: q of shape [batch, q_len,
            num_heads, D] holds q_len query tokens per sequence (the last
            q_len cached tokens, e.g. speculative drafts); query token t
            attends causally to the first cache_seqlens - (q_len - 1 - t)
            tokens, and out / lse gain the q_len dim.
        kv_cache: paged [num_blocks, page_size, head_dim_v + rope_dim] when
            block_table is given, otherwise dense [batch, max_seqlen, ...].
            A singleton kv-head dim ([..., 1, D], FlashMLA layout) is accepted.
        cache_seqlens: [batch] number of valid tokens per sequence.
        block_table: optional [batch, max_blocks_per_seq] page indices.
        head_dim_v: latent rank (512 for DeepSeek-V2/V3).
        softmax_scale: defaults to q.shape[-1] ** -0.5.
        num_splits: None (default) spreads the KV tiles of all sequences
            evenly over the GPU's compute units, computed on the device (no
            host sync, graph-capturable). An int cuts every sequence into that
            many tile-aligned pieces, as the reference's split-KV scheme does.
        return_lse: also return the natural-log log-sum-exp per head.
        single_launch: merge the split partials inside the partial kernel
            (one launch instead of two, same bits) when its workgroups fit on
            the device at once; None selects DEFAULT_SINGLE_LAUNCH.
        kv_scale: an extension for an fp8 cache (kv_cache of dtype
            torch.float8_e4m3fn, or uint8 holding E4M3 codes): the float32
            dequantisation scales, row value = e4m3 * scale -- one per page
            ([num_blocks]; dense caches: [batch]), one per token
            ([num_blocks, page_size]; dense: [batch, capacity]) or one for the
            whole cache (a float or one-element tensor). Paged fp8 caches need
            a page size that is a multiple of 16; they always run two kernels.

    Returns:
        out [batch, num_heads, head_dim_v] in q.dtype (and lse [batch,
        num_heads] float32).
    """
    single = DEFAULT_SINGLE_LAUNCH if single_launch is None else bool(single_launch)
    if not single and kv_scale is None:
        res = _fast_call(q, kv_cache, cache_seqlens, block_table, head_dim_v, softmax_scale, num_splits, return_lse)
        if res is not None:
            return res if return_lse else res[0]
    if q.dtype == torch.float32 or head_dim_v != 512 or q.shape[-1] != 576:
        if kv_scale is not None:
            raise NotImplementedError("an fp8 kv_cache is supported at head_dim_v=512, rope_dim=64")
        return _generic_decode(q, kv_cache, cache_seqlens, block_table, head_dim_v, softmax_scale, num_splits,
                               return_lse)
    call = DecodeLaunch(q, kv_cache, cache_seqlens, block_table, head_dim_v, softmax_scale, num_splits,
                        kv_scale=kv_scale)
    out, lse = call.run(single)
    if return_lse:
        return out, lse
    return out


_GENERIC_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def _generic_splits(batch, num_heads, capacity, num_sms, heads_per_wg=16):
    """Default split count of the generic decode: about four workgroups per
    compute unit of the matrix-core form (heads_per_wg 64: short workgroups
    that hide each other's latency) or one of the vector-ALU form (16: whose
    per-workgroup set-up costs more than the overlap gains), pieces of at
    least 256 tokens of the cache's capacity, at most 65535 (the launch's
    grid.y)."""
    groups = max(batch * -(-num_heads // heads_per_wg), 1)
    per_cu = 4 if heads_per_wg == 64 else 1
    by_cus = -(-per_cu * num_sms // groups)
    by_len = max(-(-capacity // 256), 1)
    return max(1, min(by_cus, by_len, 65535))


def _generic_decode(q, kv_cache, cache_seqlens, block_table, head_dim_v, softmax_scale, num_splits, return_lse):
    """``mla_decode`` at head dims or an element type the matrix-core kernels
    are not built for (tmla_mla_decode_generic): any power-of-two head_dim_v
    in [16, 1024] and rope_dim in [16, 256], bf16, fp16 or fp32 -- the
    reference's kernels take powers of two and any dtype q and the cache
    share (kernel.py:243-245). Both of the reference's stages with its
    uniform splits (kernel.py:84-86) and float32 partials; ``num_splits=None``
    takes _generic_splits of the cache's capacity (sized for the form's
    workgroups: 64 heads on matrix cores for bf16 / fp16 up to 512 + 64, 16
    on the vector ALU otherwise; no call reads ``cache_seqlens`` back to the
    host). Meant for unusual dims, not at the 512 + 64 kernels' speed."""
    # validation mirrors kernel.py:235-245
    if kv_cache.dim() == 4:
        assert kv_cache.shape[2] == 1, "MLA uses a single shared latent KV head"
        kv_cache = kv_cache.squeeze(2)
    if q.dim() == 4:
        raise NotImplementedError("multi-token queries are supported at head_dim_v=512, rope_dim=64 in bf16/fp16")
    assert q.dim() == 3 and kv_cache.dim() == 3
    batch, num_heads, d_qk = q.shape
    d_rope = d_qk - head_dim_v
    assert kv_cache.shape[-1] == d_qk
    assert q.stride(-1) == 1 and kv_cache.stride(-1) == 1
    assert _next_power_of_2(head_dim_v) == head_dim_v
    assert _next_power_of_2(d_rope) == d_rope
    assert q.dtype == kv_cache.dtype
    if q.dtype not in _GENERIC_DTYPES:
        raise NotImplementedError(f"mla_decode supports bf16, fp16 and fp32 inputs, got {q.dtype}")
    if not (16 <= head_dim_v <= 1024 and 16 <= d_rope <= 256):
        raise NotImplementedError(f"mla_decode supports head_dim_v in [16, 1024] and rope_dim in [16, 256] "
                                  f"(powers of two); got {head_dim_v}, {d_rope}")
    if q.device.type != "cuda" or kv_cache.device != q.device:
        raise RuntimeError("triton_mla.mla_decode runs on the GPU only: q and kv_cache must be "
                           "on the same HIP device")
    if softmax_scale is None:
        softmax_scale = d_qk ** -0.5  # kernel.py:247-248
    device = q.device
    cache_seqlens = cache_seqlens.to(device=device, dtype=torch.int32).contiguous()
    assert cache_seqlens.shape == (batch,), "cache_seqlens must be [batch]"
    if block_table is not None:
        block_table = block_table.to(device=device, dtype=torch.int32)
        if block_table.stride(-1) != 1:
            block_table = block_table.contiguous()
        assert block_table.dim() == 2 and block_table.shape[0] == batch
        page_size, num_blocks = kv_cache.shape[1], kv_cache.shape[0]
        capacity = block_table.shape[1] * page_size
        bt_args = (block_table.data_ptr(), block_table.stride(0), block_table.shape[1])
    else:
        assert kv_cache.shape[0] == batch  # kernel.py:258
        page_size, num_blocks = 1, kv_cache.shape[1]
        capacity = num_blocks
        bt_args = (None, 0, 1)
    if num_splits is None:
        per_wg = _native.load().tmla_generic_heads_per_workgroup(head_dim_v, d_rope, _native.DTYPE_CODE[q.dtype])
        num_splits = _generic_splits(batch, num_heads, capacity, _num_sms(device), max(per_wg, 1))
    num_splits = int(num_splits)
    assert num_splits >= 1, "num_splits must be >= 1"
    out = torch.empty(batch, num_heads, head_dim_v, dtype=q.dtype, device=device)
    lse = torch.empty(batch, num_heads, dtype=torch.float32, device=device)
    if batch:
        if block_table is not None and num_blocks == 0:
            raise ValueError("kv_cache holds no pages")
        lib = _native.load()
        ws_bytes = lib.tmla_generic_workspace_bytes(batch, num_heads, head_dim_v, num_splits)
        workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
        dev_idx = device.index if device.index is not None else torch.cuda.current_device()
        with _OnDevice(dev_idx):
            _native.check(lib.tmla_mla_decode_generic(
                q.data_ptr(), q.stride(0), q.stride(1), kv_cache.data_ptr(), kv_cache.stride(0), kv_cache.stride(1),
                num_blocks, page_size, *bt_args, cache_seqlens.data_ptr(), batch, num_heads, head_dim_v, d_rope,
                _native.DTYPE_CODE[q.dtype], float(softmax_scale), num_splits, out.data_ptr(), out.stride(0),
                out.stride(1), lse.data_ptr(), workspace.data_ptr(), ws_bytes,
                torch.cuda.current_stream(device).cuda_stream), "tmla_mla_decode_generic")
    if return_lse:
        return out, lse
    return out


class _CallShape:
    """What a two-kernel ``mla_decode`` call derives from its arguments'
    shapes, strides, dtypes and device alone: the validated geometry and the
    launch's constant arguments. Built by a full DecodeLaunch the first time
    a shape is seen, so every assertion of kernel.py:235-271 has run on it;
    later calls of the same shape only read addresses and allocate."""

    __slots__ = ("dev_idx", "device", "dtype", "out_shape", "lse_shape", "ws_alloc", "ws_bytes",
                 "a_q", "a_kv", "a_bt", "a_mid", "a_out", "fn", "fast", "plan")


_SHAPES = {}
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None) or \
    (lambda idx: torch.cuda.current_stream(idx).cuda_stream)
_capturing = getattr(torch._C, "_cuda_isCurrentStreamCapturing", None) or torch.cuda.is_current_stream_capturing
_current_device = getattr(torch._C, "_cuda_getDevice", None) or torch.cuda.current_device

# (device index, stream) -> workspace of the two-kernel calls that Python
# launches on that stream. The two kernels write every workspace byte they
# read, and calls on one stream run in order, so one buffer serves them all;
# a larger need replaces it (the caching allocator hands the old one out again
# only to work queued after the calls that use it). The library is called
# with the GIL held, so two Python threads on one stream cannot interleave
# their calls' kernels. Under graph capture each call takes its own workspace
# from the graph's memory instead, so replays share nothing with eager calls.
_STREAM_WS = {}


def _workspace(shape, stream):
    """(workspace tensor, its address) for a call of `shape` on `stream`."""
    if _capturing():
        ws = torch.empty(shape.ws_alloc, dtype=torch.uint8, device=shape.device)
        return ws, ws.data_ptr()
    key = (shape.dev_idx, stream)
    entry = _STREAM_WS.get(key)  # (tensor, address, bytes)
    if entry is None or entry[2] < shape.ws_alloc:
        ws = torch.empty(shape.ws_alloc, dtype=torch.uint8, device=shape.device)
        entry = _STREAM_WS[key] = (ws, ws.data_ptr(), shape.ws_alloc)
    return entry[0], entry[1]


def _fast_call(q, kv_cache, cache_seqlens, block_table, head_dim_v, softmax_scale, num_splits, want_lse):
    """Two-kernel decode of a shape seen before: (out, lse or None), or None
    to take the full path.

    Taken only when nothing would be copied or converted: q and the cache 3-D
    (or with the singleton kv-head dim) and 16-byte aligned, cache_seqlens
    (and block_table) int32 on q's device, the device current. The lse is
    neither allocated nor written unless asked for."""
    try:
        bt_key = None if block_table is None else (block_table.dtype, block_table.get_device(), block_table.shape,
                                                   block_table.stride())
        key = (q.shape, q.stride(), q.dtype, q.get_device(), kv_cache.shape, kv_cache.stride(), kv_cache.dtype,
               kv_cache.get_device(), cache_seqlens.dtype, cache_seqlens.get_device(), cache_seqlens.shape,
               cache_seqlens.stride(), bt_key, head_dim_v, softmax_scale, num_splits)
    except (AttributeError, TypeError):
        return None
    shape = _SHAPES.get(key)
    qp, kp = q.data_ptr(), kv_cache.data_ptr()
    if (qp | kp) & 15:
        return None
    if shape is None:
        shape = _learn_shape(key, q, kv_cache, cache_seqlens, block_table, head_dim_v, softmax_scale,
                             num_splits)
    if not shape or _current_device() != shape.dev_idx:
        return None
    out = q.new_empty(shape.out_shape)
    lse = q.new_empty(shape.lse_shape, dtype=torch.float32) if want_lse else None
    stream = _raw_stream(shape.dev_idx)
    ws, wsp = _workspace(shape, stream)
    btp = None if block_table is None else block_table.data_ptr()
    lsep = None if lse is None else lse.data_ptr()
    if shape.fast is not None:
        status = shape.fast.decode(shape.plan, qp, kp, btp, cache_seqlens.data_ptr(), out.data_ptr(), lsep, wsp,
                                   stream)
    else:
        status = shape.fn(qp, *shape.a_q, kp, *shape.a_kv, btp, *shape.a_bt, cache_seqlens.data_ptr(), *shape.a_mid,
                          out.data_ptr(), *shape.a_out, lsep, wsp, shape.ws_bytes, stream)
    if status:
        _native.check(status, "tmla_mla_decode")
    return out, lse


def _learn_shape(key, q, kv_cache, cache_seqlens, block_table, head_dim_v, softmax_scale, num_splits):
    """Validate one call of a new shape through DecodeLaunch and keep its
    constant arguments; False (kept too) when the fast path does not apply
    to the shape. q and kv_cache are 16-byte aligned here."""
    shape = False
    if q.dim() == 3 and kv_cache.dtype in _DTYPES and head_dim_v == 512 and q.shape[-1] == 576 \
            and cache_seqlens.dtype == torch.int32 \
            and cache_seqlens.device == q.device and cache_seqlens.is_contiguous() \
            and (block_table is None or (block_table.dtype == torch.int32 and block_table.device == q.device
                                         and block_table.dim() == 2 and block_table.stride(-1) == 1)):
        call = DecodeLaunch(q, kv_cache, cache_seqlens, block_table, head_dim_v, softmax_scale, num_splits)
        # no copies made (strides the kernels take as given), one query token
        if call.batch and call.q_len == 1 and not call.fp8 and call._keep[0] is q \
                and call._keep[1].data_ptr() == kv_cache.data_ptr():
            shape = _shape_of(call, q.dtype)
    if len(_SHAPES) > 1024:
        _SHAPES.clear()
    _SHAPES[key] = shape
    return shape


def _shape_of(call, dtype):
    a = call._partial_args
    shape = _CallShape()
    shape.dev_idx, shape.device, shape.dtype = call._dev_idx, call.device, dtype
    shape.out_shape, shape.lse_shape = tuple(call.out.shape), tuple(call.lse.shape)
    shape.ws_alloc, shape.ws_bytes = call.workspace.numel(), call.ws_bytes
    # _partial_args: q ptr, q strides (2), cache ptr, cache strides, blocks,
    # page size (4), table ptr, table stride, width (2), seqlens ptr, batch ..
    # workers (8), out ptr, out strides (2), lse ptr, workspace ptr, its size
    shape.a_q, shape.a_kv, shape.a_bt = a[1:3], a[4:8], a[9:11]
    shape.a_mid, shape.a_out = a[12:20], a[21:23]
    shape.fn = _native.load_gil_held().tmla_mla_decode
    # the same constant arguments packed once for the CPython entry
    shape.fast = _native.fast_module()
    shape.plan = None
    if shape.fast is not None:
        shape.plan = shape.fast.plan(*shape.a_q, *shape.a_kv, *shape.a_bt, *shape.a_mid, *shape.a_out,
                                     shape.ws_bytes)
    return shape
