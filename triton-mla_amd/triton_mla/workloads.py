"""Seeded synthetic decode workloads (inputs only; all random draws on the CPU).

Every builder draws from ``torch.Generator().manual_seed(seed)`` in a fixed
order, rounds to the element type and returns CPU tensors; callers move them
to the GPU. The shapes follow the reference benchmark's input recipe
(src/triton_mla/bench.py:20-27: randn q and cache, randperm block table,
page size 64) at the sizes the decode path is measured on.

    uniform(B, H, S)   q [B,H,576] ~ N(0,1); cache [B*cdiv(S,64),64,576] ~ N(0,1);
                       block_table = randperm(num_pages).view(B, pages_per_seq);
                       seqlens = S for every sequence.   (draw order: q, cache, perm)
    ragged(B, H, lo, hi)
                       seqlens ~ randint(lo, hi+1) first, then cache of
                       sum(cdiv(s,64)) pages, a randperm of those pages cut into
                       consecutive per-sequence chunks (table padded with 0),
                       then q.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

D_LATENT, D_ROPE = 512, 64
PAGE = 64


@dataclass
class DecodeInputs:
    name: str
    q: torch.Tensor
    kv_cache: torch.Tensor
    seqlens: torch.Tensor
    block_table: torch.Tensor
    softmax_scale: float
    head_dim_v: int = D_LATENT

    def to(self, device):
        return DecodeInputs(self.name, self.q.to(device), self.kv_cache.to(device), self.seqlens.to(device),
                            self.block_table.to(device), self.softmax_scale, self.head_dim_v)

    @property
    def batch(self):
        return self.q.shape[0]

    @property
    def heads(self):
        return self.q.shape[1]

    def algorithmic_bytes(self) -> int:
        """Bytes the decode must move at minimum (the reference bench's formula,
        src/triton_mla/bench.py:80, with the sum of sequence lengths)."""
        elt = self.q.element_size()
        tokens = int(self.seqlens.sum())
        return (tokens * self.kv_cache.shape[-1] + self.q.numel() + self.batch * self.heads * self.head_dim_v) * elt

    def flops(self) -> int:
        """2 * H * (576 + 512) per cached token at the default dims
        (src/triton_mla/bench.py:81)."""
        return int(self.seqlens.sum()) * self.heads * 2 * (self.kv_cache.shape[-1] + self.head_dim_v)


def _cdiv(a, b):
    return -(-a // b)


def uniform(batch, heads, seqlen, dtype=torch.bfloat16, seed=0, page=PAGE, name=None, d_latent=D_LATENT,
            d_rope=D_ROPE) -> DecodeInputs:
    """Uniform lengths; d_latent / d_rope as the reference's make_inputs takes
    them (bench.py:20). The softmax scale is DeepSeek's 192^-0.5 at the
    default dims, the mla_decode default (d_latent + d_rope)^-0.5 otherwise."""
    g = torch.Generator().manual_seed(seed)
    pages_per_seq = _cdiv(seqlen, page)
    num_pages = batch * pages_per_seq
    d = d_latent + d_rope
    q = torch.randn(batch, heads, d, generator=g).to(dtype)
    kv = torch.randn(num_pages, page, d, generator=g).to(dtype)
    bt = torch.randperm(num_pages, generator=g).view(batch, pages_per_seq).to(torch.int32)
    seqlens = torch.full((batch,), seqlen, dtype=torch.int32)
    scale = 192 ** -0.5 if (d_latent, d_rope) == (D_LATENT, D_ROPE) else d ** -0.5
    return DecodeInputs(name or f"uniform_b{batch}_h{heads}_s{seqlen}", q, kv, seqlens, bt, scale, d_latent)


def ragged(batch, heads, lo, hi, dtype=torch.bfloat16, seed=0, page=PAGE, name=None) -> DecodeInputs:
    g = torch.Generator().manual_seed(seed)
    seqlens = torch.randint(lo, hi + 1, (batch,), generator=g, dtype=torch.int32)
    pages = [_cdiv(int(s), page) for s in seqlens]
    num_pages = sum(pages)
    kv = torch.randn(num_pages, page, D_LATENT + D_ROPE, generator=g).to(dtype)
    perm = torch.randperm(num_pages, generator=g).to(torch.int32)
    bt = torch.zeros(batch, max(pages), dtype=torch.int32)
    start = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[start:start + n]
        start += n
    q = torch.randn(batch, heads, D_LATENT + D_ROPE, generator=g).to(dtype)
    return DecodeInputs(name or f"ragged_b{batch}_h{heads}_{lo}_{hi}", q, kv, seqlens, bt, 192 ** -0.5)


# The decode shapes the path is measured on.
def b1_h128_1k(dtype=torch.bfloat16):
    return uniform(1, 128, 1024, dtype, name="b1_h128_ctx1k")


def b8_h128_1k(dtype=torch.bfloat16):
    return uniform(8, 128, 1024, dtype, name="b8_h128_ctx1k")


def b32_h128_8k(dtype=torch.bfloat16):
    return uniform(32, 128, 8192, dtype, name="b32_h128_ctx8k")


def ragged_b64_h128(dtype=torch.bfloat16):
    return ragged(64, 128, 1024, 32768, dtype, name="ragged_b64_h128_ctx1k-32k")


def ragged_b64_h16(dtype=torch.bfloat16):
    return ragged(64, 16, 1024, 32768, dtype, name="ragged_b64_h16_ctx1k-32k")


def b8_h64_16k(dtype=torch.bfloat16):
    """64 heads (one workgroup of two 32-head blocks per worker), long context."""
    return uniform(8, 64, 16384, dtype, name="b8_h64_ctx16k")
