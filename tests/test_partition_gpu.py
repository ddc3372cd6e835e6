"""The balanced work partition in both of its forms, through the HIP kernels.

With num_splits=None the partial kernel cuts the T tiles of the batch into
ranges of c = cdiv(T, num_workers) tiles. When every sequence cut into pieces
of at most c tiles gives no more pieces than workers, each worker takes one
piece of one sequence ("snapped"); otherwise the ranges run across sequence
boundaries. The worker counts below put the same inputs on both sides of that
line (pieces == workers, pieces == workers + 1). Bar: out atol = rtol = 1e-2,
lse atol = rtol = 1e-3 against the float64 oracle, out == 0 / lse == -inf for
empty sequences, and the single-launch form equal to the two-kernel form bit
for bit (the merge inside the partial kernel uses the same slot ranges).
"""

import pytest
import torch

import oracle
from conftest import bits

pytestmark = pytest.mark.gpu

D_LATENT, D_ROPE = 512, 64
SCALE = 192 ** -0.5
OUT_TOL = dict(atol=1e-2, rtol=1e-2)
LSE_TOL = dict(atol=1e-3, rtol=1e-3)
TILE = 64


def pieces(seqlens, workers):
    tiles = [-(-n // TILE) for n in seqlens]
    c = -(-sum(tiles) // workers)
    return sum(-(-t // c) for t in tiles)


# (seqlens, workers, snapped): 257 tiles per sequence as in the DeepSeek-V3
# layer workload; a ragged batch with empty, one-token and tile-edge lengths
CASES = [
    ([16385] * 4, 64, True),
    ([16385] * 4, 63, False),
    ([0, 1, 65, 300, 4097, 2000], 20, True),
    ([0, 1, 65, 300, 4097, 2000], 19, False),
    ([700, 3, 1500], 256, True),
]


@pytest.mark.parametrize("seqlens,workers,snapped", CASES)
@pytest.mark.parametrize("heads", [16, 128])
def test_balanced_partition_forms(gpu, seqlens, workers, snapped, heads):
    from triton_mla.kernel import DecodeLaunch

    assert (pieces(seqlens, workers) <= workers) == snapped
    print(f"partition seqlens={seqlens} workers={workers} snapped={snapped} heads={heads}", flush=True)
    g = torch.Generator().manual_seed(len(seqlens) * 1000 + workers)
    lens = torch.tensor(seqlens, dtype=torch.int32)
    per_seq = max(1, -(-max(seqlens) // TILE))
    batch = len(seqlens)
    q = torch.randn(batch, heads, D_LATENT + D_ROPE, generator=g).to(torch.bfloat16)
    kv = torch.randn(batch * per_seq, TILE, D_LATENT + D_ROPE, generator=g).to(torch.bfloat16)
    bt = torch.randperm(batch * per_seq, generator=g).view(batch, per_seq).int()

    call = DecodeLaunch(q.to(gpu), kv.to(gpu), lens.to(gpu), bt.to(gpu), D_LATENT, SCALE, None, workers)
    out, lse = call.run()
    out, lse = out.clone(), lse.clone()
    out1, lse1 = call.run(single_launch=True)
    torch.cuda.synchronize()
    assert torch.equal(out, out1) and torch.equal(lse, lse1)

    ref_out, ref_lse = oracle.mla_decode_ref(bits(q), bits(kv), lens.numpy(), bt.numpy(), D_LATENT, SCALE)
    valid = lens > 0
    torch.testing.assert_close(out.float().cpu(), torch.from_numpy(ref_out), **OUT_TOL)
    torch.testing.assert_close(lse.cpu()[valid], torch.from_numpy(ref_lse)[valid], **LSE_TOL)
    assert torch.all(out.cpu()[~valid] == 0) and torch.all(torch.isneginf(lse.cpu()[~valid]))


@pytest.mark.parametrize("batch", [1, 8, 40])
def test_head_blocks_for_small_batches(gpu, batch):
    """128 heads in workgroups of 32, 64 or 128 heads: the host picks fewer
    heads per workgroup when the tile bound of the call (block-table width
    times page size) leaves compute units idle (here B = 1 -> 32, B = 8 -> 64,
    B = 40 -> 128). Every form must agree with the oracle."""
    from triton_mla import mla_decode

    g = torch.Generator().manual_seed(batch)
    lens = torch.randint(1, 1025, (batch,), generator=g, dtype=torch.int32)
    lens[0] = 1024
    q = torch.randn(batch, 128, D_LATENT + D_ROPE, generator=g).to(torch.bfloat16)
    kv = torch.randn(batch * 16, TILE, D_LATENT + D_ROPE, generator=g).to(torch.bfloat16)
    bt = torch.randperm(batch * 16, generator=g).view(batch, 16).int()
    out, lse = mla_decode(q.to(gpu), kv.to(gpu), lens.to(gpu), bt.to(gpu), softmax_scale=SCALE, return_lse=True)
    out1, lse1 = mla_decode(q.to(gpu), kv.to(gpu), lens.to(gpu), bt.to(gpu), softmax_scale=SCALE, return_lse=True,
                            single_launch=True)
    torch.cuda.synchronize()
    ref_out, ref_lse = oracle.mla_decode_ref(bits(q), bits(kv), lens.numpy(), bt.numpy(), D_LATENT, SCALE)
    for o, l in ((out, lse), (out1, lse1)):
        torch.testing.assert_close(o.float().cpu(), torch.from_numpy(ref_out), **OUT_TOL)
        torch.testing.assert_close(l.cpu(), torch.from_numpy(ref_lse), **LSE_TOL)


@pytest.mark.parametrize("heads", [16, 64, 128])
def test_ranges_across_many_sequences(gpu, heads):
    """120 short sequences over 16 workers: each straddling range holds about
    eight sequence starts (the walk charges each of them on the partition's
    line), most of its segments are whole sequences written directly, and
    its first and last ones are shared with the neighbouring workers. Both
    forms against the oracle, and the single launch equal to the two kernels."""
    from triton_mla.kernel import DecodeLaunch

    g = torch.Generator().manual_seed(heads)
    lens = torch.randint(0, 400, (120,), generator=g, dtype=torch.int32)
    lens[[5, 17, 18]] = torch.tensor([0, 1, 64], dtype=torch.int32)
    seqlens = lens.tolist()
    workers = 16
    assert pieces(seqlens, workers) > workers  # the straddling form
    batch, per_seq = len(seqlens), -(-max(seqlens) // TILE)
    q = torch.randn(batch, heads, D_LATENT + D_ROPE, generator=g).to(torch.bfloat16)
    kv = torch.randn(batch * per_seq, TILE, D_LATENT + D_ROPE, generator=g).to(torch.bfloat16)
    bt = torch.randperm(batch * per_seq, generator=g).view(batch, per_seq).int()
    call = DecodeLaunch(q.to(gpu), kv.to(gpu), lens.to(gpu), bt.to(gpu), D_LATENT, SCALE, None, workers)
    out, lse = call.run()
    out, lse = out.clone(), lse.clone()
    out1, lse1 = call.run(single_launch=True)
    torch.cuda.synchronize()
    assert torch.equal(out, out1) and torch.equal(lse, lse1)
    ref_out, ref_lse = oracle.mla_decode_ref(bits(q), bits(kv), lens.numpy(), bt.numpy(), D_LATENT, SCALE)
    valid = lens > 0
    torch.testing.assert_close(out.float().cpu(), torch.from_numpy(ref_out), **OUT_TOL)
    torch.testing.assert_close(lse.cpu()[valid], torch.from_numpy(ref_lse)[valid], **LSE_TOL)
    assert torch.all(out.cpu()[~valid] == 0) and torch.all(torch.isneginf(lse.cpu()[~valid]))
