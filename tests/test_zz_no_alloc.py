"""tmla_mla_decode_noalloc (the decode with the library's built-in device
scratch instead of a caller-owned workspace) against tmla_mla_decode with a
workspace of its own, through the C ABI: the same kernels on the same
inputs, so out and lse must agree bit for bit. Two calls in a row, the
second on a smaller input (the scratch keeps the first call's partials,
which the second must neither need cleared nor read), then the first again.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _noalloc(lib, call, stream):
    from triton_mla import _native

    call.out.fill_(1.0)  # every element must be written by the call
    call.lse.fill_(1.0)
    args = call._partial_args[:-2]  # everything but (workspace, workspace_bytes)
    _native.check(lib.tmla_mla_decode_noalloc(*args, stream), "tmla_mla_decode_noalloc")
    torch.cuda.synchronize()
    return call.out.clone(), call.lse.clone()


def _with_workspace(call):
    call.out.fill_(1.0)
    call.lse.fill_(1.0)
    call.run()  # tmla_mla_decode on the call's own workspace
    torch.cuda.synchronize()
    return call.out.clone(), call.lse.clone()


def _same(a, b, what):
    assert torch.equal(a[0].view(torch.int16), b[0].view(torch.int16)), f"{what}: out differs"
    assert torch.equal(a[1].view(torch.int32), b[1].view(torch.int32)), f"{what}: lse differs"


def test_noalloc_equals_workspace_form(gpu):
    from triton_mla import _native, workloads
    from triton_mla.kernel import DecodeLaunch

    lib = _native.load()
    stream = torch.cuda.current_stream(gpu).cuda_stream
    calls = []
    for inp in (workloads.b32_h128_8k(), workloads.ragged(5, 128, 0, 3000, seed=4)):
        d = inp.to(gpu)
        calls.append(DecodeLaunch(d.q, d.kv_cache, d.seqlens, d.block_table, 512, d.softmax_scale))
    big, small = calls
    assert small.ws_bytes < big.ws_bytes
    ref_big, ref_small = _with_workspace(big), _with_workspace(small)
    _same(_noalloc(lib, big, stream), ref_big, "first call (B=32, H=128, 8K)")
    _same(_noalloc(lib, small, stream), ref_small, "second, smaller call (ragged B=5)")
    _same(_noalloc(lib, big, stream), ref_big, "the first call again")


def test_noalloc_rejects_calls_beyond_the_scratch(gpu):
    from triton_mla import _native

    lib = _native.load()
    fake = 1 << 20  # never dereferenced: the size check comes first
    # 64 sequences x 512 heads over 256 workers: (256 + 64) * 512 partial rows of 1 KiB
    rc = lib.tmla_mla_decode_noalloc(fake, 512 * 576, 576, fake, 64 * 576, 576, 8, 64, fake, 1, 1, fake, 64, 512,
                                     512, 64, 0, 0.1, 0, 256, fake, 512 * 512, 512, fake, None)
    assert rc == 3 and b"built-in scratch" in lib.tmla_last_error()
