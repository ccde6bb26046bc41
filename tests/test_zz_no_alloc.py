"""shard_decode_attn_noalloc (no workspace argument, no allocation: the partial
rows live in the library's per-GPU scratch array) against shard_decode_attn on
the same arguments: bit-identical outputs, on two calls in a row, the second on
a smaller input, for each split kernel.  The scratch keeps the previous call's
contents, so a split that failed to write its partial row would show here."""
import pytest
import torch

from tests.helpers import random_layer, to_device

pytestmark = pytest.mark.gpu

# (B, nkv, rank, n_comp, n_stream): the second call of each pair is smaller
CALLS = [(2, 8, 192, 6000, 37), (1, 8, 128, 1500, 0)]


def _call(cuda, B, nkv, rank, n_comp, n_stream, kernel, n_splits=0):
    from shard_amd import ops
    gc, inv = random_layer(B=B, nkv=nkv, rank=rank, n_comp=n_comp, n_stream=n_stream,
                           seed=n_comp + rank)
    d = to_device(gc, cuda, inv, nkv=nkv)
    q = torch.randn(B, 4 * nkv, 128, generator=torch.Generator().manual_seed(3)).half().to(cuda)
    pos_q = 4 + n_comp + 64 + n_stream - 1
    call = ops.make_decode_args(q, d, pos_q, None, n_splits=n_splits, stream_n=n_stream)
    call.args.kernel = kernel
    return call, d


def _bits(t):
    return t.cpu().view(torch.int16)


@pytest.mark.parametrize("kernel", [0, 1, 2])
def test_noalloc_equals_workspace_entry_point(cuda, kernel):
    from shard_amd import ops
    for B, nkv, rank, n_comp, n_stream in CALLS:
        print(f"[noalloc] kernel={kernel} B={B} rank={rank} n_comp={n_comp} stream={n_stream}",
              flush=True)
        call, keep = _call(cuda, B, nkv, rank, n_comp, n_stream, kernel)
        assert call.workspace_bytes() <= ops.DECODE_NOALLOC_SCRATCH_BYTES
        want = _bits(ops.decode_attn(call).clone())
        call.out.fill_(0)
        got = _bits(ops.decode_attn_noalloc(call))
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"{int((got != want).sum())} of {got.numel()} values differ"


def test_noalloc_rejects_a_call_beyond_its_scratch(cuda):
    """A call whose workspace exceeds the scratch is refused before any launch
    (clear error), and the next call that fits runs normally."""
    from shard_amd import _lib, ops
    # one split per cost unit (3 x 125 compressed tiles + 3 extra tiles): 2 x 32
    # heads x 378 partial rows of 520 bytes = 12.6 MB
    call, keep = _call(cuda, 2, 8, 192, 4000, 0, 2, n_splits=100000)
    need = call.workspace_bytes()
    assert need > ops.DECODE_NOALLOC_SCRATCH_BYTES
    with pytest.raises(_lib.ShardHipError) as ei:
        ops.decode_attn_noalloc(call)
    assert ei.value.code == -4 and str(need) in str(ei.value)
    call2, keep2 = _call(cuda, *CALLS[1], 0)
    want = _bits(ops.decode_attn(call2).clone())
    call2.out.fill_(0)
    assert torch.equal(_bits(ops.decode_attn_noalloc(call2)), want)
