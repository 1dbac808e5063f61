"""kvskip_decode_scratch (split-K partials in the library's static device array, no allocation)
against kvskip_decode with caller-provided partials, through the C ABI: the same kernels on the
same inputs, so outputs, log-sum-exp and statistics must be bit-identical. Two calls in a row on
one GPU, the second smaller, so the second reuses the array the first left behind."""

import ctypes

import pytest
import torch

from kvskip_amd import _native
from kvskip_amd import ext as E
from kvskip_amd import workloads as W

pytestmark = pytest.mark.gpu


def _scratch_decode(q, k, v, scale, num_splits, stats=False, block_idx=None, block_cnt=None, seq_lens=None):
    """Outputs allocated here (the caller's part); the partials are the library's."""
    B, Hq, D = q.shape
    T = k.shape[2]
    nb = (T + 63) // 64
    dev = q.device
    out = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(B, Hq, dtype=torch.float32, device=dev)
    bmax = torch.empty(B, Hq, nb, dtype=torch.float32, device=dev) if stats else None
    bsum = torch.empty(B, Hq, nb, dtype=torch.float32, device=dev) if stats else None
    a = E._decode_args(q, k, v, scale, block_idx, block_cnt, num_splits, out, lse, bmax, bsum, None, None, None, None,
                       seq_lens)
    assert a.part_acc is None and a.part_ml is None
    with torch.cuda.device(dev):
        _native.check(_native.lib().kvskip_decode_scratch(ctypes.byref(a), int(stats), 1, E._stream(dev)))
    return out, lse, bmax, bsum


def test_scratch_decode_first_call_under_graph_capture(gpu):
    """The first kvskip_decode_scratch call on the device (where the library looks up its array's
    address) made under HIP graph capture, as the callers it is for make it; the graph then replayed
    three times with eager work between the replays: out and lse bit-identical to kvskip_decode on
    every replay. This test comes first in the file, before any other call of the entry point."""
    L = W.structured(1, 32, 8, 128, 3000, seed=11)
    q, k, v = L.q.cuda(), L.k.cuda(), L.v.cuda()
    S = 8
    ref = E.decode(q, k, v, L.scale, None, None, False, True, S)
    B, Hq, D = q.shape
    out = torch.empty(B, Hq, D, dtype=torch.bfloat16, device="cuda")
    lse = torch.empty(B, Hq, dtype=torch.float32, device="cuda")
    a = E._decode_args(q, k, v, L.scale, None, None, S, out, lse, None, None, None, None, None, None)
    torch.cuda.synchronize()
    print("no-alloc decode: first call under graph capture", flush=True)
    g = torch.cuda.CUDAGraph()
    rc = []
    with torch.cuda.graph(g):
        rc.append(_native.lib().kvskip_decode_scratch(ctypes.byref(a), 0, 1, E._stream(q.device)))
    assert rc == [0], _native.lib().kvskip_last_error()
    for rep in range(3):
        out.fill_(0)
        lse.fill_(0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref[0]) and torch.equal(lse, ref[1]), rep


def _case(kind):
    if kind == "cfg2_masked_stats":
        L, keep = W.cfg2()
        bi, bc = W.block_list(keep)
        return L, dict(stats=True, block_idx=bi, block_cnt=bc), 32
    if kind == "cfg2_dense":
        L, _ = W.cfg2()
        return L, {}, 32
    if kind == "small_dense":
        return W.structured(1, 32, 8, 128, 3000, seed=9), {}, 8
    if kind == "ragged":
        L = W.structured(3, 28, 4, 128, 5000, seed=10)
        return L, dict(seq_lens=torch.tensor([5000, 1200, 37], dtype=torch.int32)), 16
    raise ValueError(kind)


def _check(kind):
    L, kw, S = _case(kind)
    q, k, v = L.q.cuda(), L.k.cuda(), L.v.cuda()
    kw = {key: (val.cuda() if isinstance(val, torch.Tensor) else val) for key, val in kw.items()}
    stats = kw.pop("stats", False)
    print(f"no-alloc decode: case {kind}, q {tuple(q.shape)}, k {tuple(k.shape)}, num_splits {S}", flush=True)
    ref = E.decode(q, k, v, L.scale, kw.get("block_idx"), kw.get("block_cnt"), stats, True, S,
                   seq_lens=kw.get("seq_lens"))
    got = _scratch_decode(q, k, v, L.scale, S, stats=stats, **kw)
    torch.cuda.synchronize()
    assert torch.equal(got[0], ref[0]), "out"
    assert torch.equal(got[1], ref[1]), "lse"
    if stats:
        assert torch.equal(got[2], ref[2]) and torch.equal(got[3], ref[3]), "statistics"


@pytest.mark.parametrize("first,second", [("cfg2_masked_stats", "small_dense"), ("cfg2_dense", "ragged")])
def test_scratch_decode_matches_decode(gpu, first, second):
    """Two calls in a row, the second on a smaller input (fewer partials than the first left)."""
    _check(first)
    _check(second)


def test_scratch_decode_rejects_oversize(gpu):
    """More partials than the array holds: a clear error, nothing launched."""
    q = torch.zeros(64, 32, 128, dtype=torch.bfloat16, device="cuda")
    k = torch.zeros(64, 8, 4096, 128, dtype=torch.bfloat16, device="cuda")
    out = torch.empty(64, 32, 128, dtype=torch.bfloat16, device="cuda")
    lse = torch.empty(64, 32, dtype=torch.float32, device="cuda")
    a = E._decode_args(q, k, k, 0.1, None, None, 64, out, lse, None, None, None, None, None, None)
    rc = _native.lib().kvskip_decode_scratch(ctypes.byref(a), 0, 1, E._stream(q.device))
    assert rc == -1 and b"scratch holds" in _native.lib().kvskip_last_error()
