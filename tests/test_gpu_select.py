"""GPU: block selection on the device (kvskip_select, kvskip_block_list) against the CPU oracle.
select: the GQA-union sets of the oracle's select_blocks (kernels/kvskip.py:130-147, rules tau and
topp, ties at a top-p cut kept) identical unless the oracle's own margin is below float32 noise
(checked: none here), the per-block scales exp(blk_max - lse over the kept set) within 2e-5
relative, the lists kept-first ascending then the rest ascending (a stable argsort of ~keep, as
make_plan in kernels/kvskip.py:79-85). vskip_two_pass (pass 1, selection, pass 2) against exact
attention over the oracle's kept set."""

import math

import pytest
import torch

from kvskip_amd import ext as E
from kvskip_amd import kvskip as K
from oracle import attention as O
from oracle_side import rel_ok

pytestmark = pytest.mark.gpu


def _stats(B, Hq, nb, seed, spread=3.0, dead=0.0):
    """Random block statistics: blk_max ~ N(0, spread), blk_sum in [1, 64]; a fraction `dead` of the
    blocks unread (-inf, 0)."""
    g = torch.Generator().manual_seed(seed)
    bm = torch.randn(B, Hq, nb, generator=g) * spread
    bs = 1.0 + 63.0 * torch.rand(B, Hq, nb, generator=g)
    if dead:
        off = torch.rand(B, Hq, nb, generator=g) < dead
        bm[off], bs[off] = -math.inf, 0.0
    return bm, bs


def _oracle_sets(bm, bs, G, rule, value, local):
    logw = O.block_logw(bm.double(), bs.double())
    keep = O.select_blocks(logw, G, rule, value, local)
    if rule == "topp":
        _, margin = O.topp_heads(logw, value)
        near = float(margin.min())
    else:
        w = torch.softmax(logw, -1)
        near = float((w - value).abs().min())
    return keep, logw, near


@pytest.mark.parametrize("G", [1, 2, 4, 7, 8])
@pytest.mark.parametrize("nb", [1, 5, 64, 65, 513, 1025, 4096])
@pytest.mark.parametrize("rule,value", [("topp", 0.99), ("topp", 0.6), ("tau", 0.004)])
def test_select_matches_oracle(gpu, G, nb, rule, value):
    B, Hkv, local = 2, 3, 2
    for seed in range(nb * 10 + G, nb * 10 + G + 50):     # the first inputs with no near tie in the oracle
        bm, bs = _stats(B, Hkv * G, nb, seed=seed, dead=0.1 if nb > 64 else 0.0)
        keep_ref, logw, near = _oracle_sets(bm, bs, G, rule, value, local)
        if near > 1e-6:
            break
    assert near > 1e-6, f"oracle margin {near:.2e}: every seed tried has a near tie"
    dev = "cuda"
    keep = torch.empty(B, Hkv, nb, dtype=torch.uint8, device=dev)
    idx = torch.empty(B, Hkv, nb, dtype=torch.int32, device=dev)
    cnt = torch.empty(B, Hkv, dtype=torch.int32, device=dev)
    sc = torch.empty(B, Hkv, nb, G, dtype=torch.float32, device=dev)
    E.select(bm.cuda(), bs.cuda(), Hkv, rule, value, local, keep=keep, block_idx=idx, block_cnt=cnt, blk_scale=sc)
    keep = keep.bool().cpu()
    assert torch.equal(keep, keep_ref), (G, nb, rule, value)
    # lists: kept ascending then the rest ascending
    order = torch.argsort((~keep_ref).to(torch.int8), dim=-1, stable=True).to(torch.int32)
    assert torch.equal(idx.cpu(), order) and torch.equal(cnt.cpu(), keep_ref.sum(-1).to(torch.int32))
    # scales: exp(blk_max - lse over the kept set), 0 off the set
    kh = O.heads(keep_ref, G)
    lse_kept = logw.masked_fill(~kh, -math.inf).logsumexp(-1, keepdim=True)
    ref = torch.exp(bm.double() - lse_kept).masked_fill(~kh, 0.0)
    ref = ref.reshape(B, Hkv, G, nb).transpose(2, 3)
    got = sc.cpu().double()
    assert torch.equal(got == 0, ref == 0)
    nz = ref > 0
    assert ((got[nz] / ref[nz]) - 1).abs().max().item() <= 2e-5


def test_select_blocks_front_end(gpu):
    """kvskip.select_blocks on log-weights (unread blocks -inf) gives the oracle's sets."""
    bm, bs = _stats(1, 8, 300, seed=5, dead=0.2)
    logw = O.block_logw(bm.double(), bs.double())
    for rule, value in (("topp", 0.9), ("tau", 0.01)):
        keep = K.select_blocks(logw.float().cuda(), 4, rule, value, local=1).cpu()
        assert keep.dtype == torch.bool
        assert torch.equal(keep, O.select_blocks(logw, 4, rule, value, 1)), rule


@pytest.mark.parametrize("nb", [1, 63, 64, 65, 700])
def test_make_plan_lists(gpu, nb):
    """make_plan on the device: a stable argsort of ~keep and the counts (kernels/kvskip.py:79-85)."""
    g = torch.Generator().manual_seed(nb)
    keep = torch.rand(3, 5, nb, generator=g) < 0.3
    keep[0, 0] = False
    keep[1, 1] = True
    p = K.make_plan(keep.cuda())
    order = torch.argsort((~keep).to(torch.int8), dim=-1, stable=True).to(torch.int32)
    assert torch.equal(p.block_idx.cpu(), order) and torch.equal(p.block_cnt.cpu(), keep.sum(-1).to(torch.int32))
    assert p.max_cnt == int(keep.sum(-1).max()) and p.nb == nb
    assert K.make_plan(keep.cuda(), sync=False).max_cnt == nb


@pytest.mark.parametrize("G,D,T", [(4, 128, 32768), (7, 128, 5000), (8, 64, 3001)])
def test_vskip_two_pass_on_device(gpu, G, D, T):
    """Pass 1 -> selection -> pass 2 with no host work: the kept set of the oracle's two-pass V-skip
    on its own statistics and exact attention over it; sync=False gives the same output."""
    from kvskip_amd import workloads as W
    run = W.planner_run(layers=1, B=1, Hq=8 * G, Hkv=8, D=D, T0=T, steps=1, seed=60 + G)   # queries aimed
    qc, kc, vc = run.q0[0].to(torch.bfloat16), run.k[0][:, :, :T], run.v[0][:, :, :T]      # at planted blocks
    q, k, v = qc.cuda(), kc.cuda(), vc.cuda()
    M, S = O.block_stats(qc, kc, run.scale)
    _, margin = O.topp_heads(O.block_logw(M, S), 0.99)
    assert float(margin.min()) > 1e-6
    ref, keep = O.vskip_two_pass(qc, kc, vc, run.scale, "topp", 0.99, 2)
    assert keep.float().mean() < 0.5                              # the selection skips most V blocks
    r = K.vskip_two_pass(q, k, v, run.scale)
    assert torch.equal(r["keep"].cpu(), keep)
    assert abs(r["kept_frac"] - keep.double().mean().item()) < 1e-12
    rel_ok(r["out"], ref, (G, D, T))
    r2 = K.vskip_two_pass(q, k, v, run.scale, sync=False)
    assert r2["kept_frac"] is None and torch.equal(r2["keep"], r["keep"])
    rel_ok(r2["out"], ref, (G, D, T, "no sync"))


@pytest.mark.parametrize("G,D,T", [(4, 128, 32768), (1, 64, 200), (2, 128, 9000), (7, 128, 5000), (8, 64, 3001),
                                   (4, 64, 65536 * 4)])
@pytest.mark.parametrize("rule,value", [("topp", 0.99), ("tau", 0.004)])
def test_pv_select_matches_select_then_pv(gpu, G, D, T, rule, value):
    """kvskip_pv_select (the selection in pass 2's prologue) against kvskip_select followed by kvskip_pv
    over its lists and scales, on pass 1's statistics and P, at the same split count: every output
    bit for bit (out, out_f32, the keep mask, the lists and counts, the scales), for 1..64 statistics
    slots of 64 blocks per lane (nb 4 .. 4096)."""
    from kvskip_amd import workloads as W
    B, Hkv = (1, 8) if T <= 65536 else (1, 2)
    run = W.planner_run(layers=1, B=B, Hq=Hkv * G, Hkv=Hkv, D=D, T0=T, steps=1, seed=70 + G)
    q, k, v = run.q0[0].to(torch.bfloat16).cuda(), run.k[0][:, :, :T].cuda(), run.v[0][:, :, :T].cuda()
    first = K.decode(q, k, v, run.scale, stats=True, load_v=False, write_p=True, merge=False)
    bm, bs, P = first["blk_max"], first["blk_sum"], first["p"]
    Hq, nb = Hkv * G, bm.shape[-1]
    dev = q.device
    outs = []
    for fused in (False, True):
        keep = torch.full((B, Hkv, nb), 7, dtype=torch.uint8, device=dev)
        idx = torch.full((B, Hkv, nb), -7, dtype=torch.int32, device=dev)
        cnt = torch.full((B, Hkv), -7, dtype=torch.int32, device=dev)
        sc = torch.full((B, Hkv, nb, G), math.nan, dtype=torch.float32, device=dev)
        for S in (1, K.num_splits_for(B * Hkv, nb)):
            if fused:
                o, o32 = E.pv_select(P, v, bm, bs, rule, value, 2, S, True, keep=keep, block_idx=idx,
                                     block_cnt=cnt, blk_scale=sc)
            else:
                E.select(bm, bs, Hkv, rule, value, 2, keep=keep, block_idx=idx, block_cnt=cnt, blk_scale=sc)
                o, o32 = E.pv(P, v, sc, idx, cnt, S, True)
            outs.append((S, o, o32, keep.clone(), idx.clone(), cnt.clone(), sc.clone()))
    n = len(outs) // 2
    for a, b in zip(outs[:n], outs[n:]):
        assert a[0] == b[0]
        for x, y in zip(a[1:], b[1:]):
            assert torch.equal(x, y), (G, D, T, rule, a[0])
    assert 0 < int(outs[0][5].sum()) <= B * Hkv * nb
