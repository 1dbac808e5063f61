"""GPU: the attention passes over a paged KV cache (kvskip_attn_args.block_table: 64-token pages in a
pool, a block table per sequence) against the same passes over the contiguous cache, and against the
CPU oracle on the rows the block table addresses (gathered from the pools on the CPU). Only the
addresses differ from the contiguous cache, so outputs, log-sum-exps and block statistics must be
bit-identical to it; against the oracle, outputs within 2e-3, statistics within 2e-4, and the
decisions (V-skip votes, top-p sets, the planner's read sets) identical. The pools are built from
the contiguous cache in a random page order, and every byte the pass must not read (unused pages,
rows past a sequence's last token, pages of other sequences) holds NaN, so a wrong page or a read
past the sequence shows up in the results."""

import math

import pytest
import torch

from kvskip_amd import ext as E
from kvskip_amd import kvskip as K
from oracle import attention as O
from oracle_side import LayerOracle, gather_pages, oracle_policy, rel_ok, same_decisions

pytestmark = pytest.mark.gpu

NAN = float("nan")


def _cache(B, Hq, Hkv, D, T, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, D, generator=g).to(torch.bfloat16).cuda()
    k = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16).cuda()
    k[:, :, :64] += 0.3 * torch.randn(B, Hkv, 1, D, generator=g).to(torch.bfloat16).cuda()   # some structure
    return q, k, v


def _paginate(k, v, lens, seed, extra=5, width_pad=3):
    """Pools [P, Hkv, 64, D] holding sequence b's tokens [0, lens[b]) in random pages, NaN elsewhere,
    and the block table [B, ceil(max(lens) / 64) + width_pad] (-1 past each sequence)."""
    B, Hkv, _, D = k.shape
    nbs = [math.ceil(n / 64) for n in lens]
    P = sum(nbs) + extra
    perm = torch.randperm(P, generator=torch.Generator().manual_seed(seed)).tolist()
    kp = torch.full((P, Hkv, 64, D), NAN, dtype=torch.bfloat16, device="cuda")
    vp = torch.full((P, Hkv, 64, D), NAN, dtype=torch.bfloat16, device="cuda")
    table = torch.full((B, max(nbs) + width_pad), -1, dtype=torch.int32)
    i = 0
    for b in range(B):
        for j in range(nbs[b]):
            pg = perm[i]
            i += 1
            rows = min(64, lens[b] - 64 * j)
            kp[pg, :, :rows] = k[b, :, 64 * j:64 * j + rows]
            vp[pg, :, :rows] = v[b, :, 64 * j:64 * j + rows]
            table[b, j] = pg
    return kp, vp, table.cuda()


def _same(a, b, what):
    assert a is not None and b is not None
    assert torch.equal(a, b), (what, (a.float() - b.float()).abs().max().item())


def _gathered(kp, vp, table, lens):
    """The oracle's view of the pools: per sequence the rows its table addresses (CPU), concatenated
    into [B, Hkv, T, D] when the lengths agree."""
    ks, vs = gather_pages(kp, table, lens), gather_pages(vp, table, lens)
    if len(set(lens)) == 1:
        return torch.cat(ks), torch.cat(vs)
    return ks, vs


def _stats_close(got_max, got_sum, M, S, what):
    fin = torch.isfinite(M)
    assert torch.equal(torch.isfinite(got_max.cpu()), fin), what
    assert (got_max.cpu().double()[fin] - M[fin]).abs().max().item() <= 2e-4, what
    assert (got_sum.cpu().double()[fin] / S[fin] - 1).abs().max().item() <= 2e-4, what


@pytest.mark.parametrize("G,D", [(4, 128), (7, 128), (8, 64), (1, 64)])
@pytest.mark.parametrize("T", [4096, 3001])
def test_paged_dense_and_stats_match_contiguous(G, D, T):
    Hkv = 2
    q, k, v = _cache(2, Hkv * G, Hkv, D, T, seed=41 + G + T)
    kp, vp, table = _paginate(k, v, [T, T], seed=T)
    for S in (1, 8, 32):
        for stats in (False, True):
            ref = K.decode(q, k, v, D ** -0.5, stats=stats, num_splits=S)
            got = K.decode(q, kp, vp, D ** -0.5, stats=stats, num_splits=S, block_table=table, T=T)
            _same(got["out"], ref["out"], ("out", S, stats))
            _same(got["lse"], ref["lse"], ("lse", S, stats))
            if stats:
                _same(got["blk_max"], ref["blk_max"], ("blk_max", S))
                _same(got["blk_sum"], ref["blk_sum"], ("blk_sum", S))
    kg, vg = _gathered(kp, vp, table, [T, T])
    assert torch.equal(kg, k.cpu()) and torch.equal(vg, v.cpu())
    out, lse = O.decode(q.cpu(), kg, vg, D ** -0.5)
    rel_ok(got["out"], out, "paged dense vs oracle")
    assert (got["lse"].cpu().double() - lse).abs().max().item() <= 2e-4
    _stats_close(got["blk_max"], got["blk_sum"], *O.block_stats(q.cpu(), kg, D ** -0.5), "paged stats vs oracle")


@pytest.mark.parametrize("G,D", [(4, 128), (7, 128)])
def test_paged_masked_stats_match_contiguous(G, D):
    Hkv, T = 3, 5000
    q, k, v = _cache(2, Hkv * G, Hkv, D, T, seed=51 + G)
    kp, vp, table = _paginate(k, v, [T, T], seed=7)
    nb = math.ceil(T / 64)
    g = torch.Generator().manual_seed(52)
    keep = torch.rand(2, Hkv, nb, generator=g) < 0.35
    keep[..., 0] = True
    keep[0, 1] = False                                  # an empty list
    keep[1, 2] = True                                   # a full list
    plan = K.make_plan(keep.cuda())
    for S in (4, 16):
        ref = K.decode(q, k, v, D ** -0.5, plan=plan, stats=True, num_splits=S)
        got = K.decode(q, kp, vp, D ** -0.5, plan=plan, stats=True, num_splits=S, block_table=table, T=T)
        for key in ("out", "lse", "blk_max", "blk_sum"):
            _same(got[key], ref[key], (key, S))
    kg, vg = _gathered(kp, vp, table, [T, T])
    out, _ = O.decode(q.cpu(), kg, vg, D ** -0.5, keep=keep)
    live = O.heads(keep.any(-1, keepdim=True), G)[..., 0]                 # the empty list: out 0
    rel_ok(got["out"][live], out[live], "paged masked vs oracle")
    assert (got["out"][~live.cuda()] == 0).all()
    _stats_close(got["blk_max"], got["blk_sum"], *O.block_stats(q.cpu(), kg, D ** -0.5, keep=keep),
                 "paged masked stats vs oracle")


def test_paged_ragged_batch_matches_contiguous():
    """seq_lens with a paged cache: each sequence's table row covers only its own pages (-1 past)."""
    G, D, Hkv, Tcap = 4, 128, 2, 6000
    lens = [6000, 700, 64, 3333]
    q, k, v = _cache(4, Hkv * G, Hkv, D, Tcap, seed=61)
    kp, vp, table = _paginate(k, v, lens, seed=62)
    sl = torch.tensor(lens, dtype=torch.int32, device="cuda")
    for stats, load_v in ((False, True), (True, True), (True, False)):      # the last: the K-only pass
        ref = K.decode(q, k, v, D ** -0.5, stats=stats, load_v=load_v, seq_lens=sl)
        got = K.decode(q, kp, vp, D ** -0.5, stats=stats, load_v=load_v, seq_lens=sl, block_table=table, T=Tcap)
        if load_v:
            _same(got["out"], ref["out"], ("out", stats))
        _same(got["lse"], ref["lse"], ("lse", stats, load_v))
        if stats:
            _same(got["blk_max"], ref["blk_max"], ("blk_max", load_v))
            _same(got["blk_sum"], ref["blk_sum"], ("blk_sum", load_v))
        if load_v:
            kg, vg = _gathered(kp, vp, table, lens)
            for b, n in enumerate(lens):
                out, _ = O.decode(q[b:b + 1].cpu(), kg[b], vg[b], D ** -0.5)
                rel_ok(got["out"][b:b + 1], out, ("paged ragged vs oracle", b))


def test_paged_invalid_page_reads_as_empty_block():
    """A page id outside [0, num_pages) makes its block empty: statistics (-inf, 0) there, and the
    output equals the pass over a list without that block (within the split-order tolerance)."""
    G, D, Hkv, T = 4, 128, 2, 2048
    q, k, v = _cache(1, Hkv * G, Hkv, D, T, seed=71)
    kp, vp, table = _paginate(k, v, [T], seed=72)
    bad = 5
    table[0, bad] = kp.shape[0] + 3
    got = K.decode(q, kp, vp, D ** -0.5, stats=True, num_splits=8, block_table=table, T=T)
    assert torch.isfinite(got["out"].float()).all()
    assert torch.isinf(got["blk_max"][0, :, bad]).all() and (got["blk_max"][0, :, bad] < 0).all()
    assert (got["blk_sum"][0, :, bad] == 0).all()
    keep = torch.ones(1, Hkv, T // 64, dtype=torch.bool)
    keep[..., bad] = False
    ref = K.decode(q, k, v, D ** -0.5, plan=K.make_plan(keep.cuda()), stats=True, num_splits=8)
    a, b = got["out"].float(), ref["out"].float()
    assert ((a - b).norm() / b.norm()).item() <= 2e-3
    torch.testing.assert_close(got["lse"], ref["lse"], rtol=0, atol=1e-5)


@pytest.mark.parametrize("G,D", [(4, 128), (8, 64), (7, 128)])
def test_paged_stats_only_pass_matches_contiguous(G, D):
    """The K-only pass (statistics, fp16 P, no V) over pages: lse, statistics and P bit-identical."""
    Hkv, T = 2, 4000
    q, k, v = _cache(2, Hkv * G, Hkv, D, T, seed=101 + G)
    kp, vp, table = _paginate(k, v, [T, T], seed=102)
    nb = math.ceil(T / 64)
    keep = torch.rand(2, Hkv, nb, generator=torch.Generator().manual_seed(103)) < 0.4
    for plan in (None, K.make_plan(keep.cuda())):
        for S in (1, 16):
            ref = K.decode(q, k, v, D ** -0.5, plan=plan, stats=True, load_v=False, write_p=True, num_splits=S)
            got = K.decode(q, kp, vp, D ** -0.5, plan=plan, stats=True, load_v=False, write_p=True, num_splits=S,
                           block_table=table, T=T)
            assert got["out"] is None
            for key in ("lse", "blk_max", "blk_sum"):
                _same(got[key], ref[key], (key, S, plan is None))
            # P of a skipped block is left unwritten (an uninitialised buffer, as in the reference)
            listed = torch.ones_like(keep) if plan is None else keep
            tok = listed.cuda().repeat_interleave(G, 1).repeat_interleave(64, 2)
            _same(got["p"][tok], ref["p"][tok], ("p", S, plan is None))


@pytest.mark.parametrize("G,D", [(4, 128), (8, 64)])
@pytest.mark.parametrize("T", [4096, 2501])
def test_paged_vskip_two_pass_matches_contiguous(G, D, T):
    """Two-pass V-skip over pages (K-only pass with P, selection, pass 2 over the kept blocks' V pages)
    gives the contiguous selection and output bit for bit (sync=False: both size pass 2 by nb; the
    contiguous cache selects inside pass 2, the pages in their own launch); with sync=True the paged
    pass 2 is sized by the longest list, so its output agrees to float rounding."""
    Hkv = 2
    q, k, v = _cache(2, Hkv * G, Hkv, D, T, seed=111 + T)
    kp, vp, table = _paginate(k, v, [T, T], seed=112)
    # random scores give blocks of nearly equal weight: a small top-p mass, or tau just above the mean
    # weight, leaves blocks out of the group union
    for rule, value in (("topp", 0.3), ("tau", 1.2 / math.ceil(T / 64))):
        ref = K.vskip_two_pass(q, k, v, D ** -0.5, rule=rule, value=value)
        got = K.vskip_two_pass(q, kp, vp, D ** -0.5, rule=rule, value=value, block_table=table, T=T)
        assert torch.equal(got["keep"], ref["keep"]), rule
        assert 0 < ref["kept_frac"] < 1 and got["kept_frac"] == ref["kept_frac"], (rule, ref["kept_frac"])
        rel_ok(got["out"], ref["out"].double().cpu(), ("paged two-pass vs contiguous", rule))
        ref0 = K.vskip_two_pass(q, k, v, D ** -0.5, rule=rule, value=value, sync=False)
        got0 = K.vskip_two_pass(q, kp, vp, D ** -0.5, rule=rule, value=value, block_table=table, T=T, sync=False)
        _same(got0["out"], ref0["out"], ("out", rule))
        kg, vg = _gathered(kp, vp, table, [T, T])
        o_ref, keep = O.vskip_two_pass(q.cpu(), kg, vg, D ** -0.5, rule, value)
        assert torch.equal(got["keep"].cpu(), keep), ("paged two-pass selection vs oracle", rule)
        rel_ok(got["out"], o_ref, ("paged two-pass vs oracle", rule))


@pytest.mark.parametrize("G,D", [(4, 128), (8, 64), (1, 64)])
@pytest.mark.parametrize("T", [4096, 3001])
def test_paged_vskip_one_pass_matches_contiguous(G, D, T):
    """Single-pass V-skip over pages: output, log-sum-exp and V blocks read bit-identical, with the
    block-0 estimate and with lse_prev."""
    Hkv = 2
    q, k, v = _cache(2, Hkv * G, Hkv, D, T, seed=121 + G)
    kp, vp, table = _paginate(k, v, [T, T], seed=122)
    lse_prev = K.decode(q, k, v, D ** -0.5)["lse"]
    nb = math.ceil(T / 64)
    for S in (1, 8):
        # random scores give blocks of nearly equal weight: tau just above the mean weight skips some
        for lp, tau in ((None, 1.2), (lse_prev, 1.2 / nb)):
            ref = K.vskip_one_pass(q, k, v, D ** -0.5, tau=tau, num_splits=S, count=True, lse_prev=lp, keep=True)
            got = K.vskip_one_pass(q, kp, vp, D ** -0.5, tau=tau, num_splits=S, count=True, lse_prev=lp,
                                   block_table=table, T=T, keep=True)
            for key in ("out", "lse", "v_tiles", "v_keep"):
                _same(got[key], ref[key], (key, S, lp is None))
            assert ref["v_tiles"].sum().item() < 2 * Hkv * nb, (S, lp is None)      # some V blocks skipped
    kg, vg = _gathered(kp, vp, table, [T, T])
    for lp, tau in ((None, 1.2), (lse_prev, 1.2 / nb)):
        got = K.vskip_one_pass(q, kp, vp, D ** -0.5, tau=tau, num_splits=8, count=True, lse_prev=lp,
                               block_table=table, T=T, keep=True)
        lpd = None if lp is None else lp.cpu().double()
        o_ref, _, keep, cnt = O.vskip1(q.cpu(), kg, vg, D ** -0.5, tau, 2, lse_prev=lpd)
        _, z = O.vskip1_keep(q.cpu(), kg, D ** -0.5, tau, 2, lse_prev=lpd)
        assert float(z.abs().min()) > 1e-5                                  # no vote at float32 noise
        assert torch.equal(got["v_keep"].cpu(), keep), ("paged one-pass votes vs oracle", lp is None)
        assert torch.equal(got["v_tiles"].cpu(), cnt), ("paged one-pass votes vs oracle", lp is None)
        rel_ok(got["out"], o_ref, ("paged one-pass vs oracle", lp is None))


def test_paged_rejections():
    """Calls a paged cache cannot serve are refused instead of reading wrong memory."""
    G, D, Hkv, T = 4, 128, 1, 256
    q, k, v = _cache(1, Hkv * G, Hkv, D, T, seed=81)
    kp, vp, table = _paginate(k, v, [T], seed=82)
    big = 4097 * 64                                          # one split would gather > 4096 pages
    wide = torch.full((1, 4097), -1, dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError, match="blocks per split"):
        E.decode(q, kp, vp, 0.1, num_splits=1, block_table=wide, T=big)
    with pytest.raises(RuntimeError, match="blocks per split"):
        E.vskip1(q, kp, vp, 0.1, 1e-3, num_splits=1, block_table=wide, T=big)
    with pytest.raises(RuntimeError, match="T .* is required"):
        E.decode(q, kp, vp, 0.1, block_table=table)
    with pytest.raises(RuntimeError, match="block_table"):
        E.decode(q, kp, vp, 0.1, block_table=table[:, :2].contiguous(), T=T)


@pytest.mark.parametrize("ragged,G,D", [(False, 4, 128), (True, 4, 128), (False, 8, 64)])
def test_paged_planner_loop_matches_contiguous(ragged, G, D):
    """The device planner loop (key sums, plan with the appended key, the pass with the decision in it
    or not, updates carried by the other layer's pass) over paged caches gives the contiguous loop's
    outputs and state bit for bit; two layers share the carrier."""
    from kvskip_amd import workloads as W
    from kvskip_amd.planner import FusedPlanner, Policy, UpdateCarrier

    Hkv, steps, layers = 2, 8, 2
    lens0 = [2600, 900, 1700] if ragged else [2600]
    B = len(lens0)
    run = W.planner_run(layers=layers, B=B, Hq=Hkv * G, Hkv=Hkv, D=D, T0=max(lens0), steps=steps, seed=91,
                        ragged=lens0 if ragged else None)
    ks = [k.cuda() for k in run.k]
    vs = [v.cuda() for v in run.v]
    Tcap = ks[0].shape[2]
    qps = [W.QueryProcess(run, l, p_jump=0.2, revert=True) for l in range(layers)]
    qs = [[qps[l].next().cuda() for l in range(layers)] for _ in range(steps)]
    ids = run.ids.to(torch.int32).cuda()
    pools = [_paginate(ks[l], vs[l], [Tcap] * B, seed=92 + l) for l in range(layers)]   # random page order
    pol = lambda: Policy(calib=0.05, calib_kind="peak", calib_warm=(4, 2), calib_auto_ix=0.1)
    cr = UpdateCarrier()
    ref = [FusedPlanner(pol(), count=False) for _ in range(layers)]
    dut = [FusedPlanner(pol(), count=False, carrier=cr) for _ in range(layers)]
    keys = ("csum", "keep", "lse_ref", "cs_ref", "lse_att", "age", "trig", "block_idx", "block_cnt", "calib", "est",
            "aix")
    # the oracle's refresh_pre loop per (layer, sequence) on the rows the block tables address
    orc = [[LayerOracle(oracle_policy(pol()), run.scale) for _ in range(B)] for _ in range(layers)]
    ids_c = ids.cpu().numpy()
    for t in range(steps):
        if ragged:
            sl = torch.tensor([n + t + 1 for n in lens0], dtype=torch.int32, device="cuda")
            T = Tcap
        else:
            sl, T = None, lens0[0] + t + 1
        for l in range(layers):
            kv = (ks[l], vs[l]) if ragged else (ks[l][:, :, :T], vs[l][:, :, :T])
            kp, vp, table = pools[l]
            if t == 0:   # the paged planner's first call is step(), which starts the state on the pages
                a = ref[l].first(qs[t][l], *kv, run.scale, seq_lens=sl)
                b = dut[l].step(qs[t][l], kp, vp, run.scale, ids=ids, seq_lens=sl, block_table=table, T=T)
            else:
                a = ref[l].step(qs[t][l], *kv, run.scale, ids=ids, seq_lens=sl)
                b = dut[l].step(qs[t][l], kp, vp, run.scale, ids=ids, seq_lens=sl, block_table=table, T=T)
            assert torch.equal(a.clone(), b.clone()), (t, l)
            lens = [n + t + 1 for n in lens0]
            kg, vg = gather_pages(kp, table, lens), gather_pages(vp, table, lens)
            s = dut[l].state
            for bb in range(B):
                o_ref, read, trig, margin = orc[l][bb].step(qs[t][l][bb:bb + 1].cpu(), kg[bb], vg[bb], ids_c[bb:bb + 1])
                nb = read.shape[-1]
                dev_read = torch.zeros(1, Hkv, nb, dtype=torch.bool)
                for h in range(Hkv):
                    dev_read[0, h, s["block_idx"][bb, h, :int(s["block_cnt"][bb, h])].long().cpu()] = True
                same_decisions(dev_read, read, trig, s["trig"][bb:bb + 1].bool().cpu(), margin, (t, l, bb))
                rel_ok(b[bb:bb + 1], o_ref, (t, l, bb))
        cr.flush()
        for l in range(layers):
            for key in keys:
                assert torch.equal(ref[l].state[key], dut[l].state[key]), (t, l, key)
