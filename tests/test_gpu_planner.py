"""GPU parity of the device-side refresh planner (plan / update kernels, the fused loop, the
device initialisation, block key sums, token index) against the fp64 CPU oracle of the
reference's Python planner (refresh_pre_step, src/kvskip_attn.py:328-396).

Decisions (refresh triggers, block lists, stored sets, token-index hits, index latches) must be
identical on every head-step: any difference fails, and the failure names the oracle's margin of
that head (|estimate - delta| for a trigger, the top-p cut's distance from `level` for a stored
set), so a float32-order near-tie would show as such. Each test prints the smallest margin it
passed with. Continuous state (estimates, centroid scores, references, attended log-sum-exp,
calibration) within 1e-4 absolute; outputs within 2e-3 relative (bf16).
"""

import math

import numpy as np
import pytest
import torch

from kvskip_amd import ext as E
from kvskip_amd import kvskip as K
from kvskip_amd import workloads as W
from kvskip_amd.planner import FusedPlanner, Policy as DPolicy, PostPlanner
from oracle import attention as O
from oracle import planner as OP

pytestmark = pytest.mark.gpu



def dpolicy(p: OP.Policy) -> DPolicy:
    return DPolicy(**p.__dict__)


def test_block_sums_and_token_index(gpu):
    g = torch.Generator().manual_seed(11)
    k = torch.randn(2, 3, 1000, 128, generator=g).to(torch.bfloat16)
    cs = E.block_sums(k.cuda(), 20).cpu()
    ref = OP.centroid_sums(k)
    assert (cs[:, :, :16].double() - ref).abs().max().item() <= 1e-4 * ref.abs().max().item()
    assert (cs[:, :, 16:] == 0).all()
    ids = torch.randint(0, 50, (3, 3000), generator=g, dtype=torch.int32)
    for T in (1, 2, 63, 64, 65, 1000, 2999, 3000):
        dev = E.token_index(ids.cuda(), T, 50).cpu().numpy().astype(bool)
        ref = OP.index_blocks(ids.numpy(), T)
        nb = ref.shape[1]
        assert (dev[:, :nb] == ref).all(), T
        assert not dev[:, nb:].any()


def _state_to_oracle(p: FusedPlanner, G, scale, T, nb_ref=None) -> OP.State:
    """Oracle state built from the device state (fp32 -> fp64), so one kernel can be checked on
    exactly the inputs the device saw."""
    s = p.state
    nb = O.nblocks(T)
    nbr = nb if nb_ref is None else nb_ref
    return OP.State(scale=scale, G=G, T=T, csum=s["csum"][:, :, :nb].double().cpu(),
                    keep=s["keep"][:, :, :nbr].bool().cpu(), lse_ref=s["lse_ref"][:, :, :nbr].double().cpu(),
                    cs_ref=s["cs_ref"][:, :, :nbr].double().cpu(), lse_att=s["lse_att"].double().cpu(),
                    age=s["age"].long().cpu(), t=p.t, calib=s["calib"].double().cpu(), aix=s["aix"].bool().cpu())


def _agree(dev, ref, margin, what):
    """dev / ref bool tensors of the same shape (per head leading dims) must be equal; margin: the
    oracle's margin per head. Returns the smallest finite margin among the compared heads."""
    diff = dev != ref
    while diff.dim() > margin.dim():
        diff = diff.any(-1)
    if bool(diff.any()):
        where = torch.nonzero(diff).tolist()
        raise AssertionError(f"{what}: {len(where)} head(s) differ: {where[:8]}, oracle margins "
                             f"{[float(margin[tuple(i)]) for i in where[:8]]}")
    fin = margin[torch.isfinite(margin)]
    return float(fin.min()) if fin.numel() else math.inf


def _kv_margin(topp_heads, G):
    """Per KV head: the smallest top-p margin of its query heads (a stored set is their union)."""
    B, Hq = topp_heads.shape
    return topp_heads.reshape(B, Hq // G, G).amin(-1)


@pytest.mark.parametrize("G,D,B,Hkv,T0", [(4, 128, 2, 4, 3000), (7, 128, 2, 4, 3000), (4, 64, 2, 4, 3000),
                                          (2, 64, 1, 4, 10000), (1, 128, 1, 4, 20000), (7, 128, 1, 2, 40000),
                                          (4, 128, 1, 2, 70000), (8, 64, 1, 2, 140000)])
def test_plan_update_kernels(gpu, G, D, B, Hkv, T0):
    """One plan and one update launch each on identical inputs, after a device initialisation
    (contexts from 4 to 2189 blocks: every register tiling of update)."""
    run = W.planner_run(layers=1, B=B, Hq=Hkv * G, Hkv=Hkv, D=D, T0=T0, steps=8, seed=21 + G)
    pol = OP.Policy(calib=0.05, calib_kind="peak", calib_warm=(32, 8), dense_heads=(Hkv - 1,))
    qp = W.QueryProcess(run, 0, p_jump=0.3)
    k, v = run.k[0].cuda(), run.v[0].cuda()
    fp = FusedPlanner(dpolicy(pol))
    T = run.T0[0] + 1
    fp.first(qp.next().cuda(), k[:, :, :T], v[:, :, :T], run.scale)
    for step in range(1, 6):
        T += 1
        q = qp.next()
        nb = O.nblocks(T)
        st = _state_to_oracle(fp, G, run.scale, T - 1)
        st.csum = st.csum[:, :, :O.nblocks(T - 1)]
        pr = OP.plan(st, q, k[:, :, :T].cpu(), pol)
        s = fp.state
        qd = q.cuda()
        # the multi-workgroup plan on a copy of the state, then the one-workgroup plan on the state
        wide = {key: s[key].clone() for key in ("csum", "age", "cs_now", "trig", "block_idx", "block_cnt", "est")}
        one = {key: s[key].clone() for key in wide}
        E.plan(qd, k[:, :, :T], wide["csum"], s["lse_ref"], s["cs_ref"], s["keep"], s["lse_att"], wide["age"],
               s["flags"], wide["cs_now"], wide["trig"], wide["block_idx"], wide["block_cnt"], run.scale, pol.delta,
               OP.max_age_at(pol, step), pol.local, True, None, s["calib"], wide["est"], True,
               OP.KINDS[pol.calib_kind], None, part=s["part"])
        E.plan(qd, k[:, :, :T], s["csum"], s["lse_ref"], s["cs_ref"], s["keep"], s["lse_att"], s["age"], s["flags"],
               s["cs_now"], s["trig"], s["block_idx"], s["block_cnt"], run.scale, pol.delta, OP.max_age_at(pol, step),
               pol.local, True, None, s["calib"], s["est"], True, OP.KINDS[pol.calib_kind], None)
        # the one-launch plan (ticket: the decision by each head's last scores workgroup) on another
        # copy: bit-identical to the two launches, its tickets back to zero
        ticket = torch.zeros(B * Hkv, dtype=torch.int32, device="cuda")
        E.plan(qd, k[:, :, :T], one["csum"], s["lse_ref"], s["cs_ref"], s["keep"], s["lse_att"], one["age"],
               s["flags"], one["cs_now"], one["trig"], one["block_idx"], one["block_cnt"], run.scale, pol.delta,
               OP.max_age_at(pol, step), pol.local, True, None, s["calib"], one["est"], True,
               OP.KINDS[pol.calib_kind], None, part=s["part"], ticket=ticket)
        for key in ("csum", "cs_now", "trig", "block_cnt", "age", "est"):
            assert torch.equal(one[key], wide[key]), f"one-launch plan: {key}"
        for bb in range(B):
            for hh in range(Hkv):
                n = int(wide["block_cnt"][bb, hh])
                assert torch.equal(one["block_idx"][bb, hh, :n], wide["block_idx"][bb, hh, :n]), "one-launch plan: list"
        assert (ticket == 0).all()
        for key in ("csum", "cs_now", "trig", "block_cnt", "age"):       # same arithmetic per row
            assert torch.equal(wide[key], s[key]), f"wide plan: {key}"
        for bb in range(B):
            for hh in range(Hkv):
                n = int(s["block_cnt"][bb, hh])
                assert torch.equal(wide["block_idx"][bb, hh, :n], s["block_idx"][bb, hh, :n]), "wide plan: list"
        assert (wide["est"] - s["est"]).abs().max().item() <= 1e-6    # merge order of the partials
        fp.t, fp.T = step, T
        trig = s["trig"].bool().cpu()
        nbord = _agree(trig, pr["trig"], pr["margin"], "refresh decision")
        assert torch.equal(fp.read_mask(nb).cpu()[trig == pr["trig"]], pr["read"][trig == pr["trig"]])
        assert (s["est"].double().cpu() - pr["miss"]).abs().max().item() <= 1e-4
        assert (s["cs_now"][:, :, :nb].double().cpu() - pr["cs"]).abs().max().item() <= 1e-4
        assert (s["csum"][:, :, :nb].double().cpu() - st.csum).abs().max().item() <= 1e-3
        # update on the stats of the device's own pass
        r = K.decode(qd, k[:, :, :T], v[:, :, :T], run.scale, plan=K.Plan(s["block_idx"], s["block_cnt"], nb, nb),
                     stats=True)
        logw = O.block_logw(r["blk_max"].double().cpu(), r["blk_sum"].double().cpu())
        st_u = _state_to_oracle(fp, G, run.scale, T, nb_ref=O.nblocks(T))
        pr_u = dict(pr, trig=trig)
        # list_stats: the same update on stats that hold NaN wherever the pass read nothing must
        # leave bit-identical state (the fused loop skips the -inf / 0 fill this way)
        mut = ("keep", "lse_ref", "cs_ref", "lse_att", "calib")
        alt = {key: s[key].clone() for key in mut}
        unread = r["blk_sum"] == 0
        bmax_nan = r["blk_max"].masked_fill(unread, math.nan)
        bsum_nan = r["blk_sum"].masked_fill(unread, math.nan)
        E.update(bmax_nan, bsum_nan, s["trig"], s["cs_now"], alt["keep"], alt["lse_ref"], alt["cs_ref"],
                 alt["lse_att"], T, pol.level, pol.local, s["flags"], None, s["est"], alt["calib"], pol.calib,
                 pol.calib_free, OP.KINDS[pol.calib_kind], None, 0.0, list_stats=True)
        E.update(r["blk_max"], r["blk_sum"], s["trig"], s["cs_now"], s["keep"], s["lse_ref"], s["cs_ref"],
                 s["lse_att"], T, pol.level, pol.local, s["flags"], None, s["est"], s["calib"], pol.calib,
                 pol.calib_free, OP.KINDS[pol.calib_kind], None, 0.0)
        for key in mut:
            assert torch.equal(alt[key], s[key]), f"list_stats changed {key}"
        pr_u["miss"] = s["est"].double().cpu()
        pr_u["cs"] = s["cs_now"][:, :, :nb].double().cpu()
        OP.update(st_u, pr_u, logw, pol)
        keep_dev = s["keep"][:, :, :nb].bool().cpu()
        kb = _agree(keep_dev, st_u.keep, _kv_margin(st_u.topp_heads, G), "stored set")
        assert (s["lse_att"].double().cpu() - st_u.lse_att).abs().max().item() <= 1e-4
        assert (s["calib"].double().cpu() - st_u.calib).abs().max().item() <= 1e-4
        fin = torch.isfinite(st_u.lse_ref)
        assert torch.equal(torch.isfinite(s["lse_ref"][:, :, :nb].cpu()), fin)
        assert (s["lse_ref"][:, :, :nb].double().cpu() - st_u.lse_ref)[fin].abs().max().item() <= 1e-4
        print(f"G{G} D{D} step {step}: T {T}, refreshing {int(trig.sum())}/{trig.numel()}, smallest margin: "
              f"decision {nbord:.1e}, stored set {kb:.1e}", flush=True)


def _run_loop(pol: OP.Policy, G=4, D=128, B=1, Hkv=8, T0=4096, steps=40, seed=4, p_jump=0.03):
    run = W.planner_run(layers=1, B=B, Hq=G * Hkv, Hkv=Hkv, D=D, T0=T0, steps=steps, seed=seed)
    qp = W.QueryProcess(run, 0, p_jump=p_jump)
    k_cpu, v_cpu = run.k[0], run.v[0]
    k, v = k_cpu.cuda(), v_cpu.cuda()
    ids = run.ids.cuda()
    fp = FusedPlanner(dpolicy(pol))
    st = None
    stats = dict(head_steps=0, same=0, margin=math.inf, refresh_dev=0, refresh_ref=0, read=0, total=0, max_err=0.0)
    for t in range(steps):
        T = T0 + t + 1
        q = qp.next()
        nb = O.nblocks(T)
        idx_ref = torch.from_numpy(OP.index_blocks(run.ids.numpy(), T))
        if t == 0:
            out_d = fp.first(q.cuda(), k[:, :, :T], v[:, :, :T], run.scale)
            st, out_r = OP.init(q, k_cpu[:, :, :T], v_cpu[:, :, :T], run.scale, pol)
            read_r = torch.ones(B, Hkv, nb, dtype=torch.bool)
            read_d = fp.read_mask(nb).cpu()
            margin = torch.full((B, Hkv), math.inf, dtype=torch.float64)
        else:
            needs_index = bool(pol.index_heads) or pol.calib_auto_ix is not None
            out_d = fp.step(q.cuda(), k[:, :, :T], v[:, :, :T], run.scale, ids=ids if needs_index else None)
            out_r, pr = OP.step(st, q, k_cpu[:, :, :T], v_cpu[:, :, :T], pol, idx=idx_ref)
            read_r, margin = pr["read"], pr["margin"]
            read_d = fp.read_mask(nb).cpu()
            stats["refresh_dev"] += int(fp.state["trig"].sum())
            stats["refresh_ref"] += int(pr["trig"].sum())
        same = (read_d == read_r).all(-1)
        stats["head_steps"] += same.numel()
        stats["same"] += int(same.sum())
        stats["margin"] = min(stats["margin"], _agree(read_d, read_r, margin, f"read set at step {t}"))
        stats["read"] += int(read_r.sum())
        stats["total"] += read_r.numel()
        hq = same.repeat_interleave(G, 1)
        if bool(hq.any()):       # rel. L2 error over the heads whose read sets agree (bench/harness.py:134)
            stats["max_err"] = max(stats["max_err"], O.rel_err(out_d.float().cpu()[hq], out_r[hq]))
        if pol.calib is not None:
            # the log-odds kind differentiates logit() near its clamp, where fp32 estimates of a
            # ~1e-4 mass move it by ~1e-3 (the reference's own bar is 0.05, bench/test_planner.py:122)
            tol = 2e-3 if pol.calib_kind == "logit" else 1e-4
            assert (fp.state["calib"].double().cpu() - st.calib).abs().max().item() <= tol
        if pol.calib_auto_ix is not None:
            assert torch.equal(fp.state["aix"].bool().cpu(), st.aix)
    print(f"{pol}: identical read sets on {stats['same']}/{stats['head_steps']} head-steps "
          f"(smallest decision margin {stats['margin']:.1e}), refreshes device {stats['refresh_dev']} / oracle "
          f"{stats['refresh_ref']}, "
          f"blocks read {stats['read'] / stats['total']:.3f}, max rel. output err {stats['max_err']:.2e}, "
          f"min top-p margin {st.topp_margin:.1e}", flush=True)
    assert stats["max_err"] <= 2e-3
    return stats


POLICIES = {
    "stage3": OP.Policy(dense_heads=(6,)),
    "stage4": OP.Policy(calib=0.05, calib_kind="peak", calib_warm=(32, 8), calib_auto_ix=0.1),
    "logit": OP.Policy(calib=0.3, calib_kind="logit", calib_warm=(32, 8)),
    "add": OP.Policy(calib=0.3, calib_kind="add", calib_warm=(32, 8)),
    "index_union": OP.Policy(index_heads=(2,), index_union=True, dense_heads=(6,)),
    "index_only": OP.Policy(index_heads=(2,), index_union=False),
    "auto_index": OP.Policy(calib=0.05, calib_kind="peak", calib_warm=(32, 8), calib_auto_ix=0.001),
}


@pytest.mark.parametrize("name", list(POLICIES))
def test_planner_loop(gpu, name):
    """The fused loop (plan -> masked + stats attention -> update, device initialisation) against
    the oracle's refresh_pre_step, free-running for 40 decode steps with query drift and jumps
    (bench/test_planner.py:71-133, with the pass bar raised from 97% agreement to 100%)."""
    _run_loop(POLICIES[name], p_jump=0.05)


def test_planner_loop_gqa7_batch(gpu):
    """Config 5 shape (28 / 4 heads, G 7) at batch 3 with the stage-4 policy."""
    _run_loop(POLICIES["stage4"], G=7, Hkv=4, B=3, T0=2500, steps=30, seed=5, p_jump=0.05)


@pytest.mark.parametrize("pol", [OP.Policy(), OP.Policy(delta=0.02, max_age=8, dense_heads=(3,))],
                         ids=["default", "age8_forced"])
@pytest.mark.parametrize("B,G,Hkv,T0", [(1, 4, 8, 4096), (2, 7, 4, 4096), (1, 4, 4, 33000)])
def test_post_planner_loop(gpu, pol, B, G, Hkv, T0):
    """The refresh mode's device loop (PostPlanner: scores, attended lists, masked pass, decision
    against that pass's lse, refresh pass, update) against the oracle's post_step, free-running for
    30 steps with query drift and jumps: refresh decisions identical on every head-step (failures
    name the oracle's margin), the refresh pass's lists the blocks outside a refreshing head's
    attended set and none of the others, stored sets identical after every step, estimates within
    1e-4, outputs within 2e-3. Four KV heads at T 33k: the split count (doubled by the balanced
    partition) is capped at the 64 first-pass partial slots the refresh pass's decision merges."""
    steps = 30
    run = W.planner_run(layers=1, B=B, Hq=G * Hkv, Hkv=Hkv, D=128, T0=T0, steps=steps, seed=6)
    qp = W.QueryProcess(run, 0, p_jump=0.05)
    k_cpu, v_cpu = run.k[0], run.v[0]
    k, v = k_cpu.cuda(), v_cpu.cuda()
    pp = PostPlanner(dpolicy(pol))
    st = None
    n_trig = n_kept = 0
    margin_min = math.inf
    max_err = 0.0
    for t in range(steps):
        T = T0 + t + 1
        q = qp.next()
        nb = O.nblocks(T)
        if t == 0:
            out_d = pp.first(q.cuda(), k[:, :, :T], v[:, :, :T], run.scale)
            st, out_r = OP.init(q, k_cpu[:, :, :T], v_cpu[:, :, :T], run.scale, pol)
        else:
            out_d = pp.step(q.cuda(), k[:, :, :T], v[:, :, :T], run.scale)
            out_r, pr = OP.post_step(st, q, k_cpu[:, :, :T], v_cpu[:, :, :T], pol)
            s = pp.state
            margin_min = min(margin_min, _agree(s["trig"].bool().cpu(), pr["trig"], pr["margin"], f"trigger at step {t}"))
            rest = nb - pr["attended"].sum(-1)             # a refreshing head's blocks outside its attended set
            assert torch.equal(s["block_cnt"].cpu(), torch.where(pr["trig"], rest, 0).to(torch.int32)), t
            assert (s["est"].double().cpu() - pr["miss"]).abs().max().item() <= 1e-4, t
            n_trig += int(pr["trig"].sum())
            n_kept += int((~pr["trig"]).sum())
        _agree(pp.state["keep"][:, :, :nb].bool().cpu(), st.keep, _kv_margin(st.topp_heads, G), f"stored set at step {t}")
        max_err = max(max_err, O.rel_err(out_d.float().cpu(), out_r))
    print(f"post loop {pol}, B {B} G {G}: refreshes {n_trig}, kept {n_kept}, smallest trigger margin "
          f"{margin_min:.1e}, max rel. output err {max_err:.2e}", flush=True)
    assert n_trig > 0 and n_kept > 0
    assert max_err <= 2e-3


def test_merge_update_matches_separate_launches(gpu):
    """kvskip_merge_update (split merge + planner update in one launch) against the split merge and
    the update launched separately, on the same split pass: bit-identical output and state."""
    run = W.planner_run(layers=1, B=2, Hq=28, Hkv=4, D=128, T0=3000, steps=4, seed=31)
    pol = OP.Policy(calib=0.05, calib_kind="peak", calib_warm=(32, 8))
    qp = W.QueryProcess(run, 0, p_jump=0.3)
    k, v = run.k[0].cuda(), run.v[0].cuda()
    fp = FusedPlanner(dpolicy(pol), decide_in_pass=False)     # the test plans with plan() itself
    T = run.T0[0] + 1
    fp.first(qp.next().cuda(), k[:, :, :T], v[:, :, :T], run.scale)
    T += 1
    q = qp.next().cuda()
    s = fp.state
    nb = O.nblocks(T)
    E.plan(q, k[:, :, :T], s["csum"], s["lse_ref"], s["cs_ref"], s["keep"], s["lse_att"], s["age"], s["flags"],
           s["cs_now"], s["trig"], s["block_idx"], s["block_cnt"], run.scale, pol.delta, 32, pol.local, True, None,
           s["calib"], s["est"], True, OP.KINDS["peak"], None, part=s["part"])
    s["trig"][0, 1] = 1                                           # at least one refreshing head
    out, bmax, bsum = fp._attend(q, k[:, :, :T], v[:, :, :T], run.scale, nb)
    assert fp._S > 1
    mut = ("keep", "lse_ref", "cs_ref", "lse_att", "calib")
    alt = {key: s[key].clone() for key in mut}

    def uargs(st):
        return ((bmax, bsum, s["trig"], s["cs_now"], st["keep"], st["lse_ref"], st["cs_ref"], st["lse_att"], T,
                 pol.level, pol.local, s["flags"], None, s["est"], st["calib"], pol.calib, pol.calib_free,
                 OP.KINDS["peak"]), dict(list_stats=True))

    a, kw = uargs(s)
    E.merge_update(q, k[:, :, :T], v[:, :, :T], run.scale, fp.bufs, fp._S, a, kw, s["block_idx"], s["block_cnt"])
    out_f, lse_f = fp.bufs["out"].clone(), fp.bufs["lse"].clone()
    fp.bufs["out"].zero_()
    fp.bufs["lse"].zero_()
    E.decode_into(q, k[:, :, :T], v[:, :, :T], run.scale, fp.bufs, s["block_idx"], s["block_cnt"], stats=False,
                  num_splits=fp._S, phase=2)
    assert torch.equal(fp.bufs["out"], out_f) and torch.equal(fp.bufs["lse"], lse_f)
    a, kw = uargs(alt)
    E.update(*a, **kw)
    for key in mut:
        assert torch.equal(alt[key], s[key]), key


@pytest.mark.parametrize("ragged", [None, [2500, 700]])
def test_plan_fused_token_index(gpu, ragged):
    """plan(ids=..., idx_out=...) finds the token index inside the scores pass: the same decisions,
    lists, state and outputs as the separate token_index launch feeding plan(idx=...), and idx_out
    equal to token_index's blocks of every sequence."""
    B, Hkv, G, D, steps = (1 if ragged is None else 2), 4, 4, 128, 10
    run = W.planner_run(layers=1, B=B, Hq=Hkv * G, Hkv=Hkv, D=D, T0=3000, steps=steps, seed=41, ragged=ragged)
    k, v = run.k[0].cuda(), run.v[0].cuda()
    ids = run.ids.to(torch.int32).cuda()
    qp = W.QueryProcess(run, 0, p_jump=0.1, revert=True)
    pol = DPolicy(calib=0.05, calib_kind="peak", calib_warm=(4, 2), calib_auto_ix=0.0)   # every head on the index
    fused, sep = FusedPlanner(pol, count=False), FusedPlanner(pol, count=False)
    for t in range(steps):
        q = qp.next().cuda()
        if ragged is None:
            T = 3000 + t + 1
            kv, sl, Tv = (k[:, :, :T], v[:, :, :T]), None, T
        else:
            kv, Tv = (k, v), k.shape[2]
            sl = torch.tensor([L + t + 1 for L in ragged], dtype=torch.int32, device="cuda")
        if t == 0:
            o1 = fused.first(q, *kv, run.scale, seq_lens=sl)
            o2 = sep.first(q, *kv, run.scale, seq_lens=sl)
        else:
            o1 = fused.step(q, *kv, run.scale, ids=ids, seq_lens=sl)
            ix = E.token_index(ids, Tv, sep.NBC, seq_lens=sl)
            o2 = sep.step(q, *kv, run.scale, idx=ix, seq_lens=sl)
            lens = [Tv] if sl is None else sl.tolist()
            for b, Tb in enumerate(lens):
                nbb = math.ceil(Tb / 64)
                assert torch.equal(fused.state["idx"][b, :nbb], ix[b, :nbb]), (t, b)
        assert torch.equal(o1, o2), t
        for key in ("keep", "lse_ref", "cs_ref", "lse_att", "age", "trig", "block_idx", "block_cnt", "calib", "aix",
                    "cs_now", "est", "csum"):
            assert torch.equal(fused.state[key], sep.state[key]), (t, key)


def test_index_latch_on_heads_not_refreshing(gpu):
    """update() latches every head whose correction is above the threshold, refreshing or not
    (src/kvskip_attn.py:318-319), strictly above: corrections thr and the next float above it."""
    B, Hq, Hkv, T, NBC = 1, 8, 2, 640, 16
    nb = T // 64
    dev = "cuda"
    f32 = dict(dtype=torch.float32, device=dev)
    bmax = torch.zeros(B, Hq, nb, **f32)
    bsum = torch.ones(B, Hq, nb, **f32)
    trig = torch.zeros(B, Hkv, dtype=torch.uint8, device=dev)
    keep = torch.zeros(B, Hkv, NBC, dtype=torch.uint8, device=dev)
    lse_ref = torch.full((B, Hq, NBC), -math.inf, **f32)
    cs_ref = torch.zeros(B, Hq, NBC, **f32)
    cs_now = torch.zeros(B, Hq, NBC, **f32)
    lse_att = torch.zeros(B, Hq, **f32)
    flags = torch.zeros(Hkv, dtype=torch.int32, device=dev)
    idx = torch.zeros(B, NBC, dtype=torch.uint8, device=dev)
    est = torch.zeros(B, Hkv, **f32)
    thr = 0.25
    up = float(np.nextafter(np.float32(thr), np.float32(1.0)))
    calib = torch.tensor([[thr, up]], **f32)
    aix = torch.zeros(B, Hkv, dtype=torch.uint8, device=dev)
    E.update(bmax, bsum, trig, cs_now, keep, lse_ref, cs_ref, lse_att, T, 0.99, 2, flags, idx, est, calib, 0.05,
             False, 2, aix, thr)
    assert aix.cpu().tolist() == [[0, 1]]
    assert calib.cpu().tolist() == [[thr, up]]


@pytest.mark.parametrize("B,Hkv,G,D,ragged", [(8, 8, 4, 128, False), (16, 4, 7, 128, True), (3, 2, 8, 64, True)])
def test_plan_one_launch_loop(gpu, B, Hkv, G, D, ragged):
    """The planner loop of a batch whose lists plan decides (lengths in device memory), with plan as
    one launch (each head decided by its last scores workgroup; FusedPlanner.plan_one_launch) and as
    two: bit-identical outputs and state on every step, the tickets back to zero; then one step's
    plan captured in a HIP graph and replayed three times from a saved state, each replay against
    the two-launch plan on that state (the tickets reset themselves between replays)."""
    steps = 8
    lens = [1500 + 977 * (b % 5) for b in range(B)] if ragged else None
    run = W.planner_run(layers=1, B=B, Hq=Hkv * G, Hkv=Hkv, D=D, T0=3000 if lens is None else max(lens), steps=steps,
                        seed=61 + B + G, ragged=lens)
    k, v = run.k[0].cuda(), run.v[0].cuda()
    ids = run.ids.to(torch.int32).cuda()
    qp = W.QueryProcess(run, 0, p_jump=0.2, revert=True)
    pol = DPolicy(calib=0.05, calib_kind="peak", calib_warm=(4, 2), calib_auto_ix=0.1)
    one, two = FusedPlanner(pol, count=False, plan_one_launch=True), FusedPlanner(pol, count=False)
    keys = ("keep", "lse_ref", "cs_ref", "lse_att", "age", "trig", "block_idx", "block_cnt", "calib", "aix", "cs_now",
            "est", "csum")
    Tcap = k.shape[2]
    for t in range(steps):
        q = qp.next().cuda()
        if lens is None:
            T = 3000 + t + 1
            kv, sl = (k[:, :, :T], v[:, :, :T]), torch.full((B,), T, dtype=torch.int32, device="cuda")
        else:
            kv = (k, v)
            sl = torch.tensor([L + t + 1 for L in lens], dtype=torch.int32, device="cuda")
        outs = [(fp.first(q, *kv, run.scale, seq_lens=sl) if t == 0 else
                 fp.step(q, *kv, run.scale, ids=ids, seq_lens=sl)).clone() for fp in (one, two)]
        assert two._pargs is None                 # plan decided in its own launch(es)
        assert torch.equal(outs[0], outs[1]), t
        for key in keys:
            assert torch.equal(one.state[key], two.state[key]), (t, key)
        assert (one.state["ticket"] == 0).all()
    # graph replays of one plan call (the planner's own arguments, from a saved state)
    s = one.state
    T = (3000 + steps + 1) if lens is None else Tcap
    kk = k[:, :, :T] if lens is None else k
    sl = torch.full((B,), T, dtype=torch.int32, device="cuda") if lens is None else \
        torch.tensor([L + steps + 1 for L in lens], dtype=torch.int32, device="cuda")
    q = qp.next().cuda()
    mut = ("csum", "age", "cs_now", "trig", "block_idx", "block_cnt", "est")
    saved = {key: s[key].clone() for key in mut}

    def plan_call(st, ticket):
        E.plan(q, kk, st["csum"], s["lse_ref"], s["cs_ref"], s["keep"], s["lse_att"], st["age"], s["flags"],
               st["cs_now"], st["trig"], st["block_idx"], st["block_cnt"], run.scale, pol.delta, pol.max_age,
               pol.local, True, None, s["calib"], st["est"], True, 2, None, part=s["part"], seq_lens=sl,
               ticket=ticket)

    ref = {key: saved[key].clone() for key in mut}
    plan_call(ref, None)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        plan_call(s, s["ticket"])                 # warm-up outside the capture
        with torch.cuda.graph(g, stream=side):
            plan_call(s, s["ticket"])
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for rep in range(3):
        for key in mut:
            s[key].copy_(saved[key])
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for key in mut:
            assert torch.equal(s[key], ref[key]), (rep, key)
        assert (s["ticket"] == 0).all(), rep
