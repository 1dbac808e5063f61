"""GPU: the planner loop with an UpdateCarrier (each layer's update launched inside the next layer's
split pass, kvskip_decode_splits_update) against the same loop without one (update beside the
merge, kvskip_merge_update). Same kernels' arithmetic, so the planner state must be bit-identical
on every step and the outputs equal up to the merge kernel's summation order."""

import pytest
import torch

from kvskip_amd import ext as E
from kvskip_amd import workloads as W
from kvskip_amd.planner import FusedPlanner, Policy, UpdateCarrier

pytestmark = pytest.mark.gpu

STATE = ("keep", "lse_ref", "cs_ref", "lse_att", "age", "trig", "block_idx", "block_cnt", "calib", "est", "aix")


def _policy():
    return Policy(calib=0.05, calib_kind="peak", calib_warm=(8, 4), calib_auto_ix=0.1)


def _loop(layers, B, Hq, Hkv, D, T0, steps, seed, ragged=None):
    run = W.planner_run(layers=layers, B=B, Hq=Hq, Hkv=Hkv, D=D, T0=T0, steps=steps, seed=seed, ragged=ragged,
                        hot_shift=6.0)
    ks = [k.cuda() for k in run.k]
    vs = [v.cuda() for v in run.v]
    ids = run.ids.to(torch.int32).cuda()
    qps = [W.QueryProcess(run, l, p_jump=0.05, revert=True) for l in range(layers)]
    qs = [[qps[l].next().cuda() for l in range(layers)] for _ in range(steps)]
    carrier = UpdateCarrier()
    plain = [FusedPlanner(_policy(), count=False) for _ in range(layers)]
    carried = [FusedPlanner(_policy(), count=False, carrier=carrier) for _ in range(layers)]
    for t in range(steps):
        if ragged is None:
            T = T0 + t + 1
            kv = [(ks[l][:, :, :T], vs[l][:, :, :T]) for l in range(layers)]
            sl = None
        else:
            kv = [(ks[l], vs[l]) for l in range(layers)]
            sl = torch.tensor([T + t + 1 for T in ragged], dtype=torch.int32, device="cuda")
        for l in range(layers):
            for fp in (plain[l], carried[l]):
                if t == 0:
                    out = fp.first(qs[t][l], *kv[l], run.scale, seq_lens=sl)
                else:
                    out = fp.step(qs[t][l], *kv[l], run.scale, ids=ids, seq_lens=sl)
                fp._last_out = out.clone()
            a, b = plain[l]._last_out.float(), carried[l]._last_out.float()
            assert torch.isfinite(a).all()
            err = ((a - b).norm() / a.norm()).item()
            assert err <= 1e-6, (t, l, err)
        # every layer's update but the last one's has run (carried by the next layer's pass)
        _same_state(plain[:-1], carried[:-1], t)
    carried[-1].flush()                 # the last layer's update rides on the next step's first pass
    _same_state(plain, carried, steps)


def _same_state(plain, carried, t):
    for l, (a, b) in enumerate(zip(plain, carried)):
        for key in STATE:
            assert torch.equal(a.state[key], b.state[key]), (t, l, key)


def test_carrier_cfg4_shape(gpu):
    """3 layers of the config-4 shape (32 / 8 heads, d 128) at T 4000: every update carried by the
    next layer's pass, the last one by the next step's first pass."""
    _loop(layers=3, B=1, Hq=32, Hkv=8, D=128, T0=4000, steps=12, seed=21)


def test_carrier_group7_ragged(gpu):
    """G 7 (two query heads per wavefront in the carried update), ragged batch of 3, d 128."""
    _loop(layers=3, B=3, Hq=28, Hkv=4, D=128, T0=2600, steps=10, seed=22, ragged=[1500, 300, 2600])


def test_carrier_group8_d64_single_layer(gpu):
    """One layer (the update cannot ride on its own pass: flushed before the next plan), G 8, d 64."""
    _loop(layers=1, B=2, Hq=16, Hkv=2, D=64, T0=2000, steps=8, seed=23)


def test_carrier_long_context_two_launch_path(gpu):
    """An update over more than 1024 blocks runs as two launches inside decode_splits_update."""
    _loop(layers=2, B=1, Hq=4, Hkv=1, D=64, T0=66000, steps=4, seed=24)


def test_decode_splits_update_rejects_group_mismatch(gpu):
    q = torch.randn(1, 8, 64, device="cuda").to(torch.bfloat16)
    k = torch.randn(1, 2, 256, 64, device="cuda").to(torch.bfloat16)
    fp = FusedPlanner(_policy(), count=False)
    fp.first(q, k, k, 0.125)
    s = fp.state
    u = E.update_struct(fp.bufs["blk_max"][:8 * 4].view(1, 8, 4), fp.bufs["blk_sum"][:8 * 4].view(1, 8, 4), s["trig"],
                        s["cs_now"], s["keep"], s["lse_ref"], s["cs_ref"], s["lse_att"], 256, 0.99, 2, s["flags"],
                        list_stats=True)
    q2 = torch.randn(1, 4, 64, device="cuda").to(torch.bfloat16)        # G 2 against the update's G 4
    bufs = dict(out=torch.empty(1, 4, 64, dtype=torch.bfloat16, device="cuda"),
                lse=torch.empty(1, 4, device="cuda"), blk_max=torch.empty(16, device="cuda"),
                blk_sum=torch.empty(16, device="cuda"), part_acc=torch.empty(4 * 2 * 64, device="cuda"),
                part_ml=torch.empty(4 * 2 * 2, device="cuda"))
    bi = torch.zeros(1, 2, 4, dtype=torch.int32, device="cuda")
    bc = torch.ones(1, 2, dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError, match="group sizes"):
        E.decode_splits_update(q2, k, k, 0.125, bufs, bi, bc, 2, u)


@pytest.mark.parametrize("B", [3, 24])
@pytest.mark.parametrize("carry", [False, True])
def test_batch_balanced_partition(gpu, carry, B):
    """B 3 and 24 x 8 KV heads (24 and 192 lists, over the balanced pass's 16): the planner passes
    the lengths (all T) as seq_lens, so the ragged pass cuts the lists of all KV heads together (B 24:
    with twice the chunk slots). Against the per-(sequence, head) split (batch_balance=False):
    identical state on every step, outputs to float rounding."""
    layers, Hkv, G, D, T0, steps = 2, 8, 4, 64, 1900, 6
    run = W.planner_run(layers=layers, B=B, Hq=Hkv * G, Hkv=Hkv, D=D, T0=T0, steps=steps, seed=77)
    ks = [k.cuda() for k in run.k]
    vs = [v.cuda() for v in run.v]
    ids = run.ids.to(torch.int32).cuda()
    qps = [W.QueryProcess(run, l, p_jump=0.1, revert=True) for l in range(layers)]
    qs = [[qps[l].next().cuda() for l in range(layers)] for _ in range(steps)]
    pol = lambda: Policy(calib=0.05, calib_kind="peak", calib_warm=(4, 2), calib_auto_ix=0.1)
    cr = [UpdateCarrier(), UpdateCarrier()] if carry else [None, None]
    ref = [FusedPlanner(pol(), count=False, carrier=cr[0], batch_balance=False) for _ in range(layers)]
    dut = [FusedPlanner(pol(), count=False, carrier=cr[1]) for _ in range(layers)]
    for t in range(steps):
        T = T0 + t + 1
        for l in range(layers):
            kv = (ks[l][:, :, :T], vs[l][:, :, :T])
            outs = [(fp.first(qs[t][l], *kv, run.scale) if t == 0 else fp.step(qs[t][l], *kv, run.scale, ids=ids)).clone()
                    for fp in (ref[l], dut[l])]
            a, b = outs[0].float(), outs[1].float()
            assert float((a - b).norm() / b.norm()) <= 1e-3, (t, l)
        for c in cr:
            if c is not None:
                c.flush()
        _same_state(ref, dut, t)


@pytest.mark.parametrize("lens,Hkv,G,D", [((1700, 2900, 1100), 4, 4, 128), ((900, 4100, 2500, 3300, 1800), 2, 7, 128),
                                           ((2100,) * 8, 8, 2, 64), ((600, 3900, 2200, 1500, 3000, 2600, 800, 1900,
                                                                      3500, 1200, 2800, 700, 3300, 2400, 1000, 3100),
                                                                     2, 4, 64)])
@pytest.mark.parametrize("carry", [False, True])
def test_ragged_decision_in_pass(gpu, lens, Hkv, G, D, carry):
    """A ragged batch decided inside the masked pass (every workgroup decides its KV head's B lists,
    then takes its chunk of the ragged partition over them: B 3, 5, 8 and 16, so one, two, two and four
    lists per wavefront) against plan's own decision launch followed by the ragged pass over the
    plan's lists: bit-identical state on every step (lists, triggers, ages, references,
    calibration, latches) and bit-identical outputs (the same chunks of the same lists)."""
    layers, steps = 2, 6
    run = W.planner_run(layers=layers, B=len(lens), Hq=Hkv * G, Hkv=Hkv, D=D, T0=max(lens), steps=steps,
                        seed=90 + len(lens) + G, ragged=list(lens))
    ks = [k.cuda() for k in run.k]
    vs = [v.cuda() for v in run.v]
    ids = run.ids.to(torch.int32).cuda()
    qps = [W.QueryProcess(run, l, p_jump=0.1, revert=True) for l in range(layers)]
    qs = [[qps[l].next().cuda() for l in range(layers)] for _ in range(steps)]
    pol = lambda: Policy(calib=0.05, calib_kind="peak", calib_warm=(4, 2), calib_auto_ix=0.1)
    cr = [UpdateCarrier(), UpdateCarrier()] if carry else [None, None]
    # the reference cuts the lists per KV head as the in-pass decision does (global_partition off)
    ref = [FusedPlanner(pol(), count=False, carrier=cr[0], decide_in_pass=False, global_partition=False)
           for _ in range(layers)]
    dut = [FusedPlanner(pol(), count=False, carrier=cr[1], ragged_in_pass=True) for _ in range(layers)]
    for t in range(steps):
        sl = torch.tensor([T + t + 1 for T in lens], dtype=torch.int32, device="cuda")
        for l in range(layers):
            outs = [(fp.first(qs[t][l], ks[l], vs[l], run.scale, seq_lens=sl) if t == 0 else
                     fp.step(qs[t][l], ks[l], vs[l], run.scale, ids=ids, seq_lens=sl)).clone() for fp in (ref[l], dut[l])]
            assert torch.isfinite(outs[0].float()).all()
            assert torch.equal(outs[0], outs[1]), (t, l)
        for c in cr:
            if c is not None:
                c.flush()
        _same_state(ref, dut, t)
    assert dut[0]._pargs is not None          # the decision ran in the pass


@pytest.mark.parametrize("B,Hkv,G", [(2, 8, 2), (1, 12, 8), (4, 4, 4), (1, 1, 7)])
def test_balanced_pass_many_lists(gpu, B, Hkv, G):
    """The balanced planned pass (every workgroup decides all B * Hkv lists: 16, 12, 16 and 1 here,
    so four, three (one list decided twice), four and one list per wavefront) against plan's own
    launches: identical state on every step, outputs to float rounding."""
    layers, D, T0, steps = 2, 64, 1800, 6
    run = W.planner_run(layers=layers, B=B, Hq=Hkv * G, Hkv=Hkv, D=D, T0=T0, steps=steps, seed=40 + B * Hkv + G)
    ks = [k.cuda() for k in run.k]
    vs = [v.cuda() for v in run.v]
    ids = run.ids.to(torch.int32).cuda()
    qps = [W.QueryProcess(run, l, p_jump=0.1, revert=True) for l in range(layers)]
    qs = [[qps[l].next().cuda() for l in range(layers)] for _ in range(steps)]
    pol = lambda: Policy(calib=0.05, calib_kind="peak", calib_warm=(4, 2), calib_auto_ix=0.1)
    ref = [FusedPlanner(pol(), count=False, decide_in_pass=False) for _ in range(layers)]
    cr = UpdateCarrier()
    dut = [FusedPlanner(pol(), count=False, carrier=cr, decide_in_pass=True, balance=True) for _ in range(layers)]
    for t in range(steps):
        T = T0 + t + 1
        for l in range(layers):
            kv = (ks[l][:, :, :T], vs[l][:, :, :T])
            outs = [(fp.first(qs[t][l], *kv, run.scale) if t == 0 else fp.step(qs[t][l], *kv, run.scale, ids=ids)).clone()
                    for fp in (ref[l], dut[l])]
            a, b = outs[0].float(), outs[1].float()
            assert float((a - b).norm() / b.norm()) <= 1e-3, (t, l)
        cr.flush()
        _same_state(ref, dut, t)


@pytest.mark.parametrize("balance", [False, True])
@pytest.mark.parametrize("G,D,heads", [(4, 128, {}), (8, 64, {"dense_heads": (1,), "index_heads": (0,)}),
                                       (7, 128, {"index_heads": (2,), "index_union": True})])
def test_decision_in_pass_matches_plan(gpu, G, D, heads, balance):
    """The plan's decision made inside the masked pass (kvskip_plan_scores, then
    kvskip_decode_splits_planned; the update advances the age) against plan's own two launches:
    bit-identical state (lists, triggers, ages, references, calibration) on every step, with and
    without a carried update, dense-flagged and token-index heads included. Outputs: bit-identical
    with each head's list cut into the pass's split count; with the lists of all heads cut by one
    chunk length (balance, kvskip_plan_args.pass_budget) the split partials cover other ranges, so
    the merged outputs agree to float rounding (relative L2 <= 1e-3 of bf16 outputs)."""
    layers, Hkv, T0, steps = 2, 3, 2500, 10
    run = W.planner_run(layers=layers, B=1, Hq=Hkv * G, Hkv=Hkv, D=D, T0=T0, steps=steps, seed=25 + G)
    ks = [k.cuda() for k in run.k]
    vs = [v.cuda() for v in run.v]
    ids = run.ids.to(torch.int32).cuda()
    qps = [W.QueryProcess(run, l, p_jump=0.1, revert=True) for l in range(layers)]
    qs = [[qps[l].next().cuda() for l in range(layers)] for _ in range(steps)]
    pol = lambda: Policy(calib=0.05, calib_kind="peak", calib_warm=(4, 2), calib_auto_ix=0.1, **heads)
    for carry, dyn in ((False, False), (True, False), (True, True)):
        # dyn: the step's length in device memory (seq_lens, one sequence) over full-capacity views
        ref = [FusedPlanner(pol(), count=False, decide_in_pass=False) for _ in range(layers)]
        cr = UpdateCarrier() if carry else None
        dut = [FusedPlanner(pol(), count=False, carrier=cr, decide_in_pass=True, balance=balance)
               for _ in range(layers)]
        for t in range(steps):
            T = T0 + t + 1
            sl = torch.tensor([T], dtype=torch.int32, device="cuda") if dyn else None
            for l in range(layers):
                kv = (ks[l], vs[l]) if dyn else (ks[l][:, :, :T], vs[l][:, :, :T])
                outs = []
                for fp in (ref[l], dut[l]):
                    o = (fp.first(qs[t][l], *kv, run.scale, seq_lens=sl) if t == 0
                         else fp.step(qs[t][l], *kv, run.scale, ids=ids, seq_lens=sl))
                    outs.append(o.clone())
                if balance:
                    a, b = outs[0].float(), outs[1].float()
                    assert float((a - b).norm() / b.norm()) <= 1e-3, (carry, dyn, t, l)
                else:
                    assert torch.equal(outs[0], outs[1]), (carry, dyn, t, l)
            if cr is not None:
                cr.flush()
            _same_state(ref, dut, t)
