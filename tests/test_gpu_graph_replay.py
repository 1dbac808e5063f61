"""GPU: one HIP graph of a whole decode step (every layer's plan, pass, merge and update) captured
once and replayed for every later step. The step's length lives in device memory (seq_lens, the
ragged form, here with B 1) and the graph's first node advances it, so no launch argument changes
between steps; after the policy's warm-up (max age and calibration switch fixed) the replays must
reproduce the eager step-by-step loop bit for bit, and the oracle's refresh_pre loop on the same
inputs: identical read sets on every layer-step, outputs within 2e-3."""

import pytest
import torch

from kvskip_amd import workloads as W
from kvskip_amd.planner import FusedPlanner, Policy, UpdateCarrier
from oracle_side import LayerOracle, oracle_policy, rel_ok, same_decisions

pytestmark = pytest.mark.gpu

STATE = ("keep", "lse_ref", "cs_ref", "lse_att", "age", "trig", "block_idx", "block_cnt", "calib", "aix")


def _policy():
    return Policy(calib=0.05, calib_kind="peak", calib_warm=(4, 2), calib_auto_ix=0.1)


@pytest.mark.parametrize("carried", [False, True])
def test_one_graph_replayed_every_step(gpu, carried):
    layers, T0, steps, warm = 3, 3000, 16, 6
    run = W.planner_run(layers=layers, B=1, Hq=32, Hkv=8, D=128, T0=T0, steps=steps, seed=31, ragged=[T0])
    ks = [k.cuda() for k in run.k]
    vs = [v.cuda() for v in run.v]
    ids = run.ids.to(torch.int32).cuda()
    qps = [W.QueryProcess(run, l, p_jump=0.05, revert=True) for l in range(layers)]
    qs = torch.stack([torch.stack([qps[l].next() for l in range(layers)]) for _ in range(steps)]).cuda()

    def loop(planners, t, q, sl):
        outs = []
        for l in range(layers):
            fp = planners[l]
            if t == 0:
                outs.append(fp.first(q[l], ks[l], vs[l], run.scale, seq_lens=sl))
            else:
                outs.append(fp.step(q[l], ks[l], vs[l], run.scale, ids=ids, seq_lens=sl))
        return outs

    # the oracle's loop on the same inputs: read sets and outputs of every layer-step
    orc = [LayerOracle(oracle_policy(_policy()), run.scale) for _ in range(layers)]
    ids_c = ids.cpu().numpy()
    ref_orc = []
    for t in range(steps):
        T = T0 + t + 1
        ref_orc.append([orc[l].step(qs[t][l].cpu(), run.k[l][:, :, :T], run.v[l][:, :, :T], ids_c)
                        for l in range(layers)])

    # eager reference, one step at a time
    ce = UpdateCarrier() if carried else None
    eager = [FusedPlanner(_policy(), count=False, carrier=ce) for _ in range(layers)]
    ref_out, ref_state = [], []
    for t in range(steps):
        sl = torch.tensor([T0 + t + 1], dtype=torch.int32, device="cuda")
        outs = loop(eager, t, qs[t], sl)            # carried: the last layer's update still pending
        ref_out.append([o.clone() for o in outs])
        ref_state.append([{k: fp.state[k].clone() for k in STATE} for fp in eager])

    # warm-up eagerly, then capture one step and replay it
    cg = UpdateCarrier() if carried else None
    planners = [FusedPlanner(_policy(), count=False, carrier=cg) for _ in range(layers)]
    sl = torch.tensor([T0], dtype=torch.int32, device="cuda")
    qbuf = torch.empty_like(qs[0])
    for t in range(warm):
        sl += 1
        loop(planners, t, qs[t], sl)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        sl += 1
        outs = loop(planners, warm, qbuf, sl)
    for t in range(warm, steps):
        qbuf.copy_(qs[t])
        g.replay()
        torch.cuda.synchronize()
        assert int(sl.item()) == T0 + t + 1
        for l in range(layers):
            assert torch.equal(outs[l], ref_out[t][l]), (t, l)
            for k in STATE:
                assert torch.equal(planners[l].state[k], ref_state[t][l][k]), (t, l, k)
            o_ref, read, trig, margin = ref_orc[t][l]
            same_decisions(planners[l].read_mask(read.shape[-1]).cpu(), read, trig,
                           planners[l].state["trig"].bool().cpu(), margin, (t, l))
            rel_ok(outs[l], o_ref, (t, l))
    if carried:                  # the last replay's final update (the graph's tail holds it pending)
        ce.flush()
        cg.flush()
        torch.cuda.synchronize()
        for l in range(layers):
            for k in STATE:
                assert torch.equal(planners[l].state[k], eager[l].state[k]), ("final", l, k)


def test_refresh_mode_steps_in_a_graph(gpu):
    """The refresh mode (PostPlanner) captured: four decode steps of two layers in one HIP graph
    (each step's length in its launches), replayed three times from the same saved state with eager
    work and synchronisations between the replays; every replay must give the eager loop's outputs
    and final state bit for bit (no memset nodes: the passes and the merge write every byte they
    hand on)."""
    from kvskip_amd import kvskip as K
    from kvskip_amd.planner import PostPlanner

    layers, T0, warm, n = 2, 3000, 5, 4
    steps = warm + n
    run = W.planner_run(layers=layers, B=1, Hq=32, Hkv=8, D=128, T0=T0, steps=steps, seed=37)
    ks = [k.cuda() for k in run.k]
    vs = [v.cuda() for v in run.v]
    qps = [W.QueryProcess(run, l, p_jump=0.2) for l in range(layers)]
    qs = torch.stack([torch.stack([qps[l].next() for l in range(layers)]) for _ in range(steps)]).cuda()
    pol = Policy(delta=0.01, max_age=3)

    def step(planners, t):
        T = T0 + t + 1
        return [planners[l].step(qs[t][l], ks[l][:, :, :T], vs[l][:, :, :T], run.scale) for l in range(layers)]

    eager = [PostPlanner(pol, count=False) for _ in range(layers)]
    ref, refreshed = [], 0
    for t in range(steps):
        ref.append([o.clone() for o in step(eager, t)])
        if t >= warm:
            refreshed += sum(int(p.state["trig"].sum()) for p in eager)
    assert 0 < refreshed < n * layers * 8      # the captured steps refresh some heads and keep others
    keys = [k for k in eager[0].state if k != "part"]      # part: the scores pass's workspace

    planners = [PostPlanner(pol, count=False) for _ in range(layers)]
    for t in range(warm):
        step(planners, t)
    torch.cuda.synchronize()
    saved = [{k: p.state[k].clone() for k in keys} for p in planners]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        outs = [[o.clone() for o in step(planners, t)] for t in range(warm, steps)]
    torch.cuda.synchronize()
    for rep in range(3):
        for p, sv in zip(planners, saved):
            for k in keys:
                p.state[k].copy_(sv[k])
        K.decode(qs[0][0], ks[0], vs[0], run.scale)       # the program's own eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, t in enumerate(range(warm, steps)):
            for l in range(layers):
                assert torch.equal(outs[i][l], ref[t][l]), (rep, t, l)
        for l in range(layers):
            for k in keys:
                assert torch.equal(planners[l].state[k], eager[l].state[k]), (rep, l, k)
