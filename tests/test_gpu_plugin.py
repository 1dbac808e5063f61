"""GPU: the attention plugin's decode modes (kvskip_amd.attention.kvskip_attention_forward, the
reference's src/kvskip_attn.py:481-515) driven the way a model drives them: one call per layer per
step on the growing cache's strided views. Each mode is checked against the CPU oracle of the
reference's semantics on the same inputs: dense against exact attention, vskip2 against the oracle's
two-pass V-skip, vskip1 / vskip1sink against the oracle's keep rule (V blocks read per KV head) and
output, refresh_fused against the oracle's refresh_pre loop (read sets and refresh decisions
identical on every head-step, outputs within 2e-3), replay against exact attention over the
recorded lists. Besides, each mode gives what its kernels give when called directly (the same
launches: bit for bit), and the refresh loop with carried updates the same lists as without."""

from dataclasses import replace
from types import SimpleNamespace

import pytest
import torch

from kvskip_amd import attention as A
from kvskip_amd import kvskip as K
from kvskip_amd.planner import FusedPlanner
from oracle import attention as O
from oracle_side import LayerOracle, oracle_policy, rel_ok, same_decisions

pytestmark = pytest.mark.gpu

LAYERS, B, HQ, HKV, D, T0, STEPS = 3, 1, 16, 4, 128, 1500, 6
SCALE = D ** -0.5


def _data(seed):
    """Per layer: a prefix K/V [B, Hkv, T0, D] with a few hot blocks, the appended rows and the
    queries of every step; token ids with repeats for the index heads."""
    g = torch.Generator().manual_seed(seed)
    T = T0 + STEPS
    ks, vs, qs = [], [], []
    for _ in range(LAYERS):
        k = torch.randn(B, HKV, T, D, generator=g)
        qd = torch.randn(B, HKV, 1, D, generator=g)
        for blk in torch.randint(1, T0 // 64, (3,), generator=g).tolist():
            k[:, :, blk * 64:(blk + 1) * 64] += 0.4 * qd
        ks.append(k.to(torch.bfloat16).cuda())
        vs.append(torch.randn(B, HKV, T, D, generator=g).to(torch.bfloat16).cuda())
        qs.append([(qd.repeat_interleave(HQ // HKV, 1) + 0.3 * torch.randn(B, HQ, 1, D, generator=g))
                   .to(torch.bfloat16).cuda() for _ in range(STEPS)])
    ids = torch.randint(0, 50, (B, T), generator=g, dtype=torch.int32).cuda()
    return ks, vs, qs, ids


def _drive(cfg, ks, vs, qs, ids=None, after=None):
    """Run the plugin over every layer and step (cache appends included); outputs [step][layer].
    after(t, l, out): called after each layer's call with its output [B, Hq, D]."""
    A.KVSKIP = cfg
    cache = A.GrowingCache(capacity=T0 + 64)
    mods = [SimpleNamespace(layer_idx=l) for l in range(LAYERS)]
    for l in range(LAYERS):
        cache.update(ks[l][:, :, :T0 - 1], vs[l][:, :, :T0 - 1], l)
    outs = []
    for t in range(STEPS):
        row = []
        n = T0 + t
        if ids is not None:
            cfg.ids = ids[:, :n].contiguous()
        for l in range(LAYERS):
            kk, vv = cache.update(ks[l][:, :, n - 1:n], vs[l][:, :, n - 1:n], l)
            o, _ = A.kvskip_attention_forward(mods[l], qs[l][t], kk, vv, None, scaling=SCALE)
            assert o.shape == (B, 1, HQ, D)
            row.append(o[:, 0].clone())
            if after is not None:
                after(t, l, row[-1])
        outs.append(row)
    cfg.flush()
    return outs, cache


def test_dense_and_vskip_modes_match_direct_calls_and_oracle():
    ks, vs, qs, _ = _data(31)
    for mode in ("dense", "vskip2", "vskip1", "vskip1sink"):
        outs, cache = _drive(A.KvskipConfig(mode=mode, dense_layers=(), count=False), ks, vs, qs)
        lse = [None] * LAYERS
        for t in range(STEPS):
            n = T0 + t
            for l in range(LAYERS):
                k, v = cache.layers[l]._kbuf[:, :, :n], cache.layers[l]._vbuf[:, :, :n]
                q = qs[l][t][:, :, 0]
                qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
                if mode == "dense":
                    ref = K.decode(q, k, v, SCALE)["out"]
                    rel_ok(outs[t][l], O.decode(qc, kc, vc, SCALE)[0], (mode, t, l))
                elif mode == "vskip2":
                    ref = K.vskip_two_pass(q, k, v, SCALE, rule="topp", value=0.99, local=2, sync=False)["out"]
                    # the oracle's selection on its own statistics: identical sets unless a top-p cut is a
                    # float32 near tie (checked), then exact attention over the kept set
                    M, S = O.block_stats(qc, kc, SCALE)
                    _, margin = O.topp_heads(O.block_logw(M, S), 0.99)
                    assert float(margin.min()) > 1e-6, (mode, t, l, float(margin.min()))
                    rel_ok(outs[t][l], O.vskip_two_pass(qc, kc, vc, SCALE, "topp", 0.99, 2)[0], (mode, t, l))
                else:
                    prev = lse[l] if mode == "vskip1" else None
                    r = K.vskip_one_pass(q, k, v, SCALE, tau=1e-4, local=2, lse_prev=prev, sync=False, count=True)
                    lse[l] = r["lse"]
                    ref = r["out"]
                    o_ref, _, keep, cnt = O.vskip1(qc, kc, vc, SCALE, 1e-4, 2,
                                                   lse_prev=None if prev is None else prev.cpu().double())
                    _, z = O.vskip1_keep(qc, kc, SCALE, 1e-4, 2, lse_prev=None if prev is None else prev.cpu().double())
                    assert float(z.abs().min()) > 1e-5, (mode, t, l)        # no vote at float32 noise
                    assert torch.equal(r["v_tiles"].cpu(), cnt), (mode, t, l)
                    rel_ok(outs[t][l], o_ref, (mode, t, l))
                assert torch.equal(outs[t][l], ref), (mode, t, l)


@pytest.mark.parametrize("index", [False, True])
def test_refresh_fused_matches_planner_loop(index):
    """refresh_fused without carried updates is FusedPlanner's own loop (layer 0 dense); with them,
    the same block lists and triggers on every step and outputs within the merge's summation order."""
    ks, vs, qs, ids = _data(32)
    kw = dict(calib=0.05, calib_kind="peak", calib_warm=(4, 2), dense_heads=((2, 1),))
    if index:
        kw.update(index_heads=((1, 2),), calib_auto_ix=0.1)
    cfg = A.KvskipConfig(mode="refresh_fused", carry=False, count=False, record=True, **kw)
    outs, _ = _drive(cfg, ks, vs, qs, ids if index else None)
    plain_state = {l: cfg.state[l]["planner"].state for l in range(1, LAYERS)}
    masks = cfg.plans

    # the oracle's refresh_pre loop on the same inputs (layer 0 dense): identical decisions
    orc = {l: LayerOracle(oracle_policy(cfg.policy(l)), SCALE) for l in range(1, LAYERS)}
    ids_c = ids.cpu().numpy()
    for t in range(STEPS):
        n = T0 + t
        for l in range(LAYERS):
            qc, kc, vc = qs[l][t][:, :, 0].cpu(), ks[l][:, :, :n].cpu(), vs[l][:, :, :n].cpu()
            if l == 0:
                rel_ok(outs[t][l], O.decode(qc, kc, vc, SCALE)[0], (t, l))
                continue
            o_ref, read, trig, margin = orc[l].step(qc, kc, vc, ids_c)
            same_decisions(masks[l][t].cpu(), read, trig, trig, margin, (t, l))   # a refresh reads every block
            rel_ok(outs[t][l], o_ref, (t, l))

    fps = {l: FusedPlanner(cfg.policy(l), count=False) for l in range(1, LAYERS)}
    for t in range(STEPS):
        n = T0 + t
        for l in range(LAYERS):
            k, v = ks[l][:, :, :n], vs[l][:, :, :n]
            q = qs[l][t][:, :, 0]
            if l == 0:
                ref = K.decode(q, k, v, SCALE)["out"]
            elif t == 0:
                ref = fps[l].first(q, k, v, SCALE)
            else:
                ref = fps[l].step(q, k, v, SCALE, ids=ids[:, :n].contiguous() if index else None)
            assert torch.equal(outs[t][l], ref), (t, l)
    for l in range(1, LAYERS):
        for key in ("block_idx", "block_cnt", "trig", "age", "keep", "lse_att", "calib", "aix"):
            assert torch.equal(plain_state[l][key], fps[l].state[key]), (l, key)

    cfg2 = A.KvskipConfig(mode="refresh_fused", carry=True, count=False, record=True, **kw)
    outs2, _ = _drive(cfg2, ks, vs, qs, ids if index else None)
    for t in range(STEPS):
        for l in range(1, LAYERS):
            assert torch.equal(masks[l][t], cfg2.plans[l][t]), (t, l)
            a, b = outs[t][l].float(), outs2[t][l].float()
            assert ((a - b).norm() / a.norm()).item() <= 1e-6, (t, l)
    for l in range(1, LAYERS):
        for key in ("block_idx", "block_cnt", "trig", "age", "keep", "lse_att", "calib", "aix"):
            assert torch.equal(plain_state[l][key], cfg2.state[l]["planner"].state[key]), (l, key)


def test_refresh_mode_matches_oracle():
    """Mode "refresh" (the trigger after the masked pass, src/kvskip_attn.py:215-270) against the
    oracle's loop of that mode on the same inputs (layer 0 dense): refresh decisions and read sets
    (the attended set from the device's previous stored set, plus every block of a refreshing head)
    identical on every head-step, the refresh pass's lists the blocks outside a refreshing head's
    attended set and none of the others' blocks, stored sets identical after each step, outputs within
    2e-3; the device counters add up the blocks of both passes (src/kvskip_attn.py:256,269), each
    block once. The config also sets calibration, warm-up and token-index fields, which the reference's
    refresh_step does not read (src/kvskip_attn.py:215-270): the mode runs as without them. Then the
    same with the updates carried by the next layer's pass: the same triggers, outputs and final state."""
    ks, vs, qs, _ = _data(35)
    kw = dict(mode="refresh", count=True, delta=0.02, max_age=4, dense_heads=((2, 1),), calib=0.05,
              calib_kind="peak", calib_warm=(8, 2), calib_auto_ix=0.1)
    cfg = A.KvskipConfig(carry=False, **kw)
    ignored = dict(calib=None, calib_warm=(), calib_auto_ix=None, index_heads=(), index_union=False)
    orc = {l: LayerOracle(oracle_policy(replace(cfg.policy(l), **ignored)), SCALE, post=True) for l in range(1, LAYERS)}
    prev_keep, orc_trig = {}, {}
    seen = dict(refresh=0, kept=0, read=0)

    def check(t, l, out):
        n = T0 + t
        qc, kc, vc = qs[l][t][:, :, 0].cpu(), ks[l][:, :, :n].cpu(), vs[l][:, :, :n].cpu()
        if l == 0:
            rel_ok(out, O.decode(qc, kc, vc, SCALE)[0], (t, l))
            return
        o_ref, read, trig, margin = orc[l].step(qc, kc, vc)
        rel_ok(out, o_ref, (t, l))
        st = cfg.state[l]["post"].state
        nb = O.nblocks(n)
        if t > 0:
            dev_trig = st["trig"].bool().cpu()
            orc_trig[t, l] = trig
            sel = torch.nn.functional.pad(prev_keep[l], (0, nb - prev_keep[l].shape[-1])) | O.always_keep(nb, cfg.local)
            same_decisions(sel | dev_trig[..., None], read, trig, dev_trig, margin, (t, l))
            rest = nb - sel.sum(-1)          # a refreshing head's blocks outside its attended set
            assert torch.equal(st["block_cnt"].cpu(), torch.where(trig, rest, 0).to(torch.int32)), (t, l)
            seen["refresh"] += int(trig.sum())
            seen["kept"] += int((~trig).sum())
            # the masked pass's blocks, then the refresh pass's (the reference counts a refreshing
            # head's attended blocks again, since its refresh pass reads them again)
            seen["read"] += int(sel.sum()) + int(torch.where(trig, rest, 0).sum())
        else:
            seen["read"] += int(read.sum())
        prev_keep[l] = st["keep"][:, :, :nb].bool().cpu()
        assert torch.equal(prev_keep[l], orc[l].st.keep), (t, l)

    outs, _ = _drive(cfg, ks, vs, qs, after=check)
    assert seen["refresh"] > 0 and seen["kept"] > 0, seen
    assert int(A.log_totals()["blocks_read"]) == seen["read"], (A.log_totals(), seen)

    # with each layer's update carried by the next layer's first pass: the same triggers on every
    # step, the same outputs (within the merge's summation order) and the same final state
    trigs = {}

    def record(t, l, out):
        if l > 0:
            trigs[t, l] = cfg2.state[l]["post"].state["trig"].clone()

    cfg2 = A.KvskipConfig(carry=True, **kw)
    outs2, _ = _drive(cfg2, ks, vs, qs, after=record)
    for t in range(STEPS):
        for l in range(1, LAYERS):
            if t > 0:
                assert torch.equal(trigs[t, l].bool().cpu(), orc_trig[t, l]), (t, l)
            a, b = outs[t][l].float(), outs2[t][l].float()
            assert ((a - b).norm() / a.norm()).item() <= 1e-6, (t, l)
    for l in range(1, LAYERS):
        for key in ("keep", "lse_ref", "cs_ref", "age", "trig"):
            assert torch.equal(cfg.state[l]["post"].state[key], cfg2.state[l]["post"].state[key]), (l, key)


def test_replay_of_recorded_lists():
    """replay: the masked + statistics decode over the lists recorded by refresh_fused gives that
    run's outputs (split count may differ: within 2e-3 relative) and exact attention over those
    lists (the oracle)."""
    ks, vs, qs, _ = _data(33)
    cfg = A.KvskipConfig(mode="refresh_fused", count=False, record=True)
    outs, _ = _drive(cfg, ks, vs, qs)
    plans = {l: [K.make_plan(m) for m in cfg.plans[l]] for l in cfg.plans}
    assert sorted(plans) == list(range(1, LAYERS)) and all(len(p) == STEPS for p in plans.values())
    cfg_r = A.KvskipConfig(mode="replay", count=False, plans=plans)
    outs_r, _ = _drive(cfg_r, ks, vs, qs)
    for t in range(STEPS):
        n = T0 + t
        for l in range(LAYERS):
            a, b = outs[t][l].float(), outs_r[t][l].float()
            assert ((a - b).norm() / a.norm()).item() <= 2e-3, (t, l)
            keep = cfg.plans[l][t].cpu() if l in cfg.plans else None
            ref, _ = O.decode(qs[l][t][:, :, 0].cpu(), ks[l][:, :, :n].cpu(), vs[l][:, :, :n].cpu(), SCALE, keep=keep)
            rel_ok(outs_r[t][l], ref, (t, l))


def test_counters():
    """Per-layer counters as device tensors; log_totals sums them (blocks read <= blocks total)."""
    ks, vs, qs, _ = _data(34)
    cfg = A.KvskipConfig(mode="refresh_fused", count=True)
    _drive(cfg, ks, vs, qs)
    tot = A.log_totals()
    assert tot["blocks_total"] > 0 and 0 < tot["blocks_read"] <= tot["blocks_total"]
    assert tot["dense_heads"] >= (LAYERS - 1) * B * HKV                     # the first step reads everything
    cfg = A.KvskipConfig(mode="vskip1", dense_layers=(), count=True)
    _drive(cfg, ks, vs, qs)
    tot = A.log_totals()
    assert 0 < tot["v_tiles"] <= tot["blocks_total"]
