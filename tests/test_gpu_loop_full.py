"""The device planner loop at the full sizes of configs 4 and 5 against the oracle's refresh_pre
loop, frozen in tests/golden/planner_cfg4.npz / planner_cfg5.npz (written by
tests/golden/make_golden.py full from the pinned oracle). The inputs are regenerated from their seeds
on the CPU and checked against the fixture's digest first.

Config 4: B 1, 32 / 8 heads, D 128, T 32768 -> 32895 over 128 steps, query drift with 3% jumps,
stage-4 policy; the two planned layers run as in a model loop (each layer's update carried by the
next layer's pass, the plan's decision inside the pass, the token index found by the plan from the
ids). Config 5: B 16 ragged contexts in [4096, 65536], 28 / 4 heads (G 7), 64 steps, one layer.

Per step and (sequence, KV head), as bench/test_planner.py:100-133 compares them but with every
head-step required: identical read sets and refresh decisions; the estimate within 1e-4; after
the update, identical stored sets and index latches, calibration within 1e-4, attended
log-sum-exp within 1e-3; outputs: checksums (projections on unit vectors and norms) within 2e-3 of
the norm per query head, whole outputs every 64 steps within 2e-3 relative L2 (bf16).

A free-running loop cannot be identical on every head-step: the top-p cut of a refresh lands
within 1e-6 of the level on a few percent of refreshes here (the mass past the first blocks is
spread over hundreds of tiny blocks), below the float32 noise of the device's sums. So each KV head
is tracked as in sync (device state = oracle state) or not. While in sync every decision must be
identical, and a difference is allowed only where the oracle's own margin for that decision is
below NEAR (2e-6: |estimate - delta| for a refresh, the cut's distance from the level for a stored
set, |correction - threshold| for a latch); anything else fails. The head then leaves sync and
rejoins at the next step where both refresh it and its stored set, latch and correction agree
again (a refresh replaces the rest of its state). Printed: agreement of read sets over all
head-steps (>= 0.995; the reference's criterion is >= 0.97, bench/test_planner.py:133), the in-sync
share (>= 0.995), every near-tie event with its margin (at most MAX_NEAR per config), and the
smallest margins compared in sync. Outputs, estimates
and continuous state are checked on in-sync heads."""

import importlib.util
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from kvskip_amd.planner import FusedPlanner, Policy, UpdateCarrier
from oracle import attention as O

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
REL = 2e-3
NEAR = 2e-6            # an oracle margin below this is a float32 near tie (measured departures: 2.7e-7, 3.2e-7)
MIN_AGREE = 0.995      # the reference's own criterion is 0.97 (bench/test_planner.py:133); measured >= 0.9985
MIN_SYNC = 0.995       # measured >= 0.9983
MAX_NEAR = 2           # near-tie departures allowed per config (measured: 1 each)
AIX_THR = 0.1          # the stage-4 policy's latch threshold


def _maker():
    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _bits(a, nb):
    return np.unpackbits(a, axis=-1, count=a.shape[-1] * 8)[..., :nb].astype(bool)


class Checker:
    """Compares one (layer or sequence) record stream of the fixture with the device."""

    def __init__(self, d, part, G, u, name):
        self.d, self.part, self.G, self.u, self.name = d, part, G, u, name
        self.margin = math.inf      # smallest refresh-decision margin compared in sync
        self.topp = math.inf        # smallest top-p margin of a refresh compared in sync
        self.head_steps = self.agree = self.in_sync = 0
        self.near = []              # (step, KV head, what, oracle margin) where a head left sync
        self.rejoin = []            # (step, KV head) where it came back
        self.off = set()            # KV heads out of sync
        self.trig = None            # the device's decisions of the current step

    def _near_tie(self, t, h, what, margin):
        assert margin < NEAR, (f"{self.name} step {t} KV head {h}: {what} differs with oracle margin {margin:.3e} "
                               f"(>= {NEAR:g}: not a float32 near tie)")
        self.near.append((t, h, what, float(margin)))
        self.off.add(h)

    def _on(self, Hkv):
        return np.array([h not in self.off for h in range(Hkv)])

    def decision(self, t, read, trig, est, out):
        """read [Hkv, nb] bool, trig [Hkv] bool, est [Hkv], out [Hq, D] float (device, host copies)."""
        d, p, G = self.d, self.part, self.G
        Hkv, nb = read.shape
        ref_read = _bits(d["read"][p, t], nb)
        ref_trig = d["trig"][p, t]
        m = d["margin"][p, t]
        self.trig = trig.copy()
        same = ~(read != ref_read).any(-1)
        self.head_steps += Hkv
        self.agree += int(same.sum())
        for h in range(Hkv):
            if h in self.off:
                continue
            if trig[h] != ref_trig[h]:
                self._near_tie(t, h, "refresh decision", m[h])
            elif not same[h]:
                raise AssertionError(f"{self.name} step {t} KV head {h}: in sync, same decision, different read set")
        on = self._on(Hkv)
        self.in_sync += int(on.sum())
        fin = on & np.isfinite(m)
        if fin.any():
            self.margin = min(self.margin, float(m[fin].min()))
        if t > 0 and on.any():
            assert np.abs(est - d["miss"][p, t])[on].max() <= 1e-4, (self.name, t)
        hq = np.repeat(on, G)
        proj = out.double() @ self.u
        nrm = out.double().norm(dim=-1)
        ref_n = torch.from_numpy(d["norm"][p, t]).double()
        tol = REL * ref_n + 1e-6
        assert ((proj - torch.from_numpy(d["proj"][p, t]).double()).abs() <= tol[:, None])[hq].all(), (self.name, t)
        assert ((nrm - ref_n).abs() <= tol)[hq].all(), (self.name, t)
        fs = list(d["full_steps"])
        if t in fs and hq.any():
            ref = torch.from_numpy(d["out_full"][p, fs.index(t)]).double()
            assert O.rel_err(out[hq], ref[hq]) <= REL, (self.name, t)

    def after_update(self, t, keep, calib, aix, lse_att):
        """The state the step's update left: keep [Hkv, >= nb] bool, calib / aix [Hkv], lse_att [Hq]."""
        d, p, G = self.d, self.part, self.G
        Hkv = calib.shape[0]
        nb = O.nblocks(int(d["T0"][0 if d["T0"].size == 1 else p]) + t + 1)
        ref_keep = _bits(d["keep"][p, t], nb)
        for h in range(Hkv):
            same_keep = not (keep[h, :nb] != ref_keep[h]).any()
            same_aix = aix[h] == d["aix"][p, t, h]
            if h in self.off:
                # a common refresh replaces references, stored set and age: back in sync when the
                # stored set, the latch and the correction agree again
                if (self.trig[h] and d["trig"][p, t, h] and same_keep and same_aix
                        and abs(calib[h] - d["calib"][p, t, h]) <= 1e-4):
                    self.off.discard(h)
                    self.rejoin.append((t, h))
                continue
            if not same_keep:
                self._near_tie(t, h, "stored set", d["topp"][p, t, h])
            elif not same_aix:
                self._near_tie(t, h, "index latch", abs(float(d["calib"][p, t, h]) - AIX_THR))
        on = self._on(Hkv)
        if on.any():
            assert np.abs(calib - d["calib"][p, t])[on].max() <= 1e-4, (self.name, t)
            assert np.abs(lse_att - d["lse_att"][p, t])[np.repeat(on, G)].max() <= 1e-3, (self.name, t)
        tp = d["topp"][p, t][d["trig"][p, t] & on]
        if tp.size:
            self.topp = min(self.topp, float(tp.min()))

    def report(self):
        return (f"{self.name}: read sets identical on {self.agree}/{self.head_steps} head-steps, in sync "
                f"{self.in_sync}/{self.head_steps}; smallest margins in sync: decision {self.margin:.2e}, top-p "
                f"{self.topp:.2e}; left sync at near ties (step, KV head, what, oracle margin) {self.near}; "
                f"rejoined {self.rejoin}")


def _summary(chks, what):
    agree = sum(c.agree for c in chks) / sum(c.head_steps for c in chks)
    sync = sum(c.in_sync for c in chks) / sum(c.head_steps for c in chks)
    n_near = sum(len(c.near) for c in chks)
    print(f"{what}: read sets identical on {agree:.4f} of head-steps, in sync {sync:.4f}, {n_near} near-tie "
          f"departures (all with oracle margin < {NEAR:g})", flush=True)
    assert agree >= MIN_AGREE and sync >= MIN_SYNC and n_near <= MAX_NEAR, (agree, sync, n_near)


def _state(fp):
    """keep, calib, aix, lse_att of sequence 0 (host copies)."""
    s = fp.state
    return (s["keep"].cpu().numpy()[0].astype(bool), s["calib"].cpu().numpy()[0],
            s["aix"].cpu().numpy()[0].astype(bool), s["lse_att"].cpu().numpy()[0])


def test_planner_loop_config4(gpu):
    mk = _maker()
    d = np.load(GOLDEN / "planner_cfg4.npz", allow_pickle=False)
    run, layers, qs = mk.loop_inputs(4)
    assert mk.input_digest(run, layers, qs) == str(d["digest"]), "regenerated config-4 inputs differ"
    steps, T0 = run.steps, run.T0[0]
    G = qs[layers[0]][0].shape[1] // run.k[layers[0]].shape[1]
    u = mk.proj_dirs(run.k[layers[0]].shape[3])
    pol = Policy(**mk.stage4().__dict__)
    carrier = UpdateCarrier()
    fps = {l: FusedPlanner(pol, count=False, carrier=carrier) for l in layers}
    chk = {l: Checker(d, i, G, u, f"config 4 layer {l}") for i, l in enumerate(layers)}
    kv = {l: (run.k[l].cuda(), run.v[l].cuda()) for l in layers}
    ids = run.ids.cuda()
    print(f"config 4: layers {layers}, {steps} steps from T {T0}", flush=True)
    for t in range(steps):
        T = T0 + t + 1
        for i, l in enumerate(layers):
            k, v = kv[l][0][:, :, :T], kv[l][1][:, :, :T]
            q = qs[l][t].cuda()
            out = fps[l].first(q, k, v, run.scale) if t == 0 else fps[l].step(q, k, v, run.scale, ids=ids)
            s = fps[l].state
            chk[l].decision(t, fps[l].read_mask(O.nblocks(T)).cpu().numpy()[0], s["trig"].bool().cpu().numpy()[0],
                            s["est"].cpu().numpy()[0], out.float().cpu()[0])
            # the update of the layer before has now run inside this layer's pass
            if i > 0:
                chk[layers[i - 1]].after_update(t, *_state(fps[layers[i - 1]]))
            elif t > 0:
                chk[layers[-1]].after_update(t - 1, *_state(fps[layers[-1]]))
    carrier.flush()
    chk[layers[-1]].after_update(steps - 1, *_state(fps[layers[-1]]))
    for l in layers:
        print(chk[l].report(), flush=True)
    _summary(list(chk.values()), "config 4")


def test_planner_loop_config5(gpu):
    mk = _maker()
    d = np.load(GOLDEN / "planner_cfg5.npz", allow_pickle=False)
    run, layers, qs = mk.loop_inputs(5)
    assert mk.input_digest(run, layers, qs) == str(d["digest"]), "regenerated config-5 inputs differ"
    steps, lens = run.steps, run.T0
    B = len(lens)
    G = qs[0][0].shape[1] // run.k[0].shape[1]
    u = mk.proj_dirs(run.k[0].shape[3])
    fp = FusedPlanner(Policy(**mk.stage4().__dict__), count=False)
    chk = [Checker(d, b, G, u, f"config 5 sequence {b}") for b in range(B)]
    k, v = run.k[0].cuda(), run.v[0].cuda()
    ids = run.ids.cuda()
    base = torch.tensor(lens, dtype=torch.int32)
    print(f"config 5: B {B}, contexts {min(lens)}..{max(lens)} (sum {sum(lens)}), {steps} steps", flush=True)
    for t in range(steps):
        sl = (base + t + 1).cuda()
        q = qs[0][t].cuda()
        out = fp.first(q, k, v, run.scale, seq_lens=sl) if t == 0 else fp.step(q, k, v, run.scale, ids=ids, seq_lens=sl)
        s = fp.state
        bi, bc = s["block_idx"].cpu(), s["block_cnt"].cpu()
        trig, est = s["trig"].bool().cpu().numpy(), s["est"].cpu().numpy()
        calib, aix, la = s["calib"].cpu().numpy(), s["aix"].cpu().numpy().astype(bool), s["lse_att"].cpu().numpy()
        keep = s["keep"].cpu().numpy().astype(bool)
        out = out.float().cpu()
        for b in range(B):
            nb = O.nblocks(lens[b] + t + 1)
            read = np.zeros((bi.shape[1], nb), dtype=bool)
            for h in range(bi.shape[1]):
                lst = bi[b, h, :int(bc[b, h])].numpy()
                assert (np.diff(lst) > 0).all() and (lst < nb).all(), (b, h, t)
                read[h, lst] = True
            chk[b].decision(t, read, trig[b], est[b], out[b])
            chk[b].after_update(t, keep[b], calib[b], aix[b], la[b])
    for c in chk:
        print(c.report(), flush=True)
    _summary(chk, "config 5")
