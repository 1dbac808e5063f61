"""The HIP path against the committed golden fixtures (tests/golden/*.npz, oracle outputs on small
seeded cases): dense / masked attention with block statistics, top-p selection on the device's
statistics, single-pass V-skip decisions, and eight steps of the device planner loop."""

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from kvskip_amd import ext as E
from kvskip_amd import kvskip as K
from kvskip_amd.planner import FusedPlanner, Policy
from oracle import attention as O

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
REL, LSE_TOL = 2e-3, 2e-4


def _bf16(a):
    return torch.from_numpy(np.ascontiguousarray(a)).view(torch.bfloat16).cuda()


def test_attention_golden(gpu):
    d = np.load(GOLDEN / "attention_small.npz", allow_pickle=False)
    q, k, v = _bf16(d["q"]), _bf16(d["k"]), _bf16(d["v"])
    scale = float(d["scale"])
    G = q.shape[1] // k.shape[1]
    for S in (1, 4):
        out, lse, bmax, bsum, _, _ = E.decode(q, k, v, scale, None, None, True, True, S, 2, False, False)
        assert O.rel_err(out.float().cpu(), torch.from_numpy(d["out"])) <= REL
        assert np.abs(lse.cpu().double().numpy() - d["lse"]).max() <= LSE_TOL
        assert np.abs(bmax.cpu().double().numpy() - d["blk_max"]).max() <= LSE_TOL
        assert np.abs(bsum.cpu().double().numpy() / d["blk_sum"] - 1).max() <= 2e-4
    # masked list + statistics
    plan = K.make_plan(torch.from_numpy(d["keep"]).cuda())
    r = K.decode(q, k, v, scale, plan=plan, stats=True, num_splits=3)
    assert O.rel_err(r["out"].float().cpu(), torch.from_numpy(d["masked_out"])) <= REL
    fin = np.isfinite(d["masked_blk_max"])
    assert np.array_equal(np.isfinite(r["blk_max"].cpu().numpy()), fin)
    assert np.abs(r["blk_max"].cpu().double().numpy()[fin] - d["masked_blk_max"][fin]).max() <= LSE_TOL
    # top-p (0.9) union on the device's statistics
    logw = (bmax + torch.log(bsum))
    keep = K.select_blocks(logw, G, "topp", 0.9, local=1).cpu().numpy()
    _, margin = O.topp_heads(torch.from_numpy(d["blk_max"]) + torch.log(torch.from_numpy(d["blk_sum"])), 0.9)
    assert np.array_equal(keep, d["topp_keep"]), f"top-p sets differ (oracle margins {margin.min():.2e} and up)"
    # single-pass V-skip: V blocks read per (b, KV head)
    lp = torch.from_numpy(d["lse_prev"]).float().cuda()
    res = K.vskip_one_pass(q, k, v, scale, tau=0.02, local=1, count=True, lse_prev=lp, num_splits=2, keep=True)
    assert np.abs(d["vskip_margin"]).min() > 1e-3
    assert np.array_equal(res["v_keep"].cpu().numpy(), d["vskip_keep"])
    assert np.array_equal(res["v_tiles"].cpu().numpy(), d["vskip_keep"].sum(-1))


def test_planner_golden(gpu):
    d = np.load(GOLDEN / "planner_small.npz", allow_pickle=False)
    k, v = _bf16(d["k"]), _bf16(d["v"])
    ids = torch.from_numpy(d["ids"]).cuda()
    T0, scale = int(d["T0"]), float(d["scale"])
    fp = FusedPlanner(Policy(calib=0.05, calib_kind="peak", calib_warm=(4, 2), calib_auto_ix=0.1))
    steps = d["q"].shape[0]
    nbc = d["read"].shape[-1]
    for t in range(steps):
        T = T0 + t + 1
        q = _bf16(d["q"][t])
        if t == 0:
            out = fp.first(q, k[:, :, :T], v[:, :, :T], scale)
        else:
            out = fp.step(q, k[:, :, :T], v[:, :, :T], scale, ids=ids)
        read = fp.read_mask(math.ceil(T / 64)).cpu().numpy()
        ref = d["read"][t][..., :read.shape[-1]]
        assert np.array_equal(read, ref), f"read set at step {t} (oracle margins {d['margin'][t].tolist()})"
        assert np.array_equal(fp.state["trig"].bool().cpu().numpy(), d["trig"][t])
        assert O.rel_err(out.float().cpu(), torch.from_numpy(d["out"][t])) <= REL, t
    assert np.abs(fp.state["calib"].cpu().double().numpy() - d["calib"]).max() <= 1e-4
    assert np.array_equal(fp.state["aix"].bool().cpu().numpy(), d["aix"])
