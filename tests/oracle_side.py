"""Helpers for GPU tests that run the CPU oracle beside the device on the same inputs: the oracle's
refresh_pre loop of one layer and sequence, page gathering, and the decision comparison."""

from __future__ import annotations

import math

import numpy as np
import torch

from oracle import attention as O
from oracle import planner as OP

REL = 2e-3          # bf16 output against the fp64 oracle, relative L2


def oracle_policy(policy) -> OP.Policy:
    """The oracle's Policy of a kvskip_amd.planner.Policy (same fields)."""
    return OP.Policy(**policy.__dict__)


def gather_pages(pool: torch.Tensor, table: torch.Tensor, lens) -> list[torch.Tensor]:
    """Per sequence b: the [1, Hkv, lens[b], D] rows its block-table row addresses in a page pool
    [P, Hkv, 64, D], gathered on the CPU."""
    pool, table = pool.cpu(), table.cpu()
    out = []
    for b, n in enumerate(lens):
        pages = [int(table[b, j]) for j in range(math.ceil(n / 64))]
        rows = torch.cat([pool[p] for p in pages], dim=1)[:, :n]
        out.append(rows[None])
    return out


class LayerOracle:
    """The oracle's refresh_pre loop (OP.init, then OP.step) for one layer of one sequence; with
    post, the refresh mode's loop (OP.init, then OP.post_step)."""

    def __init__(self, policy: OP.Policy, scale: float, post: bool = False):
        self.pol, self.scale, self.st, self.post = policy, scale, None, post

    def step(self, q, k, v, ids=None):
        """q [1, Hq, D], k / v [1, Hkv, T, D] (CPU), ids [1, >= T] token ids (index heads / auto index).
        Returns (out [1, Hq, D] fp64, read [1, Hkv, nb] bool, trig [1, Hkv] bool, margin [1, Hkv])."""
        T = k.shape[2]
        if self.st is None:
            self.st, out = OP.init(q, k, v, self.scale, self.pol)
            Hkv = k.shape[1]
            return (out, torch.ones(1, Hkv, O.nblocks(T), dtype=torch.bool), torch.ones(1, Hkv, dtype=torch.bool),
                    torch.full((1, Hkv), math.inf, dtype=torch.float64))
        if self.post:
            out, pr = OP.post_step(self.st, q, k, v, self.pol)
            return out, pr["read"], pr["trig"], pr["margin"]
        idx = None if ids is None else torch.from_numpy(OP.index_blocks(np.asarray(ids)[:, :T], T))
        out, pr = OP.step(self.st, q, k, v, self.pol, idx=idx)
        return out, pr["read"], pr["trig"], pr["margin"]


def same_decisions(dev_read, ref_read, ref_trig, dev_trig, margin, what):
    """Read sets [.., Hkv, nb] and refresh decisions [.., Hkv] must be identical; the message names the
    oracle's margins of the heads that differ."""
    diff = (dev_read != ref_read).any(-1) | (dev_trig != ref_trig)
    if bool(diff.any()):
        where = torch.nonzero(diff).tolist()
        raise AssertionError(f"{what}: heads {where} differ; oracle margins "
                             f"{[float(margin[tuple(i)]) for i in where]}")


def rel_ok(out, ref, what):
    err = O.rel_err(out.double().cpu(), ref)
    assert err <= REL, (what, err)
    return err
