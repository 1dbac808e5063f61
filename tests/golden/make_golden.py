"""Writes the golden fixtures of this directory from the fp64 oracle (oracle/), whose functions are
pinned by tests/test_oracle.py (closed forms, brute force, library routines). The reference ships no
golden vectors for this path (its tests read gitignored KV dumps), so these are the oracle's outputs
on small seeded inputs, frozen: tests/test_golden.py checks that the oracle still reproduces them
(CPU), tests/test_gpu_golden.py that the HIP path matches them (GPU).

    python tests/golden/make_golden.py          # rewrites attention_small.npz, planner_small.npz
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle import attention as O  # noqa: E402
from oracle import planner as OP  # noqa: E402

SEED = 1234


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).view(torch.int16).numpy()


def from_bits(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(a).view(torch.bfloat16)


def attention_case() -> dict:
    """B 2, 8 / 2 heads (G 4), D 64, T 300 (a partial last block): dense, block statistics, a
    masked list, top-p selection, single-pass V-skip decisions."""
    g = torch.Generator().manual_seed(SEED)
    B, Hq, Hkv, D, T = 2, 8, 2, 64, 300
    q = torch.randn(B, Hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16)
    k[:, :, 64:128] += 0.5 * q.float().reshape(B, Hkv, 4, D).mean(2)[:, :, None].to(torch.bfloat16)
    scale = 0.125
    nb = O.nblocks(T)
    keep = torch.zeros(B, Hkv, nb, dtype=torch.bool)
    keep[0, 0, [0, 2, 4]] = True
    keep[0, 1, [1, 3]] = True
    keep[1, 0, [0, 1, 2, 3, 4]] = True
    keep[1, 1, [4]] = True
    out, lse = O.decode(q, k, v, scale)
    mout, mlse = O.decode(q, k, v, scale, keep=keep)
    M, S = O.block_stats(q, k, scale)
    mM, mS = O.block_stats(q, k, scale, keep=keep)
    logw = O.block_logw(M, S)
    sel = O.select_blocks(logw, 4, "topp", 0.9, local=1)
    lse_prev = lse + 0.02
    vkeep, vz = O.vskip1_keep(q, k, scale, 0.02, 1, lse_prev=lse_prev)
    return dict(q=bf16_bits(q), k=bf16_bits(k), v=bf16_bits(v), scale=np.float64(scale), keep=keep.numpy(),
                out=out.numpy(), lse=lse.numpy(), blk_max=M.numpy(), blk_sum=S.numpy(),
                masked_out=mout.numpy(), masked_lse=mlse.numpy(), masked_blk_max=mM.numpy(),
                masked_blk_sum=mS.numpy(), topp_keep=sel.numpy(), lse_prev=lse_prev.numpy(),
                vskip_keep=vkeep.numpy(), vskip_margin=vz.numpy())


def policy() -> OP.Policy:
    """Stage-4 policy with a short warm-up (first 4 steps: max age 2)."""
    return OP.Policy(calib=0.05, calib_kind="peak", calib_warm=(4, 2), calib_auto_ix=0.1)


def planner_case() -> dict:
    """B 1, 8 / 1 heads (G 8), D 64, T 2000 + 8 decode steps of the stage-4 policy with token ids:
    per step the query, the read set, the refresh decisions and margins, the attended output."""
    g = torch.Generator().manual_seed(SEED + 1)
    B, Hq, Hkv, D, T0, steps = 1, 8, 1, 64, 2000, 8
    k = torch.randn(B, Hkv, T0 + steps, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, T0 + steps, D, generator=g).to(torch.bfloat16)
    u = torch.randn(Hkv, D, generator=g)
    u = u / u.norm(dim=-1, keepdim=True)
    for h in range(Hkv):
        k[0, h, 64 * 5:64 * 6] += (8.0 * u[h]).to(torch.bfloat16)
        k[0, h, 64 * 11:64 * 12] += (8.0 * u[h]).to(torch.bfloat16)
    ids = torch.randint(0, 50, (B, T0 + steps), generator=g, dtype=torch.int32)
    pol = policy()
    q = (10.0 * u.repeat_interleave(Hq // Hkv, 0))[None] + torch.randn(B, Hq, D, generator=g)
    qs, reads, trigs, margins, outs = [], [], [], [], []
    st = None
    for t in range(steps):
        T = T0 + t + 1
        q = q + 0.25 * torch.randn(B, Hq, D, generator=g)
        if t == 4:
            q[0, 0] = -q[0, 0]                              # a jump: the estimate must fire
        qb = q.to(torch.bfloat16)
        qs.append(bf16_bits(qb))
        nb = O.nblocks(T)
        if t == 0:
            st, out = OP.init(qb, k[:, :, :T], v[:, :, :T], 0.125, pol)
            read = torch.ones(B, Hkv, nb, dtype=torch.bool)
            trig = torch.ones(B, Hkv, dtype=torch.bool)
            margin = torch.full((B, Hkv), np.inf, dtype=torch.float64)
        else:
            idx = torch.from_numpy(OP.index_blocks(ids.numpy(), T))
            out, pr = OP.step(st, qb, k[:, :, :T], v[:, :, :T], pol, idx=idx)
            read, trig, margin = pr["read"], pr["trig"], pr["margin"]
        pad = np.zeros((B, Hkv, O.nblocks(T0 + steps)), dtype=bool)
        pad[..., :nb] = read.numpy()
        reads.append(pad)
        trigs.append(trig.numpy())
        margins.append(margin.numpy())
        outs.append(out.numpy())
    return dict(k=bf16_bits(k), v=bf16_bits(v), ids=ids.numpy(), T0=np.int64(T0), scale=np.float64(0.125),
                q=np.stack(qs), read=np.stack(reads), trig=np.stack(trigs), margin=np.stack(margins),
                out=np.stack(outs), calib=st.calib.numpy(), aix=st.aix.numpy())


def main():
    np.savez_compressed(HERE / "attention_small.npz", **attention_case())
    np.savez_compressed(HERE / "planner_small.npz", **planner_case())
    for f in ("attention_small.npz", "planner_small.npz"):
        print(f, (HERE / f).stat().st_size, "bytes")


if __name__ == "__main__":
    main()
