"""Writes the golden fixtures of this directory from the fp64 oracle (oracle/), whose functions are
pinned by tests/test_oracle.py (closed forms, brute force, library routines). The reference ships no
golden vectors for this path (its tests read gitignored KV dumps), so these are the oracle's outputs
on small seeded inputs, frozen: tests/test_golden.py checks that the oracle still reproduces them
(CPU), tests/test_gpu_golden.py that the HIP path matches them (GPU).

    python tests/golden/make_golden.py          # rewrites attention_small.npz, planner_small.npz
    python tests/golden/make_golden.py full     # rewrites planner_cfg4.npz, planner_cfg5.npz (~3 min)
    python tests/golden/make_golden.py full 5   # only planner_cfg5.npz

The full-size fixtures run the oracle's refresh_pre loop on the workloads of BASELINE configs 4
and 5 (inputs regenerated from their seeds on the CPU by the tests, checked by a digest) and keep,
per decode step and (sequence, KV head): the read set, the refresh decision and its margin, the
stored set after the update and the top-p margin of a refresh, the estimate, the calibration, the
index latch; per query head the
attended log-sum-exp and output checksums (projections on seeded unit vectors and the norm), and
the whole output every 64 steps (and at the last).
"""

from __future__ import annotations

import hashlib
import math
import sys
import time
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


# ---------------------------------------------------------------- full-size planner loops

PROJ = 4              # output checksum: projections on PROJ seeded unit vectors, and the norm
FULL_EVERY = 64       # whole outputs kept every FULL_EVERY steps (and at the last step)


def stage4() -> OP.Policy:
    """The stage-4 policy of configs 4 and 5 (reproduce/04-tails.sh:16,63-69)."""
    return OP.Policy(calib=0.05, calib_kind="peak", calib_warm=(32, 8), calib_auto_ix=0.1)


def proj_dirs(D: int) -> torch.Tensor:
    u = torch.randn(D, PROJ, generator=torch.Generator().manual_seed(99), dtype=torch.float64)
    return u / u.norm(dim=0, keepdim=True)


def full_steps(steps: int) -> list[int]:
    return sorted(set(range(0, steps, FULL_EVERY)) | {steps - 1})


from kvskip_amd.workloads import cfg5_lens, input_digest, loop_inputs  # noqa: E402,F401  (fixture inputs)


def oracle_loop(k, v, qs, ids, T0, scale, pol, steps, b=0):
    """The oracle's refresh_pre loop for one sequence (row b of k / v / qs / ids, prefix T0, one
    token appended per step): per-step records (see the module docstring); read sets padded to the
    capacity of k."""
    kb, vb, idb = k[b:b + 1], v[b:b + 1], ids[b:b + 1].numpy()
    Hkv = kb.shape[1]
    G = qs[0].shape[1] // Hkv
    nbmax = O.nblocks(k.shape[2])
    u = proj_dirs(kb.shape[3])
    rec = {key: [] for key in ("read", "keep", "trig", "margin", "topp", "miss", "calib", "aix", "lse_att", "proj",
                               "norm")}
    full = []
    st = None
    for t in range(steps):
        T = T0 + t + 1
        q = qs[t][b:b + 1]
        if t == 0:
            st, out = OP.init(q, kb[:, :, :T], vb[:, :, :T], scale, pol)
            read = torch.ones(1, Hkv, O.nblocks(T), dtype=torch.bool)
            trig = torch.ones(1, Hkv, dtype=torch.bool)
            margin = torch.full((1, Hkv), math.inf, dtype=torch.float64)
            miss = torch.full((1, Hkv), math.nan, dtype=torch.float64)
        else:
            idx = torch.from_numpy(OP.index_blocks(idb, T))
            out, pr = OP.step(st, q, kb[:, :, :T], vb[:, :, :T], pol, idx=idx)
            read, trig, margin, miss = pr["read"], pr["trig"], pr["margin"], pr["miss"]
        pad = np.zeros((Hkv, nbmax), dtype=bool)
        pad[:, :read.shape[-1]] = read[0].numpy()
        rec["read"].append(np.packbits(pad, axis=-1))
        kp = np.zeros((Hkv, nbmax), dtype=bool)
        kp[:, :st.keep.shape[-1]] = st.keep[0].numpy()
        rec["keep"].append(np.packbits(kp, axis=-1))
        rec["trig"].append(trig[0].numpy())
        rec["margin"].append(margin[0].numpy().astype(np.float32))
        rec["topp"].append(st.topp_heads[0].reshape(Hkv, G).amin(-1).numpy().astype(np.float32))
        rec["miss"].append(miss[0].numpy().astype(np.float32))
        rec["calib"].append(st.calib[0].numpy().astype(np.float32))
        rec["aix"].append(st.aix[0].numpy())
        rec["lse_att"].append(st.lse_att[0].numpy().astype(np.float32))
        rec["proj"].append((out[0] @ u).numpy().astype(np.float32))
        rec["norm"].append(out[0].norm(dim=-1).numpy().astype(np.float32))
        if t in full_steps(steps):
            full.append(out[0].numpy().astype(np.float32))
    res = {key: np.stack(val) for key, val in rec.items()}
    res["out_full"] = np.stack(full)
    return res


def loop_case(cfg: int, steps: int | None = None) -> dict:
    """Config 4: records [layer, step, ...] of the two planned layers; config 5: [sequence, step, ...]
    of the planned layer (each sequence its own oracle state, as the reference planner keeps per-row
    decisions). steps: fewer steps (the CPU test's prefix check)."""
    run, layers, qs = loop_inputs(cfg)
    n = run.steps if steps is None else steps
    pol = stage4()
    parts = []
    if cfg == 4:
        for l in layers:
            parts.append(oracle_loop(run.k[l], run.v[l], qs[l], run.ids, run.T0[0], run.scale, pol, n))
    else:
        for b in range(len(run.T0)):
            parts.append(oracle_loop(run.k[0], run.v[0], qs[0], run.ids, run.T0[b], run.scale, pol, n, b=b))
    out = {key: np.stack([p[key] for p in parts]) for key in parts[0]}
    out["digest"] = np.array(input_digest(run, layers, qs))
    out["T0"] = np.array(run.T0, dtype=np.int64)
    out["layers"] = np.array(layers, dtype=np.int64)
    out["full_steps"] = np.array(full_steps(n), dtype=np.int64)
    return out


def main():
    if len(sys.argv) > 1 and sys.argv[1] == "full":
        for cfg in ((4, 5) if len(sys.argv) < 3 else (int(sys.argv[2]),)):
            t0 = time.time()
            name = f"planner_cfg{cfg}.npz"
            np.savez_compressed(HERE / name, **loop_case(cfg))
            print(name, (HERE / name).stat().st_size, "bytes", f"{time.time() - t0:.0f} s", flush=True)
        return
    np.savez_compressed(HERE / "attention_small.npz", **attention_case())
    np.savez_compressed(HERE / "planner_small.npz", **planner_case())
    for f in ("attention_small.npz", "planner_small.npz"):
        print(f, (HERE / f).stat().st_size, "bytes")


if __name__ == "__main__":
    main()
