"""Seeded synthetic inputs of the five benchmark configurations (shapes of Llama-3.2-1B,
Llama-3.1-8B, Qwen3-8B, Qwen2.5-7B attention layers; no model weights).

Everything is generated with a torch.Generator on the CPU (reproducible across machines) unless
`device` is a CUDA device, in which case the same recipe runs on that device's generator (fast,
for benchmarks; not bit-identical to the CPU stream).

Structured keys: per KV head, q_hat = normalised mean of its G queries; `hot` seeded blocks (not
block 0 and not the newest two) get k += hot_shift * q_hat; a sink bias beta * q_hat on block 0
(or on the newest two blocks) with beta solved by bisection so that the group's mean softmax mass
there is ~`sink_mass`.
"""

from __future__ import annotations

import hashlib
import math
from dataclasses import dataclass

import torch

BLOCK = 64


def _gen(device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _randn(shape, g, device):
    return torch.randn(*shape, generator=g, device=device, dtype=torch.float32)


@dataclass
class Layer:
    q: torch.Tensor        # [B, Hq, D] bf16
    k: torch.Tensor        # [B, Hkv, T, D] bf16
    v: torch.Tensor        # [B, Hkv, T, D] bf16
    scale: float
    info: dict


def _solve_bias(s_rest_lse, s_blk, c, target, iters=60):
    """beta >= 0 with mean_g [sum exp(s_blk + beta c) / (that + exp(s_rest_lse))] ~= target.
    s_rest_lse [G], s_blk [G, n], c [G]."""
    lo, hi = 0.0, 400.0

    def mass(beta):
        lb = torch.logsumexp(s_blk + beta * c[:, None], -1)
        return torch.sigmoid(lb - s_rest_lse).mean().item()

    if mass(hi) < target:
        return hi
    for _ in range(iters):
        mid = 0.5 * (lo + hi)
        if mass(mid) < target:
            lo = mid
        else:
            hi = mid
    return 0.5 * (lo + hi)


def structured(B, Hq, Hkv, D, T, seed, *, hot=3, hot_shift=2.0, sink="first", sink_mass=0.5, device="cpu"):
    """One attention layer of structured q/K/V. sink: "first" (block 0), "newest" (newest two
    blocks) or None."""
    g = _gen(device, seed)
    G = Hq // Hkv
    nb = (T + BLOCK - 1) // BLOCK
    q = _randn((B, Hq, D), g, device)
    k = _randn((B, Hkv, T, D), g, device)
    v = _randn((B, Hkv, T, D), g, device)
    q = q.to(torch.bfloat16).float()
    qhat = q.reshape(B, Hkv, G, D).mean(2)
    qhat = qhat / qhat.norm(dim=-1, keepdim=True)
    scale = 1.0 / math.sqrt(D)
    hot_blocks = torch.zeros(B, Hkv, hot, dtype=torch.long)
    betas = torch.zeros(B, Hkv)
    lo_blk, hi_blk = 1, max(1, nb - 2)                 # candidates: not block 0, not the newest two
    for b in range(B):
        for h in range(Hkv):
            if hot > 0 and hi_blk - lo_blk >= hot:
                perm = torch.randperm(hi_blk - lo_blk, generator=g, device=device)[:hot] + lo_blk
                hot_blocks[b, h] = perm.cpu()
                for blk in perm.tolist():
                    k[b, h, blk * BLOCK:min(T, (blk + 1) * BLOCK)] += hot_shift * qhat[b, h]
            if sink is None:
                continue
            t0, t1 = (0, min(T, BLOCK)) if sink == "first" else (max(0, (nb - 2) * BLOCK), T)
            qg = q[b, h * G:(h + 1) * G].double()                                      # [G, D]
            s = (qg @ k[b, h].double().T) * scale                                       # [G, T]
            c = (qg @ qhat[b, h].double()) * scale                                      # [G]
            rest = torch.cat([s[:, :t0], s[:, t1:]], -1)
            rest_lse = torch.logsumexp(rest, -1) if rest.shape[-1] else torch.full((G,), -math.inf, dtype=torch.float64)
            beta = _solve_bias(rest_lse.cpu(), s[:, t0:t1].cpu(), c.cpu(), sink_mass)
            betas[b, h] = beta
            k[b, h, t0:t1] += beta * qhat[b, h]
    info = dict(hot_blocks=hot_blocks, sink_beta=betas, sink=sink, seed=seed)
    return Layer(q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16), scale, info)


def cfg1(device="cpu", seed=1) -> Layer:
    """Llama-3.2-1B decode layer: B 1, 32 Q / 8 KV heads, D 64, T 4096, i.i.d. N(0, 1), scale 1/8."""
    g = _gen(device, seed)
    q = _randn((1, 32, 64), g, device).to(torch.bfloat16)
    k = _randn((1, 8, 4096, 64), g, device).to(torch.bfloat16)
    v = _randn((1, 8, 4096, 64), g, device).to(torch.bfloat16)
    return Layer(q, k, v, 1.0 / 8.0, dict(seed=seed))


def random_block_list(B, Hkv, nb, frac, seed, local=2, device="cpu"):
    """Per (b, KV head): a seeded random `frac` of the blocks, union block 0 and the `local` newest.
    Returns keep [B, Hkv, nb] bool."""
    g = _gen("cpu", seed)
    keep = torch.rand(B, Hkv, nb, generator=g) < frac
    keep[..., 0] = True
    if local > 0:
        keep[..., max(0, nb - local):] = True
    return keep.to(device)


def block_list(keep: torch.Tensor):
    """keep [B, Hkv, nb] -> (block_idx int32 [B, Hkv, nb] ascending kept first, block_cnt int32 [B, Hkv])."""
    cnt = keep.sum(-1, dtype=torch.int32)
    order = torch.argsort((~keep).to(torch.int8), dim=-1, stable=True).to(torch.int32)
    return order.contiguous(), cnt.contiguous()


def cfg2(device="cpu", seed=2, T=32768) -> tuple[Layer, torch.Tensor]:
    """Llama-3.1-8B layer at T 32768 with structured K (3 hot blocks + ~0.5 sink mass on block 0)
    and a per-KV-head block list: seeded 35% of blocks union {0, newest two}."""
    layer = structured(1, 32, 8, 128, T, seed, sink="first", device=device)
    nb = (T + BLOCK - 1) // BLOCK
    keep = random_block_list(1, 8, nb, 0.35, seed + 100, device=device)
    return layer, keep


def cfg3(device="cpu", seed=3, T=65536) -> Layer:
    """Qwen3-8B layer at T 65536: structured K, no sink on block 0; the ~0.5 mass sits on the
    newest two blocks instead."""
    return structured(1, 32, 8, 128, T, seed, sink="newest", device=device)


def paged_pools(ks, vs, seed, extra=16):
    """Paged copies of K / V views [B, Hkv, T, D]: one block table [B, ceil(T / 64)] int32 (a random
    page order, shared by the copies) and, per copy, pools [B ceil(T / 64) + extra, Hkv, 64, D] whose
    page table[b, j] holds tokens 64 j .. 64 j + 63 of sequence b (zeros past T and in unused pages)."""
    B, Hkv, T, D = ks[0].shape
    nb = (T + 63) // 64
    P = B * nb + extra
    perm = torch.randperm(P, generator=torch.Generator().manual_seed(seed))[: B * nb]
    table = perm.view(B, nb).to(torch.int32).to(ks[0].device)
    idx = perm.to(ks[0].device)

    def pool(x):
        y = torch.zeros(P, Hkv, 64, D, dtype=x.dtype, device=x.device)
        full = torch.zeros(B, Hkv, nb * 64, D, dtype=x.dtype, device=x.device)
        full[:, :, :T] = x
        y[idx] = full.view(B, Hkv, nb, 64, D).permute(0, 2, 1, 3, 4).reshape(B * nb, Hkv, 64, D)
        return y

    return table, [pool(k) for k in ks], [pool(v) for v in vs]


def perturbed_lse(lse_exact: torch.Tensor, seed: int, rel: float = 0.05) -> torch.Tensor:
    """lse_prev = lse_exact + log(1 + u), u ~ U[-rel, rel] per query head (the normaliser off by +-5%)."""
    g = _gen("cpu", seed)
    u = (torch.rand(lse_exact.shape, generator=g, dtype=torch.float64) * 2 - 1) * rel
    return (lse_exact.double().cpu() + torch.log1p(u)).float().to(lse_exact.device)


@dataclass
class PlannerRun:
    """Synthetic decode run for the planner loop (BASELINE configs 4 and 5): per layer a KV cache
    with capacity T0 + steps (the first T0 tokens filled), planted hot-block sets, and a query
    process; token ids with planted repeats for the token index."""
    k: list                 # per layer [B, Hkv, T0 + steps, D] bf16 (capacity)
    v: list
    dirs: list              # per layer [B, Hkv, n_sets, D] unit directions of the planted sets
    q0: list                # per layer [B, Hq, D] float32 initial queries
    aim: list               # per layer [B, Hq] int64 planted set each query head points at
    ids: torch.Tensor       # [B, T0 + steps] int32
    T0: list                # per batch element prefix length (ragged batches)
    steps: int
    scale: float
    seed: int
    alpha: float


def planner_run(layers=32, B=1, Hq=32, Hkv=8, D=128, T0=32768, steps=128, seed=4, n_sets=6, hot=3,
                hot_shift=6.0, vocab=128256, ragged=None, device="cpu") -> PlannerRun:
    """Keys / values N(0, 1); per (layer, b, KV head) n_sets planted sets of `hot` blocks whose keys
    get += hot_shift * u_j (u_j a seeded unit direction), plus a sink on block 0 holding ~0.5 of
    the group's mass at the start. hot_shift 6 (a +12-nat boost for an aimed query) makes a
    minority of blocks hold 99% of the mass, as in real decode attention; at 2 the attention is
    so flat that top-p 0.99 keeps every block and the planner has nothing to skip. Query head h starts aimed at a random set: q = alpha u_j + N(0,1)
    with alpha = 2 sqrt(D). ragged: optional list of per-batch prefix lengths (<= T0); the cache of
    element b then holds T0[b] valid tokens."""
    g = _gen(device, seed)
    G = Hq // Hkv
    T0s = list(ragged) if ragged is not None else [T0] * B
    Tcap = max(T0s) + steps
    alpha = 2.0 * math.sqrt(D)
    ks, vs, dirs, q0s, aims = [], [], [], [], []
    for layer in range(layers):
        k = _randn((B, Hkv, Tcap, D), g, device)
        v = _randn((B, Hkv, Tcap, D), g, device)
        u = _randn((B, Hkv, n_sets, D), g, device)
        u = u / u.norm(dim=-1, keepdim=True)
        aim = torch.randint(0, n_sets, (B, Hq), generator=g, device=device)
        q = _randn((B, Hq, D), g, device) + alpha * torch.gather(
            u.repeat_interleave(G, dim=1), 2, aim[..., None, None].expand(B, Hq, 1, D))[:, :, 0]
        for b in range(B):
            nb = (T0s[b] + BLOCK - 1) // BLOCK
            for h in range(Hkv):
                if nb > hot * n_sets + 3:
                    blocks = torch.randperm(nb - 3, generator=g, device=device)[:hot * n_sets] + 1
                    for j in range(n_sets):
                        for blk in blocks[j * hot:(j + 1) * hot].tolist():
                            k[b, h, blk * BLOCK:min(T0s[b], (blk + 1) * BLOCK)] += hot_shift * u[b, h, j]
                qg = q[b, h * G:(h + 1) * G].double()
                qhat = qg.mean(0)
                qhat = (qhat / qhat.norm()).float()
                s = (qg @ k[b, h, :T0s[b]].double().T) / math.sqrt(D)
                c = (qg @ qhat.double()) / math.sqrt(D)
                t1 = min(T0s[b], BLOCK)
                rest = torch.logsumexp(s[:, t1:], -1) if T0s[b] > t1 else torch.full((G,), -math.inf, dtype=torch.float64)
                beta = _solve_bias(rest.cpu(), s[:, :t1].cpu(), c.cpu(), 0.5)
                k[b, h, :t1] += beta * qhat
        ks.append(k.to(torch.bfloat16))
        vs.append(v.to(torch.bfloat16))
        dirs.append(u)
        q0s.append(q)
        aims.append(aim)
    ids = torch.randint(0, vocab, (B, Tcap), generator=g, device=device, dtype=torch.int64)
    # planted repeats: a third of the decode-step tokens copy an earlier token
    for b in range(B):
        for t in range(T0s[b], T0s[b] + steps):
            if torch.rand((), generator=g, device=device).item() < 1 / 3:
                src = int(torch.randint(0, t, (), generator=g, device=device).item())
                ids[b, t] = ids[b, src]
    return PlannerRun(ks, vs, dirs, q0s, aims, ids.to(torch.int32), T0s, steps, 1.0 / math.sqrt(D), seed, alpha)


class QueryProcess:
    """q_t = 0.97 q_{t-1} + noise N(0, 1) (noise 0.25: config 4); with probability p_jump per query
    head and step the head re-aims at another planted set: q = alpha u_new + noise N(0, 1).
    revert=True: q_t = m + 0.97 (q_{t-1} - m) + noise N(0, 1) with m = alpha u_aim, so the query
    stays on its planted set between jumps instead of decaying towards 0 (whose flat softmax puts
    the 99% set over most of the cache). Seeded, on the CPU."""

    def __init__(self, run: PlannerRun, layer: int, p_jump=0.03, seed=None, noise=0.25, revert=False):
        self.run, self.layer, self.p, self.noise, self.revert = run, layer, p_jump, noise, revert
        self.g = torch.Generator().manual_seed(run.seed * 1000 + layer if seed is None else seed)
        self.q = run.q0[layer].detach().float().cpu().clone()
        self.aim = run.aim[layer].cpu().clone()
        self.u = run.dirs[layer].float().cpu()

    def _aimed(self, G):
        B, Hq, D = self.q.shape
        return torch.gather(self.u.repeat_interleave(G, dim=1), 2, self.aim[..., None, None].expand(B, Hq, 1, D))[:, :, 0]

    def next(self) -> torch.Tensor:
        B, Hq, D = self.q.shape
        Hkv, n_sets = self.u.shape[1], self.u.shape[2]
        G = Hq // Hkv
        eps = torch.randn(B, Hq, D, generator=self.g)
        if self.revert:
            m = self.run.alpha * self._aimed(G)
            self.q = m + 0.97 * (self.q - m) + self.noise * eps
        else:
            self.q = 0.97 * self.q + self.noise * eps
        jump = torch.rand(B, Hq, generator=self.g) < self.p
        if bool(jump.any()):
            new = (self.aim + 1 + torch.randint(0, n_sets - 1, (B, Hq), generator=self.g)) % n_sets
            self.aim = torch.where(jump, new, self.aim)
            self.q = torch.where(jump[..., None], self.run.alpha * self._aimed(G) + self.noise * eps, self.q)
        return self.q.to(torch.bfloat16)


def cfg5_lens() -> list[int]:
    """Config 5's 16 contexts, log-uniform in [4096, 65536] from seed 5."""
    g = torch.Generator().manual_seed(5)
    return [int(round(math.exp(x))) for x in
            (torch.rand(16, generator=g, dtype=torch.float64) * math.log(16) + math.log(4096)).tolist()]


def loop_inputs(cfg: int):
    """The inputs of the full-size planner loops that the golden fixtures record: (run, planned
    layers, query sequences qs[layer][t] bf16 [B, Hq, D]) of config 4 (B 1, 32 / 8 heads, D 128, T0
    32768, 128 steps, jumps 0.03; layer 0 dense, layers 1 and 2 planned) or config 5 (B 16 ragged
    contexts, 28 / 4 heads, 64 steps; one planned layer), generated on the CPU."""
    if cfg == 4:
        run = planner_run(layers=3, B=1, Hq=32, Hkv=8, D=128, T0=32768, steps=128, seed=4)
        layers = [1, 2]
    elif cfg == 5:
        run = planner_run(layers=1, B=16, Hq=28, Hkv=4, D=128, T0=65536, steps=64, seed=5, ragged=cfg5_lens())
        layers = [0]
    else:
        raise ValueError(cfg)
    qs = {}
    for l in layers:
        qp = QueryProcess(run, l, p_jump=0.03)
        qs[l] = [qp.next() for _ in range(run.steps)]
    return run, layers, qs


def input_digest(run, layers, qs) -> str:
    """sha256 over the planned layers' K / V, the query sequences and the token ids."""
    h = hashlib.sha256()
    for l in layers:
        h.update(run.k[l].view(torch.int16).numpy().tobytes())
        h.update(run.v[l].view(torch.int16).numpy().tobytes())
        for q in qs[l]:
            h.update(q.view(torch.int16).numpy().tobytes())
    h.update(run.ids.numpy().tobytes())
    return h.hexdigest()
