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


def perturbed_lse(lse_exact: torch.Tensor, seed: int, rel: float = 0.05) -> torch.Tensor:
    """lse_prev = lse_exact + log(1 + u), u ~ U[-rel, rel] per query head (the normaliser off by +-5%)."""
    g = _gen("cpu", seed)
    u = (torch.rand(lse_exact.shape, generator=g, dtype=torch.float64) * 2 - 1) * rel
    return (lse_exact.double().cpu() + torch.log1p(u)).float().to(lse_exact.device)
