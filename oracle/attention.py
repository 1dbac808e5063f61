"""Attention oracle (float64, CPU): decode, per-block statistics, P, block selection, V-skip.

Test infrastructure only (see oracle/__init__.py). Units follow the reference: scores and
blk_max / lse in natural log units; blk_sum = sum exp(s - blk_max) over the block.
"""

from __future__ import annotations

import math

import torch

BLOCK = 64
NEG_INF = float("-inf")


def nblocks(T: int) -> int:
    return (T + BLOCK - 1) // BLOCK


def scores(q, k, scale, dtype=torch.float64):
    """s [B, Hq, T] = scale * q . k with query head h on KV head h // G (bench/harness.py:111-113)."""
    B, Hq, D = q.shape
    Hkv, T = k.shape[1], k.shape[2]
    G = Hq // Hkv
    s = torch.einsum("bkgd,bktd->bkgt", q.to(dtype).reshape(B, Hkv, G, D), k.to(dtype)) * scale
    return s.reshape(B, Hq, T)


def heads(x, G):
    """[B, Hkv, ...] -> [B, Hq, ...] (query head h reads KV head h // G)."""
    return x.repeat_interleave(G, dim=1)


def token_mask(keep, T):
    """Block mask [..., nb] -> token mask [..., T]."""
    return keep.repeat_interleave(BLOCK, dim=-1)[..., :T]


def decode(q, k, v, scale, keep=None, dtype=torch.float64):
    """Decode attention over the kept blocks: (out [B, Hq, D], lse [B, Hq]).

    bench/harness.py:99-118 (reference_decode); dropped blocks leave the softmax before it is
    taken. An empty kept set gives out = 0 and lse = -inf (kernels/kvskip_kernel.cu:273-286)."""
    B, Hq, D = q.shape
    Hkv, T = k.shape[1], k.shape[2]
    G = Hq // Hkv
    s = scores(q, k, scale, dtype)
    if keep is not None:
        s = s.masked_fill(~heads(token_mask(keep, T), G), NEG_INF)
    lse = torch.logsumexp(s, -1)
    p = torch.exp(s - lse[..., None].clamp_min(torch.finfo(s.dtype).min))
    p = torch.where(torch.isfinite(lse)[..., None], p, torch.zeros_like(p))
    out = torch.einsum("bkgt,bktd->bkgd", p.reshape(B, Hkv, G, T), v.to(dtype)).reshape(B, Hq, D)
    return out, lse


def block_stats(q, k, scale, keep=None, dtype=torch.float64):
    """Per-block max score and sum exp(s - max): (M, S) [B, Hq, nb] (bench/harness.py:121-131).

    Blocks outside `keep` [B, Hkv, nb] are (-inf, 0), as the masked kernel leaves them
    (kernels/kvskip_ext.cpp:51-54)."""
    B, Hq, D = q.shape
    Hkv, T = k.shape[1], k.shape[2]
    G = Hq // Hkv
    nb = nblocks(T)
    s = scores(q, k, scale, dtype)
    s = torch.nn.functional.pad(s, (0, nb * BLOCK - T), value=NEG_INF).reshape(B, Hq, nb, BLOCK)
    M = s.amax(-1)
    S = torch.exp(s - M[..., None].clamp_min(torch.finfo(s.dtype).min)).sum(-1)
    S = torch.where(torch.isfinite(M), S, torch.zeros_like(S))
    if keep is not None:
        kh = heads(keep, G)
        M = M.masked_fill(~kh, NEG_INF)
        S = S.masked_fill(~kh, 0.0)
    return M, S


def p_values(q, k, scale, dtype=torch.float64):
    """P [B, Hq, nb*64] = exp(s - block max), zero past T (pass 1 of the two-pass V-skip,
    kernels/kvskip_kernel.cu:203-216)."""
    B, Hq, D = q.shape
    T = k.shape[2]
    nb = nblocks(T)
    s = scores(q, k, scale, dtype)
    s = torch.nn.functional.pad(s, (0, nb * BLOCK - T), value=NEG_INF).reshape(B, Hq, nb, BLOCK)
    M = s.amax(-1, keepdim=True)
    return torch.exp(s - M).reshape(B, Hq, nb * BLOCK)


def block_logw(M, S):
    """Block log-weights x = M + log S (-inf where a block was not read)."""
    return M + torch.log(S)


def always_keep(nb: int, local: int) -> torch.Tensor:
    """Block 0 and the `local` newest blocks (kernels/kvskip.py:122-127)."""
    a = torch.zeros(nb, dtype=torch.bool)
    a[0] = True
    if local > 0:
        a[max(0, nb - local):] = True
    return a


def topp_heads(logw, level):
    """Per query head the fewest blocks whose weights reach `level` (ties at the threshold kept).

    kernels/kvskip.py:140-143: with weights sorted descending, block i is kept iff the mass
    ranked strictly before it is < level. Returns (keep_h [B, Hq, nb], margin [B, Hq]) where
    margin is how far the two cumulative sums around the cut are from `level` (a decision closer
    than that to `level` may flip under a different float summation order)."""
    W = torch.softmax(logw.to(torch.float64), dim=-1)
    ws, order = W.sort(-1, descending=True)
    cs = ws.cumsum(-1)
    before = cs - ws
    take = before < level
    n = take.sum(-1, keepdim=True).clamp_min(1)                       # blocks kept per head
    thr = ws.gather(-1, n - 1)                                         # weight of the last kept block
    keep_h = W >= thr                                                  # includes ties at the cut
    keep_h = keep_h | torch.zeros_like(take).scatter(-1, order, take)
    last_before = before.gather(-1, n - 1)
    last_incl = cs.gather(-1, n - 1)
    margin = torch.minimum((level - last_before).abs(), (last_incl - level).abs())[..., 0]
    return keep_h, margin


def select_blocks(logw, G, rule, value, local=2):
    """GQA-union block selection, keep [B, Hkv, nb] (kernels/kvskip.py:130-147)."""
    B, Hq, nb = logw.shape
    if rule == "tau":
        keep_h = torch.softmax(logw.to(torch.float64), dim=-1) >= value
    elif rule == "topp":
        keep_h, _ = topp_heads(logw, value)
    else:
        raise ValueError(rule)
    keep = keep_h.reshape(B, Hq // G, G, nb).any(2)
    return keep | always_keep(nb, local)


def vskip1_keep(q, k, scale, tau, local, lse_prev=None, dtype=torch.float64):
    """Blocks whose V the single-pass V-skip reads, and the signed decision margin.

    kernels/kvskip_kernel.cu:562-578,630-640 (and bench/test_decode.py:134-150): a block is read
    if it is block 0, one of the `local` newest, or some head of the group has block
    log-sum-exp - lse0 >= log(tau), lse0 = lse_prev (natural units) or the block-0 log-sum-exp.
    Returns (keep [B, Hkv, nb], z [B, Hkv, nb] = max over the group of (lse_b - lse0) - log tau)."""
    B, Hq, D = q.shape
    Hkv, T = k.shape[1], k.shape[2]
    G = Hq // Hkv
    nb = nblocks(T)
    M, S = block_stats(q, k, scale, dtype=dtype)
    lse_b = block_logw(M, S)                                           # [B, Hq, nb]
    lse0 = lse_b[..., :1] if lse_prev is None else lse_prev.to(dtype)[..., None]
    z = (lse_b - lse0 - math.log(tau)).reshape(B, Hkv, G, nb).amax(2)
    keep = (z >= 0) | always_keep(nb, local)
    return keep, z


def vskip1(q, k, v, scale, tau, local=2, lse_prev=None, dtype=torch.float64):
    """Single-pass V-skip result: (out, lse, keep, vcount [B, Hkv]). dtype: float32 for the timed CPU
    baseline (the checks use float64)."""
    keep, _ = vskip1_keep(q, k, scale, tau, local, lse_prev, dtype)
    out, lse = decode(q, k, v, scale, keep=keep, dtype=dtype)
    return out, lse, keep, keep.sum(-1).to(torch.int32)


def pv(P, v, blk_scale, keep):
    """Two-pass V-skip pass 2: out = sum over kept blocks of blk_scale[b, h, blk, g] * P . V
    (kernels/kvskip_kernel.cu:316-421). P [B, Hq, nb*64], blk_scale [B, Hkv, nb, G]."""
    B, Hq, _ = P.shape
    Hkv, T, D = v.shape[1], v.shape[2], v.shape[3]
    G = Hq // Hkv
    nb = nblocks(T)
    f = blk_scale.to(torch.float64).masked_fill(~keep[..., None], 0.0)           # [B, Hkv, nb, G]
    f = f.permute(0, 1, 3, 2).reshape(B, Hq, nb)
    w = (P.to(torch.float64).reshape(B, Hq, nb, BLOCK) * f[..., None]).reshape(B, Hq, nb * BLOCK)[..., :T]
    return torch.einsum("bkgt,bktd->bkgd", w.reshape(B, Hkv, G, T), v.to(torch.float64)).reshape(B, Hq, D)


def vskip_two_pass(q, k, v, scale, rule="topp", value=0.99, local=2):
    """Two-pass V-skip (kernels/kvskip.py:157-179): the kept set from pass-1 stats, then exact
    attention over it. Returns (out, keep)."""
    G = q.shape[1] // k.shape[1]
    M, S = block_stats(q, k, scale)
    keep = select_blocks(block_logw(M, S), G, rule, value, local)
    out, _ = decode(q, k, v, scale, keep=keep)
    return out, keep


def split_ranges(n_items: int, num_splits: int):
    """Item ranges of the split-K partition: per = ceil(n / S) (kernels/kvskip_kernel.cu:99-101)."""
    per = (n_items + num_splits - 1) // num_splits
    out = []
    for s in range(num_splits):
        i0 = min(n_items, s * per)
        out.append((i0, min(n_items, i0 + per)))
    return out


def rel_err(out, ref) -> float:
    """||out - ref||_2 / ||ref||_2 (bench/harness.py:134-135)."""
    ref = ref.to(torch.float64)
    den = ref.norm()
    return float((out.to(torch.float64) - ref).norm() / (den if den > 0 else 1.0))
