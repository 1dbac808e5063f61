"""Python front-end of the kvskip_amd decode kernels: the public API of the reference's
kernels/kvskip.py (kernels/kvskip.py:28-208) on MI355X.

    out = decode(q, k, v, scale)                         # dense
    out = decode(q, k, v, scale, plan=make_plan(keep))   # skip blocks (neither K nor V read)
    out = decode(q, k, v, scale, stats=True)             # dense + per-block max / sumexp
    out = decode(q, k, v, scale, stats=True, load_v=False)  # stats only: reads K, not V

q [B, Hq, D] or [B, Hq, 1, D]; k, v [B, Hkv, T, D] in any batch/head/token strides with D
contiguous. Blocks are 64 tokens from position 0. Any G = Hq / Hkv in {1, 2, 4, 7, 8},
D in {64, 128}.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import ext as _ext_mod

TILE = 64
WG_PER_CU = 1          # attention workgroups (4 wavefronts each) per CU in the split heuristic


def ext():
    """The operator module (the reference JIT-builds its extension here; ours is prebuilt)."""
    from . import _native
    _native.lib()
    return _ext_mod


def num_sms() -> int:
    """Compute units of the current device (256 on MI355X)."""
    return torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count


def num_splits_for(bh: int, n_tiles: int, sms: int | None = None, max_splits: int = 256,
                   min_tiles: int = 4) -> int:
    """Split count for B*Hkv work items of n_tiles blocks each (kernels/kvskip.py:51-67).

    Same rule as the reference -- best wave efficiency over the resident workgroup slots, lightly
    preferring fewer splits, at least `min_tiles` blocks per split (one per wavefront of a
    workgroup) -- with the slots counted as CUs x WG_PER_CU."""
    slots = (sms or num_sms()) * WG_PER_CU
    best, best_score = 1, -1.0
    for s in range(1, max_splits + 1):
        if s > 1 and math.ceil(n_tiles / s) < min_tiles:
            break
        waves = bh * s / slots
        eff = waves / math.ceil(waves)
        score = eff - 0.002 * s
        if score > best_score + 1e-9:
            best, best_score = s, score
    return best


def ragged_splits(B: int, Hkv: int, nb_max: int, sms: int | None = None) -> int:
    """Split budget per KV head for a ragged batch (seq_lens): about two workgroups per CU over all
    KV heads, at least 8 blocks per chunk at full length, in 2..256."""
    slots = (sms or num_sms()) * 2
    return max(2, min(256, slots // max(Hkv, 1), max(1, B * nb_max // 8)))


@dataclass
class Plan:
    """Kept-block list for the masked kernel (kernels/kvskip.py:70-76)."""
    block_idx: torch.Tensor   # int32 [B, Hkv, nb], kept blocks first, ascending
    block_cnt: torch.Tensor   # int32 [B, Hkv]
    max_cnt: int              # max kept blocks over (b, kv head), sizes the split count
    nb: int


def make_plan(keep: torch.Tensor, sync: bool = True) -> Plan:
    """keep: bool [B, Hkv, nb] -> Plan (kernels/kvskip.py:79-85). With sync=True one host sync
    sizes the split count by the largest kept list; sync=False sizes it by nb."""
    cnt = keep.sum(-1, dtype=torch.int32)
    order = torch.argsort((~keep).to(torch.int8), dim=-1, stable=True).to(torch.int32)
    return Plan(order.contiguous(), cnt.contiguous(), int(cnt.max()) if sync else keep.shape[-1], keep.shape[-1])


def decode(q, k, v, scale: float, *, plan: Plan | None = None, stats: bool = False, load_v: bool = True,
           num_splits: int | None = None, stages: int = 2, out_f32: bool = False, write_p: bool = False,
           seq_lens: torch.Tensor | None = None, block_table: torch.Tensor | None = None,
           T: int | None = None) -> dict:
    """Decode attention for one layer (kernels/kvskip.py:88-113). Returns dict(out [B, Hq, D] bf16,
    lse [B, Hq] fp32, blk_max / blk_sum [B, Hq, nb] fp32 (stats), out_f32 (if asked), p (write_p:
    fp16 [B, Hq, nb*64] = exp(s - blk_max))). Not in the reference: seq_lens (int32 [B] on the
    device): a ragged batch over views of capacity T, with the split budget shared by the batch;
    block_table (int32 [B, >= ceil(T / 64)]) with T: k, v are page pools [num_pages, Hkv, 64, D]."""
    if q.dim() == 4:
        q = q.squeeze(2)
    B, Hq, D = q.shape
    Hkv, T = k.shape[1], (k.shape[2] if block_table is None else int(T))
    nb = math.ceil(T / TILE)
    n_items = nb if plan is None else plan.max_cnt
    if num_splits is None:
        num_splits = num_splits_for(B * Hkv, n_items) if seq_lens is None else ragged_splits(B, Hkv, n_items)
    paged = {} if block_table is None else dict(block_table=block_table, T=T)
    res = ext().decode(q, k, v, float(scale), None if plan is None else plan.block_idx,
                       None if plan is None else plan.block_cnt, stats, load_v, int(num_splits), int(stages),
                       out_f32, write_p, seq_lens, **paged)
    out, lse, bmax, bsum, o32, pbuf = res
    d = {"out": out if load_v else None, "lse": lse, "num_splits": num_splits}
    if stats:
        d["blk_max"], d["blk_sum"] = bmax, bsum
    if out_f32:
        d["out_f32"] = o32
    if write_p:
        d["p"] = pbuf
    return d


def block_weights(blk_max: torch.Tensor, blk_sum: torch.Tensor) -> torch.Tensor:
    """Per-block softmax mass [B, Hq, nb] from the stats outputs (kernels/kvskip.py:116-119)."""
    logw = blk_max + torch.log(blk_sum)
    return torch.softmax(logw, dim=-1)


def always_keep(nb: int, local: int, device) -> torch.Tensor:
    """Blocks every sparse mode reads: the sink block and the `local` newest blocks."""
    a = torch.zeros(nb, dtype=torch.bool, device=device)
    a[0] = True
    if local > 0:
        a[-local:] = True
    return a


def select_blocks(logw: torch.Tensor, G: int, rule: str, value: float, local: int = 2) -> torch.Tensor:
    """GQA-union block selection from per-head block log-weights [B, Hq, nb] (kernels/kvskip.py:130-147).

    rule "tau": keep a block if any head of the group has weight >= value;
    rule "topp": keep the fewest blocks holding >= value of each head's mass (union over heads).
    Returns keep [B, Hkv, nb] bool (sink + `local` newest blocks always kept)."""
    B, Hq, nb = logw.shape
    W = torch.softmax(logw, dim=-1)
    if rule == "tau":
        keep_h = W >= value
    elif rule == "topp":
        ws, order = W.sort(-1, descending=True)
        take = (ws.cumsum(-1) - ws) < value
        keep_h = torch.zeros_like(take).scatter(-1, order, take)
    else:
        raise ValueError(rule)
    keep = keep_h.view(B, Hq // G, G, nb).any(2)
    return keep | always_keep(nb, local, logw.device)


def pv(P, v, blk_scale, plan: Plan, num_splits: int | None = None, out_f32: bool = False,
       block_table: torch.Tensor | None = None, T: int | None = None):
    """Two-pass V-skip pass 2 (kernels/kvskip.py:150-154); block_table, T: v is a page pool."""
    B, Hkv = P.shape[0], v.shape[1]
    if num_splits is None:
        num_splits = num_splits_for(B * Hkv, plan.max_cnt)
    paged = {} if block_table is None else dict(block_table=block_table, T=T)
    return ext().pv(P, v, blk_scale, plan.block_idx, plan.block_cnt, int(num_splits), out_f32, **paged)


def vskip_two_pass(q, k, v, scale: float, rule: str = "topp", value: float = 0.99, local: int = 2,
                   sync: bool = True, out_f32: bool = False, block_table: torch.Tensor | None = None,
                   T: int | None = None) -> dict:
    """Two-pass V-skip (kernels/kvskip.py:157-179): pass 1 reads all of K once and writes block stats
    and P (fp16); the GQA-union selection picks blocks; pass 2 reads P and V of the kept blocks only.
    block_table, T (not in the reference): k, v are page pools of a paged cache."""
    if q.dim() == 4:
        q = q.squeeze(2)
    B, Hq, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    paged = {} if block_table is None else dict(block_table=block_table, T=T)
    r1 = decode(q, k, v, scale, stats=True, load_v=False, write_p=True, **paged)
    logw = r1["blk_max"] + torch.log(r1["blk_sum"])                    # [B, Hq, nb]
    keep = select_blocks(logw, G, rule, value, local)                   # [B, Hkv, nb]
    keep_h = keep.repeat_interleave(G, dim=1)                           # [B, Hq, nb]
    lse_kept = logw.masked_fill(~keep_h, float("-inf")).logsumexp(-1, keepdim=True)
    scale_b = torch.exp(r1["blk_max"] - lse_kept).masked_fill(~keep_h, 0.0)
    scale_b = scale_b.view(B, Hkv, G, -1).transpose(2, 3).contiguous()  # [B, Hkv, nb, G]
    plan = make_plan(keep, sync=sync)
    out, o32 = pv(r1["p"], v, scale_b, plan, out_f32=out_f32, **paged)
    d = {"out": out, "keep": keep, "kept_frac": keep.float().mean().item() if sync else None}
    if out_f32:
        d["out_f32"] = o32
    return d


def vskip_one_pass(q, k, v, scale: float, tau: float = 1e-4, local: int = 2, num_splits: int | None = None,
                   out_f32: bool = False, count: bool = False, lse_prev: torch.Tensor | None = None,
                   sync: bool = True, block_table: torch.Tensor | None = None, T: int | None = None) -> dict:
    """Single-pass V-skip (kernels/kvskip.py:182-208): K read once, V of a block read only if some
    head of the group has estimated weight >= tau there (normaliser: lse_prev, else the sink
    block's log-sum-exp, a lower bound). With count=True "v_tiles" [B, Hkv] counts V blocks read.
    block_table, T (not in the reference): k, v are page pools of a paged cache."""
    if q.dim() == 4:
        q = q.squeeze(2)
    B, Hq, D = q.shape
    Hkv, T = k.shape[1], (k.shape[2] if block_table is None else int(T))
    paged = {} if block_table is None else dict(block_table=block_table, T=T)
    nb = math.ceil(T / TILE)
    if num_splits is None:
        num_splits = num_splits_for(B * Hkv, nb)
    out, lse, o32, cnt = ext().vskip1(q, k, v, float(scale), float(tau), int(local), int(num_splits),
                                      out_f32, count, lse_prev, **paged)
    d = {"out": out, "lse": lse, "num_splits": num_splits}
    if out_f32:
        d["out_f32"] = o32
    if count:
        d["v_tiles"] = cnt
        if sync:
            d["kept_frac"] = (cnt.sum() / (B * Hkv * nb)).item()
    return d
