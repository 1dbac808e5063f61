"""kvskip_amd's decode front-end: the Python functions a caller of the reference's
kernels/kvskip.py uses (names, arguments, defaults and result dicts of kernels/kvskip.py:47-208),
on the kvskip_amd operators. Block lists and block selection are made on the device
(kvskip_block_list, kvskip_select): vskip_two_pass is the K pass, the selection and the V pass,
with no host work in between. A host synchronisation happens only where a caller asks for a number
on the host (sync=True: the longest list sizes the split count, and the kept fraction).

    r = decode(q, k, v, scale)                              # every block
    r = decode(q, k, v, scale, plan=make_plan(keep))        # the blocks keep [B, Hkv, nb] marks
    r = decode(q, k, v, scale, stats=True)                  # + per-block blk_max / blk_sum
    r = decode(q, k, v, scale, stats=True, load_v=False)    # statistics from K alone
    out, lse = r["out"], r["lse"]

q is [B, Hq, D] or [B, Hq, 1, D]; k and v are [B, Hkv, T, D] views (D contiguous, other strides
free); a block is 64 tokens from position 0; G = Hq / Hkv in {1, 2, 4, 7, 8}; D in {64, 128}.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import ext as _ops

TILE = 64
WG_PER_CU = 1          # attention workgroups (4 wavefronts each) per CU in the split heuristic


def ext():
    """The operator module, with the native library loaded (it raises if the library is missing)."""
    from . import _native
    _native.lib()
    return _ops


def num_sms() -> int:
    """Compute units of the current device (256 on MI355X)."""
    return torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count


def _split_score(bh: int, splits: int, slots: int) -> float:
    """How fully bh * splits workgroups use whole waves of `slots`, less 0.002 per split."""
    waves = bh * splits / slots
    return waves / math.ceil(waves) - 0.002 * splits


def num_splits_for(bh: int, n_tiles: int, sms: int | None = None, max_splits: int = 256,
                   min_tiles: int = 4) -> int:
    """Split count for bh = B * Hkv work items of n_tiles blocks each. The rule of
    kernels/kvskip.py:51-67: the best wave efficiency over the resident workgroup slots (here CUs x
    WG_PER_CU), 0.002 per split against more splits, every split keeping >= min_tiles blocks; the
    smallest count wins ties."""
    slots = (sms or num_sms()) * WG_PER_CU
    most = 1                                       # ceil(n / s) only falls as s grows
    while most < max_splits and math.ceil(n_tiles / (most + 1)) >= min_tiles:
        most += 1
    best = 1
    for s in range(2, most + 1):
        if _split_score(bh, s, slots) > _split_score(bh, best, slots) + 1e-9:
            best = s
    return best


def ragged_splits(B: int, Hkv: int, nb_max: int, sms: int | None = None, G: int = 4, carry: bool = False) -> int:
    """Split budget per KV head for a ragged batch (seq_lens), at least 8 blocks per chunk at full
    length, in 2..256. Groups of up to 4 query heads: 7/8 of two workgroups per CU over all KV heads,
    the last eighth left to the sequences' partial last chunks (measured, 8 KV heads: B 8 planner
    loop 183.3 -> 178.5 us per layer-step at 64 -> 56 splits, B 32 at 64k 652.9 -> 630.0; 48 and 40
    were slower). Larger groups (more arithmetic per block): the grid's S + B chunk slots per KV head
    fill two workgroups per CU (config 5 dense 113.6 -> 112.2 us, its planner loop with the update
    beside the merge 144.0 -> 137.7), or one per CU for a pass that carries another layer's update
    (`carry`: its G-wavefront update workgroups then share the CUs; config 5's loop 125.2 at one per
    CU, 126.9 at two, 132.2 at two less the update's workgroups)."""
    cus = sms or num_sms()
    Hkv = max(Hkv, 1)
    if G <= 4:
        per_head = cus * 2 // Hkv - cus // (4 * Hkv)
    else:
        per_head = (cus if carry else cus * 2) // Hkv - B
    return max(2, min(256, per_head, max(1, B * nb_max // 8)))


@dataclass
class Plan:
    """Block lists of the masked pass (the fields of kernels/kvskip.py:70-76)."""
    block_idx: torch.Tensor   # int32 [B, Hkv, nb]: listed blocks first, ascending
    block_cnt: torch.Tensor   # int32 [B, Hkv]
    max_cnt: int              # longest list (sizes the split count); nb when not read back
    nb: int


def _lists(B: int, Hkv: int, nb: int, device):
    return (torch.empty(B, Hkv, nb, dtype=torch.int32, device=device),
            torch.empty(B, Hkv, dtype=torch.int32, device=device))


def make_plan(keep: torch.Tensor, sync: bool = True) -> Plan:
    """Lists of the blocks keep [B, Hkv, nb] (bool) marks, built on the device. sync=True reads the
    longest list back (one host synchronisation) so the split count fits it; sync=False sizes the
    split count by nb (kernels/kvskip.py:79-85)."""
    B, Hkv, nb = keep.shape
    idx, cnt = _lists(B, Hkv, nb, keep.device)
    ext().block_list(keep.contiguous(), idx, cnt)
    return Plan(idx, cnt, int(cnt.max()) if sync else nb, nb)


def _paged(block_table, T) -> dict:
    return {} if block_table is None else {"block_table": block_table, "T": int(T)}


def _as_bhd(q: torch.Tensor) -> torch.Tensor:
    return q[:, :, 0] if q.dim() == 4 else q


def decode(q, k, v, scale: float, *, plan: Plan | None = None, stats: bool = False, load_v: bool = True,
           num_splits: int | None = None, stages: int = 2, out_f32: bool = False, write_p: bool = False,
           seq_lens: torch.Tensor | None = None, block_table: torch.Tensor | None = None,
           T: int | None = None, merge: bool = True) -> dict:
    """Decode attention of one layer (kernels/kvskip.py:88-113). Returns a dict with out [B, Hq, D]
    bf16 (None with load_v=False), lse [B, Hq] fp32, num_splits, and as asked blk_max / blk_sum
    [B, Hq, nb] fp32, out_f32, p (fp16 [B, Hq, nb*64] = exp(s - blk_max)).
    Not in the reference: seq_lens (int32 [B] on the device) makes a ragged batch over views of
    capacity T, the split budget shared by the batch (with a plan, up to 512 lists, the lists of all
    KV heads cut by one chunk length: kvskip_attn_args.list_partition); block_table (int32 [B, >=
    ceil(T / 64)]) with T makes k, v page pools [num_pages, Hkv, 64, D]; merge=False (with
    load_v=False) skips the split merge, leaving lse None."""
    q = _as_bhd(q)
    B, Hkv = q.shape[0], k.shape[1]
    tokens = k.shape[2] if block_table is None else int(T)
    nb = math.ceil(tokens / TILE)
    if num_splits is None:
        items = nb if plan is None else plan.max_cnt
        num_splits = (ragged_splits(B, Hkv, items, G=q.shape[1] // Hkv) if seq_lens is not None
                      else num_splits_for(B * Hkv, items))
    lists = (None, None) if plan is None else (plan.block_idx, plan.block_cnt)
    lp = int(plan is not None and seq_lens is not None and B > 1 and B * Hkv <= 512)
    out, lse, bmax, bsum, o32, p = ext().decode(q, k, v, float(scale), *lists, stats, load_v, int(num_splits),
                                                int(stages), out_f32, write_p, seq_lens, **_paged(block_table, T),
                                                merge=merge, list_partition=lp)
    res = {"out": out, "lse": lse, "num_splits": num_splits}
    extra = {"blk_max": bmax, "blk_sum": bsum} if stats else {}
    if out_f32:
        extra["out_f32"] = o32
    if write_p:
        extra["p"] = p
    res.update(extra)
    return res


def block_weights(blk_max: torch.Tensor, blk_sum: torch.Tensor) -> torch.Tensor:
    """Each block's share of its query head's softmax mass [B, Hq, nb], from the statistics
    (kernels/kvskip.py:116-119)."""
    return torch.softmax(blk_max + blk_sum.log(), dim=-1)


def always_keep(nb: int, local: int, device) -> torch.Tensor:
    """Blocks every sparse mode reads (kernels/kvskip.py:122-127): block 0 and the `local` newest
    (none for local = 0)."""
    pos = torch.arange(nb, device=device)
    return (pos == 0) | (pos >= nb - local)


def select_blocks(logw: torch.Tensor, G: int, rule: str, value: float, local: int = 2) -> torch.Tensor:
    """GQA-union selection from block log-weights [B, Hq, nb] (kernels/kvskip.py:130-147), on the
    device: "tau" keeps a block if some head of the group gives it weight >= value, "topp" keeps per
    head the fewest blocks holding >= value of its mass (ties at the cut kept) and unites the group;
    block 0 and the `local` newest always. Returns keep [B, Hkv, nb] bool."""
    B, Hq, nb = logw.shape
    # the device selection's limits (the reference's torch rule also runs on CPU tensors and at any
    # size; here the selection is a device kernel only, with no host fallback)
    if not logw.is_cuda:
        raise RuntimeError("select_blocks runs on the device: logw must be a CUDA tensor")
    if G < 1 or Hq % G != 0 or G > 8:
        raise RuntimeError(f"select_blocks: group size G in 1..8 dividing Hq (got G={G}, Hq={Hq})")
    if nb > 4096:
        raise RuntimeError(f"select_blocks: at most 4096 blocks (got {nb})")
    if not value > 0:
        raise RuntimeError(f"select_blocks: value > 0 (got {value})")
    keep = torch.empty(B, Hq // G, nb, dtype=torch.uint8, device=logw.device)
    lw = logw.float().contiguous()
    ext().select(lw, torch.ones_like(lw), Hq // G, rule, value, local, keep=keep)
    return keep.view(torch.bool)


def pv(P, v, blk_scale, plan: Plan, num_splits: int | None = None, out_f32: bool = False,
       block_table: torch.Tensor | None = None, T: int | None = None):
    """Two-pass V-skip pass 2 over a plan's lists (kernels/kvskip.py:150-154): [out, out_f32 or None].
    block_table, T (not in the reference): v is a page pool."""
    if num_splits is None:
        num_splits = num_splits_for(P.shape[0] * v.shape[1], plan.max_cnt)
    return ext().pv(P, v, blk_scale, plan.block_idx, plan.block_cnt, int(num_splits), out_f32,
                    **_paged(block_table, T))


def vskip_two_pass(q, k, v, scale: float, rule: str = "topp", value: float = 0.99, local: int = 2,
                   sync: bool = True, out_f32: bool = False, block_table: torch.Tensor | None = None,
                   T: int | None = None) -> dict:
    """Two-pass V-skip (kernels/kvskip.py:157-179). Pass 1 reads K once, writing the block statistics
    and P (its split pass alone: the log-sum-exp merge is not needed); the device selection turns
    the statistics into the kept set and the per-block scales exp(blk_max - lse over the kept set);
    pass 2 reads P and V of the kept blocks. Over a contiguous cache the selection runs inside pass 2
    (kvskip_pv_select: two launches and the merge); over pages it is its own launch (kvskip_select)
    and, with sync=True, the read-back of the longest list sizes pass 2's split count.
    Returns out, keep [B, Hkv, nb] bool and, with sync=True, kept_frac. block_table, T (not in the
    reference): page pools."""
    q = _as_bhd(q)
    B, Hq = q.shape[:2]
    Hkv = k.shape[1]
    first = decode(q, k, v, scale, stats=True, load_v=False, write_p=True, merge=False, **_paged(block_table, T))
    nb = first["blk_max"].shape[-1]
    dev = q.device
    keep = torch.empty(B, Hkv, nb, dtype=torch.uint8, device=dev)
    if block_table is None:
        out, o32 = ext().pv_select(first["p"], v, first["blk_max"], first["blk_sum"], rule, value, local,
                                   num_splits_for(B * Hkv, nb), out_f32, keep=keep)
        res = {"out": out, "keep": keep.view(torch.bool),
               "kept_frac": float(keep.sum()) / (B * Hkv * nb) if sync else None}
        if out_f32:
            res["out_f32"] = o32
        return res
    idx, cnt = _lists(B, Hkv, nb, dev)
    scales = torch.empty(B, Hkv, nb, Hq // Hkv, dtype=torch.float32, device=dev)
    ext().select(first["blk_max"], first["blk_sum"], Hkv, rule, value, local, keep=keep, block_idx=idx,
                 block_cnt=cnt, blk_scale=scales)
    frac = None
    longest = nb
    if sync:
        longest, kept = torch.stack([cnt.max(), cnt.sum()]).tolist()
        frac = kept / (B * Hkv * nb)
    out, o32 = pv(first["p"], v, scales, Plan(idx, cnt, int(longest), nb), out_f32=out_f32,
                  block_table=block_table, T=T)
    res = {"out": out, "keep": keep.view(torch.bool), "kept_frac": frac}
    if out_f32:
        res["out_f32"] = o32
    return res


def vskip_one_pass(q, k, v, scale: float, tau: float = 1e-4, local: int = 2, num_splits: int | None = None,
                   out_f32: bool = False, count: bool = False, lse_prev: torch.Tensor | None = None,
                   sync: bool = True, block_table: torch.Tensor | None = None, T: int | None = None,
                   keep: bool = False) -> dict:
    """Single-pass V-skip (kernels/kvskip.py:182-208): K read once; a block's V is read only if some
    head of the group estimates its weight >= tau, against lse_prev (e.g. the previous step's "lse")
    or else the sink block's log-sum-exp, a lower bound of the normaliser. count=True adds v_tiles
    [B, Hkv] (V blocks read) and, with sync=True, kept_frac. block_table, T (not in the reference):
    page pools. keep=True (not in the reference) adds v_keep: bool [B, Hkv, nb], the blocks whose V
    was read."""
    q = _as_bhd(q)
    B, Hkv = q.shape[0], k.shape[1]
    nb = math.ceil((k.shape[2] if block_table is None else int(T)) / TILE)
    if num_splits is None:
        num_splits = num_splits_for(B * Hkv, nb)
    vk = torch.empty(B, Hkv, nb, dtype=torch.uint8, device=q.device) if keep else None
    out, lse, o32, vt = ext().vskip1(q, k, v, float(scale), float(tau), int(local), int(num_splits), out_f32, count,
                                     lse_prev, **_paged(block_table, T), v_keep=vk)
    res = {"out": out, "lse": lse, "num_splits": num_splits}
    if keep:
        res["v_keep"] = vk.bool()
    if out_f32:
        res["out_f32"] = o32
    if count:
        res["v_tiles"] = vt
        if sync:
            res["kept_frac"] = vt.sum().item() / (B * Hkv * nb)
    return res
