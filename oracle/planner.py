"""Planner oracle (float64, CPU): the refresh policy of the reference's Python planner
`refresh_pre_step` and helpers (src/kvskip_attn.py:166-396), the fused driver's flags
(src/kvskip_attn.py:402-432) and the token index (src/lab.py:149-167, src/run_free.py:103-113).

Test infrastructure only (see oracle/__init__.py). Split into plan() / update() at the same
place as the device kernels (before / after the attention pass) so each device kernel can be
checked on identical inputs; step() composes them with the attention oracle like
refresh_pre_step does. Decisions come with margins: a decision whose deciding quantity lies
within float32 noise of its threshold is reported as borderline.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

from . import attention as A

BLOCK = 64
NEG_INF = float("-inf")
KINDS = {"logit": 0, "add": 1, "peak": 2}
CALIB_EPS = 1e-6


@dataclass
class Policy:
    """KvskipConfig fields the planner reads (src/kvskip_attn.py:116-147), for one layer."""
    delta: float = 0.05
    max_age: int = 32
    level: float = 0.99
    local: int = 2
    calib: float | None = None          # rate of the online correction (None: off)
    calib_kind: str = "logit"
    calib_hold: int = 0
    calib_warm: tuple = ()              # (W, A): max age A during the first W steps
    calib_free: bool = False
    calib_auto_ix: float | None = None
    dense_heads: tuple = ()             # KV heads refreshed on every step
    index_heads: tuple = ()             # KV heads on the token index
    index_union: bool = False


def flags_of(policy: Policy, Hkv: int) -> list[int]:
    """Per-KV-head flags of the fused driver (src/kvskip_attn.py:413-419): bit 0 always exact,
    bit 1 token-index head, bit 2 index union. The bits are OR-ed: a head in both lists keeps
    refresh_pre's decisions (forced refresh, then the index rule, src/kvskip_attn.py:377-383),
    where _pack_fused's assignment would drop the forced refresh of an index-union head."""
    f = [0] * Hkv
    for h in policy.dense_heads:
        f[h] |= 1
    for h in policy.index_heads:
        f[h] |= 4 if policy.index_union else 2
    return f


def max_age_at(policy: Policy, t: int) -> int:
    """src/kvskip_attn.py:295-299."""
    if policy.calib_warm and t < policy.calib_warm[0]:
        return min(policy.max_age, policy.calib_warm[1])
    return policy.max_age


def logit(x):
    """src/kvskip_attn.py:290-292."""
    x = x.clamp(CALIB_EPS, 1.0 - CALIB_EPS)
    return torch.log(x) - torch.log1p(-x)


def pad_blocks(x, nb, value):
    """src/kvskip_attn.py:211-212."""
    return torch.nn.functional.pad(x, (0, nb - x.shape[-1]), value=value) if x.shape[-1] < nb else x


def centroid_sums(k) -> torch.Tensor:
    """Per-block key sums [B, Hkv, nb, D] (src/kvskip_attn.py:170-179)."""
    B, H, T, D = k.shape
    nb = A.nblocks(T)
    kk = torch.nn.functional.pad(k.to(torch.float64), (0, 0, 0, nb * BLOCK - T))
    return kk.reshape(B, H, nb, BLOCK, D).sum(3)


def centroid_scores(q, csum, T, scale) -> torch.Tensor:
    """cs[b, h, blk] = scale * q_h . (csum_blk / n_blk), n = 64 or the partial last block
    (src/kvskip_attn.py:201-208). q [B, Hq, D], csum [B, Hkv, >= nb, D] -> [B, Hq, nb]."""
    nb = A.nblocks(T)
    csum = csum[:, :, :nb].to(torch.float64)
    sizes = torch.full((nb,), float(BLOCK), dtype=torch.float64)
    sizes[-1] = T - BLOCK * (nb - 1)
    c = csum / sizes[None, None, :, None]
    B, Hq, D = q.shape
    Hkv = c.shape[1]
    return torch.einsum("bkgd,bknd->bkgn", q.to(torch.float64).reshape(B, Hkv, Hq // Hkv, D), c).reshape(B, Hq, nb) * scale


def attended_lse(logw, keep, G):
    """Log-sum-exp of block log-weights [B, Hq, nb] over the blocks in keep [B, Hkv, nb]
    (src/kvskip_attn.py:282-284)."""
    return logw.masked_fill(~A.heads(keep, G), NEG_INF).logsumexp(-1)


def topp_union(logw, G, level, local):
    """src/kvskip_attn.py:166-167 -> kernels/kvskip.py:130-147 (rule "topp"), with the per-head
    margins of the cut."""
    B, Hq, nb = logw.shape
    keep_h, margin = A.topp_heads(logw, level)
    keep = keep_h.reshape(B, Hq // G, G, nb).any(2) | A.always_keep(nb, local)
    return keep, margin


@dataclass
class State:
    """Per-layer planner state (src/kvskip_attn.py:339-354, the fields _pack_fused packs)."""
    scale: float
    G: int
    T: int
    csum: torch.Tensor        # [B, Hkv, nb, D]
    keep: torch.Tensor        # [B, Hkv, nb_ref] bool
    lse_ref: torch.Tensor     # [B, Hq, nb_ref]
    cs_ref: torch.Tensor      # [B, Hq, nb_ref]
    lse_att: torch.Tensor     # [B, Hq]
    age: torch.Tensor         # [B, Hkv] int64
    t: int
    calib: torch.Tensor       # [B, Hkv]
    aix: torch.Tensor         # [B, Hkv] bool
    topp_margin: float = math.inf    # smallest top-p margin of any refresh so far
    topp_heads: torch.Tensor | None = None   # [B, Hq] top-p margin of the last update (inf: no refresh)
    log: dict = field(default_factory=dict)


def init(q, k, v, scale, policy: Policy):
    """First decode step: dense + block stats, state initialisation (src/kvskip_attn.py:339-354).
    Returns (state, out [B, Hq, D] float64)."""
    B, Hq, D = q.shape
    Hkv, T = k.shape[1], k.shape[2]
    G = Hq // Hkv
    nb = A.nblocks(T)
    out, _ = A.decode(q, k, v, scale)
    M, S = A.block_stats(q, k, scale)
    logw = A.block_logw(M, S)
    csum = centroid_sums(k)
    keep, margin = topp_union(logw, G, policy.level, policy.local)
    cs = centroid_scores(q, csum, T, scale)
    st = State(scale=scale, G=G, T=T, csum=csum, keep=keep, lse_ref=logw, cs_ref=cs,
               lse_att=attended_lse(logw, keep | A.always_keep(nb, policy.local), G),
               age=torch.zeros(B, Hkv, dtype=torch.int64), t=0, calib=torch.zeros(B, Hkv, dtype=torch.float64),
               aix=torch.zeros(B, Hkv, dtype=torch.bool), topp_margin=float(margin.min()), topp_heads=margin)
    return st, out


def update_csum(st: State, k):
    """Add the keys appended since the last step to their blocks' sums (src/kvskip_attn.py:273-279)."""
    T = k.shape[2]
    nb = A.nblocks(T)
    csum = pad_blocks(st.csum.transpose(2, 3), nb, 0.0).transpose(2, 3).clone()
    for t in range(st.T, T):
        csum[:, :, t // BLOCK] += k[:, :, t].to(torch.float64)
    st.csum, st.T = csum, T


def plan(st: State, q, k, policy: Policy, idx=None) -> dict:
    """Everything refresh_pre_step decides before the attention pass (src/kvskip_attn.py:356-385).
    idx: bool [B, >= nb] token-index blocks of this step (needed with index heads or auto index).
    Mutates st (csum, T, t, age). Returns trig [B, Hkv], read / sel [B, Hkv, nb], miss (the
    uncorrected estimate, = the device's `est`), dec, cs [B, Hq, nb], margin [B, Hkv] (|dec - delta|,
    inf where the refresh is forced by age or flag)."""
    B, Hq, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    update_csum(st, k)
    T = st.T
    nb = A.nblocks(T)
    always = A.always_keep(nb, policy.local)
    stored = pad_blocks(st.keep, nb, False)
    sel = stored | always
    ix = list(policy.index_heads)
    if ix and policy.index_union:
        sel[:, ix] |= idx[:, None, :nb]
    if policy.calib_auto_ix is not None:
        sel |= st.aix[..., None] & idx[:, None, :nb]
    nbr = st.lse_ref.shape[-1]
    cs = centroid_scores(q, st.csum, T, st.scale)
    est = pad_blocks(st.lse_ref + cs[..., :nbr] - st.cs_ref[..., :nbr], nb, NEG_INF)
    unsel = ~sel
    unsel[..., nbr:] = False
    est = est.masked_fill(~A.heads(unsel, G), NEG_INF)
    miss = torch.sigmoid(est.logsumexp(-1) - st.lse_att).reshape(B, Hkv, G).amax(-1)
    st.t += 1
    dec = miss
    if policy.calib is not None and st.t >= policy.calib_hold:
        dec = miss + st.calib if policy.calib_kind in ("add", "peak") else torch.sigmoid(logit(miss) + st.calib)
    st.age += 1
    by_age = st.age >= max_age_at(policy, st.t)
    trig = (dec > policy.delta) | by_age
    forced = torch.zeros(Hkv, dtype=torch.bool)
    for h in policy.dense_heads:
        forced[h] = True
    trig |= forced[None]
    margin = (dec - policy.delta).abs().masked_fill(by_age | forced[None], math.inf)
    read = sel | trig[..., None]
    if ix and not policy.index_union:
        trig[:, ix] = False
        margin[:, ix] = math.inf
        read[:, ix] = (idx[:, :nb] | always)[:, None, :]
    return dict(trig=trig, read=read, sel=sel, miss=miss, dec=dec, cs=cs, margin=margin, nb=nb)


def update(st: State, pr: dict, logw, policy: Policy):
    """Everything refresh_pre_step does after the pass (src/kvskip_attn.py:387-391): calibration
    (src/kvskip_attn.py:302-319), new stored sets / references of the refreshing heads
    (src/kvskip_attn.py:182-198), attended log-sum-exp. logw [B, Hq, nb] = block log-weights of
    this step's pass (-inf where not read)."""
    B, Hq, nb = logw.shape
    G = st.G
    trig = pr["trig"]
    if policy.calib is not None:
        hsel = A.heads(pr["sel"], G)
        lin = logw.masked_fill(~hsel, NEG_INF).logsumexp(-1)
        lout = logw.masked_fill(hsel, NEG_INF).logsumexp(-1)
        real = torch.sigmoid(lout - lin).reshape(B, -1, G).amax(-1)
        est = pr["miss"]
        resid = logit(real) - logit(est) if policy.calib_kind == "logit" else real - est
        if policy.calib_kind == "peak":
            new = torch.maximum((1.0 - policy.calib) * st.calib, resid)
        else:
            new = (1.0 - policy.calib) * st.calib + policy.calib * resid
        if not policy.calib_free:
            new = new.clamp_min(0.0)
        st.calib = torch.where(trig, new, st.calib)
        if policy.calib_auto_ix is not None:
            st.aix = st.aix | (st.calib > policy.calib_auto_ix)
    keep_new, margin = topp_union(logw, G, policy.level, policy.local)
    hq = trig.repeat_interleave(G, dim=1)
    st.keep = torch.where(trig[..., None], keep_new, pad_blocks(st.keep, nb, False))
    st.lse_ref = torch.where(hq[..., None], logw, pad_blocks(st.lse_ref, nb, NEG_INF))
    st.cs_ref = torch.where(hq[..., None], pr["cs"], pad_blocks(st.cs_ref, nb, 0.0))
    st.age = torch.where(trig, torch.zeros_like(st.age), st.age)
    st.topp_heads = margin.masked_fill(~hq, math.inf)
    if bool(trig.any()):
        st.topp_margin = min(st.topp_margin, float(margin[hq].min()))
    st.lse_att = attended_lse(logw, st.keep | A.always_keep(nb, policy.local), G)


def step(st: State, q, k, v, policy: Policy, idx=None, dtype=torch.float64):
    """One decode step after the first (src/kvskip_attn.py:356-396). Returns (out, plan dict).
    dtype: the attention pass's arithmetic (float32 for the timed CPU baseline; the checks use
    float64); the planner's own arithmetic stays float64."""
    pr = plan(st, q, k, policy, idx)
    out, _ = A.decode(q, k, v, st.scale, keep=pr["read"], dtype=dtype)
    M, S = A.block_stats(q, k, st.scale, keep=pr["read"], dtype=dtype)
    update(st, pr, A.block_logw(M.double(), S.double()), policy)
    return out, pr


def post_step(st: State, q, k, v, policy: Policy, dtype=torch.float64):
    """One decode step after the first of the reference's "refresh" mode (src/kvskip_attn.py:233-270):
    attend the stored set + sink + local blocks, then decide with THIS step's attended
    log-sum-exp (not the previous step's, as refresh_pre_step does) and give each refreshing head
    a dense + statistics pass whose output replaces its masked one; the refreshing heads' sets and
    references are rebuilt from that pass (src/kvskip_attn.py:182-198). The mode knows no
    calibration, token index or warm-up age (src/kvskip_attn.py:251-254): policy must have none.
    Reuses plan() with st.lse_att set to the pass's log-sum-exp (the estimate, age and trigger
    arithmetic of src/kvskip_attn.py:241-254 is the same as :366-376) and update() for the rebuild
    (its attended log-sum-exp is not read by this mode). Returns (out, plan dict + "lse" of the
    masked pass + "attended", the blocks that pass read)."""
    assert policy.calib is None and not policy.index_heads and not policy.calib_warm \
        and policy.calib_auto_ix is None, "the refresh mode has no calibration, index or warm-up"
    update_csum(st, k)
    nb = A.nblocks(st.T)
    sel = pad_blocks(st.keep, nb, False) | A.always_keep(nb, policy.local)
    out, lse = A.decode(q, k, v, st.scale, keep=sel, dtype=dtype)
    st.lse_att = lse.to(torch.float64)
    pr = plan(st, q, k, policy)
    trig = pr["trig"]
    full = trig[..., None].expand(*trig.shape, nb)
    out2, _ = A.decode(q, k, v, st.scale, keep=full, dtype=dtype)
    out = torch.where(A.heads(trig, st.G)[..., None], out2, out)
    M, S = A.block_stats(q, k, st.scale, keep=full, dtype=dtype)
    update(st, pr, A.block_logw(M.double(), S.double()), policy)
    pr["read"] = sel | trig[..., None]
    pr["attended"] = sel
    pr["lse"] = lse
    return out, pr


# ---------------------------------------------------------------- token index

def index_blocks(ids: np.ndarray, T: int) -> np.ndarray:
    """Token-index blocks of the step whose current token is ids[:, T-1]: bool [B, nb], a block
    is hit if it holds an earlier copy of the current token or the position right after one
    (src/run_free.py:103-113; per step of src/lab.py:149-167)."""
    ids = np.asarray(ids)[:, :T]
    cur = ids[:, T - 1:T]
    same = np.zeros_like(ids, dtype=bool)
    same[:, :T - 1] = ids[:, :T - 1] == cur
    pos = same.copy()
    pos[:, 1:] |= same[:, :T - 1]
    nb = A.nblocks(T)
    pad = np.zeros((ids.shape[0], nb * BLOCK), dtype=bool)
    pad[:, :T] = pos
    return pad.reshape(ids.shape[0], nb, BLOCK).any(-1)
