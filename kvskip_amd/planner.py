"""Device-side refresh planner loop of one attention layer: the reference's "refresh_fused" mode
(src/kvskip_attn.py:399-478) on the kvskip_amd kernels, with the first step initialised on the
device too (the reference runs its Python planner for it, src/kvskip_attn.py:445-450).

Per decode step: plan (estimate, refresh decision, block list) -> masked + block-statistics
attention over the list -> update (top-p union, references, calibration, attended log-sum-exp).
Three launches per layer-step unless the batch is ragged (plan's scores pass; the split pass,
whose workgroups also make plan's decision from the scores partials, kvskip_decode_splits_planned;
the split merge and update together), four for a ragged batch (plan's decision in a launch of its
own; seq_lens with one sequence is not ragged), all on
the current stream, no host synchronisation, no allocation after the first step of a capacity: the
pass writes into buffers the planner owns. With an UpdateCarrier shared by the planners of a
model's layers, a layer's update instead runs inside the next layer's split pass and the merge runs
alone.

The policy fields follow KvskipConfig (src/kvskip_attn.py:116-147) for one layer.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import ext as E
from . import kvskip as K

TILE = 64
MARGIN = 64                      # spare block capacity of the state (src/kvskip_attn.py:399)
BALANCE_MAX_LISTS = 16           # (b, KV head) lists a balanced planned pass decides in every workgroup
RAGGED_DECIDE_MAX_B = 16         # sequences of a ragged batch whose lists a planned pass decides per KV head
GLOBAL_PARTITION_MAX_LISTS = 512  # B * Hkv bound of kvskip_attn_args.list_partition = 1
GLOBAL_PARTITION_MAX_B = 64        # sequences up to which the planner cuts all heads' lists together
POST_MAX_SLOTS = 64              # first-pass partial slots the refresh mode's decision reads (lse_slots)
KINDS = {"logit": 0, "add": 1, "peak": 2}


@dataclass
class Policy:
    delta: float = 0.05
    max_age: int = 32
    level: float = 0.99
    local: int = 2
    calib: float | None = None          # rate of the online correction of the estimate (None: off)
    calib_kind: str = "logit"           # "logit" | "add" | "peak"
    calib_hold: int = 0                 # decode steps before the correction is applied
    calib_warm: tuple = ()              # (W, A): max age A during the first W decode steps
    calib_free: bool = False            # allow negative corrections
    calib_auto_ix: float | None = None  # heads whose correction exceeds this join the token index
    dense_heads: tuple = ()             # KV heads refreshed (= exact) on every step
    index_heads: tuple = ()             # KV heads on the token index
    index_union: bool = False           # index blocks join the attended set instead of replacing it

    def flags(self, Hkv: int) -> list[int]:
        """Per-KV-head bits of the plan / update kernels (src/kvskip_attn.py:413-419): 1 refreshed on
        every step, 2 token-index head (reads index + sink + local, never refreshes), 4 index union.
        OR-ed, so a head in both lists decides as refresh_pre does (src/kvskip_attn.py:377-383)."""
        f = [0] * Hkv
        for h in self.dense_heads:
            f[h] |= 1
        for h in self.index_heads:
            f[h] |= 4 if self.index_union else 2
        return f

    def max_age_at(self, t: int) -> int:
        """src/kvskip_attn.py:295-299."""
        if self.calib_warm and t < self.calib_warm[0]:
            return min(self.max_age, self.calib_warm[1])
        return self.max_age

    @property
    def needs_index(self) -> bool:
        return bool(self.index_heads) or self.calib_auto_ix is not None


def _require_ids(ids, T):
    if not (ids.is_cuda and ids.dtype == torch.int32 and ids.dim() == 2 and ids.stride(1) == 1 and ids.shape[1] >= T):
        raise RuntimeError("ids: CUDA int32 [B, >= T]")


class UpdateCarrier:
    """Holds the update of the layer that stepped last until the next layer's split pass carries it
    (kvskip_decode_splits_update): a layer's update reads only its own statistics and is read only
    by its own next plan, so it can run under another layer's streaming. Share one carrier between
    the FusedPlanners of a model's layers. A planner flushes its own pending update before it plans
    again; call flush() before reading planner state on the host or from another stream. A ready
    idx buffer handed to step() must stay unchanged until the update has been launched (seq_lens
    may change: the update reads the plan's copy of the step's lengths)."""

    def __init__(self):
        self.pending = None          # (planner, G, UpdateArgs, tensors the struct points into)

    def take(self, planner, G):
        """The pending update if `planner`'s pass can carry it (another planner, same group size);
        a pending update it cannot carry is launched on its own first."""
        p = self.pending
        if p is None:
            return None
        if p[0] is planner or p[1] != G:
            self.flush()
            return None
        self.pending = None
        return p[2]

    def put(self, planner, G, update, refs):
        self.flush()
        self.pending = (planner, G, update, refs)

    def flush(self, planner=None):
        """Launch the pending update on its own (only `planner`'s, if given)."""
        p = self.pending
        if p is None or (planner is not None and p[0] is not planner):
            return
        self.pending = None
        E.launch_update(p[2], p[3][0]["keep"].device)


class FusedPlanner:
    """Planner state of one layer in device memory (the fields of src/kvskip_attn.py:420-432) and
    its step. Usage: out = p.first(q, k, v, scale) on the first decode step, then
    out = p.step(q, k, v, scale, idx=...) on every later one (k, v grown by one token)."""

    def __init__(self, policy: Policy, count: bool = True, carrier: UpdateCarrier | None = None,
                 decide_in_pass: bool = True, balance: bool = True, batch_balance: bool = True,
                 ragged_in_pass: bool | None = None, global_partition: bool = True, plan_one_launch: bool = False):
        self.policy = policy
        self.carrier = carrier      # shared by the layers: updates ride on the next layer's pass
        # plan's decision inside the masked pass: one launch fewer per step, the same decisions and
        # lists as plan's own decision launch
        self.decide_in_pass = decide_in_pass
        # a ragged batch (seq_lens, B > 1) of a contiguous cache: every workgroup of the pass decides
        # its KV head's B lists (B <= RAGGED_DECIDE_MAX_B), and the lists are cut per KV head. None
        # (the default): never, plan decides in its own launch and the pass cuts the lists of all
        # heads together (global_partition; measured per layer-step: config 4's shape at B 8 with
        # stable queries 92.7 -> 75.9 us, at B 8 180.7 -> 177.8, config 5 135.5 -> 132.9)
        self.ragged_in_pass = ragged_in_pass
        # with the decision in the pass and B * Hkv <= 16: the lists of all heads cut by one chunk
        # length (kvskip_plan_args.pass_budget), so a refreshing head gets more workgroups than a
        # light one; the partials get twice the split count's slots
        self.balance = balance
        # a batch of B > 1 with more than BALANCE_MAX_LISTS lists: the lists are cut over the batch
        # (the ragged partition, each KV head's lists of all sequences together) by passing the
        # lengths, all T, as seq_lens; a refreshing head of one sequence then no longer sets the
        # pass's time alone
        self.batch_balance = batch_balance
        # a ragged batch of <= GLOBAL_PARTITION_MAX_B sequences whose lists plan decided: the lists
        # of every KV head cut by one chunk length (kvskip_attn_args.list_partition = 1), so a head
        # with refreshing sequences gets more workgroups instead of longer chunks (at B 8 the
        # per-head cut's longest chunk was 1.8x the global one's; per layer-step B 8 stable 94.1 ->
        # 73.9 us, B 32 at 64k 651 -> 630, config 5 132.4 -> 131.5)
        self.global_partition = global_partition
        # plan with its decision in the scores launch (kvskip_plan_args.ticket): each head decided by
        # its last scores workgroup, one launch instead of two where plan decides. Off by default:
        # graph-replayed, the last workgroup's chain (its partial stores acknowledged at the device's
        # coherence point, the ticket's round trip, the partials read past L2) cost more than the
        # launch it saves (per layer-step: B 8 stable 75.9 -> 77.9 us, config 5 132.9 -> 134.1); it
        # saves a launch's host time where a loop is not captured
        self.plan_one_launch = plan_one_launch
        self._lp = 0
        self._pargs = None
        self._pg = {}               # this step's paged cache (block_table, T), if any
        self.state = None
        self.t = 0
        self.T = 0
        self.count = count          # per-step counters as device tensors (off under graph capture)
        self.counters = {}
        self.bufs = None

    # -- state
    def _alloc(self, q, k, NBC):
        B, Hq, D = q.shape
        Hkv = k.shape[1]
        dev = q.device
        f32 = dict(dtype=torch.float32, device=dev)
        self.NBC = NBC
        self.state = dict(
            csum=torch.zeros(B, Hkv, NBC, D, **f32),
            lse_ref=torch.full((B, Hq, NBC), -math.inf, **f32),
            cs_ref=torch.zeros(B, Hq, NBC, **f32),
            keep=torch.zeros(B, Hkv, NBC, dtype=torch.uint8, device=dev),
            lse_att=torch.zeros(B, Hq, **f32),
            age=torch.zeros(B, Hkv, dtype=torch.int32, device=dev),
            flags=torch.tensor(self.policy.flags(Hkv), dtype=torch.int32, device=dev),
            cs_now=torch.zeros(B, Hq, NBC, **f32),
            trig=torch.zeros(B, Hkv, dtype=torch.uint8, device=dev),
            block_idx=torch.zeros(B, Hkv, NBC, dtype=torch.int32, device=dev),
            block_cnt=torch.zeros(B, Hkv, dtype=torch.int32, device=dev),
            calib=torch.zeros(B, Hkv, **f32),
            est=torch.zeros(B, Hkv, **f32),
            aix=torch.zeros(B, Hkv, dtype=torch.uint8, device=dev),
            idx=torch.zeros(B, NBC, dtype=torch.uint8, device=dev),
            tlen=torch.zeros(B, dtype=torch.int32, device=dev),       # this step's lengths (ragged)
            lens=torch.zeros(B, dtype=torch.int32, device=dev),       # all T, for batch_balance
            part=torch.empty(E.plan_part_floats(B, Hq, Hkv, NBC), **f32),     # multi-workgroup plan
            ticket=torch.zeros(B * Hkv, dtype=torch.int32, device=dev),      # one-launch plan (self-resetting)
        )

    def _grow(self, NBC):
        """src/kvskip_attn.py:435-442."""
        fills = dict(keep=0, lse_ref=-math.inf, cs_ref=0.0, csum=0.0, cs_now=0.0, block_idx=0)
        for key, fill in fills.items():
            x = self.state[key]
            out = torch.full((*x.shape[:2], NBC, *x.shape[3:]), fill, dtype=x.dtype, device=x.device)
            out[:, :, :x.shape[2]] = x
            self.state[key] = out
        idx = torch.zeros(self.state["idx"].shape[0], NBC, dtype=torch.uint8, device=self.state["idx"].device)
        self.state["idx"] = idx
        B, Hq = self.state["lse_att"].shape
        Hkv = self.state["keep"].shape[1]
        self.state["part"] = torch.empty(E.plan_part_floats(B, Hq, Hkv, NBC), dtype=torch.float32, device=idx.device)
        self.NBC = NBC

    def _attend(self, q, k, v, scale, nb, seq_lens=None):
        pg = self._pg
        """Split pass (masked + statistics) over the plan's lists into the planner's buffers.
        Returns out [B, Hq, D] (valid until the next step; written by _finish when the pass is
        split) and the [B, Hq, nb] statistics views."""
        B, Hq, D = q.shape
        Hkv = k.shape[1]
        carried = self.carrier.take(self, Hq // Hkv) if self.carrier is not None else None
        # one sequence (its length in device memory) is split as an unragged batch
        S = (K.num_splits_for(B * Hkv, nb) if seq_lens is None or B == 1
             else K.ragged_splits(B, Hkv, nb, G=Hq // Hkv, carry=carried is not None))
        if seq_lens is not None and B > 16 and Hq // Hkv <= 4:
            # many lists: twice the chunk slots, so that the queued workgroups even out the chunks'
            # lengths (B 32 at 64k, all lists cut together: 629 -> 607 us per layer-step; 168 slots
            # 609; at B 8 56 stays best: 73.9 vs 78.7 at 84)
            S = min(256, 2 * S)
        budget = 0
        if (self._pargs is not None and self.balance and B * Hkv <= BALANCE_MAX_LISTS and S > 1
                and (seq_lens is None or B == 1)):
            # workgroups: S per head less the partition's B*Hkv spare chunks and room for a carried
            # update of this shape, so that the pass fits the CUs the per-head split fills (a CU
            # given a second full chunk would double the critical path); the same with and without
            # a carried update, so both cut the lists alike. S becomes the partial slots per head.
            budget, S = max(S * B * Hkv - 2 * B * Hkv, B * Hkv), min(2 * S, 256)
        S_buf = S
        if seq_lens is not None and B > 1 and Hq // Hkv > 4:
            # the budget differs with and without a carried update: partials room for the larger,
            # so that a step allocates nothing either way
            S_buf = max(S, K.ragged_splits(B, Hkv, nb, G=Hq // Hkv))
        n_st, n_part = B * Hq * self.NBC, B * Hq * S_buf * D
        b = self.bufs
        if b is None or b["blk_max"].numel() < n_st or b["part_acc"].numel() < n_part or b["out"].shape != q.shape:
            dev = q.device
            f32 = dict(dtype=torch.float32, device=dev)
            b = self.bufs = dict(out=torch.empty(B, Hq, D, dtype=torch.bfloat16, device=dev),
                                 lse=torch.empty(B, Hq, **f32), blk_max=torch.empty(n_st, **f32),
                                 blk_sum=torch.empty(n_st, **f32), part_acc=torch.empty(n_part, **f32),
                                 part_ml=torch.empty(B * Hq * S_buf * 2, **f32))
        s = self.state
        self._S = S
        self._lp = lp = int(self._pargs is None and self.global_partition and seq_lens is not None
                            and 1 < B <= GLOBAL_PARTITION_MAX_B and B * Hkv <= GLOBAL_PARTITION_MAX_LISTS)
        if self._pargs is not None:
            self._pargs.pass_budget = budget
            E.decode_splits_planned(q, k, v, scale, b, self._pargs, S, carried, seq_lens, **pg)
        elif carried is not None:
            E.decode_splits_update(q, k, v, scale, b, s["block_idx"], s["block_cnt"], S, carried, seq_lens,
                                   list_partition=lp, **pg)
        else:
            E.decode_into(q, k, v, scale, b, s["block_idx"], s["block_cnt"], stats=True, num_splits=S,
                          seq_lens=seq_lens, phase=1 if S > 1 else 3, list_partition=lp, **pg)
        n = B * Hq * nb
        return b["out"], b["blk_max"][:n].view(B, Hq, nb), b["blk_sum"][:n].view(B, Hq, nb)

    def _finish(self, q, k, v, scale, seq_lens, update_args, update_kwargs):
        """The pass's split merge and the planner update: one launch (kvskip_merge_update) when
        the pass was split, else the update alone; with a carrier, the merge alone and the update
        left to the next layer's pass."""
        s = self.state
        if self.carrier is not None:
            if self._S > 1:
                E.decode_into(q, k, v, scale, self.bufs, s["block_idx"], s["block_cnt"], stats=True,
                              num_splits=self._S, seq_lens=seq_lens, phase=2, list_partition=self._lp, **self._pg)
            G = q.shape[1] // k.shape[1]
            self.carrier.put(self, G, E.update_struct(*update_args, **update_kwargs),
                             (dict(s), self.bufs, update_args, update_kwargs))
            return
        if self._S > 1:
            E.merge_update(q, k, v, scale, self.bufs, self._S, update_args, update_kwargs, s["block_idx"],
                           s["block_cnt"], seq_lens, list_partition=self._lp, **self._pg)
        else:
            E.update(*update_args, **update_kwargs)

    def _plan(self, q, plan_args, plan_kwargs, seq_lens):
        """plan (scores + decision), or, with decide_in_pass, its scores pass alone: the decision then
        runs in the masked pass (kvskip_decode_splits_planned) and the update advances the age. A
        ragged batch decides in the pass as ragged_in_pass says (up to RAGGED_DECIDE_MAX_B sequences
        of a contiguous cache: every workgroup decides its KV head's lists over the batch); else plan
        decides."""
        B = q.shape[0]
        rag = bool(self.ragged_in_pass)
        if self.decide_in_pass and (seq_lens is None or B == 1
                                    or (rag and B <= RAGGED_DECIDE_MAX_B and not self._pg)):
            self._pargs = E.plan_struct(*plan_args, **plan_kwargs)
            E.plan_scores(self._pargs, q.device)
        else:
            self._pargs = None
            E.plan(*plan_args, ticket=self.state["ticket"] if self.plan_one_launch else None, **plan_kwargs)

    def _age(self):
        return dict(age=self.state["age"]) if self._pargs is not None else {}

    def _batch_lens(self, B, Hkv, T, seq_lens, block_table):
        """seq_lens, or (batch_balance, B > 1, more than BALANCE_MAX_LISTS lists, contiguous cache)
        the state's length buffer filled with T, so the passes cut the lists over the batch."""
        if (seq_lens is not None or block_table is not None or not self.batch_balance or B < 2
                or B * Hkv <= BALANCE_MAX_LISTS):
            return seq_lens
        self.state["lens"].fill_(T)
        return self.state["lens"]

    def _tlen(self, seq_lens):
        """The update's lengths: the plan's copy of seq_lens in the planner's state (rewritten only
        by this layer's next plan), so a carried update reads this step's lengths even after the
        caller has advanced seq_lens."""
        return None if seq_lens is None else self.state["tlen"]

    def _count(self, key, value):
        if self.count:
            self.counters[key] = self.counters.get(key, 0) + value

    def _set_idx(self, idx, ids, T, seq_lens=None):
        """This step's token-index blocks into state['idx'] ([B, NBC] uint8): from idx (bool / uint8
        [B, >= nb]) or from token ids [B, >= T] int32 with the device token-index kernel."""
        s = self.state
        nb = math.ceil(T / TILE)
        if ids is not None:
            E.token_index(ids, T, self.NBC, out=s["idx"], seq_lens=seq_lens)
        elif idx is not None and idx.dtype == torch.uint8 and idx.is_contiguous() and idx.shape[1] == self.NBC:
            return idx                                               # a ready [B, NBC] device buffer
        elif idx is not None:
            s["idx"].zero_()
            s["idx"][:, :nb] = idx[:, :nb].to(torch.uint8)
        else:
            raise RuntimeError("this policy needs the token index: pass idx or ids")
        return s["idx"]

    # -- steps
    def first(self, q, k, v, scale, seq_lens=None, block_table=None, T=None):
        """First decode step: dense + block statistics and the state initialisation
        (src/kvskip_attn.py:339-354), on the device: per-block key sums of the prefix, a plan that
        refreshes every head, the attention pass, and an update without calibration.
        seq_lens (int32 [B] on the device): a ragged batch; k, v are then views of a common
        capacity and sequence b holds seq_lens[b] tokens (every later step appends one to each).
        block_table, T (not in the reference): a paged cache, k, v page pools [num_pages, Hkv, 64, D]
        and block_table int32 [B, >= ceil(T / 64)] on the device, T the tokens (the capacity with
        seq_lens)."""
        if q.dim() == 4:
            q = q.squeeze(2)
        B, Hq, D = q.shape
        self._pg = {} if block_table is None else dict(block_table=block_table, T=int(T))
        Hkv, T = k.shape[1], (k.shape[2] if block_table is None else int(T))
        nb = math.ceil(T / TILE)
        self.flush()
        self._alloc(q, k, nb + MARGIN)
        s = self.state
        seq_lens = self._batch_lens(B, Hkv, T, seq_lens, block_table)
        E.block_sums(k, self.NBC, out=s["csum"], seq_lens=seq_lens, **self._pg)
        every = torch.ones(Hkv, dtype=torch.int32, device=q.device)      # refresh all, no index heads
        pol = self.policy
        self._plan(q, (q, k, s["csum"], s["lse_ref"], s["cs_ref"], s["keep"], s["lse_att"], s["age"], every,
                       s["cs_now"], s["trig"], s["block_idx"], s["block_cnt"], float(scale), float(pol.delta),
                       int(pol.max_age), int(pol.local), False),
                   dict(part=s["part"], seq_lens=seq_lens, seq_lens_out=self._tlen(seq_lens), **self._pg), seq_lens)
        out, bmax, bsum = self._attend(q, k, v, scale, nb, seq_lens)
        self._finish(q, k, v, scale, seq_lens,
                     (bmax, bsum, s["trig"], s["cs_now"], s["keep"], s["lse_ref"], s["cs_ref"], s["lse_att"], T,
                      float(pol.level), int(pol.local), every),
                     dict(list_stats=True, seq_lens=self._tlen(seq_lens), **self._age()))
        self.t, self.T = 0, T
        self.ragged = seq_lens is not None and seq_lens is not s["lens"]
        if self.count:
            total = B * Hkv * nb if seq_lens is None else ((seq_lens + TILE - 1) // TILE).sum() * Hkv
            self._count("dense_heads", B * Hkv)
            self._count("blocks_read", total)
            self._count("blocks_total", total)
        return out

    def step(self, q, k, v, scale, idx=None, ids=None, seq_lens=None, block_table=None, T=None):
        """One later decode step (src/kvskip_attn.py:451-478): plan -> masked + stats attention ->
        update. idx: this step's token-index blocks (bool [B, >= nb], or a uint8 [B, NBC] device
        buffer used as is) or ids: token ids [B, >= T] int32 (index heads / auto index only).
        seq_lens: the ragged batch's lengths after this step's token (one more per sequence).
        block_table, T: a paged cache, as in first()."""
        if self.state is None:
            return self.first(q, k, v, scale, seq_lens, block_table=block_table, T=T)
        if q.dim() == 4:
            q = q.squeeze(2)
        B, Hq, D = q.shape
        self._pg = {} if block_table is None else dict(block_table=block_table, T=int(T))
        Hkv, T = k.shape[1], (k.shape[2] if block_table is None else int(T))
        nb = math.ceil(T / TILE)
        self.flush()                                                  # this layer's last update
        if nb > self.NBC:
            self._grow(nb + MARGIN)
        s = self.state
        pol = self.policy
        if seq_lens is not None:
            add_token = True                                          # one token per sequence per step
        else:
            add_token = T == self.T + 1
            if not add_token and T != self.T:
                E.block_sums(k, self.NBC, out=s["csum"], **self._pg)  # several tokens appended: resum
        self.t += 1
        self.T = T
        seq_lens = self._batch_lens(B, Hkv, T, seq_lens, block_table)
        fuse_ix = pol.needs_index and ids is not None and idx is None     # the plan finds the index itself
        if fuse_ix:
            _require_ids(ids, T)
            ix = s["idx"]
        else:
            ix = self._set_idx(idx, ids, T, seq_lens) if pol.needs_index else None
        cal = pol.calib is not None
        kind = KINDS[pol.calib_kind]
        self._plan(q, (q, k, s["csum"], s["lse_ref"], s["cs_ref"], s["keep"], s["lse_att"], s["age"], s["flags"],
                       s["cs_now"], s["trig"], s["block_idx"], s["block_cnt"], float(scale), float(pol.delta),
                       int(pol.max_age_at(self.t)), int(pol.local), add_token, None if fuse_ix else ix,
                       s["calib"] if cal else None, s["est"], cal and self.t >= pol.calib_hold, kind,
                       s["aix"] if pol.calib_auto_ix is not None else None),
                   dict(part=s["part"], seq_lens=seq_lens, seq_lens_out=self._tlen(seq_lens),
                        ids=ids if fuse_ix else None, idx_out=ix if fuse_ix else None, **self._pg), seq_lens)
        out, bmax, bsum = self._attend(q, k, v, scale, nb, seq_lens)
        self._finish(q, k, v, scale, seq_lens,
                     (bmax, bsum, s["trig"], s["cs_now"], s["keep"], s["lse_ref"], s["cs_ref"], s["lse_att"], T,
                      float(pol.level), int(pol.local), s["flags"], ix, s["est"], s["calib"] if cal else None,
                      float(pol.calib or 0.0), bool(pol.calib_free), kind,
                      s["aix"] if pol.calib_auto_ix is not None else None, float(pol.calib_auto_ix or 0.0)),
                     dict(list_stats=True, seq_lens=self._tlen(seq_lens), **self._age()))
        if self.count:
            self._count("blocks_read", s["block_cnt"].sum())
            self._count("blocks_total", B * Hkv * nb if seq_lens is None
                        else ((seq_lens + TILE - 1) // TILE).sum() * Hkv)
            self._count("masked_heads", B * Hkv)
            self._count("dense_heads", s["trig"].sum())
        return out

    def flush(self):
        """Launch this planner's update if a carrier still holds it (before reading its state)."""
        if self.carrier is not None:
            self.carrier.flush(self)

    def read_mask(self, nb):
        """Blocks read this step per (b, KV head): bool [B, Hkv, nb] (host-side view for checks)."""
        s = self.state
        bi, bc = s["block_idx"], s["block_cnt"]
        B, H, n = bi.shape
        ar = torch.arange(n, device=bi.device)
        valid = ar[None, None, :] < bc[..., None]
        m = torch.zeros(B, H, n + 1, dtype=torch.bool, device=bi.device)
        m.scatter_(-1, torch.where(valid, bi.long(), n), True)
        return m[..., :nb]


class PostPlanner(FusedPlanner):
    """The reference's "refresh" mode (src/kvskip_attn.py:215-270) on the device: the trigger is
    decided AFTER a masked pass over the stored sets, against that pass's own log-sum-exp, and a
    refreshing head's output is then its attention over every block (with the statistics of every
    block, from which the update rebuilds its set).
    Per later step, four launches on the current stream, no host synchronisation: plan's scores pass
    (estimate partials, the appended key's sum) -> the masked + statistics split pass over the
    attended sets (kvskip_decode_splits_planned, DECIDE_LISTS: every workgroup takes its list from
    the scores partials) into partial slots [0, S) -> the refresh pass (DECIDE_POST: every workgroup
    merges the first pass's partials of its heads into their log-sum-exp, decides against it, and a
    refreshing head reads the blocks OUTSIDE its attended set) into slots [S, 2S) -> one split merge
    over the 2S slots with the update of the refreshing heads. A head that does not refresh has only
    first-pass partials, so its output is its masked attention; a refreshing head's merge joins its
    attended and its other blocks, so every block is read once per step (the reference reads the
    attended blocks of a refreshing head twice, and counts them twice).
    Up to BALANCE_MAX_LISTS lists, both passes cut all lists by one chunk length (pass_budget), so a
    single refreshing head's blocks spread over the whole GPU. With an UpdateCarrier shared by the
    layers' planners, the update runs inside the next layer's first pass instead (the merge then
    runs alone), as FusedPlanner's does. The first step is FusedPlanner.first (dense + statistics and
    the state initialisation, src/kvskip_attn.py:223-231). The mode has no calibration, token index or
    warm-up age, and takes contiguous caches without seq_lens (as the reference's, which reads
    k.shape[2] as every sequence's length)."""

    def __init__(self, policy: Policy, count: bool = True, carrier: UpdateCarrier | None = None, balance: bool = True):
        if (policy.calib is not None or policy.index_heads or policy.calib_warm
                or policy.calib_auto_ix is not None):
            raise ValueError("the refresh mode has no calibration, token index or warm-up age")
        super().__init__(policy, count, carrier=carrier, decide_in_pass=False, balance=balance, batch_balance=False)
        self.post = None

    def _post_bufs(self, q, S):
        """Buffers of both passes: out / lse of the merge, statistics, and 2 S partial slots per
        query head (the first pass's S, then the refresh pass's S)."""
        B, Hq, D = q.shape
        p = self.post
        n_st = B * Hq * self.NBC
        if (p is None or p["blk_max"].numel() < n_st or p["part_acc"].numel() < B * Hq * 2 * S * D
                or p["out"].shape != q.shape):
            dev = q.device
            f32 = dict(dtype=torch.float32, device=dev)
            p = self.post = dict(out=torch.empty(B, Hq, D, dtype=torch.bfloat16, device=dev),
                                 lse=torch.empty(B, Hq, **f32),
                                 blk_max=torch.empty(n_st, **f32), blk_sum=torch.empty(n_st, **f32),
                                 part_acc=torch.empty(B * Hq * 2 * S * D, **f32),
                                 part_ml=torch.empty(B * Hq * 2 * S * 2, **f32))
        return p

    def step(self, q, k, v, scale, seq_lens=None, block_table=None, T=None):
        """One decode step (k, v grown by one token, or several: the key sums are then rebuilt).
        Returns out [B, Hq, D], valid until the next step."""
        if seq_lens is not None or block_table is not None:
            raise ValueError("the refresh mode takes a contiguous cache without seq_lens")
        if self.state is None:
            return self.first(q, k, v, scale)
        if q.dim() == 4:
            q = q.squeeze(2)
        B, Hq, D = q.shape
        Hkv, T = k.shape[1], k.shape[2]
        nb = math.ceil(T / TILE)
        dev = q.device
        self.flush()                                                  # this layer's last update
        if nb > self.NBC:
            self._grow(nb + MARGIN)
        s = self.state
        pol = self.policy
        G = Hq // Hkv
        add_token = T == self.T + 1
        if not add_token and T != self.T:
            E.block_sums(k, self.NBC, out=s["csum"])
        self.t += 1
        self.T = T
        # 2 S slots per head in all; the refresh pass's decision merges the first pass's S slots into
        # its attended log-sum-exp, at most POST_MAX_SLOTS of them
        S = min(K.num_splits_for(B * Hkv, nb), POST_MAX_SLOTS)
        budget = 0
        if self.balance and B * Hkv <= BALANCE_MAX_LISTS and S > 1:
            budget, S = max(S * B * Hkv - 2 * B * Hkv, B * Hkv), min(2 * S, POST_MAX_SLOTS)
        b = self._post_bufs(q, S)
        pargs = E.plan_struct(q, k, s["csum"], s["lse_ref"], s["cs_ref"], s["keep"], s["lse_att"], s["age"],
                              s["flags"], s["cs_now"], s["trig"], s["block_idx"], s["block_cnt"], float(scale),
                              float(pol.delta), int(pol.max_age), int(pol.local), add_token, est=s["est"],
                              part=s["part"])
        pargs.pass_budget = budget
        pargs.slot_count = S
        E.plan_scores(pargs, dev)
        pargs.decide_mode, pargs.slot_base = E.DECIDE_LISTS, 0
        carried = self.carrier.take(self, G) if self.carrier is not None else None
        E.decode_splits_planned(q, k, v, scale, b, pargs, 2 * S, carried)
        if self.count:
            self._count("blocks_read", s["block_cnt"].sum())
        pargs.decide_mode, pargs.slot_base = E.DECIDE_POST, S
        pargs.lse_part, pargs.lse_slots, pargs.lse_stride = b["part_ml"].data_ptr(), S, 2 * S
        E.decode_splits_planned(q, k, v, scale, b, pargs, 2 * S)
        n = B * Hq * nb
        uargs = (b["blk_max"][:n].view(B, Hq, nb), b["blk_sum"][:n].view(B, Hq, nb), s["trig"], s["cs_now"],
                 s["keep"], s["lse_ref"], s["cs_ref"], s["lse_att"], T, float(pol.level), int(pol.local), s["flags"])
        ukw = dict(list_stats=True, age=s["age"])
        if self.carrier is not None:
            E.decode_into(q, k, v, scale, b, s["block_idx"], s["block_cnt"], stats=True, num_splits=2 * S, phase=2)
            self.carrier.put(self, G, E.update_struct(*uargs, **ukw), (dict(s), b, uargs, ukw))
        else:
            E.merge_update(q, k, v, scale, b, 2 * S, uargs, ukw, s["block_idx"], s["block_cnt"])
        if self.count:
            self._count("blocks_read", s["block_cnt"].sum())
            self._count("blocks_total", B * Hkv * nb)
            self._count("masked_heads", B * Hkv)
            self._count("dense_heads", s["trig"].sum())
        return b["out"]
