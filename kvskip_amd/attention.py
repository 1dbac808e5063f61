"""Attention plugin of a transformers model on the kvskip_amd kernels: the per-layer forward that the
model calls through AttentionInterface under the name "kvskip" (src/kvskip_attn.py:481-520), its
configuration (src/kvskip_attn.py:116-147) and a growing KV cache whose layers hand the forward
strided views of one preallocated buffer (src/kvskip_attn.py:68-113).

Prefill (more than one query position) goes to SDPA, as in the reference. A decode step dispatches
on KVSKIP.mode (layers in dense_layers always run dense):
  "dense"          split-K decode over every block (kvskip_decode)
  "vskip2"         two-pass V-skip, top-p(level) GQA union (kvskip.vskip_two_pass)
  "vskip1"         single-pass V-skip against the layer's previous-step LSE (kept per layer)
  "vskip1sink"     the same against the sink block's bound (no previous LSE)
  "refresh_fused"  the device-side refresh planner loop (planner.FusedPlanner: plan -> masked +
                   statistics pass -> update, no host synchronisation); "refresh_pre" is accepted
                   as the same loop: the fused loop reproduces that mode's decisions
                   (src/kvskip_attn.py:399-478), here on the device from the first step on
  "refresh"        the trigger decided after a masked pass over the stored sets, against that
                   pass's log-sum-exp; a refreshing head's output is its attention over every
                   block, with every block's statistics (src/kvskip_attn.py:215-270;
                   planner.PostPlanner, on the device, each block read once, no host
                   synchronisation where the reference syncs once per step to skip an empty
                   second pass)
  "replay"         masked + statistics decode over KVSKIP.plans[layer][t] (one kvskip.Plan per step)

Not in the reference: KVSKIP.ids (token ids [B, >= T] int32 on the device) lets the planner find the
token index itself instead of reading idx_blocks, and KVSKIP.carry lets each layer's planner update
run inside the next layer's split pass (planner.UpdateCarrier; flush() before reading the state).
"""

from __future__ import annotations


import collections
import math
from dataclasses import dataclass, field, replace

import torch
import torch.nn.functional as F

from . import kvskip as K
from .planner import FusedPlanner, Policy, PostPlanner, UpdateCarrier

BLOCK = 64

try:  # the plugin registry and the cache base classes come from transformers when it is present
    from transformers import AttentionInterface
    from transformers.cache_utils import Cache, DynamicLayer
    from transformers.integrations.sdpa_attention import sdpa_attention_forward
    from transformers.masking_utils import AttentionMaskInterface, sdpa_mask
    HAVE_TRANSFORMERS = True
except ImportError:  # pragma: no cover - transformers is part of the image
    HAVE_TRANSFORMERS = False
    DynamicLayer = object


@dataclass
class KvskipConfig:
    """Plugin configuration; the fields and defaults of src/kvskip_attn.py:116-140 plus ids, carry."""
    mode: str = "dense"
    level: float = 0.99
    tau: float = 1e-4
    delta: float = 0.05
    max_age: int = 32
    local: int = 2
    dense_layers: tuple = (0,)
    dense_heads: tuple = ()          # (layer, kv_head) pairs refreshed on every step
    index_heads: tuple = ()          # (layer, kv_head) pairs on the token index
    index_union: bool = False
    idx_blocks: object = None        # this step's token-index blocks [B, >= nb] bool (set by the driver)
    calib: float | None = None
    calib_hold: int = 0
    calib_warm: tuple = ()
    calib_free: bool = False
    calib_kind: str = "logit"
    calib_auto_ix: float | None = None
    count: bool = True
    record: bool = False             # refresh modes: append each step's read mask to plans[layer]
    ids: object = None               # token ids [B, >= T] int32 on the device (index found on the device)
    carry: bool = True               # updates ride on the next layer's split pass
    state: dict = field(default_factory=dict)
    log: dict = field(default_factory=dict)
    plans: dict = field(default_factory=dict)
    carrier: UpdateCarrier = field(default_factory=UpdateCarrier)

    def policy(self, layer: int) -> Policy:
        """The planner policy of one layer (its dense and index KV heads)."""
        return Policy(delta=self.delta, max_age=self.max_age, level=self.level, local=self.local,
                      calib=self.calib, calib_kind=self.calib_kind, calib_hold=self.calib_hold,
                      calib_warm=tuple(self.calib_warm), calib_free=self.calib_free,
                      calib_auto_ix=self.calib_auto_ix,
                      dense_heads=tuple(h for (l, h) in self.dense_heads if l == layer),
                      index_heads=tuple(h for (l, h) in self.index_heads if l == layer),
                      index_union=self.index_union)

    def flush(self):
        """Launch a layer update still held by the carrier (before reading planner state)."""
        self.carrier.flush()

    def reset(self):
        self.flush()
        self.state.clear()
        self.log.clear()


KVSKIP = KvskipConfig()


def _tally(layer, **amounts):
    """Add device (or host) amounts to a layer's counters; nothing when counting is off."""
    if KVSKIP.count:
        counters = KVSKIP.log.setdefault(layer, {})
        for name, amount in amounts.items():
            counters[name] = counters.get(name, 0.0) + amount


def log_totals() -> dict:
    """Every counter summed over the layers, as floats (src/kvskip_attn.py:155-163; reading a device
    counter synchronises once)."""
    acc = collections.Counter()
    for counters in KVSKIP.log.values():
        acc.update({name: float(amount) for name, amount in counters.items()})
    return dict(acc)


def _prefill(module, query, key, value, attention_mask, scaling, dropout, **kwargs):
    if HAVE_TRANSFORMERS:
        return sdpa_attention_forward(module, query, key, value, attention_mask, dropout=dropout, scaling=scaling,
                                      **kwargs)
    G = query.shape[1] // key.shape[1]  # pragma: no cover
    out = F.scaled_dot_product_attention(query, key.repeat_interleave(G, 1), value.repeat_interleave(G, 1),
                                         attn_mask=attention_mask, dropout_p=dropout, scale=scaling,
                                         is_causal=attention_mask is None and query.shape[2] > 1)
    return out.transpose(1, 2).contiguous(), None


def _refresh(layer, q, k, v, scale):
    st = KVSKIP.state.setdefault(layer, {})
    fp = st.get("planner")
    nb = math.ceil(k.shape[2] / BLOCK)
    if fp is None:
        fp = st["planner"] = FusedPlanner(KVSKIP.policy(layer), count=KVSKIP.count,
                                          carrier=KVSKIP.carrier if KVSKIP.carry else None)
        if KVSKIP.count:
            KVSKIP.log[layer] = fp.counters       # the planner's device counters are the layer's
        out = fp.first(q, k, v, scale)
    elif KVSKIP.ids is not None and fp.policy.needs_index:
        out = fp.step(q, k, v, scale, ids=KVSKIP.ids)
    else:
        out = fp.step(q, k, v, scale, idx=KVSKIP.idx_blocks if fp.policy.needs_index else None)
    if KVSKIP.record:
        KVSKIP.plans.setdefault(layer, []).append(fp.read_mask(nb))
    return out


def _dense(layer, q, k, v, scale):
    return K.decode(q, k, v, scale)["out"]


def _two_pass(layer, q, k, v, scale):
    return K.vskip_two_pass(q, k, v, scale, rule="topp", value=KVSKIP.level, local=KVSKIP.local, sync=False)["out"]


def _one_pass(layer, q, k, v, scale, *, sink_bound=False):
    """Single-pass V-skip; the layer's normaliser estimate is its previous step's log-sum-exp, or with
    sink_bound the sink block's own bound (mode vskip1sink)."""
    mem = KVSKIP.state.setdefault(layer, {})
    res = K.vskip_one_pass(q, k, v, scale, tau=KVSKIP.tau, local=KVSKIP.local,
                           lse_prev=None if sink_bound else mem.get("lse"), count=KVSKIP.count, sync=False)
    mem["lse"] = res["lse"]
    if KVSKIP.count:
        vt = res["v_tiles"]
        _tally(layer, v_tiles=vt.sum(), blocks_total=vt.numel() * math.ceil(k.shape[2] / BLOCK))
    return res["out"]


def _replay(layer, q, k, v, scale):
    """Masked + statistics decode over the lists recorded for this layer, one per step in order."""
    mem = KVSKIP.state.setdefault(layer, {"t": 0})
    plan = KVSKIP.plans[layer][mem["t"]]
    mem["t"] += 1
    return K.decode(q, k, v, scale, plan=plan, stats=True)["out"]


def _refresh_post(layer, q, k, v, scale):
    """Mode "refresh" (src/kvskip_attn.py:215-270): the layer's PostPlanner; its device counters are
    the layer's."""
    st = KVSKIP.state.setdefault(layer, {})
    pp = st.get("post")
    if pp is None:
        # the reference's refresh_step reads delta, max_age, local, level and the dense heads only
        # (src/kvskip_attn.py:215-270): the calibration, warm-up and token-index fields of the
        # config are ignored there, so they are dropped here too
        pol = replace(KVSKIP.policy(layer), calib=None, calib_warm=(), calib_auto_ix=None,
                                  index_heads=(), index_union=False)
        pp = st["post"] = PostPlanner(pol, count=KVSKIP.count, carrier=KVSKIP.carrier if KVSKIP.carry else None)
        if KVSKIP.count:
            KVSKIP.log[layer] = pp.counters
        return pp.first(q, k, v, scale)
    return pp.step(q, k, v, scale)


# Decode-step handlers by KVSKIP.mode (src/kvskip_attn.py:487-513).
MODES = {
    "dense": _dense,
    "vskip2": _two_pass,
    "vskip1": _one_pass,
    "vskip1sink": lambda layer, q, k, v, scale: _one_pass(layer, q, k, v, scale, sink_bound=True),
    "refresh_fused": _refresh,
    "refresh_pre": _refresh,
    "replay": _replay,
    "refresh": _refresh_post,
}


def kvskip_attention_forward(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
    """AttentionInterface forward (src/kvskip_attn.py:481-515): query [B, Hq, Sq, D], key / value
    [B, Hkv, T, D] (the cache's views); returns ([B, Sq, Hq, D], None). Prefill goes to SDPA; a
    decode step to the handler of KVSKIP.mode, or dense for a layer in dense_layers."""
    if query.shape[2] != 1:
        return _prefill(module, query, key, value, attention_mask, scaling, dropout, **kwargs)
    layer = module.layer_idx
    mode = "dense" if layer in KVSKIP.dense_layers else KVSKIP.mode
    handler = MODES.get(mode)
    if handler is None:
        raise ValueError(f"unknown kvskip mode {mode!r}")
    scale = query.shape[-1] ** -0.5 if scaling is None else scaling
    out = handler(layer, query[:, :, 0], key, value, scale)
    return out.unsqueeze(1), None


def register():
    """Register the forward and its mask under the name "kvskip" (src/kvskip_attn.py:518-520)."""
    if not HAVE_TRANSFORMERS:
        raise RuntimeError("transformers is not importable: nothing to register with")
    AttentionInterface.register("kvskip", kvskip_attention_forward)
    AttentionMaskInterface.register("kvskip", sdpa_mask)


class GrowingLayer(DynamicLayer):
    """One layer of the growing cache: keys and values live in a [B, H, capacity, D] buffer whose
    capacity is a whole number of 64-token blocks; the layer exposes views of its first n tokens
    (head stride capacity * D, which every kvskip entry point takes). Growth at least doubles the
    capacity, so appends cost amortised O(1) copies."""

    capacity = 0        # tokens allocated at the first update (the class attribute of GrowingCache(capacity))
    headroom = 512      # tokens beyond the need allocated on growth

    def lazy_initialization(self, key_states, value_states):
        super().lazy_initialization(key_states, value_states)
        self._kbuf = self._vbuf = None
        self._n = 0

    def _reserve(self, need, like):
        have = 0 if self._kbuf is None else self._kbuf.shape[-2]
        if need <= have:
            return
        cap = max(need + self.headroom, 2 * have, self.capacity)
        cap = (cap + BLOCK - 1) // BLOCK * BLOCK
        B, H, _, D = like.shape
        kb = torch.empty(B, H, cap, D, dtype=like.dtype, device=like.device)
        vb = torch.empty_like(kb)
        if self._n:
            kb[:, :, :self._n].copy_(self._kbuf[:, :, :self._n])
            vb[:, :, :self._n].copy_(self._vbuf[:, :, :self._n])
        self._kbuf, self._vbuf = kb, vb

    def _views(self):
        self.keys = self._kbuf[:, :, :self._n]
        self.values = self._vbuf[:, :, :self._n]

    def update(self, key_states, value_states, *args, **kwargs):
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        t = key_states.shape[-2]
        self._reserve(self._n + t, key_states)
        self._kbuf[:, :, self._n:self._n + t].copy_(key_states)
        self._vbuf[:, :, self._n:self._n + t].copy_(value_states)
        self._n += t
        self._views()
        return self.keys, self.values

    def get_seq_length(self) -> int:
        return self._n if self.is_initialized else 0

    def crop(self, tokens_to_remove: int) -> None:
        """A negative count drops that many tokens; a positive one is the length to keep (the legacy
        form of DynamicLayer.crop)."""
        if not self.is_initialized:
            return
        keep = max(0, min(self._n, tokens_to_remove)) if tokens_to_remove > 0 else max(0, self._n + tokens_to_remove)
        self._n = keep
        if self._kbuf is not None:
            self._views()

    def batch_repeat_interleave(self, repeats: int) -> None:
        if self.get_seq_length() > 0:
            self._kbuf = self._kbuf.repeat_interleave(repeats, dim=0)
            self._vbuf = self._vbuf.repeat_interleave(repeats, dim=0)
            self._views()

    def batch_select_indices(self, indices: torch.Tensor) -> None:
        if self.get_seq_length() > 0:
            self._kbuf = self._kbuf[indices].contiguous()
            self._vbuf = self._vbuf[indices].contiguous()
            self._views()


def GrowingCache(capacity: int = 0):
    """A transformers Cache of GrowingLayers; capacity: tokens allocated at the first update
    (src/kvskip_attn.py:110-113)."""
    if not HAVE_TRANSFORMERS:
        raise RuntimeError("transformers is not importable")
    layer = GrowingLayer if not capacity else type("GrowingLayerCap", (GrowingLayer,), {"capacity": int(capacity)})
    return Cache(layer_class_to_replicate=layer)
