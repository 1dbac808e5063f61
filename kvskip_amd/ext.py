"""Operator surface of the reference's torch extension `kvskip_ext`, on the kvskip_amd C ABI.

Same functions, positional/keyword signatures, defaults, output lists and validation messages as
kernels/kvskip_ext.cpp:327-351 (decode, pv, vskip1, plan, update, read_bw). Outputs are allocated
with torch on the inputs' device; launches go to torch's current stream; nothing synchronises.
Absent outputs are returned as None (the reference returns undefined tensors).

Extra operators with no counterpart in kvskip_ext: block_sums and token_index (the device-side
planner initialisation and token index) and decode_into (decode into caller-owned buffers).
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _native
from ._native import AttnArgs, PlanArgs, UpdateArgs

TILE = 64


def _fail(msg: str):
    raise RuntimeError(msg)


def _require(cond: bool, msg: str):
    if not cond:
        _fail(msg)


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream(dev: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def check_kv(t: torch.Tensor, name: str):
    """kernels/kvskip_ext.cpp:12-19."""
    _require(t.is_cuda and t.dtype == torch.bfloat16, f"{name} must be a CUDA bf16 tensor")
    _require(t.dim() == 4, f"{name} must be [B, Hkv, T, D]")
    _require(t.stride(3) == 1, f"{name} must have a contiguous last dim")
    _require(t.stride(2) % 8 == 0 and t.stride(1) % 8 == 0 and t.stride(0) % 8 == 0,
             f"{name} strides must be multiples of 8 elements (16-byte rows)")
    _require(t.data_ptr() % 16 == 0, f"{name} must be 16-byte aligned")
    T, D = t.shape[2], t.shape[3]
    _require((T - 1) * t.stride(2) + D < 2**30, f"{name}: one head's rows must span < 2 GiB")


def check_q(q: torch.Tensor):
    _require(q.is_cuda and q.dtype == torch.bfloat16 and q.dim() == 3, "q must be CUDA bf16 [B, Hq, D]")
    _require(q.stride(2) == 1 and q.stride(1) % 8 == 0 and q.stride(0) % 8 == 0 and q.data_ptr() % 16 == 0,
             "q rows must be 16-byte aligned")


def check_f32(t: torch.Tensor, name: str):
    _require(t.is_cuda and t.dtype == torch.float32 and t.is_contiguous(), f"{name} must be contiguous CUDA fp32")


def _attn_args(q, k, v, scale, B, Hq, Hkv, T, D) -> AttnArgs:
    a = AttnArgs()
    if q is not None:
        a.q = q.data_ptr()
        a.q_sb, a.q_sh = q.stride(0), q.stride(1)
    if k is not None:
        a.k = k.data_ptr()
        a.k_sb, a.k_sh, a.k_st = k.stride(0), k.stride(1), k.stride(2)
    if v is not None:
        a.v = v.data_ptr()
        a.v_sb, a.v_sh, a.v_st = v.stride(0), v.stride(1), v.stride(2)
    a.B, a.Hq, a.Hkv, a.T, a.D = B, Hq, Hkv, T, D
    a.scale = float(scale)
    return a


def _kv_dims(q, k, v, block_table=None, T=None):
    """(B, Hq, D, Hkv, T) of an attention call over views [B, Hkv, T, D], or (block_table given, not
    in the reference) over page pools k, v [num_pages, Hkv, 64, D] whose page block_table[b, j] holds
    tokens 64 j .. 64 j + 63 of sequence b; T is then required (the tokens, or the capacity with
    seq_lens)."""
    B, Hq, D = q.shape
    Hkv = k.shape[1]
    if block_table is None:
        # every kernel reads v (and k) as [B, Hkv, T, D] of k's sizes: a shorter or narrower view
        # would be read past its end
        _require(k.dim() == 4 and v.dim() == 4 and k.shape[0] == B and k.shape[3] == D
                 and tuple(v.shape) == tuple(k.shape), "shape mismatch between q, k, v")
        return B, Hq, D, Hkv, k.shape[2]
    return B, Hq, D, Hkv, _pool_tokens((k, v), B, Hkv, D, block_table, T)


def _pool_tokens(pools, B, Hkv, D, block_table, T) -> int:
    """T of a paged call, after checking the page pools [num_pages, Hkv, 64, D] and the table."""
    _require(T is not None and int(T) >= 1, "paged cache: T (tokens per sequence, or the capacity) is required")
    T = int(T)
    _require(all(x.dim() == 4 and tuple(x.shape[1:]) == (Hkv, TILE, D) and x.shape[0] == pools[0].shape[0]
                 for x in pools), "paged cache: k, v must be page pools [num_pages, Hkv, 64, D]")
    _require(block_table.is_cuda and block_table.dtype == torch.int32 and block_table.dim() == 2
             and block_table.shape[0] == B and block_table.stride(1) == 1
             and block_table.shape[1] >= (T + TILE - 1) // TILE,
             "block_table: int32 [B, >= ceil(T / 64)] on the device, rows contiguous")
    return T


def _set_pages(a, block_table, pool):
    if block_table is not None:          # page pools: the dim-0 strides of k / v are the page strides
        a.block_table, a.bt_stride, a.num_pages = block_table.data_ptr(), block_table.stride(0), pool.shape[0]


def decode(q, k, v, scale, block_idx=None, block_cnt=None, stats=False, load_v=True, num_splits=1, stages=2,
           want_f32=False, write_p=False, seq_lens=None, block_table=None, T=None, merge=True, list_partition=0):
    """Split-K decode attention (kernels/kvskip_ext.cpp:25-101).

    Returns [out bf16 [B,Hq,D], lse fp32 [B,Hq], blk_max, blk_sum ([B,Hq,nb] or None), out_f32 (or None),
    P fp16 [B,Hq,nb*64] (write_p) or None].

    seq_lens (not in the reference): int32 [B] on the device, a ragged batch; sequence b attends
    tokens [0, clamp(seq_lens[b], 1, T)) of its view; num_splits is then the per-KV-head split
    budget over the whole batch (>= 2). list_partition (not in the reference; block lists with
    seq_lens): 0 cuts each KV head's lists over the batch, 1 all B * Hkv lists by one chunk length
    (kvskip_attn_args.list_partition).
    block_table, T (not in the reference): a paged cache, see _kv_dims (the pass with V, MFMA engine).
    merge=False (not in the reference; load_v=False): the split pass alone, no merge launch; the block
    statistics and P are whole, lse is not computed (returned as None)."""
    check_q(q)
    check_kv(k, "k")
    check_kv(v, "v")
    B, Hq, D, Hkv, T = _kv_dims(q, k, v, block_table, T)
    if block_table is None:
        _require(k.shape[0] == B and v.shape[0] == B and k.shape[3] == D and v.shape[3] == D and v.shape[1] == Hkv
                 and v.shape[2] == T, "shape mismatch between q, k, v")
    _require(Hq % Hkv == 0, "Hq must be a multiple of Hkv")
    _require(1 <= num_splits <= 256, "num_splits in 1..256")
    _require(load_v or stats, "load_v=false only makes sense with stats=true")
    _require(not write_p or stats, "write_p needs stats=true")
    _require(merge or not load_v, "merge=False needs load_v=False")
    _require(stages in (2, 3), "kvskip: unsupported head dim / stages")
    nb = (T + TILE - 1) // TILE
    dev = q.device
    f32 = dict(dtype=torch.float32, device=dev)
    out = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=dev) if load_v else None
    out32 = torch.empty(B, Hq, D, **f32) if (load_v and want_f32) else None
    lse = torch.empty(B, Hq, **f32)
    bmax = bsum = None
    if stats:                           # every block is written (-inf / 0 where a list skips it)
        bmax = torch.empty(B, Hq, nb, **f32)
        bsum = torch.empty(B, Hq, nb, **f32)
    pbuf = torch.empty(B, Hq, nb * TILE, dtype=torch.float16, device=dev) if write_p else None
    part_acc = part_ml = None
    if num_splits > 1:
        part_acc = torch.empty(B, Hq, num_splits, D, **f32) if load_v else None
        part_ml = torch.empty(B, Hq, num_splits, 2, **f32)
    split_only = not merge and num_splits > 1
    _launch_decode(q, k, v, scale, block_idx, block_cnt, stats, load_v, num_splits, out, lse, bmax, bsum, out32,
                   pbuf, part_acc, part_ml, seq_lens, phase=1 if split_only else 3, block_table=block_table, T=T,
                   list_partition=list_partition)
    return [out, None if split_only else lse, bmax, bsum, out32, pbuf]


def decode_into(q, k, v, scale, bufs: dict, block_idx=None, block_cnt=None, stats=False, num_splits=1,
                seq_lens=None, phase=3, block_table=None, T=None, list_partition=0):
    """decode() into caller-owned buffers, allocating nothing (not in the reference): bufs holds
    out bf16, lse fp32 and, as needed, blk_max / blk_sum fp32 (>= B*Hq*nb elements, written as
    [B, Hq, nb], -inf / 0 where a list skips a block) and part_acc / part_ml fp32
    (>= B*Hq*num_splits*D / *2 elements). The fused planner loop runs its passes this way.
    phase: 3 = the whole op, 1 = the split pass only (its merge left to merge_splits / merge_update),
    2 = that merge alone (given the pass's list_partition). block_table, T: a paged cache (see _kv_dims)."""
    check_q(q)
    check_kv(k, "k")
    check_kv(v, "v")
    B, Hq, D, Hkv, T = _kv_dims(q, k, v, block_table, T)
    _require(1 <= num_splits <= 256, "num_splits in 1..256")
    nb = (T + TILE - 1) // TILE
    out, lse = bufs["out"], bufs["lse"]
    _require(out.dtype == torch.bfloat16 and out.is_contiguous() and out.numel() >= B * Hq * D, "bufs: out")
    _require(lse.dtype == torch.float32 and lse.is_contiguous() and lse.numel() >= B * Hq, "bufs: lse")
    bmax = bsum = part_acc = part_ml = None
    if stats:
        bmax, bsum = bufs["blk_max"], bufs["blk_sum"]
        for t in (bmax, bsum):
            _require(t.dtype == torch.float32 and t.is_contiguous() and t.numel() >= B * Hq * nb, "bufs: stats")
    if num_splits > 1:
        part_acc, part_ml = bufs["part_acc"], bufs["part_ml"]
        _require(part_acc.dtype == torch.float32 and part_acc.is_contiguous()
                 and part_acc.numel() >= B * Hq * num_splits * D, "bufs: part_acc")
        _require(part_ml.dtype == torch.float32 and part_ml.is_contiguous()
                 and part_ml.numel() >= B * Hq * num_splits * 2, "bufs: part_ml")
    _launch_decode(q, k, v, scale, block_idx, block_cnt, stats, True, num_splits, out, lse, bmax, bsum, None, None,
                   part_acc, part_ml, seq_lens, phase, block_table, T, list_partition)


class DecodeOp:
    """One decode-attention op with its arguments and outputs built once (fixed q, k, v views):
    run() = decode(); splits() then merge() = its two launches (kvskip_decode_splits /
    kvskip_merge_splits), for timing each kernel or placing work between them. Not in the
    reference. Outputs: .out bf16 [B, Hq, D], .lse fp32 [B, Hq]."""

    def __init__(self, q, k, v, scale, num_splits, block_idx=None, block_cnt=None):
        check_q(q)
        check_kv(k, "k")
        check_kv(v, "v")
        _require(2 <= num_splits <= 256, "DecodeOp: num_splits in 2..256")
        B, Hq, D = q.shape
        Hkv, T = k.shape[1], k.shape[2]
        dev = q.device
        f32 = dict(dtype=torch.float32, device=dev)
        self.out = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=dev)
        self.lse = torch.empty(B, Hq, **f32)
        self._keep = [q, k, v, block_idx, block_cnt,
                      torch.empty(B, Hq, num_splits, D, **f32), torch.empty(B, Hq, num_splits, 2, **f32)]
        a = _attn_args(q, k, v, scale, B, Hq, Hkv, T, D)
        if block_idx is not None:
            a.block_idx, a.block_cnt, a.max_blocks = block_idx.data_ptr(), block_cnt.data_ptr(), block_idx.shape[2]
        a.num_splits = int(num_splits)
        a.part_acc, a.part_ml = self._keep[5].data_ptr(), self._keep[6].data_ptr()
        a.out, a.lse = self.out.data_ptr(), self.lse.data_ptr()
        self.args, self.dev = a, dev
        self.lib = _native.lib()

    def _call(self, fn):
        _native.check(fn(ctypes.byref(self.args), 0, 1, _stream(self.dev)))

    def run(self):
        self._call(self.lib.kvskip_decode)

    def splits(self):
        self._call(self.lib.kvskip_decode_splits)

    def merge(self):
        self._call(self.lib.kvskip_merge_splits)


def _decode_args(q, k, v, scale, block_idx, block_cnt, num_splits, out, lse, bmax, bsum, out32, pbuf, part_acc,
                 part_ml, seq_lens=None, block_table=None, T=None, list_partition=0) -> AttnArgs:
    B, Hq, D, Hkv, T = _kv_dims(q, k, v, block_table, T)
    a = _attn_args(q, k, v, scale, B, Hq, Hkv, T, D)
    _set_pages(a, block_table, k)
    if seq_lens is not None:
        _require(seq_lens.is_cuda and seq_lens.dtype == torch.int32 and seq_lens.is_contiguous()
                 and seq_lens.numel() == B, "seq_lens: contiguous CUDA int32 [B]")
        a.seq_lens = seq_lens.data_ptr()
    if block_idx is not None:
        _require(block_cnt is not None, "block_cnt is required with block_idx")
        bi, bc = block_idx, block_cnt
        _require(bi.is_cuda and bi.dtype == torch.int32 and bi.dim() == 3 and bi.is_contiguous()
                 and bi.shape[0] == B and bi.shape[1] == Hkv, "block_idx must be contiguous int32 [B, Hkv, max_blocks]")
        _require(bc.is_cuda and bc.dtype == torch.int32 and bc.is_contiguous() and bc.numel() == B * Hkv,
                 "block_cnt must be contiguous int32 [B, Hkv]")
        a.block_idx, a.block_cnt, a.max_blocks = bi.data_ptr(), bc.data_ptr(), bi.shape[2]
    a.num_splits = int(num_splits)
    a.part_acc, a.part_ml = _ptr(part_acc), _ptr(part_ml)
    a.out, a.out_f32, a.lse = _ptr(out), _ptr(out32), lse.data_ptr()
    a.blk_max, a.blk_sum = _ptr(bmax), _ptr(bsum)
    a.p_out = _ptr(pbuf)
    a.list_partition = int(list_partition)
    return a


_PHASES = {3: "kvskip_decode", 1: "kvskip_decode_splits", 2: "kvskip_merge_splits"}


def _launch_decode(q, k, v, scale, block_idx, block_cnt, stats, load_v, num_splits, out, lse, bmax, bsum, out32,
                   pbuf, part_acc, part_ml, seq_lens=None, phase=3, block_table=None, T=None, list_partition=0):
    a = _decode_args(q, k, v, scale, block_idx, block_cnt, num_splits, out, lse, bmax, bsum, out32, pbuf, part_acc,
                     part_ml, seq_lens, block_table, T, list_partition)
    dev = q.device
    with torch.cuda.device(dev):
        _native.check(getattr(_native.lib(), _PHASES[phase])(ctypes.byref(a), int(bool(stats)), int(bool(load_v)),
                                                              _stream(dev)))


def pv(P, v, blk_scale, block_idx, block_cnt, num_splits=1, want_f32=False, block_table=None, T=None):
    """Two-pass V-skip, pass 2 (kernels/kvskip_ext.cpp:106-146). Returns [out bf16, out_f32 or None].
    block_table, T (not in the reference): v is the page pool of a paged cache (see _kv_dims)."""
    check_kv(v, "v")
    _require(P.is_cuda and P.dtype == torch.float16 and P.dim() == 3 and P.is_contiguous(), "P: fp16 [B, Hq, t_pad]")
    _require(blk_scale.is_cuda and blk_scale.dtype == torch.float32 and blk_scale.dim() == 4
             and blk_scale.is_contiguous(), "blk_scale: contiguous fp32 [B, Hkv, nb, G]")
    B, Hkv, T, D = v.shape if block_table is None else (P.shape[0], v.shape[1], T, v.shape[3])
    if block_table is not None:
        T = _pool_tokens((v,), B, Hkv, D, block_table, T)
    Hq = P.shape[1]
    _require(Hq % Hkv == 0, "Hq must be a multiple of Hkv")
    G = Hq // Hkv
    nb = (T + TILE - 1) // TILE
    _require(P.shape[0] == B and P.shape[2] == nb * TILE, "P shape")
    _require(tuple(blk_scale.shape) == (B, Hkv, nb, G), "blk_scale shape")
    _require(block_idx.dtype == torch.int32 and block_idx.is_contiguous() and block_idx.shape[0] == B
             and block_idx.shape[1] == Hkv, "block_idx")
    _require(block_cnt.dtype == torch.int32 and block_cnt.is_contiguous() and block_cnt.numel() == B * Hkv,
             "block_cnt")
    _require(num_splits >= 1, "num_splits >= 1")
    dev = v.device
    f32 = dict(dtype=torch.float32, device=dev)
    out = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=dev)
    out32 = torch.empty(B, Hq, D, **f32) if want_f32 else None
    part_acc = torch.empty(B, Hq, num_splits, D, **f32) if num_splits > 1 else None
    part_ml = torch.empty(B, Hq, num_splits, 2, **f32) if num_splits > 1 else None
    a = _attn_args(None, None, v, 1.0, B, Hq, Hkv, T, D)
    a.block_idx, a.block_cnt, a.max_blocks = block_idx.data_ptr(), block_cnt.data_ptr(), block_idx.shape[2]
    a.num_splits = int(num_splits)
    a.part_acc, a.part_ml = _ptr(part_acc), _ptr(part_ml)
    a.out, a.out_f32 = out.data_ptr(), _ptr(out32)
    a.p_in, a.blk_scale = P.data_ptr(), blk_scale.data_ptr()
    _set_pages(a, block_table, v)
    with torch.cuda.device(dev):
        _native.check(_native.lib().kvskip_pv(ctypes.byref(a), _stream(dev)))
    return [out, out32]


def vskip1(q, k, v, scale, tau, local=2, num_splits=1, want_f32=False, count=False, lse_prev=None,
           block_table=None, T=None, v_keep=None):
    """Single-pass V-skip (kernels/kvskip_ext.cpp:149-195). Returns [out, lse, out_f32 or None, vcount or None].
    block_table, T (not in the reference): a paged cache (see _kv_dims; the MFMA engine).
    v_keep (not in the reference): uint8 [B, Hkv, ceil(T / 64)] on the device, set to 1 where a block's V
    was read, else 0."""
    check_q(q)
    check_kv(k, "k")
    check_kv(v, "v")
    _require(tau > 0.0 and local >= 0 and num_splits >= 1, "tau > 0, local >= 0, num_splits >= 1")
    B, Hq, D, Hkv, T = _kv_dims(q, k, v, block_table, T)
    if block_table is None:
        _require(k.shape[0] == B and v.shape[0] == B and k.shape[3] == D and v.shape[3] == D and v.shape[1] == Hkv
                 and v.shape[2] == T, "shape mismatch between q, k, v")
    _require(Hq % Hkv == 0, "Hq must be a multiple of Hkv")
    dev = q.device
    f32 = dict(dtype=torch.float32, device=dev)
    out = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=dev)
    out32 = torch.empty(B, Hq, D, **f32) if want_f32 else None
    lse = torch.empty(B, Hq, **f32)
    vcount = torch.zeros(B, Hkv, dtype=torch.int32, device=dev) if count else None
    part_acc = part_ml = None
    if num_splits > 1:
        part_acc = torch.empty(B, Hq, num_splits, D, **f32)
        part_ml = torch.empty(B, Hq, num_splits, 2, **f32)
    a = _attn_args(q, k, v, scale, B, Hq, Hkv, T, D)
    a.num_splits = int(num_splits)
    a.part_acc, a.part_ml = _ptr(part_acc), _ptr(part_ml)
    a.out, a.out_f32, a.lse = out.data_ptr(), _ptr(out32), lse.data_ptr()
    a.tau, a.local, a.vcount = float(tau), int(local), _ptr(vcount)
    if lse_prev is not None:
        _require(lse_prev.is_cuda and lse_prev.dtype == torch.float32 and lse_prev.is_contiguous()
                 and lse_prev.numel() == B * Hq, "lse_prev: contiguous fp32 [B, Hq]")
        a.lse_prev = lse_prev.data_ptr()
    if v_keep is not None:
        _require(v_keep.is_cuda and v_keep.dtype == torch.uint8 and v_keep.is_contiguous()
                 and tuple(v_keep.shape) == (B, Hkv, (T + TILE - 1) // TILE), "v_keep: contiguous uint8 [B, Hkv, nb]")
        a.v_keep = v_keep.data_ptr()
    _set_pages(a, block_table, k)
    with torch.cuda.device(dev):
        _native.check(_native.lib().kvskip_vskip1(ctypes.byref(a), _stream(dev)))
    return [out, lse, out32, vcount]


def plan(q, k, csum, lse_ref, cs_ref, keep, lse_att, age, flags, cs_now, trig, block_idx, block_cnt, scale, delta,
         max_age, local, add_token, idx=None, calib=None, est=None, calib_on=False, calib_kind=0, aix=None,
         part=None, seq_lens=None, seq_lens_out=None, ids=None, idx_out=None, block_table=None, T=None,
         ticket=None):
    """Device-side refresh planner before the pass (kernels/kvskip_ext.cpp:205-267); in place.

    part (not in the reference): fp32 workspace of plan_part_floats(...) elements; with it the
    centroid pass is spread over all compute units (two launches instead of one).
    seq_lens (not in the reference): int32 [B] on the device, a ragged batch over views of
    capacity T (sequence b holds seq_lens[b] tokens; add_token adds each one's last row).
    seq_lens_out (not in the reference): int32 [B] on the device; receives each sequence's length
    this step (for the step's update, which may run later).
    ids, idx_out (not in the reference; need part, and idx None): token ids int32 [B, >= T]; the
    plan finds this step's token-index blocks itself and writes them to idx_out (uint8 [B, NBC]).
    block_table, T (not in the reference): k is the page pool of a paged cache (see _kv_dims).
    ticket (not in the reference; needs part): int32 [B * Hkv] on the device, zero before the first
    call and left zero by each call; the plan is then one launch (each head decided by its last
    scores workgroup, kvskip_plan_args.ticket). Calls sharing one must not overlap in time."""
    p = _plan_args(q, k, csum, lse_ref, cs_ref, keep, lse_att, age, flags, cs_now, trig, block_idx, block_cnt, scale,
                   delta, max_age, local, add_token, idx, calib, est, calib_on, calib_kind, aix, part, seq_lens,
                   seq_lens_out, ids, idx_out, block_table, T, ticket)
    dev = q.device
    with torch.cuda.device(dev):
        _native.check(_native.lib().kvskip_plan(ctypes.byref(p), _stream(dev)))


def plan_struct(*plan_args, **plan_kwargs) -> PlanArgs:
    """The argument block of plan(*plan_args, **plan_kwargs), checked (it holds raw pointers)."""
    return _plan_args(*plan_args, **plan_kwargs)


def plan_scores(pargs: PlanArgs, device):
    """plan's first launch alone (kvskip_plan_scores; needs part); its decision then runs in
    decode_splits_planned. Not in the reference."""
    dev = torch.device(device)
    with torch.cuda.device(dev):
        _native.check(_native.lib().kvskip_plan_scores(ctypes.byref(pargs), _stream(dev)))


DECIDE_PLAN, DECIDE_LISTS, DECIDE_POST = 0, 1, 2      # kvskip_plan_args.decide_mode


def decode_splits_planned(q, k, v, scale, bufs: dict, pargs: PlanArgs, num_splits, update: UpdateArgs | None = None,
                          seq_lens=None, block_table=None, T=None):
    """plan's decision and the masked + statistics split pass in one launch (kvskip_decode_splits_planned;
    after plan_scores(pargs)); the whole op when num_splits == 1. The layer's update must advance the
    age (update_struct(..., age=...)). update: another layer's update to carry, or None. seq_lens: the
    plan's (one sequence, B 1). pargs.decide_mode picks the decision (DECIDE_PLAN, DECIDE_LISTS,
    DECIDE_POST), pargs.slot_base / slot_count the partial slots the pass writes."""
    check_q(q)
    check_kv(k, "k")
    check_kv(v, "v")
    B, Hq, D = q.shape
    _, _, _, Hkv, T = _kv_dims(q, k, v, block_table, T)
    _require(1 <= num_splits <= 256, "num_splits in 1..256")
    nb = (T + TILE - 1) // TILE
    bmax, bsum = bufs["blk_max"], bufs["blk_sum"]
    for t in (bmax, bsum):
        _require(t.dtype == torch.float32 and t.is_contiguous() and t.numel() >= B * Hq * nb, "bufs: stats")
    part_acc = part_ml = None
    if num_splits > 1:
        part_acc, part_ml = bufs["part_acc"], bufs["part_ml"]
        _require(part_acc.numel() >= B * Hq * num_splits * D and part_ml.numel() >= B * Hq * num_splits * 2,
                 "bufs: split partials")
    a = _decode_args(q, k, v, scale, None, None, num_splits, bufs["out"], bufs["lse"], bmax, bsum, None, None,
                     part_acc, part_ml, seq_lens, block_table, T)
    dev = q.device
    with torch.cuda.device(dev):
        _native.check(_native.lib().kvskip_decode_splits_planned(ctypes.byref(a), ctypes.byref(pargs),
                                                                 None if update is None else ctypes.byref(update),
                                                                 _stream(dev)))


def _plan_args(q, k, csum, lse_ref, cs_ref, keep, lse_att, age, flags, cs_now, trig, block_idx, block_cnt, scale, delta,
         max_age, local, add_token, idx=None, calib=None, est=None, calib_on=False, calib_kind=0, aix=None,
         part=None, seq_lens=None, seq_lens_out=None, ids=None, idx_out=None, block_table=None, T=None,
               ticket=None):
    """kvskip_plan_args of plan(), validated. block_table, T: a paged cache (see _kv_dims)."""
    _require(q.is_cuda and q.dtype == torch.bfloat16 and q.dim() == 3 and q.stride(2) == 1, "q: CUDA bf16 [B, Hq, D]")
    check_kv(k, "k")
    B, Hq, D = q.shape
    _, _, _, Hkv, T = _kv_dims(q, k, k, block_table, T)
    for t, n in ((csum, "csum"), (lse_ref, "lse_ref"), (cs_ref, "cs_ref"), (lse_att, "lse_att"), (cs_now, "cs_now")):
        check_f32(t, n)
    NBC = keep.shape[2]
    _require((T + TILE - 1) // TILE <= NBC, "block capacity exceeded")
    _require(csum.shape[2] == NBC and lse_ref.shape[2] == NBC and cs_ref.shape[2] == NBC and cs_now.shape[2] == NBC
             and block_idx.shape[2] == NBC, "capacity mismatch")
    _require(age.dtype == torch.int32 and age.is_contiguous() and age.numel() == B * Hkv, "age: int32 [B, Hkv]")
    _require(flags.dtype == torch.int32 and flags.numel() == Hkv, "flags: int32 [Hkv]")
    _require(keep.dtype == torch.uint8 and keep.is_contiguous(), "keep: contiguous uint8 [B, Hkv, NBC]")
    _require(trig.dtype == torch.uint8 and block_idx.dtype == torch.int32 and block_cnt.dtype == torch.int32,
             "trig uint8, block_idx / block_cnt int32")
    p = PlanArgs()
    p.q, p.q_sb, p.q_sh = q.data_ptr(), q.stride(0), q.stride(1)
    p.k, p.k_sb, p.k_sh, p.k_st = k.data_ptr(), k.stride(0), k.stride(1), k.stride(2)
    p.csum, p.lse_ref, p.cs_ref, p.keep = csum.data_ptr(), lse_ref.data_ptr(), cs_ref.data_ptr(), keep.data_ptr()
    p.lse_att, p.age, p.flags = lse_att.data_ptr(), age.data_ptr(), flags.data_ptr()
    if idx is not None:
        _require(idx.is_cuda and idx.dtype == torch.uint8 and idx.is_contiguous() and idx.shape[0] == B
                 and idx.shape[1] == NBC, "idx: contiguous uint8 [B, NBC]")
        p.idx = idx.data_ptr()
    if calib is not None:
        check_f32(calib, "calib")
        _require(calib.numel() == B * Hkv, "calib: [B, Hkv]")
        p.calib = calib.data_ptr()
    if est is not None:
        check_f32(est, "est")
        _require(est.numel() == B * Hkv, "est: [B, Hkv]")
        p.est = est.data_ptr()
    p.calib_on, p.calib_kind = int(bool(calib_on)), int(calib_kind)
    if aix is not None:
        _require(aix.is_cuda and aix.dtype == torch.uint8 and aix.is_contiguous() and aix.numel() == B * Hkv,
                 "aix: contiguous uint8 [B, Hkv]")
        _require(idx is not None or ids is not None, "aix needs idx")
        p.aix = aix.data_ptr()
    p.cs_now, p.trig = cs_now.data_ptr(), trig.data_ptr()
    p.block_idx, p.block_cnt = block_idx.data_ptr(), block_cnt.data_ptr()
    p.B, p.Hq, p.Hkv, p.T, p.D, p.NBC = B, Hq, Hkv, T, D, NBC
    p.local, p.max_age, p.add_token = int(local), int(max_age), int(bool(add_token))
    p.scale, p.delta = float(scale), float(delta)
    if part is not None:
        check_f32(part, "part")
        _require(part.numel() >= plan_part_floats(B, Hq, Hkv, NBC), "part: too small")
        p.part = part.data_ptr()
    p.seq_lens = _seq_lens_ptr(seq_lens, B)
    if block_table is not None:
        p.block_table, p.bt_stride, p.num_pages = block_table.data_ptr(), block_table.stride(0), k.shape[0]
    if seq_lens_out is not None:
        _require(seq_lens_out.is_cuda and seq_lens_out.dtype == torch.int32 and seq_lens_out.is_contiguous()
                 and seq_lens_out.numel() == B, "seq_lens_out: contiguous int32 [B] on the device")
        p.seq_lens_out = seq_lens_out.data_ptr()
    if ids is not None:
        _require(part is not None and idx is None and idx_out is not None, "plan: ids needs part and idx_out, and no idx")
        _require(ids.is_cuda and ids.dtype == torch.int32 and ids.dim() == 2 and ids.stride(1) == 1
                 and ids.shape[0] == B and ids.shape[1] >= T, "ids: CUDA int32 [B, >= T]")
        _require(idx_out.dtype == torch.uint8 and idx_out.is_contiguous() and tuple(idx_out.shape) == (B, NBC),
                 "idx_out: uint8 [B, NBC]")
        p.ids, p.ids_sb, p.idx_out = ids.data_ptr(), ids.stride(0), idx_out.data_ptr()
    if ticket is not None:
        _require(part is not None, "plan: ticket needs part")
        _require(ticket.is_cuda and ticket.dtype == torch.int32 and ticket.is_contiguous() and ticket.numel() == B * Hkv,
                 "ticket: contiguous int32 [B * Hkv] on the device")
        p.ticket = ticket.data_ptr()
    return p


def plan_part_floats(B, Hq, Hkv, NBC) -> int:
    """fp32 elements of plan()'s `part` workspace for a state of capacity NBC blocks."""
    return int(_native.lib().kvskip_plan_part_floats(int(B), int(Hq), int(Hkv), int(NBC)))


def _update_args(blk_max, blk_sum, trig, cs_now, keep, lse_ref, cs_ref, lse_att, T, level, local, flags=None,
                 idx=None, est=None, calib=None, calib_rate=0.0, calib_free=False, calib_kind=0, aix=None,
                 aix_thr=0.0, list_stats=False, seq_lens=None, age=None) -> UpdateArgs:
    """kvskip_update_args of update() (kernels/kvskip_ext.cpp:270-319), validated."""
    check_f32(blk_max, "blk_max")
    check_f32(blk_sum, "blk_sum")
    B, Hkv, NBC = keep.shape
    Hq = lse_att.shape[1]
    _require(blk_max.shape[2] == (T + TILE - 1) // TILE, "stats length mismatch")
    _require(keep.dtype == torch.uint8 and keep.is_contiguous(), "keep: contiguous uint8 [B, Hkv, NBC]")
    p = UpdateArgs()
    p.blk_max, p.blk_sum, p.trig, p.cs_now = blk_max.data_ptr(), blk_sum.data_ptr(), trig.data_ptr(), cs_now.data_ptr()
    p.keep, p.lse_ref, p.cs_ref, p.lse_att = keep.data_ptr(), lse_ref.data_ptr(), cs_ref.data_ptr(), lse_att.data_ptr()
    p.B, p.Hq, p.Hkv, p.T, p.NBC, p.local = B, Hq, Hkv, int(T), NBC, int(local)
    p.level = float(level)

    def set_flags_idx():
        _require(flags.is_cuda and flags.dtype == torch.int32 and flags.numel() == Hkv, "flags: int32 [Hkv]")
        p.flags = flags.data_ptr()
        if idx is not None:
            _require(idx.is_cuda and idx.dtype == torch.uint8 and idx.is_contiguous() and idx.shape[0] == B
                     and idx.shape[1] == NBC, "idx: contiguous uint8 [B, NBC]")
            p.idx = idx.data_ptr()

    if calib is not None:
        _require(flags is not None and est is not None, "calibration needs flags and est")
        _require(flags.is_cuda and flags.dtype == torch.int32 and flags.numel() == Hkv, "flags: int32 [Hkv]")
        check_f32(est, "est")
        check_f32(calib, "calib")
        _require(est.numel() == B * Hkv and calib.numel() == B * Hkv, "est / calib: [B, Hkv]")
        p.flags, p.est, p.calib = flags.data_ptr(), est.data_ptr(), calib.data_ptr()
        p.calib_rate, p.calib_free, p.calib_kind = float(calib_rate), int(bool(calib_free)), int(calib_kind)
        if aix is not None:
            _require(aix.is_cuda and aix.dtype == torch.uint8 and aix.is_contiguous() and aix.numel() == B * Hkv,
                     "aix: contiguous uint8 [B, Hkv]")
            _require(idx is not None, "aix needs idx")
            p.aix, p.aix_thr = aix.data_ptr(), float(aix_thr)
        set_flags_idx()
    if list_stats:
        _require(flags is not None, "list_stats needs flags")
        set_flags_idx()
        p.list_stats = 1
    p.seq_lens = _seq_lens_ptr(seq_lens, B)
    if age is not None:
        _require(age.is_cuda and age.dtype == torch.int32 and age.is_contiguous() and age.numel() == B * Hkv,
                 "age: contiguous int32 [B, Hkv]")
        p.age = age.data_ptr()
    return p


def update(blk_max, blk_sum, trig, cs_now, keep, lse_ref, cs_ref, lse_att, T, level, local, flags=None, idx=None,
           est=None, calib=None, calib_rate=0.0, calib_free=False, calib_kind=0, aix=None, aix_thr=0.0,
           list_stats=False, seq_lens=None, age=None):
    """Device-side refresh planner after the pass (kernels/kvskip_ext.cpp:270-319); in place.

    list_stats (not in the reference): blk_max / blk_sum hold values only for the blocks of this
    step's plan (the masked pass ran on unfilled buffers); the kernel derives the read set from
    trig, keep, flags and idx and ignores the rest. Needs flags (and idx if the plan had one).
    age (not in the reference): advance the plan's age here (after decode_splits_planned)."""
    p = _update_args(blk_max, blk_sum, trig, cs_now, keep, lse_ref, cs_ref, lse_att, T, level, local, flags, idx,
                     est, calib, calib_rate, calib_free, calib_kind, aix, aix_thr, list_stats, seq_lens, age)
    dev = keep.device
    with torch.cuda.device(dev):
        _native.check(_native.lib().kvskip_update(ctypes.byref(p), _stream(dev)))


def merge_update(q, k, v, scale, bufs: dict, num_splits, update_args: tuple, update_kwargs: dict,
                 block_idx=None, block_cnt=None, seq_lens=None, block_table=None, T=None, list_partition=0):
    """The split merge of a decode_into(..., phase=1) pass (same q, k, v, bufs, list, num_splits >= 2)
    and update(*update_args, **update_kwargs), in one launch (kvskip_merge_update; not in the
    reference). block_table, T: the pass's paged cache (see _kv_dims); list_partition: the pass's."""
    B, Hq, D = q.shape
    _require(num_splits >= 2, "merge_update needs num_splits >= 2")
    a = _decode_args(q, k, v, scale, block_idx, block_cnt, num_splits, bufs["out"], bufs["lse"], None, None, None,
                     None, bufs["part_acc"], bufs["part_ml"], seq_lens, block_table, T, list_partition)
    u = _update_args(*update_args, **update_kwargs)
    dev = q.device
    with torch.cuda.device(dev):
        _native.check(_native.lib().kvskip_merge_update(ctypes.byref(a), ctypes.byref(u), _stream(dev)))


def update_struct(*update_args, **update_kwargs) -> UpdateArgs:
    """The argument block of update(*update_args, **update_kwargs), checked, for a later launch
    (decode_splits_update, launch_update); it holds raw pointers, so the tensors must outlive its use."""
    return _update_args(*update_args, **update_kwargs)


def launch_update(update: UpdateArgs, device):
    """update() from an update_struct, on the current stream of `device`."""
    dev = torch.device(device)
    with torch.cuda.device(dev):
        _native.check(_native.lib().kvskip_update(ctypes.byref(update), _stream(dev)))


def decode_splits_update(q, k, v, scale, bufs: dict, block_idx, block_cnt, num_splits, update: UpdateArgs,
                         seq_lens=None, block_table=None, T=None, list_partition=0):
    """decode_into(..., stats=True, phase=1) over a block list (the whole op when num_splits == 1)
    and the update of ANOTHER layer (an update_struct), in one launch (kvskip_decode_splits_update;
    not in the reference). The update reads only its own layer's buffers. block_table, T: a paged cache."""
    check_q(q)
    check_kv(k, "k")
    check_kv(v, "v")
    B, Hq, D, Hkv, T = _kv_dims(q, k, v, block_table, T)
    _require(1 <= num_splits <= 256, "num_splits in 1..256")
    nb = (T + TILE - 1) // TILE
    bmax, bsum = bufs["blk_max"], bufs["blk_sum"]
    for t in (bmax, bsum):
        _require(t.dtype == torch.float32 and t.is_contiguous() and t.numel() >= B * Hq * nb, "bufs: stats")
    part_acc = part_ml = None
    if num_splits > 1:
        part_acc, part_ml = bufs["part_acc"], bufs["part_ml"]
        _require(part_acc.numel() >= B * Hq * num_splits * D and part_ml.numel() >= B * Hq * num_splits * 2,
                 "bufs: split partials")
    a = _decode_args(q, k, v, scale, block_idx, block_cnt, num_splits, bufs["out"], bufs["lse"], bmax, bsum, None,
                     None, part_acc, part_ml, seq_lens, block_table, T, list_partition)
    dev = q.device
    with torch.cuda.device(dev):
        _native.check(_native.lib().kvskip_decode_splits_update(ctypes.byref(a), ctypes.byref(update), _stream(dev)))


def read_bw(x, out, blocks):
    """Streaming read of x (bandwidth ceiling), kernels/kvskip_ext.cpp:321-325."""
    _require(x.is_cuda and x.is_contiguous() and (x.numel() * x.element_size()) % 16 == 0,
             "x: contiguous CUDA, 16-byte multiple")
    dev = x.device
    with torch.cuda.device(dev):
        _native.check(_native.lib().kvskip_read(x.data_ptr(), x.numel() * x.element_size(), out.data_ptr(),
                                                int(blocks), _stream(dev)))


def _seq_lens_ptr(seq_lens, B):
    if seq_lens is None:
        return None
    _require(seq_lens.is_cuda and seq_lens.dtype == torch.int32 and seq_lens.is_contiguous()
             and seq_lens.numel() == B, "seq_lens: contiguous CUDA int32 [B]")
    return seq_lens.data_ptr()


def block_sums(k, NBC, out=None, seq_lens=None, block_table=None, T=None):
    """Per-block key sums [B, Hkv, NBC, D] fp32 of k [B, Hkv, T, D] (blocks >= nb are zero);
    seq_lens: ragged batch (sequence b sums its first seq_lens[b] rows). block_table, T (not in the
    reference): k is a page pool [num_pages, Hkv, 64, D] of a paged cache (see _kv_dims)."""
    check_kv(k, "k")
    if block_table is None:
        B, Hkv, T, D = k.shape
        bt = (None, 0, 0)
    else:
        _require(T is not None and k.dim() == 4 and k.shape[2] == TILE, "paged cache: k [num_pages, Hkv, 64, D] and T")
        _require(block_table.is_cuda and block_table.dtype == torch.int32 and block_table.dim() == 2
                 and block_table.stride(1) == 1, "block_table: int32 [B, >= ceil(T / 64)] on the device, rows contiguous")
        B, (Hkv, D), T = block_table.shape[0], (k.shape[1], k.shape[3]), int(T)
        bt = (block_table.data_ptr(), block_table.stride(0), k.shape[0])
    _require((T + TILE - 1) // TILE <= NBC, "block capacity exceeded")
    if out is None:
        out = torch.empty(B, Hkv, NBC, D, dtype=torch.float32, device=k.device)
    check_f32(out, "csum")
    _require(tuple(out.shape) == (B, Hkv, NBC, D), "csum: [B, Hkv, NBC, D]")
    with torch.cuda.device(k.device):
        _native.check(_native.lib().kvskip_block_sums(k.data_ptr(), k.stride(0), k.stride(1), k.stride(2), B, Hkv, T, D,
                                                      out.data_ptr(), NBC, _seq_lens_ptr(seq_lens, B), *bt,
                                                      _stream(k.device)))
    return out


def token_index(ids, T, NBC, out=None, seq_lens=None):
    """Token-index blocks [B, NBC] uint8 of the step whose current token is ids[:, T-1]
    (ids[b, seq_lens[b] - 1] with seq_lens: ragged batch)."""
    _require(ids.is_cuda and ids.dtype == torch.int32 and ids.dim() == 2 and ids.stride(1) == 1,
             "ids: CUDA int32 [B, >= T]")
    B = ids.shape[0]
    _require(ids.shape[1] >= T >= 1, "ids: CUDA int32 [B, >= T]")
    if out is None:
        out = torch.empty(B, NBC, dtype=torch.uint8, device=ids.device)
    _require(out.dtype == torch.uint8 and out.is_contiguous() and tuple(out.shape) == (B, NBC), "idx: uint8 [B, NBC]")
    with torch.cuda.device(ids.device):
        _native.check(_native.lib().kvskip_token_index(ids.data_ptr(), ids.stride(0), B, int(T), out.data_ptr(), NBC,
                                                       _seq_lens_ptr(seq_lens, B), _stream(ids.device)))
    return out


_RULES = {"tau": 0, "topp": 1}


def select(blk_max, blk_sum, Hkv, rule, value, local=2, keep=None, block_idx=None, block_cnt=None, blk_scale=None):
    """GQA-union block selection on the device (kvskip_select; not in kvskip_ext): from per-block
    statistics [B, Hq, nb] fp32, rule "tau" (weight >= value) or "topp" (fewest blocks reaching value)
    per query head, the union over each KV head's group plus block 0 and the `local` newest blocks.
    Fills whichever outputs are given: keep uint8 [B, Hkv, nb], block_idx / block_cnt int32 ([B, Hkv, nb]
    kept first ascending, [B, Hkv]) and blk_scale fp32 [B, Hkv, nb, G] (exp(blk_max - lse over the kept
    blocks), 0 off the set)."""
    a = _select_args(blk_max, blk_sum, Hkv, rule, value, local, keep, block_idx, block_cnt, blk_scale)
    dev = blk_max.device
    with torch.cuda.device(dev):
        _native.check(_native.lib().kvskip_select(ctypes.byref(a), _stream(dev)))


def _select_args(blk_max, blk_sum, Hkv, rule, value, local, keep, block_idx, block_cnt, blk_scale):
    _require(rule in _RULES, "rule must be tau or topp")
    check_f32(blk_max, "blk_max")
    check_f32(blk_sum, "blk_sum")
    _require(blk_max.dim() == 3 and blk_sum.shape == blk_max.shape, "blk_max / blk_sum: [B, Hq, nb]")
    B, Hq, nb = blk_max.shape
    _require(Hq % Hkv == 0, "Hq must be a multiple of Hkv")
    G = Hq // Hkv
    a = _native.SelectArgs()
    a.blk_max, a.blk_sum = blk_max.data_ptr(), blk_sum.data_ptr()
    a.B, a.Hq, a.Hkv, a.nb = B, Hq, Hkv, nb
    a.rule, a.value, a.local = _RULES[rule], float(value), int(local)
    for t, shape, dtype, name in ((keep, (B, Hkv, nb), torch.uint8, "keep"), (block_idx, (B, Hkv, nb), torch.int32,
                                  "block_idx"), (block_cnt, (B, Hkv), torch.int32, "block_cnt"),
                                  (blk_scale, (B, Hkv, nb, G), torch.float32, "blk_scale")):
        if t is not None:
            _require(t.is_cuda and t.dtype == dtype and t.is_contiguous() and tuple(t.shape) == shape,
                     f"{name}: contiguous {dtype} {list(shape)} on the device")
            setattr(a, name, t.data_ptr())
    _require(block_idx is None or block_cnt is not None, "block_cnt is required with block_idx")
    return a


def pv_select(P, v, blk_max, blk_sum, rule, value, local=2, num_splits=1, want_f32=False, keep=None,
              block_idx=None, block_cnt=None, blk_scale=None):
    """Two-pass V-skip pass 2 with the selection in it (kvskip_pv_select; not in kvskip_ext): select()
    on pass 1's statistics, then pv() over the kept blocks and their scales, in one launch (+ the split
    merge), the same results bit for bit. Contiguous cache. keep / block_idx / block_cnt / blk_scale:
    select()'s outputs, filled if given. Returns [out bf16, out_f32 or None]."""
    check_kv(v, "v")
    _require(P.is_cuda and P.dtype == torch.float16 and P.dim() == 3 and P.is_contiguous(), "P: fp16 [B, Hq, t_pad]")
    B, Hkv, T, D = v.shape
    Hq = P.shape[1]
    nb = (T + TILE - 1) // TILE
    _require(P.shape[0] == B and P.shape[2] == nb * TILE, "P shape")
    _require(tuple(blk_max.shape) == (B, Hq, nb), "blk_max: [B, Hq, nb] of the pass's cache")
    _require(num_splits >= 1, "num_splits >= 1")
    sa = _select_args(blk_max, blk_sum, Hkv, rule, value, local, keep, block_idx, block_cnt, blk_scale)
    dev = v.device
    f32 = dict(dtype=torch.float32, device=dev)
    out = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=dev)
    out32 = torch.empty(B, Hq, D, **f32) if want_f32 else None
    part_acc = torch.empty(B, Hq, num_splits, D, **f32) if num_splits > 1 else None
    part_ml = torch.empty(B, Hq, num_splits, 2, **f32) if num_splits > 1 else None
    a = _attn_args(None, None, v, 1.0, B, Hq, Hkv, T, D)
    a.num_splits = int(num_splits)
    a.part_acc, a.part_ml = _ptr(part_acc), _ptr(part_ml)
    a.out, a.out_f32 = out.data_ptr(), _ptr(out32)
    a.p_in = P.data_ptr()
    with torch.cuda.device(dev):
        _native.check(_native.lib().kvskip_pv_select(ctypes.byref(a), ctypes.byref(sa), _stream(dev)))
    return [out, out32]


def block_list(keep, block_idx, block_cnt):
    """The kept-first block list of a keep mask [B, Hkv, nb] (bool or uint8) on the device
    (kvskip_block_list; not in kvskip_ext): block_idx int32 [B, Hkv, nb] (kept blocks ascending, then
    the others ascending), block_cnt int32 [B, Hkv]."""
    _require(keep.is_cuda and keep.dtype in (torch.bool, torch.uint8) and keep.dim() == 3 and keep.is_contiguous(),
             "keep: contiguous bool / uint8 [B, Hkv, nb] on the device")
    B, Hkv, nb = keep.shape
    _require(block_idx.dtype == torch.int32 and block_idx.is_contiguous() and tuple(block_idx.shape) == (B, Hkv, nb),
             "block_idx: int32 [B, Hkv, nb]")
    _require(block_cnt.dtype == torch.int32 and block_cnt.is_contiguous() and tuple(block_cnt.shape) == (B, Hkv),
             "block_cnt: int32 [B, Hkv]")
    dev = keep.device
    with torch.cuda.device(dev):
        _native.check(_native.lib().kvskip_block_list(keep.data_ptr(), B, Hkv, nb, block_idx.data_ptr(),
                                                      block_cnt.data_ptr(), _stream(dev)))
