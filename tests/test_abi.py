"""CPU checks of the native boundary: the library loads, exports every entry point that
include/kvskip_amd.h declares, its struct layouts match the ctypes mirrors, and argument
validation fails with the reference's messages before any device work (no GPU needed)."""

import ctypes
import re
from pathlib import Path

import pytest
import torch

from kvskip_amd import _native, ext
from kvskip_amd._native import AttnArgs, PlanArgs, SelectArgs, UpdateArgs

HEADER = Path(__file__).resolve().parent.parent / "include" / "kvskip_amd.h"


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(kvskip_\w+)\s*\(", text, re.M)))


def test_header_symbols_exported():
    lib = _native.lib()
    names = declared()
    assert "kvskip_decode" in names and "kvskip_plan" in names and len(names) >= 11
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(_native.SIGNATURES) == names
    assert b"gfx950" in lib.kvskip_version()


def test_struct_layouts():
    lib = _native.lib()
    assert lib.kvskip_struct_size(0) == ctypes.sizeof(AttnArgs)
    assert lib.kvskip_struct_size(1) == ctypes.sizeof(PlanArgs)
    assert lib.kvskip_struct_size(2) == ctypes.sizeof(UpdateArgs)
    assert lib.kvskip_struct_size(3) == ctypes.sizeof(SelectArgs)
    assert lib.kvskip_struct_size(4) == -1


def _args(**kw):
    a = AttnArgs()
    a.q, a.k, a.v = 0x1000, 0x2000, 0x3000
    a.q_sb, a.q_sh = 32 * 128, 128
    a.k_sb, a.k_sh, a.k_st = 8 * 4096 * 128, 4096 * 128, 128
    a.v_sb, a.v_sh, a.v_st = a.k_sb, a.k_sh, a.k_st
    a.B, a.Hq, a.Hkv, a.T, a.D = 1, 32, 8, 4096, 128
    a.scale = 128 ** -0.5
    a.num_splits = 1
    a.out, a.lse = 0x4000, 0x5000
    for k_, v_ in kw.items():
        setattr(a, k_, v_)
    return a


@pytest.mark.parametrize("kw,code,msg", [
    (dict(D=96), -2, "unsupported head dim"),
    (dict(Hq=30), -1, "Hq must be a multiple of Hkv"),
    (dict(k_st=100), -1, "k strides must be multiples of 8"),
    (dict(v=0x3008), -1, "v must be 16-byte aligned"),
    (dict(q=0), -1, "q must be CUDA bf16"),
    (dict(num_splits=0), -1, "num_splits >= 1"),
    (dict(num_splits=4), -1, "split partial buffers"),
    (dict(T=0), -1, "sizes must be positive"),
    (dict(block_idx=0x6000), -1, "block_cnt is required with block_idx"),
    (dict(list_partition=2), -1, "list_partition in {0, 1}"),
    (dict(list_partition=1), -1, "list_partition 1 partitions a masked ragged pass"),
    (dict(list_partition=1, block_idx=0x6000, block_cnt=0x7000, num_splits=4, part_acc=0x8000, part_ml=0x9000,
          B=65, seq_lens=0xa000), -2, "list_partition 1: B * Hkv <= 512"),
])
def test_decode_validation(kw, code, msg):
    lib = _native.lib()
    rc = lib.kvskip_decode(ctypes.byref(_args(**kw)), 0, 1, None)
    assert rc == code
    assert msg in lib.kvskip_last_error().decode()


def test_flag_validation():
    lib = _native.lib()
    assert lib.kvskip_decode(ctypes.byref(_args()), 0, 0, None) == -1
    assert "load_v=false only makes sense" in lib.kvskip_last_error().decode()
    assert lib.kvskip_decode(ctypes.byref(_args(p_out=0x7000)), 0, 1, None) == -1
    assert "write_p needs stats" in lib.kvskip_last_error().decode()
    assert lib.kvskip_vskip1(ctypes.byref(_args(tau=0.0)), None) == -1
    assert "tau > 0" in lib.kvskip_last_error().decode()
    assert lib.kvskip_read(0x1000, 17, 0x2000, 4, None) == -1


def test_planner_validation():
    lib = _native.lib()
    p = PlanArgs()
    p.q, p.k, p.k_sb, p.k_sh, p.k_st = 0x1000, 0x2000, 8 * 4096 * 128, 4096 * 128, 128
    for f in ("csum", "lse_ref", "cs_ref", "keep", "lse_att", "age", "flags", "cs_now", "trig", "block_idx",
              "block_cnt"):
        setattr(p, f, 0x10000)
    p.B, p.Hq, p.Hkv, p.T, p.D, p.NBC = 1, 32, 8, 4096, 128, 32
    assert lib.kvskip_plan(ctypes.byref(p), None) == -1
    assert "block capacity exceeded" in lib.kvskip_last_error().decode()
    p.NBC, p.D = 64, 80
    assert lib.kvskip_plan(ctypes.byref(p), None) == -2
    u = UpdateArgs()
    assert lib.kvskip_update(ctypes.byref(u), None) == -1
    assert lib.kvskip_block_sums(0, 0, 0, 0, 1, 1, 1, 128, 0, 1, None, None, 0, 0, None) == -1
    assert lib.kvskip_token_index(0x1000, 10, 1, 20, 0x2000, 1, None, None) == -1


def test_python_shim_messages():
    """The torch-level checks of kernels/kvskip_ext.cpp raise RuntimeError with the same text."""
    q = torch.zeros(1, 32, 128, dtype=torch.bfloat16)
    k = torch.zeros(1, 8, 64, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match=r"q must be CUDA bf16 \[B, Hq, D\]"):
        ext.decode(q, k, k, 0.1)
    with pytest.raises(RuntimeError, match="k must be a CUDA bf16 tensor"):
        ext.check_kv(k, "k")
    with pytest.raises(RuntimeError, match="x: contiguous CUDA"):
        ext.read_bw(k, torch.zeros(1), 4)


def test_scratch_decode_validation():
    """kvskip_decode_scratch refuses more split partials than its static array holds, before any
    device call, and otherwise validates like kvskip_decode."""
    lib = _native.lib()
    a = _args(B=64, num_splits=64)           # 64 * 32 * 64 * 130 * 4 bytes > 16 MiB
    assert lib.kvskip_decode_scratch(ctypes.byref(a), 0, 1, None) == -1
    assert "the scratch holds 16777216" in lib.kvskip_last_error().decode()
    assert lib.kvskip_decode_scratch(ctypes.byref(_args(D=96)), 0, 1, None) == -2
    assert lib.kvskip_decode_scratch(None, 0, 1, None) == -1


def test_select_validation():
    """kvskip_select / kvskip_block_list refuse bad arguments before any device work."""
    lib = _native.lib()
    a = SelectArgs()
    a.blk_max, a.blk_sum = 0x1000, 0x2000
    a.B, a.Hq, a.Hkv, a.nb, a.rule, a.value, a.local = 1, 32, 8, 512, 1, 0.99, 2
    for kw, code, msg in ((dict(rule=2), -1, "rule must be tau or topp"), (dict(Hq=30), -1, "multiple of Hkv"),
                          (dict(Hq=72), -2, "G <= 8"), (dict(nb=5000), -2, "at most 4096 blocks"),
                          (dict(value=0.0), -1, "value > 0"), (dict(blk_sum=0), -1, "blk_max / blk_sum"),
                          (dict(block_idx=0x3000), -1, "block_cnt is required")):
        b = SelectArgs.from_buffer_copy(a)
        for k_, v_ in kw.items():
            setattr(b, k_, v_)
        assert lib.kvskip_select(ctypes.byref(b), None) == code, kw
        assert msg in lib.kvskip_last_error().decode(), kw
    assert lib.kvskip_block_list(0, 1, 1, 4, 0x1000, 0x2000, None) == -1
    assert lib.kvskip_block_list(0x1000, 1, 0, 4, 0x1000, 0x2000, None) == -1


def test_planned_pass_validation():
    """kvskip_decode_splits_planned refuses an unknown decide_mode, a pass budget out of range or over
    more than 16 lists, and mismatched shapes, before any device work."""
    lib = _native.lib()
    p = PlanArgs()
    p.q, p.k, p.k_sb, p.k_sh, p.k_st = 0x1000, 0x2000, 8 * 4096 * 128, 4096 * 128, 128
    for f in ("csum", "lse_ref", "cs_ref", "keep", "lse_att", "age", "flags", "cs_now", "trig", "block_idx",
              "block_cnt", "part"):
        setattr(p, f, 0x10000)
    p.B, p.Hq, p.Hkv, p.T, p.D, p.NBC = 1, 32, 8, 4096, 128, 128
    for kw, code, msg in ((dict(decide_mode=3), -1, "decide_mode in {0, 1, 2}"),
                          (dict(decide_mode=-1), -1, "decide_mode in {0, 1, 2}"),
                          (dict(pass_budget=-1), -1, "pass_budget in 0..65536"),
                          (dict(pass_budget=70000), -1, "pass_budget in 0..65536")):
        q = PlanArgs.from_buffer_copy(p)
        for k_, v_ in kw.items():
            setattr(q, k_, v_)
        assert lib.kvskip_decode_splits_planned(ctypes.byref(_args(num_splits=4, part_acc=0x8000, part_ml=0x9000)),
                                                ctypes.byref(q), None, None) == code, kw
        assert msg in lib.kvskip_last_error().decode(), kw
    q = PlanArgs.from_buffer_copy(p)
    q.B, q.Hkv, q.Hq, q.pass_budget = 4, 8, 32, 100
    a = _args(B=4, num_splits=4, part_acc=0x8000, part_ml=0x9000)
    assert lib.kvskip_decode_splits_planned(ctypes.byref(a), ctypes.byref(q), None, None) == -2
    assert "pass_budget needs B * Hkv <= 16" in lib.kvskip_last_error().decode()
    assert lib.kvskip_decode_splits_planned(ctypes.byref(_args(T=2048)), ctypes.byref(p), None, None) == -1
    assert "attention and plan shapes differ" in lib.kvskip_last_error().decode()


def test_planned_ragged_validation():
    """A ragged batch (seq_lens, B > 1) in kvskip_decode_splits_planned: at most 16 sequences, a
    contiguous cache, and no pass budget, partial slots, lse_part or DECIDE_POST; refused before any
    device work."""
    lib = _native.lib()
    p = PlanArgs()
    p.q, p.k, p.k_sb, p.k_sh, p.k_st = 0x1000, 0x2000, 8 * 4096 * 128, 4096 * 128, 128
    for f in ("csum", "lse_ref", "cs_ref", "keep", "lse_att", "age", "flags", "cs_now", "trig", "block_idx",
              "block_cnt", "part"):
        setattr(p, f, 0x10000)
    p.Hq, p.Hkv, p.T, p.D, p.NBC, p.seq_lens = 32, 8, 4096, 128, 128, 0x20000
    cases = ((dict(B=17), {}, "at most 16 sequences"),
             (dict(B=4, pass_budget=100), {}, "takes no pass_budget"),
             (dict(B=4, slot_count=2), {}, "takes no pass_budget"),
             (dict(B=4, decide_mode=2), {}, "takes no pass_budget"),
             (dict(B=4), dict(block_table=0x30000, bt_stride=64, num_pages=64), "contiguous cache"))
    for pk, ak, msg in cases:
        q = PlanArgs.from_buffer_copy(p)
        for k_, v_ in pk.items():
            setattr(q, k_, v_)
        a = _args(B=q.B, num_splits=4, part_acc=0x8000, part_ml=0x9000, seq_lens=0x20000, **ak)
        assert lib.kvskip_decode_splits_planned(ctypes.byref(a), ctypes.byref(q), None, None) == -2, (pk, ak)
        assert msg in lib.kvskip_last_error().decode(), (pk, ak, lib.kvskip_last_error())
