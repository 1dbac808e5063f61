"""ctypes binding of libkvskip_amd.so (the C ABI declared in include/kvskip_amd.h).

Loads the in-tree library built by __graft_entry__.build() / kvskip_amd/build.py. There is no
fallback: if the library is missing or does not load, every operator raises.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_uint8, c_void_p
from pathlib import Path

LIB_PATH = Path(os.environ.get("KVSKIP_AMD_LIB", Path(__file__).resolve().parent / "libkvskip_amd.so"))


class AttnArgs(ctypes.Structure):
    """kvskip_attn_args."""
    _fields_ = [
        ("q", c_void_p), ("k", c_void_p), ("v", c_void_p),
        ("q_sb", c_int64), ("q_sh", c_int64),
        ("k_sb", c_int64), ("k_sh", c_int64), ("k_st", c_int64),
        ("v_sb", c_int64), ("v_sh", c_int64), ("v_st", c_int64),
        ("B", c_int32), ("Hq", c_int32), ("Hkv", c_int32), ("T", c_int32), ("D", c_int32),
        ("scale", c_float),
        ("block_idx", c_void_p), ("block_cnt", c_void_p), ("max_blocks", c_int32),
        ("num_splits", c_int32), ("part_acc", c_void_p), ("part_ml", c_void_p),
        ("out", c_void_p), ("out_f32", c_void_p), ("lse", c_void_p),
        ("blk_max", c_void_p), ("blk_sum", c_void_p),
        ("p_out", c_void_p), ("p_in", c_void_p), ("blk_scale", c_void_p),
        ("tau", c_float), ("local", c_int32), ("vcount", c_void_p), ("lse_prev", c_void_p),
        ("seq_lens", c_void_p), ("block_table", c_void_p), ("bt_stride", c_int64), ("num_pages", c_int32),
        ("v_keep", c_void_p), ("list_partition", c_int32),
    ]


class PlanArgs(ctypes.Structure):
    """kvskip_plan_args."""
    _fields_ = [
        ("q", c_void_p), ("q_sb", c_int64), ("q_sh", c_int64),
        ("k", c_void_p), ("k_sb", c_int64), ("k_sh", c_int64), ("k_st", c_int64),
        ("csum", c_void_p), ("lse_ref", c_void_p), ("cs_ref", c_void_p), ("keep", c_void_p),
        ("lse_att", c_void_p), ("age", c_void_p), ("flags", c_void_p), ("idx", c_void_p),
        ("calib", c_void_p), ("est", c_void_p), ("aix", c_void_p), ("cs_now", c_void_p),
        ("trig", c_void_p), ("block_idx", c_void_p), ("block_cnt", c_void_p),
        ("B", c_int32), ("Hq", c_int32), ("Hkv", c_int32), ("T", c_int32), ("D", c_int32),
        ("NBC", c_int32), ("local", c_int32), ("max_age", c_int32), ("add_token", c_int32),
        ("calib_on", c_int32), ("calib_kind", c_int32),
        ("scale", c_float), ("delta", c_float),
        ("part", c_void_p), ("seq_lens", c_void_p), ("seq_lens_out", c_void_p),
        ("ids", c_void_p), ("ids_sb", c_int64), ("idx_out", c_void_p),
        ("block_table", c_void_p), ("bt_stride", c_int64), ("num_pages", c_int32), ("pass_budget", c_int32),
        ("decide_mode", c_int32), ("slot_base", c_int32), ("slot_count", c_int32),
        ("lse_part", c_void_p), ("lse_slots", c_int32), ("lse_stride", c_int32), ("ticket", c_void_p),
    ]


class UpdateArgs(ctypes.Structure):
    """kvskip_update_args."""
    _fields_ = [
        ("blk_max", c_void_p), ("blk_sum", c_void_p), ("trig", c_void_p), ("cs_now", c_void_p),
        ("keep", c_void_p), ("lse_ref", c_void_p), ("cs_ref", c_void_p), ("lse_att", c_void_p),
        ("flags", c_void_p), ("idx", c_void_p), ("est", c_void_p), ("calib", c_void_p), ("aix", c_void_p),
        ("calib_rate", c_float), ("aix_thr", c_float), ("level", c_float),
        ("calib_free", c_int32), ("calib_kind", c_int32),
        ("B", c_int32), ("Hq", c_int32), ("Hkv", c_int32), ("T", c_int32), ("NBC", c_int32), ("local", c_int32),
        ("list_stats", c_int32), ("seq_lens", c_void_p), ("age", c_void_p),
    ]


class SelectArgs(ctypes.Structure):
    """kvskip_select_args."""
    _fields_ = [
        ("blk_max", c_void_p), ("blk_sum", c_void_p),
        ("B", c_int32), ("Hq", c_int32), ("Hkv", c_int32), ("nb", c_int32),
        ("rule", c_int32), ("value", c_float), ("local", c_int32),
        ("keep", c_void_p), ("block_idx", c_void_p), ("block_cnt", c_void_p), ("blk_scale", c_void_p),
    ]


# Every entry point of include/kvskip_amd.h with its argument types.
SIGNATURES = {
    "kvskip_decode": ([POINTER(AttnArgs), c_int, c_int, c_void_p], c_int),
    "kvskip_decode_splits": ([POINTER(AttnArgs), c_int, c_int, c_void_p], c_int),
    "kvskip_merge_splits": ([POINTER(AttnArgs), c_int, c_int, c_void_p], c_int),
    "kvskip_decode_scratch": ([POINTER(AttnArgs), c_int, c_int, c_void_p], c_int),
    "kvskip_pv": ([POINTER(AttnArgs), c_void_p], c_int),
    "kvskip_vskip1": ([POINTER(AttnArgs), c_void_p], c_int),
    "kvskip_read": ([c_void_p, c_int64, c_void_p, c_int32, c_void_p], c_int),
    "kvskip_plan": ([POINTER(PlanArgs), c_void_p], c_int),
    "kvskip_plan_part_floats": ([c_int32, c_int32, c_int32, c_int32], c_int64),
    "kvskip_update": ([POINTER(UpdateArgs), c_void_p], c_int),
    "kvskip_merge_update": ([POINTER(AttnArgs), POINTER(UpdateArgs), c_void_p], c_int),
    "kvskip_decode_splits_update": ([POINTER(AttnArgs), POINTER(UpdateArgs), c_void_p], c_int),
    "kvskip_plan_scores": ([POINTER(PlanArgs), c_void_p], c_int),
    "kvskip_decode_splits_planned": ([POINTER(AttnArgs), POINTER(PlanArgs), POINTER(UpdateArgs), c_void_p], c_int),
    "kvskip_block_sums": ([c_void_p, c_int64, c_int64, c_int64, c_int32, c_int32, c_int32, c_int32, c_void_p,
                           c_int32, c_void_p, c_void_p, c_int64, c_int32, c_void_p], c_int),
    "kvskip_token_index": ([c_void_p, c_int64, c_int32, c_int32, c_void_p, c_int32, c_void_p, c_void_p], c_int),
    "kvskip_select": ([POINTER(SelectArgs), c_void_p], c_int),
    "kvskip_pv_select": ([POINTER(AttnArgs), POINTER(SelectArgs), c_void_p], c_int),
    "kvskip_block_list": ([c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p], c_int),
    "kvskip_last_error": ([], c_char_p),
    "kvskip_version": ([], c_char_p),
    "kvskip_struct_size": ([c_int], c_int),
}

_LIB = None


def lib() -> ctypes.CDLL:
    """The loaded native library (raises if it is not built)."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"kvskip_amd: native library {LIB_PATH} is missing; "
                               "build it with `python -c 'import __graft_entry__ as g; g.build()'`")
        h = ctypes.CDLL(str(LIB_PATH))
        for name, (argtypes, restype) in SIGNATURES.items():
            fn = getattr(h, name)
            fn.argtypes = argtypes
            fn.restype = restype
        _LIB = h
    return _LIB


def check(rc: int) -> None:
    """Raise RuntimeError with the library's message if rc != 0."""
    if rc != 0:
        msg = lib().kvskip_last_error().decode(errors="replace")
        raise RuntimeError(msg or f"kvskip_amd: error {rc}")
