"""kvskip_amd: the kvskip decode-attention hot path (dense / block-list / per-block statistics /
V-skip split-K decode and the device-side refresh planner) as hand-written HIP kernels for
MI355X (gfx950), behind the reference's `kvskip_ext` operator surface (kvskip_amd.ext), the
Python API of its kernels/kvskip.py (kvskip_amd.kvskip) and a device-side planner loop
(kvskip_amd.planner). The native library is libkvskip_amd.so (C ABI: include/kvskip_amd.h).
"""

__all__ = ["ext", "kvskip"]
