"""Build libkvskip_amd.so in-tree for gfx950 with hipcc (objects in _build/, one per source, in
parallel). Usage: python -m kvskip_amd.build"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "kvskip_amd" / "csrc"
OUT = ROOT / "kvskip_amd" / "libkvskip_amd.so"
BUILD = ROOT / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
SOURCES = ["attn_decode.hip", "attn_decode_paged.hip", "attn_vskip.hip", "planner.hip", "split_update.hip", "split_update_paged.hip", "planned.hip", "planned_paged.hip", "planned_ragged.hip", "select.hip", "capi.hip"]
# Packed FP32 (v_pk_*_f32) stays off: hipcc would otherwise form it from plain float code.
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", f"-I{ROOT / 'include'}",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _compile(src: str) -> Path:
    obj = BUILD / (Path(src).stem + ".o")
    cmd = [HIPCC, *FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = OUT.with_suffix(".so.tmp")
    r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-o", str(tmp), *map(str, objs)],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT} ({OUT.stat().st_size} bytes)", flush=True)
    return OUT


if __name__ == "__main__":
    build()
    sys.exit(0)
