"""Build libictc_mi355x.so for gfx950 (in-tree, no JIT).

1. ``gen_tables.py`` emits ``generated/ictc_tables.h`` from the frozen basis.
2. Each ``*.hip`` translation unit is compiled in parallel with hipcc.
3. The objects are linked into ``ictc_o3/_lib/libictc_mi355x.so``.

Usage: python csrc/build.py [--jobs N]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
OUT_DIR = os.path.join(PKG, "ictc_o3", "_lib")
LIB = os.path.join(OUT_DIR, "libictc_mi355x.so")
BUILD_DIR = os.path.join(HERE, "_build")
SOURCES = ["capi.hip", "misc.hip", "radial_mlp.hip", "gate_gemm.hip", "gemm_tn.hip", "gemm_nt.hip", "species.hip", "linear.hip", "geometry.hip", "neighbors.hip", "sc.hip", "tp_edge.hip", "msg_fwd.hip", "pairs.hip",
           "msg_bwd.hip", "msg_bwd_tan.hip", "msg_fused.hip", "tp_second.hip", "msg_second_rcv.hip", "msg_second_src.hip", "sc_part_low.hip", "sc_part_l3_t0.hip", "sc_part_l3_t1.hip", "sc_part_l3_t2.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
         # Packed FP32 (v_pk_*_f32) stays off for all device code.
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-munsafe-fp-atomics"]


def _includes(path, seen):
    """Local headers reachable from ``path`` through #include "..." lines."""
    import re
    for line in open(path):
        m = re.match(r'\s*#include\s+"([^"]+)"', line)
        if not m:
            continue
        dep = os.path.normpath(os.path.join(os.path.dirname(path), m.group(1)))
        if os.path.exists(dep) and dep not in seen:
            seen.add(dep)
            _includes(dep, seen)
    return seen


def _deps_mtime(src):
    path = os.path.join(HERE, src)
    deps = _includes(path, set()) | {path}
    return max(os.path.getmtime(p) for p in deps)


def _compile(src, force=True):
    obj = os.path.join(BUILD_DIR, src.replace(".hip", ".o"))
    if (not force and os.path.exists(obj)
            and os.path.getmtime(obj) > _deps_mtime(src)):
        return obj
    cmd = [HIPCC, *FLAGS, "-c", os.path.join(HERE, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr[-6000:]}")
    return obj


def build(jobs: int | None = None, force: bool = True) -> str:
    """Compile every translation unit (``force=False``: only those older than their inputs)."""
    sys.path.insert(0, HERE)
    import gen_sc
    import gen_tables
    gen_tables.generate(os.path.join(HERE, "generated", "ictc_tables.h"))
    gen_sc.generate(os.path.join(HERE, "generated", "ictc_sc.h"))
    os.makedirs(BUILD_DIR, exist_ok=True)
    os.makedirs(OUT_DIR, exist_ok=True)
    jobs = jobs or min(len(SOURCES), max(1, (os.cpu_count() or 2)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda src: _compile(src, force), SOURCES))
    tmp = LIB + ".tmp"
    r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp],
                       capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"link failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--incremental", action="store_true", help="skip objects newer than their inputs")
    a = ap.parse_args()
    print(build(a.jobs, force=not a.incremental))
