"""Builds libexl3_amd.so (gfx950) in-tree with hipcc, one object per bit width in
parallel, then links.  Usage: python -m dsv4_carve_amd.build [--jobs N]"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libexl3_amd.so")
# The HBM read-ceiling and decode-rate probes the benchmark times beside the
# decode kernels (not part of the decode path's ABI, so a library of its own).
PROBE_LIB = os.path.join(HERE, "libexl3_probe.so")
# Timing-only twin of libexl3_amd.so built with EXL3_NULL_DECODE=1: the same
# kernels with each decoded weight replaced by a loaded tile word, so the
# benchmark can time the loads, MFMAs, stores and launches without the decode
# (its outputs are meaningless; nothing but the benchmark loads it).
NULL_LIB = os.path.join(HERE, "libexl3_null.so")
NULL_DIR = os.path.join(OUT_DIR, "null")
ARCH = os.environ.get("EXL3_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # packed-fp32 instructions are disabled for every HIP object on this target
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{CSRC}",
]

# (source, extra defines, object name)
UNITS = [("exl3_capi.hip", [], "exl3_capi.o")]
UNITS += [("exl3_dense_inst.hip", [f"-DEXL3_BITS={b}"], f"exl3_dense_b{b}.o") for b in range(1, 9)]
UNITS += [("exl3_moe_capi.hip", [], "exl3_moe_capi.o")]
# (bit-width mask, codebook) instances of the MoE kernel; keep in sync with
# EXL3_MOE_INSTANCES in csrc/exl3_moe_capi.hip.
MOE_UNITS = [(0x004, 1), (0x008, 1), (0x010, 1), (0x040, 1), (0x00C, 1), (0x01C, 1), (0x04C, 1),
             (0x1FE, 1), (0x1FE, 0), (0x1FE, 2)]
UNITS += [("exl3_moe_inst.hip", [f"-DEXL3_MOE_MASK=0x{m:03X}u", f"-DEXL3_MOE_CB={c}"],
           f"exl3_moe_m{m:03x}_c{c}.o") for m, c in MOE_UNITS]
UNITS += [("exl3_prefill_capi.hip", [], "exl3_prefill_capi.o")]
UNITS += [("exl3_prefill_inst.hip", [f"-DEXL3_BITS={b}"], f"exl3_pf_b{b}.o") for b in range(1, 9)]
UNITS += [("exl3_prefill_inst.hip", ["-DEXL3_BITS=3", "-DEXL3_BITS2=2"], "exl3_pf_b32.o")]


def _stale(src: str, out: str) -> bool:
    """True unless `out` is newer than the unit's source and every header."""
    if not os.path.isfile(out):
        return True
    t = os.path.getmtime(out)
    deps = [os.path.join(CSRC, src)] + [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hpp")]
    return any(os.path.getmtime(d) > t for d in deps)


def _compile(unit, incremental=False):
    src, defs, obj = unit
    out = obj if os.path.isabs(obj) else os.path.join(OUT_DIR, obj)
    if incremental and not _stale(src, out):
        return out
    cmd = [HIPCC, *COMMON, *defs, "-c", os.path.join(CSRC, src), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "packed-fp32-ops"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src} {defs}:\n{err}")
    return out


def _link(objs, lib):
    tmp = lib + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link of {lib} failed:\n" + r.stderr)
    os.replace(tmp, lib)


def build(jobs: int | None = None, verbose: bool = True, null: bool = True, incremental: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    os.makedirs(NULL_DIR, exist_ok=True)
    units = [u for u in UNITS if os.path.isfile(os.path.join(CSRC, u[0]))]
    null_units = [(src, [*defs, "-DEXL3_NULL_DECODE=1"], os.path.join(NULL_DIR, obj)) for src, defs, obj in units]
    jobs = jobs or min(8, os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda u: _compile(u, incremental), units + (null_units if null else [])))
    _link(objs[:len(units)], LIB)
    if null:
        _link(objs[len(units):], NULL_LIB)
    tmp = PROBE_LIB + ".tmp"
    cmd = [HIPCC, *COMMON, "-shared", "-o", tmp, os.path.join(CSRC, "exl3_probe.hip")]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("probe build failed:\n" + r.stderr)
    os.replace(tmp, PROBE_LIB)
    if verbose:
        print(f"built {LIB} from {len(units)} objects, {PROBE_LIB}" + (f" and {NULL_LIB}" if null else ""),
              file=sys.stderr)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--no-null", action="store_true", help="skip the timing-only null-decode library")
    ap.add_argument("--incremental", action="store_true",
                    help="recompile only units older than their sources (development; build() always compiles all)")
    a = ap.parse_args()
    build(a.jobs, null=not a.no_null, incremental=a.incremental)
