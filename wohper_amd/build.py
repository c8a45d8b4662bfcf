"""Builds the gfx950 library libwohper_hip.so in-tree.

Steps: compile and run the libm table generator (host glibc is the
specification it verifies against; the table is cached by content hash of
its inputs), then hipcc the single HIP translation unit.
"""
from __future__ import annotations

import hashlib
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
GEN = CSRC / "_gen"
LIB = PKG / "libwohper_hip.so"

HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the MI355X library cannot be built")


def _glibc_version() -> str:
    try:
        return os.confstr("CS_GNU_LIBC_VERSION") or "unknown"
    except (ValueError, OSError):
        return "unknown"


def build_libm_tables(verbose: bool = True) -> Path:
    GEN.mkdir(exist_ok=True)
    src = CSRC / "gen_libm_tables.c"
    hdr = CSRC / "libm_emul.h"
    key = hashlib.sha256(src.read_bytes() + hdr.read_bytes() + _glibc_version().encode()).hexdigest()
    inc = GEN / "libm_tables.inc"
    stamp = GEN / "libm_tables.key"
    if inc.exists() and stamp.exists() and stamp.read_text() == key:
        return inc
    exe = GEN / "gen_libm_tables"
    subprocess.run(
        ["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-I", str(CSRC), str(src), "-o", str(exe),
         "-lm", "-lpthread"],
        check=True,
    )
    if verbose:
        print("[wohper_amd] generating glibc-exact libm tables (exhaustive check, ~15 s)", flush=True)
    tmp = GEN / "libm_tables.inc.tmp"
    subprocess.run([str(exe), str(tmp)], check=True)
    tmp.replace(inc)
    stamp.write_text(key)
    return inc


def build(verbose: bool = True, timeline: Path | None = None) -> Path:
    """Builds libwohper_hip.so in the package.  timeline: instead build the
    per-wave timeline variant (-DWH_TIMELINE: the persistent expert kernels
    stamp s_memrealtime at fixed points, read back with wh_debug_timeline)
    to that path; it is a measuring build, not the product."""
    build_libm_tables(verbose)
    out = Path(timeline) if timeline else LIB
    cmd = [_hipcc(), *HIP_FLAGS, *(["-DWH_TIMELINE"] if timeline else []), "-I", str(ROOT / "include"),
           "-I", str(CSRC), "-I", str(GEN), "-o", str(out) + ".tmp", str(CSRC / "wohper_hip.hip")]
    if verbose:
        print("[wohper_amd] " + " ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass reports the device-only feature flag as unknown: harmless
    noise = [ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln]
    if res.returncode != 0:
        sys.stderr.write("\n".join(noise) + "\n")
        raise RuntimeError("hipcc failed building libwohper_hip.so")
    if noise and verbose:
        sys.stderr.write("\n".join(noise) + "\n")
    os.replace(str(out) + ".tmp", out)
    return out


if __name__ == "__main__":
    import argparse

    ap = argparse.ArgumentParser()
    ap.add_argument("--timeline", type=Path, default=None,
                    help="build the per-wave timeline variant to this path instead of the product library")
    build(timeline=ap.parse_args().timeline)
