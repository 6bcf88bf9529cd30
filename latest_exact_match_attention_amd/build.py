"""Build liblema_hip.so in-tree from csrc/*.hip with hipcc for gfx950.

    python -m latest_exact_match_attention_amd.build          # compile + link
    python -m latest_exact_match_attention_amd.build --check  # is the built library current?
    python -m latest_exact_match_attention_amd.build --stamps # diagnostics library (below)

`--stamps` builds liblema_hip_stamps.so beside the product library: the same sources with the
decode-step kernel reading the clock after each of its phases (LEMA_STEP_STAMPS), for
`bench.py --workload decode --step-stamps`. Nothing else loads it.

hipcc cross-compiles without a GPU. Objects go to `_build/` at the repository root, the
library next to this file, where `_lib.py` loads it.
"""
from __future__ import annotations

import argparse
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
ROOT = PKG.parent
BUILD = ROOT / "_build"
LIB = PKG / "liblema_hip.so"
STAMPS_LIB = PKG / "liblema_hip_stamps.so"
INCLUDE = ROOT / "include"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# The compiler is kept from forming packed-FP32 instructions (v_pk_{add,mul,fma}_f32) out of
# plain float code: no kernel here needs them and some of their forms are unreliable on
# this hardware class.
FLAGS = [f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _deps() -> list[Path]:
    return sources() + sorted(CSRC.glob("*.h")) + sorted(INCLUDE.glob("*.h"))


def is_current() -> bool:
    if not LIB.exists():
        return False
    t = LIB.stat().st_mtime
    return all(p.stat().st_mtime <= t for p in _deps())


def _compile(src: Path, extra: tuple = (), suffix: str = "") -> tuple[Path, str]:
    obj = BUILD / (src.stem + suffix + ".o")
    cmd = [HIPCC, *FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    log = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                    if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{log}")
    return obj, log


def build(verbose: bool = False, stamps: bool = False) -> Path:
    """Compile every csrc/*.hip for gfx950 and link liblema_hip.so (always rebuilds); with
    `stamps` the diagnostics library liblema_hip_stamps.so instead."""
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    extra, suffix, lib = (("-DLEMA_STEP_STAMPS",), "_stamps", STAMPS_LIB) if stamps else ((), "", LIB)
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        results = list(ex.map(lambda src: _compile(src, extra, suffix), srcs))
    for _, log in results:
        if verbose and log.strip():
            print(log, file=sys.stderr)
    tmp = lib.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC",
           *[str(o) for o, _ in results], "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, lib)
    return lib


def ensure_built() -> Path:
    """Build only when the library is missing or older than its sources."""
    return LIB if is_current() else build()


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--check", action="store_true")
    ap.add_argument("-v", "--verbose", action="store_true")
    ap.add_argument("--stamps", action="store_true")
    a = ap.parse_args(argv)
    if a.check:
        print("current" if is_current() else "stale")
        return 0 if is_current() else 1
    print(build(verbose=a.verbose, stamps=a.stamps))
    return 0


if __name__ == "__main__":
    sys.exit(main())
