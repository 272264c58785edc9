"""Build ``libwinnow_hip.so`` in-tree for gfx950 with hipcc.

    python -m winnow_amd.build            # compile every source, link the library

Each ``csrc/*.hip`` file compiles to an object in ``winnow_amd/_build/`` (in
parallel), then one ``hipcc -shared`` link writes ``winnow_amd/libwinnow_hip.so``.
Packed-FP32 instruction selection is disabled for device code
(``-target-feature -packed-fp32-ops``); the host pass ignores the flag with a
warning.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OUT_DIR = HERE / "_build"
LIB = HERE / "libwinnow_hip.so"
PROBE_LIB = HERE / "libwinnow_probe.so"  # bench.py's measurement probes (csrc/probe/), not the product
ARCH = os.environ.get("WN_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CFLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _run(cmd):
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(map(str, cmd))}\n"
                           f"{proc.stdout}\n{proc.stderr}")
    return proc


# Sources that take longest to compile (many kernel instantiations) start first.
_SLOW_FIRST = ("decode_split_any256", "decode_rows", "decode_split_any128", "decode_split_any64",
               "decode_split_any16", "decode_split_any32", "decode")


def sources():
    def rank(p):
        for i, prefix in enumerate(_SLOW_FIRST):
            if p.stem.startswith(prefix):
                return i
        return len(_SLOW_FIRST)
    return sorted(CSRC.glob("*.hip"), key=lambda p: (rank(p), p.name))


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every HIP source for ``ARCH`` and link the shared library."""
    OUT_DIR.mkdir(exist_ok=True)
    srcs = sources()
    objs = [OUT_DIR / (s.stem + ".o") for s in srcs]

    def compile_one(pair):
        src, obj = pair
        cmd = [HIPCC, *CFLAGS, "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        _run(cmd)
        return obj

    probe_srcs = sorted((CSRC / "probe").glob("*.hip"))
    probe_objs = [OUT_DIR / ("probe_" + s.stem + ".o") for s in probe_srcs]
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(compile_one, zip(srcs + probe_srcs, objs + probe_objs)))
    for lib, lib_objs in ((LIB, objs), (PROBE_LIB, probe_objs)):
        tmp = lib.with_suffix(".so.tmp")
        _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, lib_objs), "-o", str(tmp)])
        os.replace(tmp, lib)
        if verbose:
            print(f"built {lib}", flush=True)
    return LIB


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
