"""Build the gfx950 HIP library ``libsuperl8_kv.so`` in-tree.

Every ``csrc/*.hip`` file is compiled for gfx950 with hipcc (in parallel) and
linked into one shared library next to this file.  Packed-fp32 VALU ops are
disabled (``-packed-fp32-ops``); fp16 packed math and MFMA are unaffected.

A second library, ``libsuperl8_kv_trace.so``, is the same code with the
decode kernel built with ``-DS8KV_DECODE_TRACE``: per-workgroup timestamps of
each decode launch (a diagnostics build for ``bench.py --trace-decode``; the
ops never load it).

Usage: ``python -m superl8_serve_amd.build_ext`` or ``build()`` from Python.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
INCLUDE = PKG_DIR.parent / "include"
LIB_NAME = "libsuperl8_kv.so"
LIB_PATH = PKG_DIR / LIB_NAME
TRACE_LIB_PATH = PKG_DIR / "libsuperl8_kv_trace.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}",
]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the HIP library cannot be built")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in proc.stdout.splitlines() if "packed-fp32-ops" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile all HIP sources and link ``libsuperl8_kv.so`` (and the decode
    trace build ``libsuperl8_kv_trace.so``).  Always rebuilds."""
    hipcc = _hipcc()
    obj_dir = PKG_DIR / "_build"
    obj_dir.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    objs = [obj_dir / (s.stem + ".o") for s in sources]
    cmds = [[hipcc, *HIPCC_FLAGS, "-c", str(s), "-o", str(o)] for s, o in zip(sources, objs)]
    decode_src = CSRC / "s8kv_decode.hip"
    trace_obj = obj_dir / "s8kv_decode_trace.o"
    cmds.append([hipcc, *HIPCC_FLAGS, "-DS8KV_DECODE_TRACE", "-c", str(decode_src), "-o", str(trace_obj)])
    workers = jobs or min(len(cmds), max(1, (os.cpu_count() or 4)))
    with ThreadPoolExecutor(max_workers=workers) as ex:
        for cmd, fut in zip(cmds, [ex.submit(_run, c) for c in cmds]):
            if verbose:
                print(" ".join(cmd))
            fut.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB_PATH)
    trace_objs = [trace_obj if o.stem == "s8kv_decode" else o for o in objs]
    tmp = TRACE_LIB_PATH.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, trace_objs)])
    os.replace(tmp, TRACE_LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
