"""Build liblogkv_hip.so (gfx950) from logkv_amd/csrc with hipcc.

Flags: -ffp-contract=off (no fused multiply-add anywhere, so every kernel keeps
the exact float32 operation order its comments state), packed fp32 ops
disabled, -O3. Objects go to logkv_amd/_build; the library lands next to this
file, where ``logkv_amd._lib`` loads it.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "liblogkv_hip.so"
ARCH = os.environ.get("LOGKV_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (Path(cand).exists() or cand == "hipcc"):
            return cand
    raise RuntimeError("hipcc not found")


def sources():
    return sorted(CSRC.glob("*.hip"))


def build(verbose: bool = False, jobs: int = 8) -> Path:
    """Compile every HIP source for gfx950 and link the shared library (always rebuilds)."""
    BUILD.mkdir(exist_ok=True)
    cc = hipcc()
    procs = []
    objs = []
    for src in sources():
        obj = BUILD / (src.stem + ".o")
        objs.append(obj)
        cmd = [cc, *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
        if len(procs) >= jobs:
            _wait(procs.pop(0))
    for p in procs:
        _wait(p)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    out = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if out.returncode:
        raise RuntimeError(f"link failed:\n{out.stdout}")
    os.replace(tmp, LIB)
    return LIB


def _wait(item):
    src, proc = item
    out, _ = proc.communicate()
    if proc.returncode:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{out}")
    warn = [line for line in out.splitlines() if "packed-fp32-ops" not in line and line.strip()]
    if warn:
        print(f"[{src.name}]\n" + "\n".join(warn), file=sys.stderr)


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
