"""Compile the gfx950 HIP sources into the in-tree shared library.

``python -m local_kimi_amd._build`` (or ``__graft_entry__.build()``) compiles
every ``csrc/*.hip`` with hipcc for gfx950 into ``local_kimi_amd/liblkamd.so``,
and the measurement probes of ``probe/*.hip`` (used by the benchmark only)
into ``local_kimi_amd/liblkprobe.so``. Objects are compiled in parallel and
each library is linked once. The product library exports only the C ABI
declared in ``include/lk_*.h`` (``lk_probe.h`` belongs to the probe library).
"""

from __future__ import annotations

import concurrent.futures
import glob
import os
import shutil
import subprocess

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
PROBE = os.path.join(PKG, "probe")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "liblkamd.so")
PROBE_LIB = os.path.join(PKG, "liblkprobe.so")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Wall",
    "-Wno-unused-function",
    # packed fp32 ops are kept out of the generated code on this target
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the HIP library cannot be built")
    return path


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", src, "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{proc.stdout}\n{proc.stderr}")
    noise = "is not a recognized feature for this target"
    warnings = "\n".join(line for line in proc.stderr.splitlines() if noise not in line).strip()
    if warnings:
        print(warnings)
    return obj


def _link(sources: list[str], out: str) -> None:
    workers = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(workers) as pool:
        objects = list(pool.map(_compile, sources))
    tmp = out + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objects]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, out)


def build(verbose: bool = True) -> str:
    """Compile all HIP sources, link ``liblkamd.so`` and the probe library;
    returns the product library's path."""
    os.makedirs(BUILD, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    probes = sorted(glob.glob(os.path.join(PROBE, "*.hip")))
    _link(sources, LIB)
    if probes:
        _link(probes, PROBE_LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources" +
              (f" and {PROBE_LIB} from {len(probes)}" if probes else ""))
    return LIB


if __name__ == "__main__":
    build()
