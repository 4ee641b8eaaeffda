"""Host-side AddressSanitizer run of the C-ABI library (CPU only, no GPU).

``python tests/host_asan.py`` compiles every ``csrc/*.hip`` with the host
pass instrumented by AddressSanitizer (the gfx950 device code is compiled as
usual, without it) into ``local_kimi_amd/_build/asan/liblkamd_asan.so``, then
runs the CPU tests that call into the library (exported symbols, argument
and workspace refusals, size queries, path knobs) against that build, with
clang's ASan runtime preloaded into the Python process. Any invalid host
memory access stops the run with the sanitizer's report and a nonzero exit.
Not collected by pytest (its name has no ``test_`` prefix): the build takes a
few minutes. Leak checking is off (the Python interpreter itself is not
instrumented).
"""

from __future__ import annotations

import concurrent.futures
import glob
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "local_kimi_amd", "csrc")
OUT = os.path.join(ROOT, "local_kimi_amd", "_build", "asan")
LIB = os.path.join(OUT, "liblkamd_asan.so")
TESTS = ["tests/test_capi.py", "tests/test_host_validation.py"]

FLAGS = ["--offload-arch=gfx950", "-O1", "-g", "-fno-omit-frame-pointer", "-std=c++17", "-fPIC",
         "-fvisibility=hidden", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}"]
SANITIZE = ["-Xarch_host", "-fsanitize=address"]  # host pass only


def hipcc() -> str:
    return "/opt/rocm/bin/hipcc"


def asan_runtime() -> str:
    found = sorted(glob.glob("/opt/rocm/lib/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not found:
        raise SystemExit("clang's ASan runtime (libclang_rt.asan-x86_64.so) not found")
    return found[-1]


def build() -> None:
    os.makedirs(OUT, exist_ok=True)

    def compile_one(src: str) -> str:
        obj = os.path.join(OUT, os.path.basename(src) + ".o")
        proc = subprocess.run([hipcc(), *FLAGS, *SANITIZE, "-c", src, "-o", obj],
                              capture_output=True, text=True)
        if proc.returncode != 0:
            raise SystemExit(f"hipcc failed for {src}:\n{proc.stderr}")
        return obj

    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    with concurrent.futures.ThreadPoolExecutor(min(8, os.cpu_count() or 1)) as pool:
        objects = list(pool.map(compile_one, sources))
    proc = subprocess.run([hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *SANITIZE,
                           "-o", LIB, *objects], capture_output=True, text=True)
    if proc.returncode != 0:
        raise SystemExit(f"link failed:\n{proc.stderr}")


RUNNER = """
import sys
sys.path.insert(0, {root!r})
from local_kimi_amd import _lib
_lib.LIB_PATH = {lib!r}
import pytest
sys.exit(pytest.main(["-q", "-m", "not gpu", "-p", "no:cacheprovider", *{tests!r}]))
"""


def main() -> int:
    build()
    env = dict(os.environ)
    env["LD_PRELOAD"] = asan_runtime()
    env["ASAN_OPTIONS"] = "detect_leaks=0:halt_on_error=1"
    code = RUNNER.format(root=ROOT, lib=LIB, tests=TESTS)
    return subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env).returncode


if __name__ == "__main__":
    sys.exit(main())
