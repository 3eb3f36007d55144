"""Host-sanitizer build of libxrmm and the job-JSON runner (CPU checks only).

``python -m xrgpu_amd.build_sanitized`` compiles the host code of the C ABI
(``xrmm_api.cpp``, ``xrmm_operator.cpp``: argument checks, planning, the
request lifecycle) and the runner (``xrmm_execute.cpp``: the hand-written JSON
parser of job files) with AddressSanitizer and UndefinedBehaviorSanitizer, and
links them with the kernel objects of the regular build (device code is not
instrumented: GPU sanitizers are not used here). Outputs go to
``xrgpu_amd/lib/sanitize/``. Run the CPU tests of the runner and of the plan
path against it::

    python -m xrgpu_amd.build_sanitized
    XRMM_LIB_PATH=xrgpu_amd/lib/sanitize/libxrmm.so \\
    XRMM_EXECUTE=xrgpu_amd/lib/sanitize/xrmm_execute \\
    LD_PRELOAD=$(python -m xrgpu_amd.build_sanitized --runtime) \\
    ASAN_OPTIONS=detect_leaks=0 UBSAN_OPTIONS=halt_on_error=1:print_stacktrace=1 \\
    python -m pytest tests/test_runner.py tests/test_operator_plan.py -m "not gpu"

(the Python interpreter is not instrumented, so the sanitizer runtime is
preloaded into it; leak checking is off because the interpreter's own
allocations would be reported).
"""
from __future__ import annotations

import os
import subprocess
import sys

from xrgpu_amd import build as B

SAN_DIR = os.path.join(B.LIB_DIR, "sanitize")
SAN_OBJ = os.path.join(B.OBJ_DIR, "sanitize")
HOST_UNITS = ("xrmm_api.cpp", "xrmm_operator.cpp")
# hipcc: the sanitizers apply to the host compilation only
HOST_SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer",
            "-Xarch_host", "-shared-libsan"]
# the runner is plain host C++, compiled and linked by clang (the same
# sanitizer runtime as the library)
RUNNER_SAN = ["-fsanitize=address", "-fsanitize=undefined", "-fno-sanitize-recover=undefined",
              "-fno-omit-frame-pointer", "-shared-libsan"]


def clangxx() -> str:
    return os.path.join(os.path.dirname(os.path.realpath(B.hipcc())), "..", "llvm", "bin", "clang++")


def runtime() -> str:
    """Path of the shared AddressSanitizer runtime the sanitized build links."""
    r = subprocess.run([clangxx(), "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True,
                       check=True)
    return os.path.realpath(r.stdout.strip())


def build_sanitized(verbose: bool = False) -> str:
    if not os.path.exists(B.LIB):
        B.build(verbose=verbose)
    os.makedirs(SAN_DIR, exist_ok=True)
    os.makedirs(SAN_OBJ, exist_ok=True)
    cc = B.hipcc()
    inc = ["-I", os.path.join(B.ROOT, "include"), "-I", B.CSRC]
    host_objs = []
    for src in HOST_UNITS:
        obj = os.path.join(SAN_OBJ, src.replace(".cpp", ".o"))
        B._run([cc, *B.FLAGS, *HOST_SAN, "-O1", *inc, "-c", os.path.join(B.CSRC, src), "-o", obj], verbose)
        host_objs.append(obj)
    host_names = {src.replace("xrmm_", "").replace(".cpp", ".o") for src in HOST_UNITS}
    kernel_objs = [os.path.join(B.OBJ_DIR, obj) for _, _, obj in B.UNITS if obj not in host_names]
    lib = os.path.join(SAN_DIR, "libxrmm.so")
    B._run([cc, "-shared", "-fPIC", f"--offload-arch={B.ARCH}", *HOST_SAN, *kernel_objs, *host_objs, "-o", lib],
           verbose)
    runner = os.path.join(SAN_DIR, "xrmm_execute")
    rt_dir = os.path.dirname(runtime())  # the runner also starts without a preload
    B._run([clangxx(), "-O1", "-g", "-std=c++17", *RUNNER_SAN, "-I", os.path.join(B.ROOT, "include"),
            os.path.join(B.CSRC, "xrmm_execute.cpp"), "-L", SAN_DIR, "-lxrmm", "-Wl,-rpath,$ORIGIN",
            f"-Wl,-rpath,{rt_dir}", "-o", runner], verbose)
    return lib


if __name__ == "__main__":
    if "--runtime" in sys.argv:
        print(runtime())
    else:
        print(build_sanitized(verbose=True))
