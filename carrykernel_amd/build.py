"""Build recipe for the gfx950 HIP library behind the C ABI.

Compiles every ``csrc/*.hip`` into one shared object,
``carrykernel_amd/lib/libcarrykernel_gdn.so``, with hipcc, and the host-only
CPython extension ``csrc/front.cpp`` (the packed decode's argument checks and
launch for its Python front end) with g++ against torch's headers. Both are
built in-tree so that they travel with the source tree to the GPU host.

Run ``python -m carrykernel_amd.build`` (or ``__graft_entry__.build()``).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC_DIR = os.path.join(PKG_DIR, "csrc")
INCLUDE_DIR = os.path.join(REPO_DIR, "include")
LIB_DIR = os.path.join(PKG_DIR, "lib")
LIB_NAME = "libcarrykernel_gdn.so"
LIB_PATH = os.path.join(LIB_DIR, LIB_NAME)
TIMELINE_LIB_PATH = os.path.join(LIB_DIR, "libcarrykernel_gdn_timeline.so")
OBJ_DIR = os.path.join(LIB_DIR, "_obj")
FRONT_SRC = os.path.join(CSRC_DIR, "front.cpp")
FRONT_PATH = os.path.join(LIB_DIR, "_ck_front" + sysconfig.get_config_var("EXT_SUFFIX"))

ARCH = "gfx950"

# -ffp-contract=off: every fma in the kernels is an explicit fmaf(), so the
# fp32 operation sequence is fixed (and replayed by the CPU oracle).
# -packed-fp32-ops: packed fp32 VALU forms are disabled.
HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-mcode-object-version=5",
    "-ffp-contract=off",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # the bandwidth decode kernel's 12 leading scalar arguments (launch
    # geometry) go to SGPRs at dispatch
    "-mllvm", "-amdgpu-kernarg-preload-count=12",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc_path() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def sources() -> list[str]:
    return sorted(os.path.join(CSRC_DIR, f) for f in os.listdir(CSRC_DIR) if f.endswith(".hip"))


def front_command(out_path: str) -> list[str]:
    """g++ line of the front end's CPython extension (host code, no HIP)."""
    import torch
    from torch.utils import cpp_extension
    cxx = os.environ.get("CXX") or shutil.which("g++") or "g++"
    incs = [*cpp_extension.include_paths(), sysconfig.get_paths()["include"], INCLUDE_DIR]
    libdirs = cpp_extension.library_paths()
    return [cxx, "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall",
            f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
            *(f"-I{d}" for d in incs), FRONT_SRC, "-o", out_path,
            *(f"-L{d}" for d in libdirs), "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python",
            *(f"-Wl,-rpath,{d}" for d in libdirs)]


def _run(cmd: list[str]) -> str:
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"{os.path.basename(cmd[0])} failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    return err


def build(verbose: bool = False, extra_flags: list[str] | None = None, jobs: int | None = None,
          timeline: bool = False) -> str:
    """Compile every source (in parallel) and link the library; returns its
    path. Always recompiles. ``timeline=True`` builds the measurement variant
    (``CK_TIMELINE``: per-workgroup timestamps in the decode kernel) as
    ``libcarrykernel_gdn_timeline.so`` beside the product library."""
    obj_dir = OBJ_DIR + ("_timeline" if timeline else "")
    lib_path = TIMELINE_LIB_PATH if timeline else LIB_PATH
    os.makedirs(obj_dir, exist_ok=True)
    hipcc = hipcc_path()
    flags = [*HIPCC_FLAGS, *(["-DCK_TIMELINE=1"] if timeline else []), *(extra_flags or []),
             f"-I{INCLUDE_DIR}", f"-I{CSRC_DIR}"]
    srcs = sources()
    objs = [os.path.join(obj_dir, os.path.basename(f)[:-4] + ".o") for f in srcs]
    cmds = [[hipcc, *flags, "-c", src, "-o", obj] for src, obj in zip(srcs, objs)]
    if not timeline:   # the front end's extension: one build, bound to whichever library is loaded
        cmds.append(front_command(FRONT_PATH + ".tmp"))
    jobs = jobs or max(1, min(16, len(os.sched_getaffinity(0))))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        for cmd, err in zip(cmds, pool.map(_run, cmds)):
            if verbose:
                print(" ".join(cmd), flush=True)
                if err.strip():
                    print(err, file=sys.stderr)
    tmp = lib_path + ".tmp"
    link = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    if verbose:
        print(" ".join(link), flush=True)
    _run(link)
    os.replace(tmp, lib_path)
    if not timeline:
        os.replace(FRONT_PATH + ".tmp", FRONT_PATH)
    return lib_path


if __name__ == "__main__":
    print(build(verbose=True, timeline="--timeline" in sys.argv[1:]))
