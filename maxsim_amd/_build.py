"""In-tree build of the native parts of maxsim_amd.

Produces, next to this file:

* ``libmaxsim_amd.so`` -- the HIP kernels and the C ABI of
  ``include/maxsim_amd.h`` (hipcc, gfx950; no torch dependency);
* ``_maxsim_amd_torch.so`` -- the torch operator registrations
  (``torch_binding.cpp``), linked against ``libmaxsim_amd.so``.

Run ``python maxsim_amd/_build.py`` (or ``__graft_entry__.build()``); not as
``python -m``, which would import the package and its previous build first.  The HIP
objects are compiled in parallel; nothing is cached between runs.
"""

from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
REPO = PKG.parent
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = os.environ.get("MAXSIM_AMD_ARCH", "gfx950")

HIP_SOURCES = ["maxsim_fwd.hip", "maxsim_bwd.hip", "maxsim_pack.hip", "maxsim_ce.hip", "maxsim_capi.hip"]
LIB = PKG / "libmaxsim_amd.so"
TORCH_LIB = PKG / "_maxsim_amd_torch.so"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-munsafe-fp-atomics",
    # Packed fp32 VALU ops are kept out of the generated code on purpose.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def _run(cmds: list[list[str]]) -> None:
    procs = [
        (cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True))
        for cmd in cmds
    ]
    failed = []
    for cmd, p in procs:
        out, _ = p.communicate()
        lines = [
            ln for ln in out.splitlines()
            if "packed-fp32-ops' is not a recognized feature" not in ln
        ]
        if p.returncode != 0:
            failed.append((cmd, "\n".join(lines)))
        elif lines:
            print("\n".join(lines), file=sys.stderr)
    if failed:
        msg = "\n\n".join(f"$ {' '.join(c)}\n{o}" for c, o in failed)
        raise RuntimeError(f"native build failed:\n{msg}")


def build_hip_library() -> Path:
    hipcc = str(ROCM / "bin" / "hipcc")
    objdir = PKG / "_objs"
    objdir.mkdir(exist_ok=True)
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = objdir / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append([hipcc, *HIPCC_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
    _run(cmds)
    tmp = LIB.with_suffix(".so.tmp")
    _run([[hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objs)]])
    os.replace(tmp, LIB)
    return LIB


def build_torch_binding() -> Path:
    import torch

    tdir = Path(torch.__file__).resolve().parent
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = TORCH_LIB.with_suffix(".so.tmp")
    cmd = [
        "g++", "-O2", "-std=c++17", "-shared", "-fPIC",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        "-I", str(tdir / "include"),
        "-I", str(tdir / "include" / "torch" / "csrc" / "api" / "include"),
        "-I", str(ROCM / "include"),
        str(CSRC / "torch_binding.cpp"),
        "-o", str(tmp),
        "-L", str(PKG), "-lmaxsim_amd",
        "-L", str(tdir / "lib"), "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch_hip",
        "-Wl,-rpath,$ORIGIN",
        "-Wl,-rpath," + str(tdir / "lib"),
    ]
    _run([cmd])
    os.replace(tmp, TORCH_LIB)
    return TORCH_LIB


BUILD_INFO = PKG / "_build_info.json"


def write_build_info() -> None:
    """Record the source revision the libraries were built from
    (``_build_info.json``, next to them): the GPU box receives the tree
    without its git metadata, and the benchmark's result records name the
    commit."""
    import json

    info = {"git_commit": "unknown", "git_dirty": False}
    try:
        head = subprocess.run(["git", "-C", str(REPO), "rev-parse", "HEAD"],
                              capture_output=True, text=True, timeout=20)
        if head.returncode == 0:
            info["git_commit"] = head.stdout.strip()
            st = subprocess.run(["git", "-C", str(REPO), "status", "--porcelain", "--",
                                 "maxsim_amd", "include", "oracle", "bench.py"],
                                capture_output=True, text=True, timeout=20)
            info["git_dirty"] = st.returncode == 0 and bool(st.stdout.strip())
    except (OSError, subprocess.SubprocessError):
        pass
    BUILD_INFO.write_text(json.dumps(info) + "\n")


def build() -> None:
    build_hip_library()
    build_torch_binding()
    write_build_info()


if __name__ == "__main__":
    build()
    print(f"built {LIB.name} and {TORCH_LIB.name} in {PKG}")
