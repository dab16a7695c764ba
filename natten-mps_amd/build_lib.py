"""Build libnatten_hip.so (gfx950) in-tree with hipcc.

    python natten-mps_amd/build_lib.py            # build
    python natten-mps_amd/build_lib.py --check    # print the commands only

Objects go to natten-mps_amd/_build/, the library to
natten-mps_amd/natten_mps_amd/libnatten_hip.so (git-ignored; it travels to
the GPU box with the working tree).

It also builds natten-mps_amd/natten_mps_amd/_natten_torch.so, the C++ host
binding of the fused forward / backward (csrc/na_torch.cpp, g++ against the
installed torch headers), linked to libnatten_hip.so beside it.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "natten_mps_amd", "libnatten_hip.so")
BIND_NAME = "_natten_torch"
BIND = os.path.join(HERE, "natten_mps_amd", BIND_NAME + ".so")
CXX = os.environ.get("CXX", "g++")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["na_generic.hip", "na_mfma.hip", "na_lean.hip", "na_global.hip", "na_rpb.hip", "na_profile.hip", "na_capi.hip"]

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # keep hipcc from forming packed-fp32 (v_pk_*_f32) instructions
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in ordinary VGPRs (no AGPR copies around the softmax)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wno-unused-command-line-argument",
    "-I" + os.path.join(ROOT, "include"),
    "-I" + CSRC,
]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return r


def commands():
    objs, cmds = [], []
    for src in SOURCES:
        path = os.path.join(CSRC, src)
        if not os.path.exists(path):
            continue
        obj = os.path.join(OBJ, src.replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([HIPCC, *FLAGS, "-c", path, "-o", obj])
    link = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-Wl,-soname,libnatten_hip.so", *objs, "-o", LIB]
    return cmds, link


def binding_commands():
    """Compile and link commands of the torch host binding (g++, host code
    only: the HIP runtime headers, no device code)."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension as E

    src = os.path.join(CSRC, "na_torch.cpp")
    obj = os.path.join(OBJ, "na_torch.o")
    abi = int(getattr(torch._C, "_GLIBCXX_USE_CXX11_ABI", True))
    inc = [f"-I{os.path.join(ROOT, 'include')}"] + [f"-isystem{p}" for p in E.include_paths()]
    inc.append(f"-isystem{sysconfig.get_paths()['include']}")
    # torch's HIP headers (the caching allocator's empty tensor, the current
    # stream) include the HIP runtime's
    inc += ["-D__HIP_PLATFORM_AMD__", "-isystem/opt/rocm/include"]
    comp = [CXX, "-O2", "-std=c++17", "-fPIC", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
            f"-DTORCH_EXTENSION_NAME={BIND_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H", *inc, "-c", src, "-o", obj]
    tlib = E.library_paths()[0]
    link = [CXX, "-shared", obj, "-o", BIND, f"-L{os.path.dirname(LIB)}", "-lnatten_hip", "-Wl,-rpath,$ORIGIN",
            f"-L{tlib}", "-lc10", "-ltorch_cpu", "-ltorch", "-ltorch_python", "-ltorch_hip", "-lc10_hip"]
    return comp, link


LLVM = "/opt/rocm/llvm/bin"


def outlined_device_functions(obj: str) -> list:
    """Device functions of a built object that are not kernels.

    The kernels' non-finite recomputation paths read the kernel-argument
    segment pointer (kernargs() in na_tile.h), which is only meaningful in
    the kernel's own code: a copy of such a path compiled out of line would
    read another address.  So every device function must be inlined into a
    kernel: each FUNC symbol of the gfx950 code object needs a kernel
    descriptor (<name>.kd).  Returns the names that have none."""
    import tempfile

    if ".hip_fatbin" not in _run([os.path.join(LLVM, "llvm-readelf"), "-S", "-W", obj]).stdout:
        return []  # host code only
    with tempfile.TemporaryDirectory() as tmp:
        fat, co = os.path.join(tmp, "fat.bin"), os.path.join(tmp, "dev.co")
        _run([os.path.join(LLVM, "llvm-objcopy"), f"--dump-section=.hip_fatbin={fat}", obj,
              os.path.join(tmp, "rest.o")])
        _run([os.path.join(LLVM, "clang-offload-bundler"), "--type=o", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950",
              f"--input={fat}", f"--output={co}", "--unbundle"])
        syms = _run([os.path.join(LLVM, "llvm-readelf"), "-s", "-W", co]).stdout.split("\n")
    funcs, kds = set(), set()
    for line in syms:
        parts = line.split()
        if len(parts) >= 8 and parts[3] == "FUNC":
            funcs.add(parts[7])
        elif len(parts) >= 8 and parts[7].endswith(".kd"):
            kds.add(parts[7][:-3])
    return sorted(funcs - kds)


def check_inlined(verbose: bool = False) -> None:
    cmds, _ = commands()
    for cmd in cmds:
        obj = cmd[-1]
        bad = outlined_device_functions(obj)
        if bad:
            raise RuntimeError(f"{obj}: device functions compiled out of line (must be inlined into kernels): "
                               f"{bad[:5]}")
    if verbose:
        print(f"checked {len(cmds)} objects: every device function is inlined into a kernel")


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    cmds, link = commands()
    bcomp, blink = binding_commands()
    cmds = cmds + [bcomp]
    with cf.ThreadPoolExecutor(max_workers=min(len(cmds), 8)) as ex:
        for cmd, _ in zip(cmds, ex.map(_run, cmds)):
            if verbose:
                print(" ".join(cmd))
    tmp = LIB + ".tmp"
    link = link[:-1] + [tmp]
    _run(link)
    os.replace(tmp, LIB)
    if verbose:
        print(" ".join(link[:-1] + [LIB]))
    check_inlined(verbose)
    btmp = BIND + ".tmp"
    _run([btmp if x == BIND else x for x in blink])
    os.replace(btmp, BIND)
    if verbose:
        print(" ".join(blink))
    return LIB


if __name__ == "__main__":
    if "--check" in sys.argv:
        c, l = commands()
        for x in c + [l, *binding_commands()]:
            print(" ".join(x))
    else:
        print(build(verbose=True))
