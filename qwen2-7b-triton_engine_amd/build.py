"""Build recipe for the W4A16 AWQ HIP library (gfx950).

``python qwen2-7b-triton_engine_amd/build.py`` compiles every ``csrc/*.hip``
with hipcc for gfx950 and links ``lib/libawq_w4a16.so``, then compiles the
torch binding of the eager entry point (``csrc/awq_torch_binding.cpp``, host
C++) into ``lib/_awq_torch*.so``.  Objects go to ``_build/`` next to this
file.  hipcc cross-compiles without a GPU.
"""
from __future__ import annotations

import glob
import os
import re
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ_DIR = os.path.join(HERE, "_build")
LIB_DIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIB_DIR, "libawq_w4a16.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Packed-FP32 instructions are switched off for device code: hipcc forms them
# from ordinary float code on its own, and this build wants none of them.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON_FLAGS = ["--offload-arch=" + ARCH, "-O3", "-std=c++17", "-fPIC", "-Wall",
                "-Wno-unused-command-line-argument", "-munsafe-fp-atomics"]


# Per-kernel resource remarks (registers, LDS, scratch), read below: no kernel
# may spill registers to scratch memory.
RESOURCE_FLAGS = ["-Rpass-analysis=kernel-resource-usage"]


def _spills(remarks: str) -> list:
    """(kernel, bytes per lane) of every kernel whose remarks report scratch."""
    out, name = [], None
    for line in remarks.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and int(m.group(1)) > 0:
            out.append((name, int(m.group(1))))
    return out


def _compile(src: str, verbose: bool) -> str:
    obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, *DEVICE_FLAGS, *RESOURCE_FLAGS, "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the device feature above and says so; drop that line.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    lines = [l for l in r.stderr.splitlines() if noise not in l]
    err = "\n".join(l for l in lines if "remark:" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    spills = _spills("\n".join(lines))
    if spills:
        raise RuntimeError(f"{src}: kernels spill registers to scratch: {spills}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)
    return obj


# The torch binding of the eager entry point (csrc/awq_torch_binding.cpp):
# host C++ against torch's headers and libraries, linked to the library
# above and found next to it at run time.
BINDING_SRC = os.path.join(CSRC, "awq_torch_binding.cpp")


def _binding_path() -> str:
    import sysconfig
    return os.path.join(LIB_DIR, "_awq_torch" + sysconfig.get_config_var("EXT_SUFFIX"))


def build_binding(verbose: bool = False) -> str:
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    out = _binding_path()
    tmp = out + ".tmp"
    torch_lib = cpp_extension.library_paths()[0]
    incs = [*cpp_extension.include_paths(), sysconfig.get_paths()["include"], "/opt/rocm/include"]
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
           "-DTORCH_EXTENSION_NAME=_awq_torch", "-DTORCH_API_INCLUDE_EXTENSION_H", "-D__HIP_PLATFORM_AMD__=1",
           "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
           *[f"-isystem{d}" for d in incs], BINDING_SRC, "-o", tmp,
           f"-L{LIB_DIR}", "-lawq_w4a16", f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu",
           "-ltorch_python", "-lamdhip64", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"building the torch binding failed:\n{r.stderr}")
    os.replace(tmp, out)
    return out


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ_DIR, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    build_binding(verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
