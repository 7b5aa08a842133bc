"""Build libqlka.so (the gfx950 HIP kernels + C ABI) and its PyTorch extension in-tree.

Every ``csrc/*.hip`` is compiled with hipcc for gfx950 only, with packed-fp32 code generation disabled, into objects
under ``csrc/_build/`` and linked into ``qlka/libqlka.so``: plain HIP + C, no hipify, no torch headers.
``csrc/torch_ext.cpp`` (host C++ only: the pybind module the drop-in packages call, checks, allocation, autograd) is
compiled with the host compiler against torch's headers into ``qlka/_qlka_torch.so``, linked to libqlka.so (found
next to it through an $ORIGIN run path).

    python quasi-linear-kernel-attention_amd/qlka/build.py [--jobs N]
"""

import argparse
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REPO_ROOT = os.path.dirname(PKG_ROOT)
CSRC = os.path.join(PKG_ROOT, "csrc")
BUILD_DIR = os.path.join(CSRC, "_build")
INCLUDE = os.path.join(REPO_ROOT, "include")
LIB_PATH = os.path.join(PKG_ROOT, "qlka", "libqlka.so")
EXT_NAME = "_qlka_torch"
EXT_PATH = os.path.join(PKG_ROOT, "qlka", EXT_NAME + ".so")
CXX = os.environ.get("CXX", "c++")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    # packed fp32 (v_pk_*_f32) code generation is off for every device function
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _run(cmd):
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in res.stdout.splitlines()
                    if "packed-fp32-ops" not in line and "argument unused" not in line)
    return res.returncode, out


def _torch_ext_flags():
    """Compile and link flags of the torch extension (those torch.utils.cpp_extension uses for a ROCm build)."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension as ce
    inc = [f"-I{INCLUDE}", "-I/opt/rocm/include"]
    for d in ce.include_paths() + [sysconfig.get_paths()["include"]]:
        inc += ["-isystem", d]
    cflags = [f"-DTORCH_EXTENSION_NAME={EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H", "-D__HIP_PLATFORM_AMD__=1",
              "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}", "-fPIC",
              "-std=c++17", "-O2", *inc]
    libdir = ce.library_paths()[0]
    ldflags = ["-shared", f"-L{libdir}", "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch", "-ltorch_python",
               f"-L{os.path.dirname(LIB_PATH)}", "-lqlka", "-Wl,-rpath,$ORIGIN"]
    return cflags, ldflags


def build(jobs=None, verbose=False):
    """Compile every csrc/*.hip for gfx950 and link qlka/libqlka.so, then build qlka/_qlka_torch.so. Raises
    RuntimeError on failure."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = sources()
    objs = [os.path.join(BUILD_DIR, os.path.basename(s)[:-4] + ".o") for s in srcs]
    cmds = [[HIPCC, *COMMON_FLAGS, "-c", s, "-o", o] for s, o in zip(srcs, objs)]
    ext_cflags, ext_ldflags = _torch_ext_flags()
    ext_obj = os.path.join(BUILD_DIR, "torch_ext.o")
    cmds.append([CXX, *ext_cflags, "-c", os.path.join(CSRC, "torch_ext.cpp"), "-o", ext_obj])
    jobs = jobs or min(len(cmds), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        results = list(ex.map(_run, cmds))
    failed = [(c, out) for c, (rc, out) in zip(cmds, results) if rc != 0]
    if verbose:
        for (rc, out) in results:
            if out.strip():
                print(out)
    if failed:
        msg = "\n\n".join(" ".join(c) + "\n" + out for c, out in failed)
        raise RuntimeError(f"compile failed:\n{msg}")
    tmp = LIB_PATH + ".tmp"
    rc, out = _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-soname,libqlka.so", *objs, "-o", tmp])
    if rc != 0:
        raise RuntimeError(f"link failed:\n{out}")
    os.replace(tmp, LIB_PATH)
    tmp = EXT_PATH + ".tmp"
    rc, out = _run([CXX, ext_obj, *ext_ldflags, "-o", tmp])
    if rc != 0:
        raise RuntimeError(f"link of {EXT_NAME} failed:\n{out}")
    os.replace(tmp, EXT_PATH)
    return LIB_PATH


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("-v", "--verbose", action="store_true")
    args = ap.parse_args()
    path = build(jobs=args.jobs, verbose=args.verbose)
    print(path)
    sys.exit(0)
