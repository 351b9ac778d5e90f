"""Build recipe for the gfx950 kernels and the genie_tk._C binding.

Produces, inside the package directory (so they travel with the source tree):
  genie_tk/libgenie_tk_hip.so   the C-ABI library (include/genie_tk.h), hipcc
  genie_tk/_C.<abi>.so          the PyTorch binding, g++, linked to the above

Only gfx950 code objects are built.  Usage: ``python genie-tk_amd/build.py``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
CSRC = PKG_ROOT / "csrc"
OUT = PKG_ROOT / "genie_tk"
BUILD = PKG_ROOT / "_build"
REPO = PKG_ROOT.parent
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")
ARCH = "gfx950"

HIP_SOURCES = ["layernorm.hip", "tri_mul.hip", "tri_mul_bwd.hip", "tri_attn.hip", "tri_attn_bwd.hip",
               "pair_transition.hip",
               "capi.cpp"]
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    # never emit packed fp32 VALU ops
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{REPO / 'include'}",
]
LIB_NAME = "libgenie_tk_hip.so"


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


# Per-source extra flags.  tri_attn.hip: the softmax never sees NaN, and
# without NaN semantics chains of fmaxf fuse into v_max3_f32.
EXTRA_FLAGS = {"tri_attn.hip": ["-fno-honor-nans"]}


def _compile_hip(src: str) -> Path:
    obj = BUILD / (Path(src).stem + ".o")
    lang = ["-x", "hip"] if src.endswith(".cpp") else []
    _run([HIPCC, *HIP_FLAGS, *EXTRA_FLAGS.get(src, []), *lang, "-c", str(CSRC / src), "-o", str(obj)])
    return obj


def build_hip_library() -> Path:
    BUILD.mkdir(parents=True, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(HIP_SOURCES))) as ex:
        objs = list(ex.map(_compile_hip, HIP_SOURCES))
    lib = OUT / LIB_NAME
    tmp = lib.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp),
          "-Wl,-soname," + LIB_NAME])
    os.replace(tmp, lib)
    return lib


def build_torch_binding() -> Path:
    import torch  # noqa: F401  (paths only)
    from torch.utils import cpp_extension

    import pybind11

    ext_suffix = sysconfig.get_config_var("EXT_SUFFIX")
    target = OUT / f"_C{ext_suffix}"
    tmp = target.with_suffix(".tmp")
    torch_lib = cpp_extension.library_paths()[0]
    inc = [f"-I{p}" for p in cpp_extension.include_paths()]
    inc += [f"-I{pybind11.get_include()}", f"-I{sysconfig.get_paths()['include']}",
            f"-I{ROCM / 'include'}", f"-I{REPO / 'include'}"]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-w",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-DTORCH_EXTENSION_NAME=_C", "-DTORCH_API_INCLUDE_EXTENSION_H",
        *inc,
        str(CSRC / "torch_ext.cpp"),
        "-o", str(tmp),
        f"-L{OUT}", "-l:" + LIB_NAME,
        f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
        "-ltorch_python",
        "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}",
    ]
    _run(cmd)
    os.replace(tmp, target)
    return target


def build(verbose: bool = True) -> None:
    lib = build_hip_library()
    if verbose:
        print(f"built {lib.relative_to(REPO)}")
    ext = build_torch_binding()
    if verbose:
        print(f"built {ext.relative_to(REPO)}")


if __name__ == "__main__":
    build()
    sys.exit(0)
