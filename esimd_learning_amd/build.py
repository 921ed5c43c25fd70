"""Build recipe for the gfx950 op pack.

Two products, both in-tree under ``python/custom_esimd_kernels_vllm/``:

* ``libcek.so`` -- the C-ABI library (``include/cek.h``): every HIP kernel
  and its ``extern "C"`` launcher, compiled by ``hipcc --offload-arch=gfx950``.
* ``custom_esimd_kernels*.so`` / ``custom_esimd_kernels_gemm*.so`` -- the
  torch extension modules (PyTorch-ROCm ``cpp_extension``) that register the
  ``torch.ops.custom_esimd_kernels_vllm`` schemas and call into ``libcek.so``
  (linked with an ``$ORIGIN`` rpath).

Usage:  python -m esimd_learning_amd.build [--cabi-only] [-j N]
"""

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
PYPKG = PKG / "python" / "custom_esimd_kernels_vllm"
OBJDIR = PKG / "_build" / "cabi"
LIBCEK = PYPKG / "libcek.so"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: keep the compiler from emitting packed fp32 VALU ops.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    f"-I{INCLUDE}", f"-I{CSRC}",
]

CABI_SOURCES = ["cek_api.cpp", "cek_gemv.hip", "cek_norm.hip", "cek_act.hip", "cek_gemm.hip", "cek_probe.hip"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + r.stdout + r.stderr)
        raise RuntimeError(f"build step failed: {cmd[-1]}")
    return r


def build_cabi(jobs=8):
    """Compile every C-ABI source for gfx950 and link libcek.so."""
    OBJDIR.mkdir(parents=True, exist_ok=True)

    def compile_one(src):
        obj = OBJDIR / (src + ".o")
        lang = ["-x", "hip"] if src.endswith(".hip") else []
        _run([HIPCC, *HIP_FLAGS, *lang, "-c", str(CSRC / src), "-o", str(obj)])
        return obj

    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(compile_one, CABI_SOURCES))
    tmp = LIBCEK.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs),
          "-Wl,-soname,libcek.so", "-Wl,--no-undefined"])
    os.replace(tmp, LIBCEK)
    return LIBCEK


def build_torch_ext():
    """Build the torch extension modules in place (setup.py build_ext)."""
    env = dict(os.environ)
    env.setdefault("PYTORCH_ROCM_ARCH", ARCH)
    env.setdefault("MAX_JOBS", "8")
    r = subprocess.run([sys.executable, "setup.py", "build_ext", "--inplace"], cwd=str(PKG),
                       env=env, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout[-20000:] + r.stderr[-20000:])
        raise RuntimeError("torch extension build failed")


def build_all(jobs=8):
    build_cabi(jobs)
    build_torch_ext()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--cabi-only", action="store_true")
    ap.add_argument("-j", type=int, default=8)
    a = ap.parse_args()
    build_cabi(a.j)
    if not a.cabi_only:
        build_torch_ext()
    print("built", LIBCEK)


if __name__ == "__main__":
    main()
