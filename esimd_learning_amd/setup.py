"""custom-esimd-kernels-vllm for AMD Instinct MI355X (gfx950).

Drop-in replacement of the Intel-XPU package of the same name (reference
setup.py:64-71): the same Python package ``custom_esimd_kernels_vllm`` with
its two extension modules ``custom_esimd_kernels`` and
``custom_esimd_kernels_gemm``, built here with PyTorch-ROCm's
``torch.utils.cpp_extension`` for gfx950 only.

The HIP kernels live in ``libcek.so`` (C ABI, ``include/cek.h``), compiled
by ``build.py`` with hipcc before the extension modules, which link it with
an ``$ORIGIN`` rpath and ship it as package data.

    python setup.py build_ext --inplace      # in-tree build
    pip install . --no-build-isolation        # installed build
"""

import os
import sys
from pathlib import Path

from setuptools import find_packages, setup

os.environ.setdefault("PYTORCH_ROCM_ARCH", "gfx950")

from torch.utils.cpp_extension import BuildExtension, CUDAExtension  # noqa: E402

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
import build as cek_build  # noqa: E402

INCLUDE = [str(HERE.parent / "include"), str(HERE / "csrc")]
LIBDIR = str(cek_build.PYPKG)
CXX = ["-O3", "-std=c++17", "-D__HIP_PLATFORM_AMD__=1"]
LINK = ["-Wl,-rpath,$ORIGIN", "-Wl,-rpath,$ORIGIN/../torch/lib"]


class BuildWithCabi(BuildExtension):
    """Builds libcek.so (hipcc, gfx950) before the torch extension modules."""

    def run(self):
        cek_build.build_cabi(int(os.environ.get("MAX_JOBS", "8")))
        super().run()


def ext(name, sources):
    return CUDAExtension(
        name=f"custom_esimd_kernels_vllm.{name}",
        sources=[f"csrc/{s}" for s in sources],
        include_dirs=INCLUDE,
        library_dirs=[LIBDIR],
        libraries=["cek"],
        extra_compile_args={"cxx": CXX, "nvcc": []},
        extra_link_args=LINK,
        py_limited_api=False,
    )


setup(
    name="custom-esimd-kernels-vllm",
    version="0.1.0",
    packages=find_packages(where="python"),
    package_dir={"": "python"},
    package_data={"custom_esimd_kernels_vllm": ["libcek.so"]},
    ext_modules=[
        ext("custom_esimd_kernels", ["esimd_kernel.cpp", "torch_extension.cpp"]),
        ext("custom_esimd_kernels_gemm", ["esimd_kernel_gemm.cpp", "torch_extension_gemm.cpp"]),
    ],
    cmdclass={"build_ext": BuildWithCabi.with_options(use_ninja=True)},
)
