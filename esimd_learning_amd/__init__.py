"""esimd_learning_amd -- MI355X (gfx950) build of the custom_esimd_kernels_vllm op pack.

Layout:
  csrc/                      HIP kernels (libcek.so, C ABI in include/cek.h) and
                             the torch op shims / registration
  python/custom_esimd_kernels_vllm/
                             the drop-in Python package (same module names and
                             wrappers as the reference), where the built
                             .so files are placed
  build.py, setup.py         build recipe (hipcc for libcek.so, PyTorch-ROCm
                             cpp_extension for the torch modules)
  cabi.py                    ctypes binding of include/cek.h
  synthetic.py               seeded synthetic inputs (quantisation recipe)

``import esimd_learning_amd`` puts the drop-in package on ``sys.path`` so
that ``import custom_esimd_kernels_vllm`` finds the in-tree build.
"""

import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
PY_DIR = PKG_DIR / "python"
LIB_DIR = PY_DIR / "custom_esimd_kernels_vllm"
LIBCEK = LIB_DIR / "libcek.so"

if str(PY_DIR) not in sys.path:
    sys.path.insert(0, str(PY_DIR))


def built() -> bool:
    """True if libcek.so and both torch extension modules are present."""
    return LIBCEK.exists() and any(LIB_DIR.glob("custom_esimd_kernels.*.so")) and \
        any(LIB_DIR.glob("custom_esimd_kernels_gemm.*.so"))


def ops():
    """Import and return the drop-in package (raises if it is not built)."""
    import custom_esimd_kernels_vllm
    return custom_esimd_kernels_vllm
