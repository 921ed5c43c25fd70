"""ctypes binding of the C ABI in ``include/cek.h`` (libcek.so).

This is the binding a non-torch host would write; the parity tests use it to
exercise the C ABI directly with device pointers of torch-allocated tensors.
Loading the library does not touch the GPU; calls do.
"""

import ctypes as C
import re
from pathlib import Path

from . import LIBCEK, PKG_DIR

HEADER = PKG_DIR.parent / "include" / "cek.h"

CEK_F16, CEK_BF16, CEK_F32 = 0, 1, 2
CEK_E4M3, CEK_E5M2 = 0, 1
CEK_OK, CEK_ERR_INVALID, CEK_ERR_UNSUPPORTED, CEK_ERR_HIP, CEK_ERR_SCRATCH = 0, 1, 2, 3, 4

_p, _i64, _i, _f = C.c_void_p, C.c_int64, C.c_int, C.c_float

SIGNATURES = {
    "cek_error_string": (C.c_char_p, [_i]),
    "cek_last_hip_error": (C.c_char_p, []),
    "cek_version": (_i, []),
    "cek_gemv_fp8_pern": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _i, _i, _i, _p]),
    "cek_gemv_fp8_pert": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _i, _i, _p]),
    "cek_gemv_fp8_pern_multi": (_i, [_p, _i, _p, _p, _p, _p, _i64, _i64, _i, _i, _i, _p]),
    "cek_gemv_fp8_pert_multi": (_i, [_p, _i, _p, _p, _p, _p, _i64, _i64, _i, _i, _p]),
    "cek_gemm_fp8_pert": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _i, _i, _p]),
    "cek_gemm_fp8_pert_workspace_size": (_i64, [_i64, _i64, _i64]),
    "cek_gemm_fp8_pert_ws": (_i, [_p, _p, _p, _p, _i64, _i64, _i64, _i, _i, _p, _i64, _p]),
    "cek_fused_add_rms_norm": (_i, [_p, _p, _p, _i64, _i64, _f, _i, _p]),
    "cek_fused_add_rms_norm_quant_fp8": (_i, [_p, _p, _p, _i64, _i64, _f, _i, _p, _p, _p]),
    "cek_per_token_quant_fp8": (_i, [_p, _i64, _i64, _i, _p, _p, _p]),
    "cek_gemm_fp8_a8w8": (_i, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i, _p]),
    "cek_gemm_fp8_a8w8_workspace_size": (_i64, [_i64, _i64, _i64]),
    "cek_gemm_fp8_a8w8_ws": (_i, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i, _p, _i64, _p]),
    "cek_gemm_fp8_a8w8_noalloc": (_i, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i, _p]),
    "cek_gelu_and_mul": (_i, [_p, _p, _i64, _i64, _i64, _i64, _i, _p]),
    "cek_gemv_fp8_gelu_and_mul": (_i, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i, _i, _i, _p]),
    "cek_add_rms_norm_gemv_fp8": (_i, [_p, _p, _p, _f, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i, _i, _i, _i,
                                       _p]),
    "cek_qk_norm_rope": (_i, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _f, _f, _i, _i, _p]),
    "cek_gemv_fp8_qk_norm_rope": (_i, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _f, _f, _i, _p, _p, _i64, _i64,
                                       _i64, _i, _i, _i, _p]),
    "cek_gemv_fp8_add_rms_norm_defer_groups": (_i64, [_i64]),
    "cek_defer_norm_shift": (_i, [_f]),
    "cek_gemv_fp8_add_rms_norm_defer": (_i, [_p, _p, _p, _p, _p, _p, _p, _i, _i64, _i64, _i64, _i, _i, _i, _p]),
    "cek_gemv_fp8_pern_rs": (_i, [_p, _p, _p, _p, _p, _i64, _f, _i64, _i64, _i64, _i, _i, _i, _p]),
    "cek_gemv_fp8_gelu_and_mul_rs": (_i, [_p, _p, _p, _p, _p, _i64, _f, _i64, _i64, _i64, _i, _i, _i, _p]),
    "cek_gemv_fp8_qk_norm_rope_rs": (_i, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _f, _f, _i, _p, _p, _p,
                                          _i64, _f, _i64, _i64, _i64, _i, _i, _i, _p]),
    "cek_hbm_read_probe": (_i, [_p, _i64, _p, _p]),
}


def header_functions(path=HEADER):
    """Names of the functions ``include/cek.h`` declares."""
    text = Path(path).read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cek_[a-z0-9_]+)\s*\(", text)))


_lib = None


def load(path=LIBCEK):
    """dlopen libcek.so and attach the signatures (no GPU work)."""
    global _lib
    if _lib is None:
        lib = C.CDLL(str(path))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(rc):
    if rc != CEK_OK:
        lib = load()
        msg = lib.cek_error_string(rc).decode()
        if rc == CEK_ERR_HIP:
            msg += " -- " + lib.cek_last_hip_error().decode()
        raise RuntimeError(f"cek status {rc}: {msg}")


def ptr(t):
    """Device pointer of a torch tensor as a ctypes void*."""
    return C.c_void_p(t.data_ptr())


def stream_ptr(stream=None):
    """hipStream_t of a torch stream (default: the current stream)."""
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)
