"""C ABI (include/cek.h, libcek.so): load, exports, host-side argument checks.

CPU tests: the library loads, exports every function the header declares,
the ctypes signatures cover exactly those, and invalid arguments are rejected
on the host before any GPU work.  GPU tests: calls through the C ABI with
device pointers agree with the torch ops and the oracle.
"""

import ctypes as C
from pathlib import Path
import subprocess

import numpy as np
import pytest
import torch

from conftest import assert_close_fp
from esimd_learning_amd import LIBCEK, cabi, synthetic
from oracle import gemv as ogemv
from oracle import norm as onorm


def test_library_exports_header_functions():
    assert LIBCEK.exists(), "libcek.so not built"
    declared = cabi.header_functions()
    assert len(declared) >= 12
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIBCEK)], capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.split()[-2:-1] == ["T"]}
    missing = [f for f in declared if f not in exported]
    assert not missing, missing
    assert sorted(cabi.SIGNATURES) == declared


def test_c_host_program(tmp_path):
    """A C99 program built against include/cek.h and libcek.so (gcc, no GPU
    calls): the header is plain C and the argument checks hold from C."""
    import shutil
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    src = Path(__file__).parent / "c" / "abi_host.c"
    exe = tmp_path / "abi_host"
    libdir = Path(cabi.LIBCEK).parent
    subprocess.run([gcc, "-std=c99", "-Wall", "-Wextra", "-Werror", "-I", str(cabi.HEADER.parent), str(src),
                    "-o", str(exe), "-L", str(libdir), "-lcek", f"-Wl,-rpath,{libdir}"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("ok")


def test_c_host_program_sanitized(tmp_path):
    """The same host program built with AddressSanitizer and
    UndefinedBehaviorSanitizer (host code only; libcek.so itself is the
    normal build, seen through the sanitizer's interceptors): no invalid
    access, undefined behaviour or leak on the argument-check paths."""
    import os
    import shutil
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    src = Path(__file__).parent / "c" / "abi_host.c"
    exe = tmp_path / "abi_host_asan"
    libdir = Path(cabi.LIBCEK).parent
    b = subprocess.run([gcc, "-std=c99", "-Wall", "-Wextra", "-Werror", "-g", "-fno-omit-frame-pointer",
                        "-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-I", str(cabi.HEADER.parent),
                        str(src), "-o", str(exe), "-L", str(libdir), "-lcek", f"-Wl,-rpath,{libdir}"],
                       capture_output=True, text=True)
    if b.returncode != 0 and "asan" in (b.stderr + b.stdout).lower():
        pytest.skip("no sanitizer runtime: " + b.stderr[-200:])
    assert b.returncode == 0, b.stdout + b.stderr
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1", UBSAN_OPTIONS="halt_on_error=1")
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("ok")


def test_library_loads_and_reports():
    lib = cabi.load()
    assert lib.cek_version() == 100
    assert lib.cek_error_string(cabi.CEK_OK) == b"ok"
    assert b"invalid" in lib.cek_error_string(cabi.CEK_ERR_INVALID)
    assert lib.cek_last_hip_error() == b""


def test_defer_norm_groups():
    """Partial sums per row of the deferred-norm producer: N / 12 where the
    16-column runs give fewer than 256 workgroups and N is a multiple of 48
    (the consumers take a multiple of 4, at most 256), else N / 16; 0 for N
    not a multiple of 16.  Host arithmetic only."""
    lib = cabi.load()
    g = lib.cek_gemv_fp8_add_rms_norm_defer_groups
    assert [g(n) for n in (3072, 1536, 4096, 512, 2048, 5120, 48 * 100)] == [256, 128, 256, 32, 128, 320, 300]
    assert [g(n) for n in (0, 100, -16)] == [0, 0, 0]


def test_defer_norm_shift():
    """The deferred-norm producer's shift for a norm weight's max |w|: the
    smallest E with 2^E >= max|w| (so residual * w * 2^-E never exceeds the
    residual), clamped to [-24, 24]; 0 for 0 and NaN.  Host arithmetic only."""
    lib = cabi.load()
    f = lib.cek_defer_norm_shift
    cases = {1.0: 0, 1.36: 1, 2.0: 1, 2.01: 2, 8.0: 3, 8.31: 4, 0.3: -1, 0.5: -1, 0.75: 0, 65504.0: 16,
             0.0: 0, -3.0: 2, 1e-30: -24, 1e30: 24, float("nan"): 0, float("inf"): 24}
    for m, e in cases.items():
        assert f(m) == e, (m, f(m), e)
    for m in (0.37, 1.0001, 3.9, 4.0, 123.4, 6e-5):
        e = f(m)
        assert 2.0 ** e >= m > 2.0 ** (e - 1), (m, e)


def test_host_rejects_invalid_arguments():
    """Argument checks return before any HIP call, so they run without a GPU."""
    lib = cabi.load()
    p = C.c_void_p(16)   # never dereferenced: every call below fails validation first
    E = cabi.CEK_ERR_INVALID
    assert lib.cek_gemv_fp8_pern(p, p, p, p, -1, 8, 64, 0, 0, 2, None) == E          # M < 0
    assert lib.cek_gemv_fp8_pern(p, p, p, p, 17, 8, 64, 0, 0, 9, None) == E          # scale dtype, M > 16
    assert lib.cek_gemv_fp8_pern(p, p, p, p, 1, 8, 64, 0, 0, 7, None) == E           # scale dtype
    assert lib.cek_gemv_fp8_pert(p, p, p, p, 1, 8, 0, 0, 0, None) == E               # K = 0
    assert lib.cek_gemv_fp8_pert(None, p, p, p, 1, 8, 64, 0, 0, None) == E           # null x
    assert lib.cek_gemv_fp8_pert(p, p, p, p, 1, 8, 64, 5, 0, None) == E              # io dtype
    assert lib.cek_gemm_fp8_pert(p, p, p, p, 1, 8, 64, 0, 9, None) == E              # fp8 fmt
    assert lib.cek_gemm_fp8_a8w8(p, p, p, p, p, 4, 4, 40, 0, None) == E              # K % 16
    assert lib.cek_gemm_fp8_a8w8(C.c_void_p(17), p, p, p, p, 4, 4, 64, 0, None) == E  # alignment
    assert lib.cek_fused_add_rms_norm(p, p, p, 4, 0, 1e-6, 0, None) == E             # H = 0
    assert lib.cek_fused_add_rms_norm_quant_fp8(p, p, p, 4, 64, 1e-6, 0, None, p, None) == E
    assert lib.cek_per_token_quant_fp8(p, -1, 64, 0, p, p, None) == E
    assert lib.cek_gelu_and_mul(p, p, 4, 64, 100, 64, 0, None) == E                  # x stride < 2d
    assert lib.cek_qk_norm_rope(p, p, p, p, p, 4, 2, 2, 1024, 2048, 2048, 1e-6, 1e4, 1, 0, None) == E
    assert lib.cek_qk_norm_rope(p, p, p, p, p, 4, 2, 2, 128, 100, 256, 1e-6, 1e4, 1, 0, None) == E
    assert lib.cek_hbm_read_probe(p, 1000, p, None) == E                               # bytes % 16
    assert lib.cek_hbm_read_probe(C.c_void_p(8), 1024, p, None) == E                   # alignment
    assert lib.cek_hbm_read_probe(p, 0, p, None) == E
    # multi-matrix GEMV: count out of range, null tables
    P3 = C.c_void_p * 3
    Ns = (C.c_int64 * 3)(8, 8, 8)
    assert lib.cek_gemv_fp8_pern_multi(p, 0, P3(p, p, p), P3(p, p, p), P3(p, p, p), Ns, 1, 64, 0, 0, 2, None) == E
    assert lib.cek_gemv_fp8_pern_multi(p, 9, P3(p, p, p), P3(p, p, p), P3(p, p, p), Ns, 1, 64, 0, 0, 2, None) == E
    assert lib.cek_gemv_fp8_pert_multi(p, 3, None, P3(p, p, p), P3(p, p, p), Ns, 1, 64, 0, 0, None) == E
    # fused gate/up GEMV + gelu_and_mul: bad enums, a8w8 contract, then shapes
    # the fused kernel leaves to the caller's two-launch path
    glu = lib.cek_gemv_fp8_gelu_and_mul
    U = cabi.CEK_ERR_UNSUPPORTED
    assert glu(p, None, p, p, p, 4, 64, 4096, 5, 0, 2, None) == E                     # io dtype
    assert glu(p, None, p, p, p, 4, 64, 4096, 0, 0, 7, None) == E                     # scale dtype
    assert glu(p, p, p, p, p, 4, 64, 4096, 0, 1, 2, None) == E                        # a8w8 with e5m2
    assert glu(p, p, p, p, p, 4, 64, 4096, 0, 0, 0, None) == E                        # a8w8 with fp16 scales
    assert glu(p, None, p, p, p, -1, 64, 4096, 0, 0, 2, None) == E
    assert glu(None, None, p, p, p, 4, 64, 4096, 0, 0, 2, None) == E                  # null x
    assert glu(p, None, p, p, p, 17, 64, 4096, 0, 0, 2, None) == U                    # M > 16
    assert glu(p, None, p, p, p, 4, 64, 2048, 0, 0, 2, None) == U                     # K outside 3-5 KiB
    assert glu(p, None, p, p, p, 4, 64, 4100, 0, 0, 2, None) == U
    assert glu(C.c_void_p(24), None, p, p, p, 4, 64, 4096, 0, 0, 2, None) == U        # alignment
    assert glu(None, None, None, None, None, 0, 64, 4096, 0, 0, 2, None) == cabi.CEK_OK
    # add+RMSNorm fused into the GEMV: quant form needs e4m3 weights, fp32
    # scales and no hidden_out; unsupported shapes and aliasing side outputs
    # are left to the caller's two launches
    ng = lib.cek_add_rms_norm_gemv_fp8
    q = C.c_void_p(4096)
    assert ng(p, p, p, 1e-6, q, None, p, p, p, p, p, 4, 64, 4096, 0, 0, 1, 2, None) == E   # quant with e5m2
    assert ng(p, p, p, 1e-6, q, None, p, None, p, p, p, 4, 64, 4096, 0, 0, 0, 2, None) == E  # no scale output
    assert ng(p, p, p, 1e-6, q, p, p, p, p, p, p, 4, 64, 4096, 0, 0, 0, 2, None) == E      # quant with hidden_out
    assert ng(p, p, p, 1e-6, q, None, None, None, p, p, p, 4, 65, 4096, 1, 0, 0, 2, None) == E  # odd 2d
    assert ng(p, None, p, 1e-6, q, None, None, None, p, p, p, 4, 64, 4096, 0, 0, 0, 2, None) == E  # null residual
    assert ng(p, p, p, 1e-6, q, None, None, None, p, p, p, 5, 64, 4096, 0, 0, 0, 2, None) == U   # M > 4
    assert ng(p, p, p, 1e-6, q, None, None, None, p, p, p, 4, 64, 2048, 0, 0, 0, 2, None) == U   # K
    assert ng(p, p, p, 1e-6, q, None, None, None, p, p, p, 4, 64, 4096, 0, 0, 1, 2, None) == U   # e5m2
    assert ng(p, p, p, 1e-6, p, None, None, None, p, p, p, 4, 64, 4096, 0, 0, 0, 2, None) == U   # r_out aliases
    # the quantising form fuses one row only (two launches are faster from two
    # rows on); outputs at distinct fake addresses, so only the row count decides
    h_, r_, w_, ro, qo, qs = (C.c_void_p(a) for a in (1 << 20, 2 << 20, 3 << 20, 4 << 20, 5 << 20, 6 << 20))
    assert ng(h_, r_, w_, 1e-6, ro, None, qo, qs, p, p, p, 2, 64, 4096, 0, 0, 0, 2, None) == U
    assert ng(None, None, None, 1e-6, None, None, None, None, None, None, None, 0, 64, 4096, 0, 0, 0, 2,
              None) == cabi.CEK_OK
    # split-K workspace: size query, and a negative or missing workspace
    assert lib.cek_gemm_fp8_a8w8_workspace_size(2048, 6144, 4096) == 0
    ws = lib.cek_gemm_fp8_a8w8_workspace_size(512, 4096, 14336)           # K split in parts
    assert ws > 0 and ws % (512 * 4096 * 4) == 0 and ws // (512 * 4096 * 4) in (2, 4)
    assert lib.cek_gemm_fp8_a8w8_ws(p, p, p, p, p, 512, 4096, 14336, 0, None, 64, None) == E
    assert lib.cek_gemm_fp8_a8w8_ws(p, p, p, p, p, 512, 4096, 14336, 0, p, -1, None) == E
    assert lib.cek_gemm_fp8_a8w8_ws(p, p, p, p, p, 512, 4096, 14336, 0, C.c_void_p(18), 64, None) == E  # misaligned
    # the w8a16 GEMM's split-K workspace: the same contract
    assert lib.cek_gemm_fp8_pert_workspace_size(2048, 6144, 4096) == 0
    ws = lib.cek_gemm_fp8_pert_workspace_size(512, 4096, 14336)
    assert ws > 0 and ws % (512 * 4096 * 4) == 0
    assert lib.cek_gemm_fp8_pert_workspace_size(64, 4096, 14336) == 0  # below the round model: unsplit
    assert lib.cek_gemm_fp8_pert_ws(p, p, p, p, 512, 4096, 14336, 0, 0, None, 64, None) == E
    assert lib.cek_gemm_fp8_pert_ws(p, p, p, p, 512, 4096, 14336, 0, 0, p, -1, None) == E
    assert lib.cek_gemm_fp8_pert_ws(p, p, p, p, 512, 4096, 14336, 0, 0, C.c_void_p(18), 64, None) == E
    # the no-allocation a8w8 entry point refuses plans beyond its 32 MiB
    # static scratch buffer before any HIP call
    assert lib.cek_gemm_fp8_a8w8_workspace_size(768, 6144, 24576) > (32 << 20)
    assert lib.cek_gemm_fp8_a8w8_noalloc(p, p, p, p, p, 768, 6144, 24576, 0, None) == cabi.CEK_ERR_SCRATCH
    assert b"scratch" in lib.cek_error_string(cabi.CEK_ERR_SCRATCH)
    # empty problems are no-ops that succeed without touching memory
    assert lib.cek_gemv_fp8_pern(None, None, None, None, 0, 8, 64, 0, 0, 2, None) == cabi.CEK_OK
    assert lib.cek_fused_add_rms_norm(None, None, None, 0, 64, 1e-6, 0, None) == cabi.CEK_OK


# ------------------------------------------------------------------ GPU
@pytest.mark.gpu
def test_cabi_gemv_matches_torch_op(ops, dev):
    lib = cabi.load()
    M, K, N = 3, 4096, 2048
    W8, s = synthetic.weight_fp8(N, K, seed=21)
    x = synthetic.activations(M, K, seed=22)
    xd, wd, sd = x.to(dev), W8.to(dev), s.to(dev)
    y1 = torch.zeros(M, N, dtype=torch.float16, device=dev)
    y2 = torch.zeros(M, N, dtype=torch.float16, device=dev)
    cabi.check(lib.cek_gemv_fp8_pern(cabi.ptr(xd), cabi.ptr(wd), cabi.ptr(sd), cabi.ptr(y1), M, N, K,
                                     cabi.CEK_F16, cabi.CEK_E4M3, cabi.CEK_F32, cabi.stream_ptr()))
    ops.esimd_gemv_fp8_pern(xd, wd, sd, y2, N, K)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    assert_close_fp(y1.cpu(), ogemv.gemv_fp8_pern(x, W8, s), "cabi gemv")


@pytest.mark.gpu
def test_cabi_norm_quant_on_side_stream(ops, dev):
    lib = cabi.load()
    T, H = 8, 4096
    h = synthetic.activations(T, H, seed=31)
    r = synthetic.activations(T, H, seed=32)
    w = synthetic.norm_weight(H)
    hd, rd, wd = h.to(dev), r.to(dev), w.to(dev)
    q = torch.empty(T, H, dtype=torch.uint8, device=dev)
    s = torch.empty(T, dtype=torch.float32, device=dev)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        cabi.check(lib.cek_fused_add_rms_norm_quant_fp8(cabi.ptr(hd), cabi.ptr(rd), cabi.ptr(wd), T, H, 1e-6,
                                                        cabi.CEK_F16, cabi.ptr(q), cabi.ptr(s),
                                                        cabi.stream_ptr(side)))
    side.synchronize()
    r_ref, _, s_ref, _ = onorm.fused_add_rms_norm_quant(h, r, w, 1e-6)
    assert torch.equal(rd.cpu(), r_ref)
    assert np.allclose(s.cpu().numpy(), s_ref.numpy(), rtol=1e-3)


@pytest.mark.gpu
def test_cabi_error_string_after_invalid(ops, dev):
    lib = cabi.load()
    rc = lib.cek_gemv_fp8_pern(None, None, None, None, 1, 8, 64, 0, 0, 2, None)
    assert rc == cabi.CEK_ERR_INVALID
    with pytest.raises(RuntimeError, match="invalid argument"):
        cabi.check(rc)


@pytest.mark.gpu
def test_cabi_multi_gemv_matches_single(ops, dev):
    """cek_gemv_fp8_pern_multi over three matrices (host pointer tables) gives
    each matrix's cek_gemv_fp8_pern result bit for bit, at M on both sides of
    the v_dot2 / LDS-kernel switch."""
    lib = cabi.load()
    K = 4096
    Ns = [1024, 520, 2048]
    mats = [synthetic.weight_fp8(n, K, seed=40 + i) for i, n in enumerate(Ns)]
    wd = [w.to(dev) for w, _ in mats]
    sd = [s.to(dev) for _, s in mats]
    for M in (1, 5):
        x = synthetic.activations(M, K, seed=41).to(dev)
        ys = [torch.zeros(M, n, dtype=torch.float16, device=dev) for n in Ns]
        P = C.c_void_p * 3
        cabi.check(lib.cek_gemv_fp8_pern_multi(cabi.ptr(x), 3, P(*[t.data_ptr() for t in wd]),
                                               P(*[t.data_ptr() for t in sd]), P(*[t.data_ptr() for t in ys]),
                                               (C.c_int64 * 3)(*Ns), M, K, cabi.CEK_F16, cabi.CEK_E4M3,
                                               cabi.CEK_F32, cabi.stream_ptr()))
        for w, s, y, n in zip(wd, sd, ys, Ns):
            y1 = torch.zeros(M, n, dtype=torch.float16, device=dev)
            cabi.check(lib.cek_gemv_fp8_pern(cabi.ptr(x), cabi.ptr(w), cabi.ptr(s), cabi.ptr(y1), M, n, K,
                                             cabi.CEK_F16, cabi.CEK_E4M3, cabi.CEK_F32, cabi.stream_ptr()))
            torch.cuda.synchronize()
            assert torch.equal(y, y1), f"M={M} N={n}"


@pytest.mark.gpu
@pytest.mark.parametrize("nbytes", [16, 4096, 1 << 20, 58720256 + 48])
def test_cabi_read_probe_reads_every_byte_once(dev, nbytes):
    """The XOR of the probe's 1024 workgroup words equals the XOR of the
    buffer's 32-bit words: every 16-byte unit is read exactly once (a unit
    read twice or skipped changes the XOR for random data)."""
    import numpy as np
    lib = cabi.load()
    g = torch.Generator().manual_seed(nbytes)
    buf = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, generator=g)
    sink = torch.full((1024,), 0x5A5A5A5A, dtype=torch.int32, device=dev)
    bd = buf.to(dev)
    cabi.check(lib.cek_hbm_read_probe(cabi.ptr(bd), nbytes, cabi.ptr(sink), cabi.stream_ptr()))
    torch.cuda.synchronize()
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    want = np.bitwise_xor.reduce(buf.numpy().view(np.uint32))
    assert got == want
    # the timed mode (no sink) runs the same loads and writes nothing
    cabi.check(lib.cek_hbm_read_probe(cabi.ptr(bd), nbytes, None, cabi.stream_ptr()))
    torch.cuda.synchronize()
