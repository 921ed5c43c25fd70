"""GPU parity of cek_gemm_fp8_a8w8_noalloc, the a8w8 entry point that
allocates nothing (its split-K partial sums go to a static per-GPU buffer in
the library instead of a caller workspace).

Against cek_gemm_fp8_a8w8_ws with a workspace of the plan's size (the same
kernels and plan, so bit for bit) and against the CPU oracle to the op
pack's tolerance, on calls in a row that share the static buffer: the
largest split plan the buffer holds (M = 512, K = 14336, N = 4096: 4 parts,
32 MiB), then a smaller one (M = 64, K = 4096, N = 6144: 4 parts, 6 MiB),
then the first again; a shape that runs unsplit uses no scratch; a plan
larger than the buffer is refused with CEK_ERR_SCRATCH before any launch.
"""

import sys

import pytest
import torch

from conftest import assert_close_fp
from esimd_learning_amd import cabi, synthetic
from oracle import gemm as ogemm

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 32 << 20


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _inputs(M, K, N, seed):
    x = synthetic.activations(M, K, seed=seed).float()
    sa = torch.clamp(x.abs().amax(dim=1) / 448.0, min=1.0 / (448.0 * 512.0))
    q = (x / sa[:, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8)
    W8, sb = synthetic.weight_fp8(N, K, seed=seed + 1)
    return q, sa, W8.view(torch.uint8), sb


def _run_pair(lib, dev, M, K, N, seed, expect_split):
    _say(f"a8w8 noalloc M={M} K={K} N={N}")
    need = lib.cek_gemm_fp8_a8w8_workspace_size(M, N, K)
    assert (need > 0) == expect_split and need <= SCRATCH_BYTES, need
    q, sa, W8, sb = _inputs(M, K, N, seed)
    qd, sad, Wd, sbd = q.to(dev), sa.to(dev), W8.to(dev), sb.to(dev)
    st = cabi.stream_ptr(torch.cuda.current_stream())
    y_na = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    rc = lib.cek_gemm_fp8_a8w8_noalloc(qd.data_ptr(), sad.data_ptr(), Wd.data_ptr(), sbd.data_ptr(), y_na.data_ptr(),
                                       M, N, K, 0, st)
    assert rc == 0, lib.cek_error_string(rc)
    y_ws = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    ws = torch.empty(max(need, 4) // 4, dtype=torch.float32, device=dev)
    assert lib.cek_gemm_fp8_a8w8_ws(qd.data_ptr(), sad.data_ptr(), Wd.data_ptr(), sbd.data_ptr(), y_ws.data_ptr(),
                                    M, N, K, 0, ws.data_ptr(), need, st) == 0
    torch.cuda.synchronize()
    assert torch.equal(y_na, y_ws), f"noalloc differs from the workspace call at M={M} K={K} N={N}"
    assert_close_fp(y_na.cpu(), ogemm.gemm_a8w8(q, sa, W8, sb), f"noalloc M={M} K={K} N={N}")


def test_a8w8_noalloc_calls_in_a_row(dev):
    assert torch.cuda.is_available()
    lib = cabi.load()
    _run_pair(lib, dev, 512, 14336, 4096, seed=3, expect_split=True)
    _run_pair(lib, dev, 64, 4096, 6144, seed=4, expect_split=True)
    _run_pair(lib, dev, 512, 14336, 4096, seed=5, expect_split=True)
    _run_pair(lib, dev, 2048, 4096, 6144, seed=6, expect_split=False)


def test_a8w8_noalloc_refuses_plans_beyond_scratch(dev):
    lib = cabi.load()
    M, K, N = 768, 24576, 6144  # 4 parts: 72 MiB of partial sums
    assert lib.cek_gemm_fp8_a8w8_workspace_size(M, N, K) > SCRATCH_BYTES
    # refused on the host before anything is launched; the operands are full
    # size all the same, so no launch could read past them
    a = torch.zeros(M, K, dtype=torch.uint8, device=dev)
    b = torch.zeros(N, K, dtype=torch.uint8, device=dev)
    sa = torch.ones(M, dtype=torch.float32, device=dev)
    sb = torch.ones(N, dtype=torch.float32, device=dev)
    y = torch.full((M, N), 7.0, dtype=torch.float16, device=dev)
    rc = lib.cek_gemm_fp8_a8w8_noalloc(a.data_ptr(), sa.data_ptr(), b.data_ptr(), sb.data_ptr(), y.data_ptr(),
                                       M, N, K, 0, cabi.stream_ptr(torch.cuda.current_stream()))
    torch.cuda.synchronize()
    assert rc == cabi.CEK_ERR_SCRATCH
    assert "scratch" in lib.cek_error_string(rc).decode()
    assert bool((y == 7.0).all()), "a refused call wrote its output"
