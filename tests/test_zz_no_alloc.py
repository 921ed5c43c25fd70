"""GPU parity of cek_gemm_fp8_a8w8_noalloc, the a8w8 entry point that
allocates nothing (its split-K partial sums go to a static per-GPU buffer in
the library instead of a caller workspace).

Against cek_gemm_fp8_a8w8_ws with a workspace of the plan's size (the same
kernels and plan, so bit for bit) and against the CPU oracle to the op
pack's tolerance, on calls in a row that share the static buffer: the
largest split plan the buffer holds (M = 512, K = 14336, N = 4096: 4 parts,
32 MiB), then a smaller one (M = 64, K = 4096, N = 6144: 4 parts, 6 MiB),
then the first again; a shape that runs unsplit uses no scratch; a plan
larger than the buffer is refused with CEK_ERR_SCRATCH before any launch;
an eager call allocates nothing, and the call captured in a HIP graph
replays to the eager result.
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


def test_a8w8_noalloc_allocates_nothing_and_captures(dev):
    """What the entry point exists for: an eager split-K call (M = 512,
    K = 14336, N = 4096: 4 parts in the static buffer) leaves torch's
    allocator and the device's free memory unchanged; the same call captured
    in a torch.cuda graph (the first call on the device, which looks the
    buffer up, made before the capture) and replayed three times with new
    activations and unrelated eager work between the replays gives, each
    time, the eager workspace call's result bit for bit."""
    lib = cabi.load()
    M, K, N = 512, 14336, 4096
    _say(f"a8w8 noalloc graph M={M} K={K} N={N}")
    need = lib.cek_gemm_fp8_a8w8_workspace_size(M, N, K)
    assert 0 < need <= SCRATCH_BYTES
    q, sa, W8, sb = _inputs(M, K, N, seed=9)
    qd, sad, Wd, sbd = q.to(dev), sa.to(dev), W8.to(dev), sb.to(dev)
    y = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    ref = torch.empty_like(y)
    ws = torch.empty(need // 4, dtype=torch.float32, device=dev)
    cur = cabi.stream_ptr(torch.cuda.current_stream())
    call = lambda s: lib.cek_gemm_fp8_a8w8_noalloc(qd.data_ptr(), sad.data_ptr(), Wd.data_ptr(),  # noqa: E731
                                                   sbd.data_ptr(), y.data_ptr(), M, N, K, 0, s)
    assert call(cur) == 0        # set-up call (and the buffer's address lookup on this device)
    torch.cuda.synchronize()
    alloc0, free0 = torch.cuda.memory_allocated(), torch.cuda.mem_get_info()[0]
    assert call(cur) == 0
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == alloc0
    assert torch.cuda.mem_get_info()[0] == free0
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        assert call(cabi.stream_ptr(side)) == 0
    torch.cuda.current_stream().wait_stream(side)
    gen = torch.Generator().manual_seed(12)
    for rep in range(3):
        qd.copy_(torch.randint(0, 0x7E, (M, K), generator=gen, dtype=torch.uint8))   # finite e4m3 codes
        assert lib.cek_gemm_fp8_a8w8_ws(qd.data_ptr(), sad.data_ptr(), Wd.data_ptr(), sbd.data_ptr(),
                                        ref.data_ptr(), M, N, K, 0, ws.data_ptr(), need, cur) == 0
        torch.cuda.synchronize()
        y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, ref), f"replay {rep}"
        torch.randn(4096, device=dev).sum().item()   # unrelated eager work between replays


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
