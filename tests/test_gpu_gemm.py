"""GPU parity of the fp8 GEMMs.

esimd_gemm_fp8_pert: the reference's GEMM test grid (reference
tests/test_gemm_fp8.py:13-23: M in {1..64} x 6 (N, K), e4m3/e5m2,
fp16/bf16 IO, scale 0.05..0.15) plus prefill M.
esimd_gemm_fp8_a8w8: every BASELINE config-4 shape (M in {512, 2048, 4096}
x (K, N) in {(4096, 6144), (4096, 28672), (14336, 4096)}) against the CPU
oracle (an fp32 CPU matmul of the dequantised codes: about a second per
shape on the host's cores); tile and split-K edge cases against the same
CPU oracle.
"""

import sys

import numpy as np
import pytest
import torch

from conftest import assert_close_fp
from esimd_learning_amd import synthetic
from oracle import gemm as ogemm
from oracle import gemv as ogemv
from oracle import norm as onorm

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


REF_SHAPES = [(2560, 2048), (512, 2048), (2048, 512), (128, 2048), (3072, 2048), (1024, 1024)]


@pytest.mark.parametrize("fmt", [torch.float8_e4m3fn, torch.float8_e5m2])
@pytest.mark.parametrize("io", [torch.float16, torch.bfloat16])
def test_gemm_pert_reference_grid(ops, dev, fmt, io):
    g = torch.Generator().manual_seed(0)
    for N, K in REF_SHAPES:
        for M in (1, 2, 4, 8, 16, 32, 64):
            _say(f"gemm pert M={M} N={N} K={K} {fmt} {io}")
            W8 = (torch.randn(N, K, generator=g).half() * 0.1).to(fmt)
            sv = torch.tensor(0.05 + torch.rand(1, generator=g).item() * 0.1)
            x = (torch.randn(M, K, generator=g) * 0.1).to(io)
            y = torch.zeros(M, N, dtype=io, device=dev)
            ops.esimd_gemm_fp8_pert(x.to(dev), W8.to(dev), sv.to(dev), y)
            torch.cuda.synchronize()
            assert_close_fp(y.cpu(), ogemv.gemm_fp8_pert(x, W8, sv), f"M={M} N={N} K={K}")


@pytest.mark.parametrize("M,K,N", [(128, 4096, 6144), (512, 4096, 4096), (100, 1000, 300), (33, 64, 17)])
def test_gemm_pert_prefill(ops, dev, M, K, N):
    _say(f"gemm pert prefill M={M} K={K} N={N}")
    W8, _ = synthetic.weight_fp8(N, K, seed=M)
    x = synthetic.activations(M, K, seed=M + 1)
    sv = torch.tensor(0.01)
    y = torch.zeros(M, N, dtype=torch.float16, device=dev)
    ops.esimd_gemm_fp8_pert(x.to(dev), W8.to(dev), sv.to(dev), y)
    torch.cuda.synchronize()
    assert_close_fp(y.cpu(), ogemv.gemm_fp8_pert(x, W8, sv), f"prefill M={M}")


@pytest.mark.parametrize("M,K,N,parts,io,fmt", [
    (276, 2048, 130, 2, torch.float16, torch.float8_e4m3fn),     # 256 x 128, 2 parts
    (1736, 16384, 847, 4, torch.bfloat16, torch.float8_e4m3fn),  # 256 x 128, 4 parts
    (2977, 2048, 1325, 0, torch.float16, torch.float8_e5m2),     # 256 x 128
    (1444, 2048, 5388, 0, torch.float16, torch.float8_e4m3fn),   # 256 x 192
    (1298, 2048, 8256, 0, torch.bfloat16, torch.float8_e5m2),    # 256 x 256
    (787, 128, 8256, 0, torch.float16, torch.float8_e4m3fn),     # 256 x 256, one K step
    (641, 2048, 5388, 0, torch.float16, torch.float8_e4m3fn),    # 128 x 256
    (130, 128, 369, 0, torch.bfloat16, torch.float8_e4m3fn),     # 128 x 256, one K step
    (130, 2048, 369, 2, torch.float16, torch.float8_e4m3fn),     # 128 x 256, 2 parts
    (130, 8192, 6344, 4, torch.float16, torch.float8_e5m2),      # 128 x 256, 4 parts
    (1000, 8192, 1000, 4, torch.float16, torch.float8_e4m3fn),   # 128 x 128, 4 parts
    (130, 130, 4096, 0, torch.float16, torch.float8_e4m3fn),     # K = 130: not a multiple of 64
    (130, 4096, 130, 4, torch.float16, torch.float8_e4m3fn),     # 128 x 128, 4 parts
    (130, 8192, 130, 8, torch.bfloat16, torch.float8_e4m3fn),    # 128 x 128, 8 parts
    (500, 2048, 6000, 0, torch.float16, torch.float8_e4m3fn),    # 128 x 96 (4 x 2 waves, padded epilogue rows)
    (450, 4096, 5000, 0, torch.bfloat16, torch.float8_e5m2),     # 128 x 96
])
def test_gemm_pert_round_model(ops, dev, M, K, N, parts, io, fmt):
    """Ragged shapes (M and N not multiples of the tile) on which the w8a16
    round-model plan (M, N >= 128) picks each register-pipelined tile,
    unsplit or split in `parts` (0: unsplit; the op allocates the
    workspace); the bare C-ABI call (no workspace) runs the unsplit plan.
    Both against the CPU oracle; two calls of the op agree bit for bit."""
    from esimd_learning_amd import cabi
    _say(f"gemm pert round model M={M} K={K} N={N} parts={parts} {io} {fmt}")
    lib = cabi.load()
    assert lib.cek_gemm_fp8_pert_workspace_size(M, N, K) == (parts * M * N * 4 if parts else 0)
    g = torch.Generator().manual_seed(M + K + N)
    W8 = (torch.randn(N, K, generator=g) * 0.05).to(fmt)
    x = (torch.randn(M, K, generator=g) * 0.5).to(io)
    sv = torch.tensor(0.02)
    xd, Wd, svd = x.to(dev), W8.to(dev), sv.to(dev)
    y1 = torch.full((M, N), float("nan"), dtype=io, device=dev)
    y2 = torch.full((M, N), float("nan"), dtype=io, device=dev)
    ops.esimd_gemm_fp8_pert(xd, Wd, svd, y1)
    ops.esimd_gemm_fp8_pert(xd, Wd, svd, y2)
    y3 = torch.full((M, N), float("nan"), dtype=io, device=dev)
    io_code = cabi.CEK_F16 if io == torch.float16 else cabi.CEK_BF16
    fmt_code = cabi.CEK_E4M3 if fmt == torch.float8_e4m3fn else cabi.CEK_E5M2
    assert lib.cek_gemm_fp8_pert(xd.data_ptr(), Wd.data_ptr(), svd.data_ptr(), y3.data_ptr(), M, N, K, io_code,
                                 fmt_code, cabi.stream_ptr(torch.cuda.current_stream())) == 0
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    ref = ogemv.gemm_fp8_pert(x, W8, sv)
    assert_close_fp(y1.cpu(), ref, f"w8a16 op M={M} K={K} N={N}")
    assert_close_fp(y3.cpu(), ref, f"w8a16 unsplit M={M} K={K} N={N}")


def _a8w8_inputs(M, K, N, seed):
    x = synthetic.activations(M, K, seed=seed)
    q, sa = onorm.per_token_quant(x)
    W8, sb = synthetic.weight_fp8(N, K, seed=seed + 1)
    return q, sa, W8.view(torch.uint8), sb


def _a8w8_inputs_config4(M, K, N, seed):
    """Config-4 operands at full size: A per-token e4m3 from fp16 N(0, 1), B
    per-channel e4m3 from N(0, 0.02) (the synthetic recipe).  A's codes come
    from torch's CPU e4m3 conversion of x / s (RNE, the oracle's formula; the
    numpy oracle codec is pinned to it and takes tens of seconds at this size)."""
    x = synthetic.activations(M, K, seed=seed).float()
    sa = torch.clamp(x.abs().amax(dim=1) / 448.0, min=1.0 / (448.0 * 512.0))
    q = (x / sa[:, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8)
    W8, sb = synthetic.weight_fp8(N, K, seed=seed + 1)
    return q, sa, W8.view(torch.uint8), sb


@pytest.mark.parametrize("M", [512, 2048, 4096])
@pytest.mark.parametrize("K,N", [(4096, 6144), (4096, 28672), (14336, 4096)])
def test_a8w8_config4(ops, dev, M, K, N):
    """BASELINE config 4, every (M, K, N), against the CPU oracle."""
    _say(f"a8w8 config 4 M={M} K={K} N={N}")
    q, sa, W8, sb = _a8w8_inputs_config4(M, K, N, seed=M + K + N)
    y = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    ops.esimd_gemm_fp8_a8w8(q.to(dev), sa.to(dev), W8.to(dev), sb.to(dev), y)
    torch.cuda.synchronize()
    out = y.cpu()
    del y
    assert_close_fp(out, ogemm.gemm_a8w8(q, sa, W8, sb), f"a8w8 M={M} K={K} N={N}")


@pytest.mark.parametrize("M,K,N", [(1, 128, 16), (17, 48, 33), (64, 256, 64), (130, 1040, 250)])
def test_a8w8_ragged(ops, dev, M, K, N):
    _say(f"a8w8 ragged M={M} K={K} N={N}")
    q, sa, W8, sb = _a8w8_inputs(M, K, N, seed=M * 31 + K)
    for out_dt in (torch.float16, torch.bfloat16):
        y = torch.zeros(M, N, dtype=out_dt, device=dev)
        ops.esimd_gemm_fp8_a8w8(q.to(dev), sa.to(dev), W8.to(dev), sb.to(dev), y)
        torch.cuda.synchronize()
        assert_close_fp(y.cpu(), ogemm.gemm_a8w8(q, sa, W8, sb), f"ragged {out_dt}")


def test_a8w8_rejects_bad_k(ops, dev):
    a = torch.zeros(4, 40, dtype=torch.uint8, device=dev)
    with pytest.raises(RuntimeError, match="multiple of 16"):
        ops.esimd_gemm_fp8_a8w8(a, torch.ones(4, device=dev), a, torch.ones(4, device=dev),
                                torch.zeros(4, 4, dtype=torch.float16, device=dev))


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 13, 16])
@pytest.mark.parametrize("K,N", [(1024, 600), (4096, 1040)])
def test_a8w8_decode_rows(ops, dev, M, K, N):
    """M <= 16 takes the weight-streaming GEMV kernels with fp8 activations."""
    _say(f"a8w8 decode M={M} K={K} N={N}")
    q, sa, W8, sb = _a8w8_inputs(M, K, N, seed=M * 7 + K + N)
    ref = ogemm.gemm_a8w8(q, sa, W8, sb)
    for out_dt in (torch.float16, torch.bfloat16):
        y = torch.zeros(M, N, dtype=out_dt, device=dev)
        ops.esimd_gemm_fp8_a8w8(q.to(dev), sa.to(dev), W8.to(dev), sb.to(dev), y)
        torch.cuda.synchronize()
        assert_close_fp(y.cpu(), ref, f"a8w8 decode M={M} {out_dt}")


@pytest.mark.parametrize("M,K,N", [(4096, 1024, 8192), (4000, 512, 8150), (2000, 1024, 6100), (2048, 512, 6144),
                                   (2048, 640, 6144), (2048, 128, 6144), (2048, 256, 6144), (2040, 384, 6100),
                                   (2000, 768, 6100), (2048, 896, 6144), (520, 1024, 28800),
                                   (4100, 512, 6150), (100, 256, 3000), (200, 512, 100), (70, 384, 130)])
def test_a8w8_large_tiles(ops, dev, M, K, N):
    """The tile configurations (256 x 256, 256 x 192, 128 x 128, 64 x 128),
    including ragged M and N, against the CPU oracle.  The register-pipelined kernel moves a last tile that
    would cross M or N back onto the previous one and stores only its own
    rows and columns (ragged shapes here); N < 128 (200 x 100) takes the
    clamping LDS kernel.  K = 640 and 128 give an odd number of K steps and a
    single one; K = 128, 256 and 384 (one to three steps) also cover the
    8-wave tiles' load chunks at the ends of the K loop (the prologue loads
    steps 0 and 1 whole, later steps go out in chunks).  256 x 192 (M near
    2048, N near 6144) runs the 3-slot B ring: K = 128 .. 896 (1 to 7 steps)
    cover its prologue (A 0-1, B 0-2), the slot cycle of period 3 against the
    A ring's 2, and its tail waits."""
    _say(f"a8w8 large tiles M={M} K={K} N={N}")
    q, sa, W8, sb = _a8w8_inputs(M, K, N, seed=M + N)
    qd, Wd = q.to(dev), W8.to(dev)
    ref = ogemm.gemm_a8w8(q, sa, W8, sb)
    for out_dt in (torch.float16, torch.bfloat16):
        y = torch.zeros(M, N, dtype=out_dt, device=dev)
        ops.esimd_gemm_fp8_a8w8(qd, sa.to(dev), Wd, sb.to(dev), y)
        torch.cuda.synchronize()
        assert_close_fp(y.cpu(), ref, f"a8w8 M={M} K={K} N={N} {out_dt}")


@pytest.mark.parametrize("M,K,N", [(65, 4096, 200), (100, 2048, 512), (300, 8192, 4096), (300, 14336, 4096),
                                   (512, 14336, 4096), (200, 8192, 2048), (150, 4096, 1000), (65, 4096, 203),
                                   (100, 2048, 1001),
                                   (64, 4096, 6144), (64, 14336, 4096), (64, 4096, 300), (64, 4096, 28672)])
def test_a8w8_split_k(ops, dev, M, K, N):
    """Shapes with too few output tiles split K (the op allocates the
    workspace the plan asks for): 64 x 128 tiles in 8, 4 and 2 parts (M = 64
    included, which without a workspace takes the weight-streaming kernels;
    at N = 6144 on 64 x 96 tiles, 256 parts), 128 x 256 in 4 parts, 128 x 128
    (four waves) in 8 and 4 parts.  Against the CPU oracle;
    the unsplit C-ABI call (no workspace) agrees within the same tolerance;
    two split calls agree bit for bit (the parts are added in order), and a
    workspace 4 bytes off 16-byte alignment (the finalize's element-by-element
    form, also taken for N % 4 != 0) gives the same outputs."""
    from esimd_learning_amd import cabi
    _say(f"a8w8 split K M={M} K={K} N={N}")
    lib = cabi.load()
    need = lib.cek_gemm_fp8_a8w8_workspace_size(M, N, K)
    assert need > 0 and need % (M * N * 4) == 0, need
    q, sa, W8, sb = _a8w8_inputs(M, K, N, seed=M + K)
    qd, Wd, sad, sbd = q.to(dev), W8.to(dev), sa.to(dev), sb.to(dev)
    ref = ogemm.gemm_a8w8(q, sa, W8, sb)
    y1 = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    y2 = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    ops.esimd_gemm_fp8_a8w8(qd, sad, Wd, sbd, y1)
    ops.esimd_gemm_fp8_a8w8(qd, sad, Wd, sbd, y2)
    y3 = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    st = cabi.stream_ptr(torch.cuda.current_stream())
    assert lib.cek_gemm_fp8_a8w8(qd.data_ptr(), sad.data_ptr(), Wd.data_ptr(), sbd.data_ptr(), y3.data_ptr(),
                                 M, N, K, 0, st) == 0
    yb = torch.zeros(M, N, dtype=torch.bfloat16, device=dev)
    ws = torch.empty(need // 4, dtype=torch.float32, device=dev)
    assert lib.cek_gemm_fp8_a8w8_ws(qd.data_ptr(), sad.data_ptr(), Wd.data_ptr(), sbd.data_ptr(), yb.data_ptr(),
                                    M, N, K, 1, ws.data_ptr(), need, st) == 0
    y4 = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    ws4 = torch.empty(need // 4 + 1, dtype=torch.float32, device=dev)
    assert lib.cek_gemm_fp8_a8w8_ws(qd.data_ptr(), sad.data_ptr(), Wd.data_ptr(), sbd.data_ptr(), y4.data_ptr(),
                                    M, N, K, 0, ws4.data_ptr() + 4, need, st) == 0
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    assert torch.equal(y1, y4)
    assert_close_fp(y1.cpu(), ref, f"a8w8 split M={M} K={K} N={N}")
    assert_close_fp(y3.cpu(), ref, f"a8w8 unsplit M={M} K={K} N={N}")
    assert_close_fp(yb.cpu(), ref, f"a8w8 split bf16 M={M} K={K} N={N}")


@pytest.mark.parametrize("M,K,N,parts", [(225, 4096, 339, 4), (516, 2048, 7302, 0), (710, 2048, 5403, 0),
                                         (537, 16384, 5000, 2), (516, 8192, 1605, 4), (225, 16384, 339, 8),
                                         (2720, 16384, 1100, 2), (1583, 8192, 550, 4), (419, 16384, 339, 8),
                                         (500, 2048, 6000, 0), (300, 4096, 3000, 0)])
def test_a8w8_round_model_tiles(ops, dev, M, K, N, parts):
    """Shapes (ragged in M and N) on which the round-model plan for M >= 128
    picks each 8-wave, 3-slot tile (128 x 128, 128 x 256, 256 x 128, and
    128 x 96 with its padded epilogue rows: 500 x 6000, 300 x 3000) unsplit
    or split in 2, 4 or 8 parts (`parts`, 0: unsplit; the op allocates the
    workspace), and without a workspace (the bare C-ABI call) the unsplit
    plan, which at 225 x 339 is the 8-wave 128 x 128 tile.  Both against the
    CPU oracle; two calls of the op agree bit for bit."""
    from esimd_learning_amd import cabi
    _say(f"a8w8 round-model tiles M={M} K={K} N={N} parts={parts}")
    lib = cabi.load()
    need = lib.cek_gemm_fp8_a8w8_workspace_size(M, N, K)
    assert need == (parts * M * N * 4 if parts else 0), need
    q, sa, W8, sb = _a8w8_inputs_config4(M, K, N, seed=M + K + N)
    qd, Wd, sad, sbd = q.to(dev), W8.to(dev), sa.to(dev), sb.to(dev)
    y1 = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    y2 = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    ops.esimd_gemm_fp8_a8w8(qd, sad, Wd, sbd, y1)
    ops.esimd_gemm_fp8_a8w8(qd, sad, Wd, sbd, y2)
    y3 = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
    st = cabi.stream_ptr(torch.cuda.current_stream())
    assert lib.cek_gemm_fp8_a8w8(qd.data_ptr(), sad.data_ptr(), Wd.data_ptr(), sbd.data_ptr(), y3.data_ptr(),
                                 M, N, K, 1, st) == 0
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    ref = ogemm.gemm_a8w8(q, sa, W8, sb)
    assert_close_fp(y1.cpu(), ref, f"a8w8 op M={M} K={K} N={N}")
    assert_close_fp(y3.cpu(), ref, f"a8w8 unsplit bf16 M={M} K={K} N={N}")


def test_a8w8_split_k_graph_replays(ops, dev):
    """The split-K op captured in a HIP graph (its workspace then comes from
    the graph's memory pool): three replays, with eager work on the same
    buffers and synchronisations between them, each equal bit for bit to the
    eager call on fresh inputs."""
    M, K, N = 512, 14336, 4096
    _say(f"a8w8 split K graph M={M} K={K} N={N}")
    q, sa, W8, sb = _a8w8_inputs(M, K, N, seed=7)
    qd, Wd, sad, sbd = q.to(dev), W8.to(dev), sa.to(dev), sb.to(dev)
    y = torch.zeros(M, N, dtype=torch.float16, device=dev)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):  # warm-up outside the capture
        ops.esimd_gemm_fp8_a8w8(qd, sad, Wd, sbd, y)
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.esimd_gemm_fp8_a8w8(qd, sad, Wd, sbd, y)
    g2 = torch.Generator().manual_seed(11)
    for r in range(3):
        qd.view(torch.uint8).copy_(torch.randint(0, 0x7E, (M, K), generator=g2, dtype=torch.uint8))  # finite codes
        sad.mul_(1.0 + 0.25 * r)
        eager = torch.empty_like(y)
        ops.esimd_gemm_fp8_a8w8(qd, sad, Wd, sbd, eager)
        torch.cuda.synchronize()
        y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), f"replay {r}"


@pytest.mark.parametrize("M,K,N", [(4096, 1024, 4096), (4000, 576, 4090), (2048, 512, 6144), (2000, 576, 6100),
                                   (2048, 512, 4096), (2000, 576, 4000)])
@pytest.mark.parametrize("io,fmt", [(torch.float16, torch.float8_e4m3fn), (torch.bfloat16, torch.float8_e5m2)])
def test_gemm_pert_large_tiles(ops, dev, M, K, N, io, fmt):
    """w8a16 256 x 256, 256 x 192 and 256 x 128 tiles (8 waves), ragged edges, both activation types
    and fp8 formats, against the CPU oracle."""
    _say(f"gemm pert large tiles M={M} K={K} N={N} {io} {fmt}")
    g = torch.Generator().manual_seed(M + K)
    W8 = (torch.randn(N, K, generator=g).half() * 0.1).to(fmt)
    x = (torch.randn(M, K, generator=g) * 0.5).to(io)
    sv = torch.tensor(0.05)
    y = torch.zeros(M, N, dtype=io, device=dev)
    ops.esimd_gemm_fp8_pert(x.to(dev), W8.to(dev), sv.to(dev), y)
    torch.cuda.synchronize()
    assert_close_fp(y.cpu(), ogemv.gemm_fp8_pert(x, W8, sv), f"pert large M={M} {io} {fmt}")


@pytest.mark.parametrize("M,N,K", [(17, 1, 64), (64, 5, 2048), (300, 16, 4160), (2048, 8, 2048), (33, 16, 64)])
@pytest.mark.parametrize("io,fmt", [(torch.float16, torch.float8_e4m3fn), (torch.bfloat16, torch.float8_e5m2)])
def test_gemm_pert_tiny_n(ops, dev, M, N, K, io, fmt):
    """N <= 16 with M > 16: the activation-streaming kernel (reference tiny-N
    M-parallel path), against the CPU oracle."""
    _say(f"gemm pert tiny N M={M} N={N} K={K} {io} {fmt}")
    g = torch.Generator().manual_seed(M * 7 + N)
    W8 = (torch.randn(N, K, generator=g).half() * 0.1).to(fmt)
    x = (torch.randn(M, K, generator=g) * 0.5).to(io)
    sv = torch.tensor(0.08)
    y = torch.zeros(M, N, dtype=io, device=dev)
    ops.esimd_gemm_fp8_pert(x.to(dev), W8.to(dev), sv.to(dev), y)
    torch.cuda.synchronize()
    assert_close_fp(y.cpu(), ogemv.gemm_fp8_pert(x, W8, sv), f"tiny N M={M} N={N} K={K}")
