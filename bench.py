"""Benchmark of the fp8 decode GEMV (headline) and the fp8 prefill GEMM.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--warm-s S] [--no-cpu] [--no-gemm] [--no-layer] [--no-tables]

Headline workload (headline shape): esimd_gemv_fp8_pern
with M = 1, K = 4096, N = 14336: fp16 activations, e4m3 weights with an fp32
per-output-channel scale, fp16 output.  A step is one GEMV call; step i reads
weight copy i % C, with C copies totalling > 2 GB so that no step finds its
weights in the 256 MB Infinity Cache.  All inputs are resident in HBM before
the timed region.

Timing: W untimed warm-up steps, then exactly K steps captured in one HIP
graph (one graph launch instead of K kernel launches from the host); the
graph is replayed untimed for WARM_S seconds (a cold MI355X runs the first
replays 7-20% slower while its clocks settle), then replayed once, timed,
between device synchronisations; ms_per_step = wall time / K.  The dominant
kernel's average launch duration is measured with HIP events on the launch
stream around one more replay of the same graph; it feeds roofline.achieved.

Further legs (same JSON line): "gemm" (a8w8 at M = 2048,
three projections), "gemm_pert" (the reference's esimd_gemm_fp8_pert, w8a16,
same shapes), "decoder_layer" (config 5, one graph-replayed step),
"gemv_shapes" (config 2, every M x shape), "norm_quant_gemv" (config 3,
fused add+RMSNorm+quant then the fp8 GEMV/GEMM to N = 6144), "small_ops"
(the norm, quant, gelu_and_mul and QK-norm+RoPE kernels at T = 4 and 64;
--small-ops-only runs just this leg), and the device
copy rate the headline is also quoted against (roofline.copy_GBps).
roofline.read_ceiling_us is cek_hbm_read_probe (a read-only kernel) over
the same rotating weight copies, timed the same way: the practical ceiling
of one pass over those bytes on this GPU, beside the 8 TB/s spec peak.

cpu_baseline: the reference's torch CPU path restated in oracle/
((x.float() @ W8.to(fp16).float().T) * s) on this host's cores, timed on the
same shape (2 warm-ups, median of 5); sub-keys time the CPU path of the other
legs (GEMV M = 16, norm+quant T = 64, a8w8 GEMM M = 2048, decoder step).
"""

import argparse
import json
import math
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, spec
FP8_PEAK_TFLOPS = 5000.0       # MI355X dense fp8 MFMA, spec
FP16_PEAK_TFLOPS = 2500.0      # MI355X dense fp16 MFMA, spec
ROTATE_BYTES = 2.2e9
WARM_S = 1.0                   # graph replays before each headline timing (clock settling)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def gemv_bytes(M, N, K):
    # weights + activations + fp32 scales + fp16 outputs
    return N * K + M * K * 2 + N * 4 + M * N * 2


def gemm_a8w8_bytes(M, N, K):
    return M * K + N * K + 2 * M * N + 4 * M + 4 * N


def time_graph(fn_list, torch, stream, warm_s=0.0):
    """Capture fn_list (one launch each) in a graph, replay it for warm_s
    seconds (the GPU's clocks take about a second of load to settle: a cold
    GPU runs the first replays 7% (GEMV) to 20% (GEMM) slower), then time one
    replay between device synchronisations (wall clock: nothing else in the
    bracket -- two event records there added ~14 us to a 20-launch replay)
    and one more between events on its stream (GPU time); returns
    (wall_s, event_ms, graph)."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for fn in fn_list:
            fn()
    torch.cuda.synchronize()
    g.replay()                      # warm replay (graph upload)
    torch.cuda.synchronize()
    t_end = time.perf_counter() + warm_s
    while time.perf_counter() < t_end:
        g.replay()
        torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        g.replay()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        e0.record(stream)
        g.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    return wall, e0.elapsed_time(e1), g


def load_traffic(kernel_key):
    p = ROOT / "profiles" / "traffic.json"
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text()).get(kernel_key)
    except Exception:
        return None


def bench_gemv(ops, torch, steps, warmup, M=1, K=4096, N=14336):
    from esimd_learning_amd import synthetic
    dev = "cuda:0"
    W8, s = synthetic.weight_fp8(N, K, seed=0)
    x = synthetic.activations(M, K, seed=1).to(dev)
    copies = max(2, math.ceil(ROTATE_BYTES / (N * K)))
    log(f"gemv: M={M} K={K} N={N}, {copies} weight copies ({copies * N * K / 1e9:.2f} GB)")
    Wd = W8.to(dev)
    Ws = [Wd] + [Wd.clone() for _ in range(copies - 1)]
    Ss = [s.to(dev).clone() for _ in range(copies)]
    y = torch.empty(M, N, dtype=torch.float16, device=dev)
    stream = torch.cuda.Stream()

    def step(i):
        return lambda: ops.esimd_gemv_fp8_pern(x, Ws[i % copies], Ss[i % copies], y, N, K)

    with torch.cuda.stream(stream):
        for i in range(warmup):
            step(i)()
    torch.cuda.synchronize()
    wall, ev_ms, _ = time_graph([step(i) for i in range(steps)], torch, stream, warm_s=WARM_S)
    nbytes = gemv_bytes(M, N, K)
    avg_launch_us = ev_ms * 1e3 / steps
    res = {
        "ms_per_step": wall * 1e3 / steps,
        "value": nbytes * steps / wall / 1e9,
        "avg_launch_us": avg_launch_us,
        "achieved": nbytes / (avg_launch_us * 1e-6) / 1e9,
        "bytes": nbytes,
    }
    # eager launches with one event pair each (host launch cost excluded from
    # each pair only if the queue stays ahead; reported for reference)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(64)]
    with torch.cuda.stream(stream):
        for i, (a, b) in enumerate(evs):
            a.record(stream)
            step(i)()
            b.record(stream)
    torch.cuda.synchronize()
    per = sorted(a.elapsed_time(b) * 1e3 for a, b in evs)
    res["eager_event_us"] = {"p10": round(per[len(per) // 10], 2), "median": round(per[len(per) // 2], 2),
                             "p90": round(per[(9 * len(per)) // 10], 2)}
    # One-pass read ceiling: cek_hbm_read_probe over the same rotating weight
    # copies, timed the same way (graph of K launches, warmed).
    from esimd_learning_amd import cabi
    lib = cabi.load()

    def probe(i):  # timed mode (no sink)
        return lambda: cabi.check(lib.cek_hbm_read_probe(Ws[i % copies].data_ptr(), N * K, None,
                                                         cabi.stream_ptr(stream)))

    _, pev_ms, _ = time_graph([probe(i) for i in range(steps)], torch, stream, warm_s=WARM_S)
    res["read_ceiling_us"] = pev_ms * 1e3 / steps
    # correctness spot check against the first copy (cheap, CPU oracle at M=1)
    return res, (x, Wd, s, y)


def launch_floor_us(torch, steps=400):
    """Per-launch time of a trivial kernel (a 4-element fill) replayed from a
    graph: the fixed cost every kernel launch in a sequence pays."""
    dev = "cuda:0"
    t = torch.empty(4, dtype=torch.float32, device=dev)
    stream = torch.cuda.Stream()
    _, ev_ms, _ = time_graph([lambda: t.fill_(1.0)] * steps, torch, stream)
    return ev_ms * 1e3 / steps


def copy_bandwidth(torch, nbytes=1 << 30, reps=5):
    """Device-to-device copy rate (read + write bytes / s) of a 1 GiB buffer."""
    dev = "cuda:0"
    src = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    return 2 * nbytes * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9


def bench_gemv_table(ops, torch, shapes=((4096, 14336), (4096, 6144), (4096, 4096), (4096, 28672), (14336, 4096)),
                     Ms=(1, 2, 4, 8, 16)):
    """every (M, K, N), per-launch time over > 2 GB of
    rotating weights (graph of two passes over the copies, event-timed), and
    per shape the one-pass read ceiling of its weight bytes
    (cek_hbm_read_probe over the same copies, timed the same way)."""
    from esimd_learning_amd import cabi, synthetic
    lib = cabi.load()
    dev = "cuda:0"
    stream = torch.cuda.Stream()
    rows = []
    for K, N in shapes:
        W8, s = synthetic.weight_fp8(N, K, seed=0)
        copies = max(2, math.ceil(ROTATE_BYTES / (N * K)))
        Wd = W8.to(dev)
        Ws = [Wd] + [Wd.clone() for _ in range(copies - 1)]
        sd = s.to(dev)
        pfns = [(lambda W=W: cabi.check(lib.cek_hbm_read_probe(W.data_ptr(), N * K, None, cabi.stream_ptr(stream))))
                for W in Ws] * 2
        _, pev_ms, _ = time_graph(pfns, torch, stream, warm_s=0.1)
        ceil_us = pev_ms * 1e3 / len(pfns)
        for M in Ms:
            x = synthetic.activations(M, K, seed=1).to(dev)
            y = torch.empty(M, N, dtype=torch.float16, device=dev)
            fns = [(lambda W=W: ops.esimd_gemv_fp8_pern(x, W, sd, y, N, K)) for W in Ws] * 2
            with torch.cuda.stream(stream):
                for f in fns[:copies]:
                    f()
            torch.cuda.synchronize()
            _, ev_ms, _ = time_graph(fns, torch, stream, warm_s=0.1)
            us = ev_ms * 1e3 / len(fns)
            rows.append({"M": M, "K": K, "N": N, "us": round(us, 2),
                         "GBps": round(gemv_bytes(M, N, K) / (us * 1e-6) / 1e9, 1),
                         "read_ceiling_us": round(ceil_us, 2), "frac_of_read_ceiling": round(ceil_us / us, 3)})
        del Ws, Wd
        torch.cuda.empty_cache()
    return rows


def bench_gemv_scaling(ops, torch, K=4096, N0=14336, mults=(1, 2, 4, 8, 16)):
    """The M = 1 GEMV and the read probe at K = 4096 over N = 14336 x
    (1, 2, 4, 8, 16) rows (58.7 to 940 MB of weights; random finite e4m3
    codes, made on the device), each timed over > 2 GB of rotating copies
    (graph of two passes over the copies, event-timed), and per kernel a
    least-squares line t = fixed + bytes / rate through its five times: the
    fixed cost of a launch (ramp-up, first-byte latency, the last
    workgroups' tail) and the marginal streaming rate.  best_frac_of_spec is
    what one pass over the headline's 58.7 MB reaches on this part: those
    bytes over the probe's time at that size, against 8 TB/s."""
    import numpy as np
    from esimd_learning_amd import cabi
    lib = cabi.load()
    dev = "cuda:0"
    stream = torch.cuda.Stream()
    gen = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(1, K, device=dev, generator=gen).half()
    rows = []
    for mlt in mults:
        N = N0 * mlt
        wb = N * K
        copies = max(2, math.ceil(ROTATE_BYTES / wb))
        Ws = [torch.randint(0, 0x7E, (N, K), device=dev, dtype=torch.uint8, generator=gen).view(torch.float8_e4m3fn)
              for _ in range(copies)]
        sd = torch.rand(N, device=dev, generator=gen) * 1e-3
        y = torch.empty(1, N, dtype=torch.float16, device=dev)
        pfns = [(lambda W=W: cabi.check(lib.cek_hbm_read_probe(W.data_ptr(), wb, None, cabi.stream_ptr(stream))))
                for W in Ws] * 2
        gfns = [(lambda W=W: ops.esimd_gemv_fp8_pern(x, W, sd, y, N, K)) for W in Ws] * 2
        _, p_ms, _ = time_graph(pfns, torch, stream, warm_s=0.2)
        _, g_ms, _ = time_graph(gfns, torch, stream, warm_s=0.2)
        rows.append({"N": N, "weight_MB": round(wb / 1e6, 1), "gemv_us": round(g_ms * 1e3 / len(gfns), 3),
                     "probe_us": round(p_ms * 1e3 / len(pfns), 3)})
        del Ws
        torch.cuda.empty_cache()
    b = np.array([r["weight_MB"] * 1e6 for r in rows])
    fit = {}
    for key in ("gemv_us", "probe_us"):
        t = np.array([r[key] for r in rows])
        slope, icpt = np.polyfit(b, t, 1)          # us per byte, us
        resid = t - (slope * b + icpt)
        fit[key[:-3]] = {"fixed_us": round(float(icpt), 3), "marginal_TBps": round(1e6 / float(slope) / 1e12, 3),
                         "max_residual_us": round(float(np.abs(resid).max()), 3)}
    hb = N0 * K
    return {"K": K, "rows": rows, "fit": fit,
            "best_frac_of_spec": round(hb / (rows[0]["probe_us"] * 1e-6) / (HBM_PEAK_GBS * 1e9), 4),
            "gemv_frac_of_probe": round(rows[0]["probe_us"] / rows[0]["gemv_us"], 4)}


def bench_norm_quant_gemv(ops, torch, reps=50, N=6144):
    """fused add+RMSNorm+per-token e4m3 quant, then the
    fp8 x fp8 GEMV/GEMM to N = 6144 on its codes and scales.  Per (T, H):
    the two kernels' times (each a graph of `reps` launches, event-timed;
    the GEMV rotates over > 2 GB of weights), the pair back to back, and for
    T <= 4 the single launch that computes the same outputs (fused_us)."""
    from esimd_learning_amd import synthetic
    dev = "cuda:0"
    stream = torch.cuda.Stream()
    rows = []
    for H in (4096, 5120):
        W8, sb = synthetic.weight_fp8(N, H, seed=4)
        copies = max(2, math.ceil(ROTATE_BYTES / (N * H)))
        Wd = W8.view(torch.uint8).to(dev)
        Ws = [Wd] + [Wd.clone() for _ in range(copies - 1)]
        sbd = sb.to(dev)
        w = synthetic.norm_weight(H, seed=H).to(dev)
        for T in (1, 8, 32, 64):
            h = synthetic.activations(T, H, seed=T).to(dev)
            r = synthetic.activations(T, H, seed=T + 1).to(dev)
            q = torch.empty(T, H, dtype=torch.float8_e4m3fn, device=dev)
            sa = torch.empty(T, dtype=torch.float32, device=dev)
            y = torch.empty(T, N, dtype=torch.float16, device=dev)
            norm = lambda: ops.esimd_fused_add_rms_norm_quant_fp8(h, r, w, 1e-6, q, sa)  # noqa: E731
            gemv = [(lambda W=W: ops.esimd_gemm_fp8_a8w8(q.view(torch.uint8), sa, W, sbd, y)) for W in Ws]
            with torch.cuda.stream(stream):
                norm()
                gemv[0]()
            torch.cuda.synchronize()
            _, n_ms, _ = time_graph([norm] * reps, torch, stream, warm_s=0.05)
            _, g_ms, _ = time_graph(gemv * 2, torch, stream, warm_s=0.05)
            pair = []
            for i in range(reps):
                pair += [norm, gemv[i % copies]]
            _, p_ms, _ = time_graph(pair, torch, stream, warm_s=0.05)
            row = {"T": T, "H": H, "norm_quant_us": round(n_ms * 1e3 / reps, 2),
                   "gemv_us": round(g_ms * 1e3 / (2 * copies), 2),
                   "pair_us": round(p_ms * 1e3 / reps, 2)}
            if T <= 4:
                # the same outputs from one launch: norm + quant in the GEMV's prologue
                r_out = torch.empty_like(r)
                fused = [(lambda W=W: ops.esimd_fused_add_rms_norm_quant_gemv_fp8(h, r, w, 1e-6, r_out, q, sa, W,
                                                                                    sbd, y)) for W in Ws]
                _, f_ms, _ = time_graph(fused * 2, torch, stream, warm_s=0.05)
                row["fused_us"] = round(f_ms * 1e3 / (2 * copies), 2)
            rows.append(row)
        del Ws, Wd
        torch.cuda.empty_cache()
    return rows


def bench_gemm(ops, torch, steps, warmup, M=2048, K=4096, N=6144, rotate=False):
    """One a8w8 shape: `steps` launches in one graph, event-timed.  With
    rotate, launch i reads weight copy i % C of C copies totalling > 2 GB
    (weights from HBM, as a prefill streaming fresh layers sees them);
    otherwise every launch re-reads one copy (Infinity Cache resident)."""
    from esimd_learning_amd import synthetic
    dev = "cuda:0"
    log(f"gemm a8w8: M={M} K={K} N={N}" + (" (rotating weights)" if rotate else ""))
    x = synthetic.activations(M, K, seed=2).to(dev)
    q = torch.empty(M, K, dtype=torch.float8_e4m3fn, device=dev)
    sa = torch.empty(M, dtype=torch.float32, device=dev)
    ops.esimd_per_token_quant_fp8(x, q, sa)
    W8, sb = synthetic.weight_fp8(N, K, seed=3)
    Wd, sbd = W8.to(dev), sb.to(dev)
    copies = max(2, math.ceil(ROTATE_BYTES / (N * K))) if rotate else 1
    Ws = [Wd] + [Wd.clone() for _ in range(copies - 1)]
    y = torch.empty(M, N, dtype=torch.float16, device=dev)
    stream = torch.cuda.Stream()
    fns = [(lambda W=W: ops.esimd_gemm_fp8_a8w8(q, sa, W, sbd, y)) for W in Ws]
    fn = fns[0]
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            fn()
    torch.cuda.synchronize()
    if rotate:
        steps = max(steps, copies)
    wall, ev_ms, _ = time_graph([fns[i % copies] for i in range(steps)], torch, stream, warm_s=WARM_S)
    del Ws
    flops = 2.0 * M * N * K
    us = ev_ms * 1e3 / steps
    return {"config": f"a8w8 M={M} K={K} N={N}", "avg_launch_us": us,
            "tflops": flops / (us * 1e-6) / 1e12,
            "wall_tflops": flops * steps / wall / 1e12,
            "roofline": {"bound": "mfma", "achieved": flops / (us * 1e-6) / 1e12, "peak": FP8_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": flops / (us * 1e-6) / 1e12 / FP8_PEAK_TFLOPS,
                         "traffic": None}}


def bench_gemm_all(ops, torch, steps, warmup, all_m=True):
    """the headline M = 2048, (K, N) = (4096, 6144), plus
    the other two projections ("shapes"), each timed the same way (one weight
    copy re-read by every launch, so it stays in the Infinity Cache); with
    all_m M = 512, 2048 and 4096 with weights rotating from HBM ("m_table",
    each row with the roofline time
    max(flop / fp8 peak, bytes / HBM peak), bytes = M K + N K + 2 M N + 4 M +
    4 N: M = 512 sits near the ridge point)."""
    head = bench_gemm(ops, torch, steps, warmup)
    head["weights"] = "one copy re-read across launches (Infinity Cache resident); m_table: from HBM"
    head["shapes"] = []
    for K, N in ((4096, 6144), (4096, 28672), (14336, 4096)):
        r = head if (K, N) == (4096, 6144) else bench_gemm(ops, torch, steps, warmup, K=K, N=N)
        head["shapes"].append({"config": r["config"], "avg_launch_us": round(r["avg_launch_us"], 2),
                               "tflops": round(r["tflops"], 1)})
    if all_m:
        head["m_table"] = []
        for M in (512, 2048, 4096):
            for K, N in ((4096, 6144), (4096, 28672), (14336, 4096)):
                r = bench_gemm(ops, torch, steps, warmup, M=M, K=K, N=N, rotate=True)
                flops = 2.0 * M * N * K
                byts = M * K + N * K + 2 * M * N + 4 * M + 4 * N
                roof_us = max(flops / (FP8_PEAK_TFLOPS * 1e12), byts / (HBM_PEAK_GBS * 1e9)) * 1e6
                head["m_table"].append({"M": M, "K": K, "N": N, "avg_launch_us": round(r["avg_launch_us"], 2),
                                        "tflops": round(r["tflops"], 1), "roofline_us": round(roof_us, 2),
                                        "frac_of_roofline": round(roof_us / r["avg_launch_us"], 3),
                                        "weights": "rotating copies over > 2 GB (read from HBM)"})
    return head


def bench_gemm_k_scaling(ops, torch, M=2048, N=6144, Ks=(1024, 2048, 4096, 8192, 12288), reps=20):
    """The headline a8w8 shape's time against K (M = 2048, N = 6144: one
    256 x 192 tile per CU, K / 128 steps each; random finite e4m3 codes,
    operands re-read from the Infinity Cache; a graph of `reps` launches,
    event-timed, warmed) and a least-squares line t = fixed + steps x
    per_step: the fixed cost of a launch (its dispatch, the first loads, the
    epilogue's output stores) and the time of one K step (48 MFMAs per SIMD).
    Also the same flops on 256 x 256 tiles with 24 steps each (M = 2048,
    K = 3072, N = 8192): the step count a stream-K schedule of the
    headline's 192 tiles of 256 x 256 would give every CU, before any
    fix-up of the tiles it splits."""
    import numpy as np
    dev = "cuda:0"
    stream = torch.cuda.Stream()
    gen = torch.Generator(device=dev).manual_seed(7)

    def timed(M_, K_, N_):
        a = torch.randint(0, 0x7E, (M_, K_), device=dev, dtype=torch.uint8, generator=gen)
        b = torch.randint(0, 0x7E, (N_, K_), device=dev, dtype=torch.uint8, generator=gen)
        sa = torch.rand(M_, device=dev, generator=gen) * 1e-3
        sb = torch.rand(N_, device=dev, generator=gen) * 1e-3
        y = torch.empty(M_, N_, dtype=torch.float16, device=dev)
        fn = lambda: ops.esimd_gemm_fp8_a8w8(a, sa, b, sb, y)  # noqa: E731
        with torch.cuda.stream(stream):
            fn()
        torch.cuda.synchronize()
        _, ms, _ = time_graph([fn] * reps, torch, stream, warm_s=0.3)
        return ms * 1e3 / reps

    rows = [{"K": K, "steps": K // 128, "us": round(timed(M, K, N), 2)} for K in Ks]
    st = np.array([r["steps"] for r in rows], dtype=np.float64)
    t = np.array([r["us"] for r in rows])
    per_step, fixed = np.polyfit(st, t, 1)
    mfma_us = 48 * 32 / 2.4e3  # one step's MFMA cycles per SIMD at the 2.4 GHz of the 5 PF spec
    return {"M": M, "N": N, "tile": "256 x 192, one per CU", "rows": rows,
            "fixed_us": round(float(fixed), 2), "per_step_us": round(float(per_step), 4),
            "per_step_mfma_us_at_2p4GHz": round(mfma_us, 4),
            "equal_flops_256x256_24_steps_us": round(timed(2048, 3072, 8192), 2)}


def bench_gemm_pert(ops, torch, steps, warmup, M=2048, rotate=False):
    """The reference's prefill op esimd_gemm_fp8_pert (fp16 activations, e4m3
    weights, fp32 per-tensor scale; the w8a16 fp16-MFMA path) at the three
    config-4 projections, timed like the a8w8 leg (with rotate, launch i
    reads weight copy i % C of C copies over > 2 GB: weights from HBM); rate
    against the 2.5 PFLOP/s dense fp16 MFMA peak."""
    from esimd_learning_amd import synthetic
    dev = "cuda:0"
    stream = torch.cuda.Stream()
    rows = []
    for K, N in ((4096, 6144), (4096, 28672), (14336, 4096)):
        x = synthetic.activations(M, K, seed=2).to(dev)
        W8, _ = synthetic.weight_fp8(N, K, seed=3)
        Wd = W8.to(dev)
        copies = max(2, math.ceil(ROTATE_BYTES / (N * K))) if rotate else 1
        Ws = [Wd] + [Wd.clone() for _ in range(copies - 1)]
        sv = torch.tensor(0.01, dtype=torch.float32, device=dev)
        y = torch.empty(M, N, dtype=torch.float16, device=dev)
        fns = [(lambda W=W: ops.esimd_gemm_fp8_pert(x, W, sv, y)) for W in Ws]
        with torch.cuda.stream(stream):
            for _ in range(warmup):
                fns[0]()
        torch.cuda.synchronize()
        n = max(steps, copies) if rotate else steps
        _, ev_ms, _ = time_graph([fns[i % copies] for i in range(n)], torch, stream, warm_s=WARM_S / 2)
        us = ev_ms * 1e3 / n
        tf = 2.0 * M * N * K / (us * 1e-6) / 1e12
        row = {"config": f"w8a16 M={M} K={K} N={N}", "avg_launch_us": round(us, 2), "tflops": round(tf, 1),
               "frac_of_fp16_peak": round(tf / FP16_PEAK_TFLOPS, 4)}
        if rotate:
            row["weights"] = "rotating copies over > 2 GB (read from HBM)"
        rows.append(row)
        del x, Wd, Ws, y
    return rows


def bench_small_ops(ops, torch, reps=200):
    """The HBM/latency-bound small kernels at decode (T = 4, the config-5
    shapes) and prefill (T = 64) sizes: add+RMSNorm, add+RMSNorm+quant,
    per-token quant (H = 3072), gelu_and_mul (d = 24576) and QK-norm+RoPE
    (16 q + 16 k heads x 256 in a [T, 12288] QKV buffer).  Each a graph of
    `reps` launches over one set of buffers, event-timed; bytes are the
    algorithmic bytes per launch (reads + writes)."""
    from esimd_learning_amd import synthetic
    dev = "cuda:0"
    stream = torch.cuda.Stream()
    H, d, hd, nq, nk = 3072, 24576, 256, 16, 16
    rows = []
    for T in (4, 64):
        h = synthetic.activations(T, H, seed=T).to(dev)
        r = synthetic.activations(T, H, seed=T + 1).to(dev)
        w = synthetic.norm_weight(H, seed=H).to(dev)
        q8 = torch.empty(T, H, dtype=torch.float8_e4m3fn, device=dev)
        s8 = torch.empty(T, dtype=torch.float32, device=dev)
        gu = synthetic.activations(T, 2 * d, seed=T + 2).to(dev)
        act = torch.empty(T, d, dtype=torch.float16, device=dev)
        qkv = synthetic.activations(T, (nq + 2 * nk) * hd, seed=T + 3).to(dev)
        qw, kw = synthetic.norm_weight(hd, 1).to(dev), synthetic.norm_weight(hd, 2).to(dev)
        pos = synthetic.positions(T, seed=T).to(dev)
        legs = {
            # in place: reads hidden and residual, writes both
            "add_rmsnorm": (lambda: ops.esimd_fused_add_rms_norm_batched(h, r, w, 1e-6), 4 * T * H * 2 + H * 2),
            "add_rmsnorm_quant": (lambda: ops.esimd_fused_add_rms_norm_quant_fp8(h, r, w, 1e-6, q8, s8),
                                  3 * T * H * 2 + H * 2 + T * H + T * 4),
            "per_token_quant": (lambda: ops.esimd_per_token_quant_fp8(h, q8, s8), T * H * 2 + T * H + T * 4),
            "gelu_and_mul": (lambda: ops.esimd_gelu_and_mul(act, gu), T * 2 * d * 2 + T * d * 2),
            "qk_norm_rope": (lambda: ops.esimd_qk_norm_rope(qkv[:, : nq * hd], qkv[:, nq * hd:(nq + nk) * hd], qw, kw,
                                                            pos, 1e-6, 10000.0, True),
                             2 * T * (nq + nk) * hd * 2 + 2 * hd * 2 + T * 8),
        }
        for name, (fn, nbytes) in legs.items():
            with torch.cuda.stream(stream):
                fn()
            torch.cuda.synchronize()
            # (the norms update the residual in place, so it grows by about
            # one unit per call: a short warm keeps every value finite)
            _, ms, _ = time_graph([fn] * reps, torch, stream, warm_s=0.02)
            us = ms * 1e3 / reps
            rows.append({"op": name, "T": T, "us": round(us, 2), "bytes": nbytes,
                         "GBps": round(nbytes / (us * 1e-6) / 1e9, 1)})
    return rows


# Decoder-step variants timed side by side: the default step (add+RMSNorms
# deferred across the GEMVs around them, gelu_and_mul in the gate/up GEMV's
# epilogue, QK-norm+RoPE and the attention stand-in's copy of q in the QKV
# GEMV's last workgroup of each head), the same with the norms as launches of
# their own (equal to the separate ops bit for bit), with QK-norm+RoPE as its
# own launch too, the e4m3 hand-off, every op its own launch, and the
# add+RMSNorms in the GEMV prologues.
LAYER_VARIANTS = {"us_per_step": dict(),
                  "no_defer_us_per_step": dict(defer_norm=False),
                  "no_tails_us_per_step": dict(fuse_tails=False),
                  "act_fp8_us_per_step": dict(act_fp8=True),
                  "unfused_us_per_step": dict(fuse_glu=False, fuse_tails=False),
                  "norm_fused_us_per_step": dict(fuse_norm=True)}


LAYERS = 8  # decoder layers per captured forward, each with its own weight copy (2.2 GB: read from HBM)


def bench_layer(torch, steps, M=4, rounds=5, layers=LAYERS):
    """the Gemma-style decoder-layer decode step, as a
    multi-layer model runs it: `layers` chained layers (each layer's output
    the next one's hidden state, each with its own copy of the weights, so
    that every step reads its 277 MB from HBM) captured in one HIP graph; a
    step is the graph's time / `layers`.  Every variant of LAYER_VARIANTS is
    captured first, then the variants are timed in turn, `rounds` times
    round-robin (so that all see the same clock state), and each reports its
    median round.  Also: the default step captured alone and its graph
    replayed back to back (`single_step_graphs_us`: each replay adds the
    graph-to-graph launch gap), and the read probe over the layers' weight
    matrices in one graph the same way (the one-pass floor of a step's
    GEMVs)."""
    from esimd_learning_amd import synthetic
    from esimd_learning_amd.layer import GemmaDecodeLayer, capture_forward, forward
    dev = "cuda:0"
    p = synthetic.gemma_layer(seed=10)
    p0 = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in p.items()}
    psets = [p0] + [{k: (v.clone() if torch.is_tensor(v) else v) for k, v in p0.items()} for _ in range(layers - 1)]
    h = synthetic.activations(M, p["hidden"], seed=20).to(dev)
    r = synthetic.activations(M, p["hidden"], seed=21).to(dev)
    pos = synthetic.positions(M, seed=22).to(dev)
    reps = max(1, -(-steps // layers))
    graphs, stacks = {}, {}
    for key, kw in LAYER_VARIANTS.items():
        stack = [GemmaDecodeLayer(ps, M, dev, **kw) for ps in psets]
        forward(stack, h, r, pos)
        torch.cuda.synchronize()
        graphs[key] = capture_forward(stack, h, r, pos)
        stacks[key] = stack
    t_end = time.perf_counter() + WARM_S
    while time.perf_counter() < t_end:
        for g in graphs.values():
            g.replay()
        torch.cuda.synchronize()
    times = {key: [] for key in graphs}
    for _ in range(rounds):
        for key, g in graphs.items():
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                g.replay()
            e1.record()
            torch.cuda.synchronize()
            times[key].append(e0.elapsed_time(e1) * 1e3 / (reps * layers))
    med = {key: sorted(v)[len(v) // 2] for key, v in times.items()}
    # the default step alone in a graph, replayed back to back
    one = stacks["us_per_step"][0]
    g1 = one.capture(h, r, pos)
    for _ in range(10):
        g1.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        g1.replay()
    e1.record()
    torch.cuda.synchronize()
    single_us = e0.elapsed_time(e1) * 1e3 / steps
    wb = one.weight_bytes()
    # the layers' weight matrices read once each by cek_hbm_read_probe, in
    # one graph the same way: the one-pass read floor of a step's GEMVs
    from esimd_learning_amd import cabi
    lib = cabi.load()
    mats = [w for ly in stacks["us_per_step"] for w in (ly.Wqkv, ly.Wo, ly.Wgu, ly.Wd)]
    stream = torch.cuda.Stream()
    pfns = [(lambda w=w: cabi.check(lib.cek_hbm_read_probe(w.data_ptr(), w.numel(), None, cabi.stream_ptr(stream))))
            for w in mats] * reps
    _, pev_ms, _ = time_graph(pfns, torch, stream, warm_s=WARM_S / 2)
    floor_us = pev_ms * 1e3 / (reps * layers)
    us = med["us_per_step"]
    out = {"config": "Gemma-style decoder layer decode step, M=4, hidden 3072, 16q/16kv x 256, MLP 24576 "
                     "(attention stood in by a copy of q)",
           "us_per_step": round(us, 2), "weight_bytes": wb, "weight_GBps": round(wb / us / 1e3, 1),
           "weight_read_floor_us": round(floor_us, 2)}
    for key in LAYER_VARIANTS:
        if key != "us_per_step":
            out[key] = round(med[key], 2)
    out["single_step_graphs_us"] = round(single_us, 2)
    out["timing"] = (f"{layers} chained layers (own weight copies) per HIP graph, {reps} replays back to back, "
                     f"per step = time / {reps * layers}; variants timed round-robin {rounds} times, median round")
    return out


def bench_parity(ops, torch, eps=1e-6):
    """Parity of the measured paths against the CPU oracle, computed after
    every timed region (nothing here is timed):
      * config 3 (T in {1, 8, 32, 64} x H in {4096, 5120}, the norm+quant
        leg's inputs): the per-token e4m3 quant of the device's normed rows
        against the oracle's quant of the same rows -- code and scale
        mismatches (expected 0) and the rounding ties among them; the fused
        add+RMSNorm+quant against the oracle's -- residual mismatches
        (expected 0), rows whose scale differs, and codes that differ (by at
        most one step: the normed value rounds differently where the sum of
        squares is taken in another order);
      * config 5: the decode forward bench_layer times (eight layers of one
        weight set, the default deferred-norm step), run once eagerly,
        against eight oracle decoder steps: max-abs error / max|ref| of the
        output and of the residual."""
    from esimd_learning_amd import synthetic
    from esimd_learning_amd.layer import GemmaDecodeLayer, forward
    from oracle import fp8 as ofp8
    from oracle import layer as olayer
    from oracle import norm as onorm
    import numpy as np
    dev = "cuda:0"
    mag = lambda c: np.where(c & 0x80, -(c & 0x7F), c & 0x7F).astype(np.int64)  # noqa: E731  monotone code order
    tot = {"elements": 0, "quant_code_mismatches": 0, "quant_scale_mismatches": 0, "quant_ties": 0,
           "fused_residual_mismatches": 0, "fused_rows_scale_differs": 0, "fused_code_diffs": 0,
           "fused_code_max_step": 0}
    rows = []
    for H in (4096, 5120):
        w = synthetic.norm_weight(H, seed=H)
        for T in (1, 8, 32, 64):
            h = synthetic.activations(T, H, seed=T)
            r = synthetic.activations(T, H, seed=T + 1)
            hd, rd, wd = h.to(dev), r.to(dev), w.to(dev)
            # per-token quant of the device's normed rows
            h2, r2 = hd.clone(), rd.clone()
            ops.esimd_fused_add_rms_norm_batched(h2, r2, wd, eps)
            q = torch.empty(T, H, dtype=torch.float8_e4m3fn, device=dev)
            s = torch.empty(T, dtype=torch.float32, device=dev)
            ops.esimd_per_token_quant_fp8(h2, q, s)
            # fused add+RMSNorm+quant
            r1 = rd.clone()
            q1 = torch.empty_like(q)
            s1 = torch.empty_like(s)
            ops.esimd_fused_add_rms_norm_quant_fp8(hd, r1, wd, eps, q1, s1)
            torch.cuda.synchronize()
            xf = h2.cpu().float().numpy()
            q_ref, s_ref = ofp8.per_token_quant(xf)
            sn = s.cpu().numpy()
            v = np.clip((xf / sn[:, None]).astype(np.float32), -448, 448).astype(np.float32)
            qm = int((q.view(torch.uint8).cpu().numpy() != q_ref).sum())
            sm = int((sn.view(np.uint32) != s_ref.view(np.uint32)).sum())
            ties = int(ofp8.e4m3_is_tie(v).sum())
            r_ref, qf_ref, sf_ref, _ = onorm.fused_add_rms_norm_quant(h, r, w, eps)
            rm = int((r1.cpu() != r_ref).sum())
            srows = int((s1.cpu().numpy() != sf_ref.numpy()).sum())
            d = np.abs(mag(q1.view(torch.uint8).cpu().numpy()) - mag(qf_ref.numpy()))
            row = {"T": T, "H": H, "quant_code_mismatches": qm, "quant_scale_mismatches": sm, "quant_ties": ties,
                   "fused_residual_mismatches": rm, "fused_rows_scale_differs": srows,
                   "fused_code_diffs": int((d != 0).sum()), "fused_code_max_step": int(d.max())}
            rows.append(row)
            tot["elements"] += T * H
            for k in row:
                if k == "fused_code_max_step":
                    tot[k] = max(tot[k], row[k])
                elif k not in ("T", "H"):
                    tot[k] += row[k]
    out = {"config3_norm_quant": {"totals": tot, "rows": rows}}
    # config 5: the benchmarked forward against the oracle
    M, L = 4, LAYERS
    p = synthetic.gemma_layer(seed=10)
    pd = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in p.items()}
    stack = [GemmaDecodeLayer(pd, M, dev) for _ in range(L)]
    h = synthetic.activations(M, p["hidden"], seed=20)
    r = synthetic.activations(M, p["hidden"], seed=21)
    pos = synthetic.positions(M, seed=22)
    rd = r.to(dev)
    y = forward(stack, h.to(dev), rd, pos.to(dev))
    torch.cuda.synchronize()
    ho, ro = h, r
    for _ in range(L):
        o, ro, _ = olayer.decoder_step(p, ho, ro, pos)
        ho = o.to(h.dtype)
    frac = lambda a, b: round(float((a.cpu().float() - b.float()).abs().max() / b.float().abs().max()), 6)  # noqa: E731
    out["config5_forward"] = {"layers": L, "defer_norm": all(ly.defer_norm for ly in stack),
                              "output_maxerr_over_maxref": frac(y, o),
                              "residual_maxerr_over_maxref": frac(rd, ro), "bound": 0.01}
    return out


def _cpu_model():
    """The host CPU's model name (lscpu, else /proc/cpuinfo) and socket/core counts."""
    import subprocess
    model, extra = "", ""
    try:
        txt = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        kv = {}
        for line in txt.splitlines():
            if ":" in line:
                k, v = line.split(":", 1)
                kv[k.strip()] = v.strip()
        model = kv.get("Model name", "")
        extra = ", ".join(f"{k} {kv[k]}" for k in ("Socket(s)", "Core(s) per socket", "Thread(s) per core",
                                                   "CPU(s)") if k in kv)
    except (OSError, subprocess.SubprocessError):
        pass
    if not model:
        try:
            for line in open("/proc/cpuinfo"):
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
        except OSError:
            pass
    return model, extra


def _time_cpu(fn, reps, warm=2):
    """Median wall time (s) of fn over reps calls after warm calls."""
    ts = []
    for i in range(warm + reps):
        t0 = time.perf_counter()
        fn()
        if i >= warm:
            ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2]


def cpu_baseline(torch, M=1, K=4096, N=14336, reps=5):
    """The reference's torch CPU path, restated in oracle/, on this host's
    cores beside each GPU leg: the headline GEMV (value), plus the batched
    GEMV at M = 16, add+RMSNorm+quant at T = 64, the a8w8 GEMM at M = 2048
    and the decoder-layer step (sub-keys).  About 10-20 s in all."""
    from esimd_learning_amd import synthetic
    from oracle import gemm as ogemm
    from oracle import gemv as ogemv
    from oracle import layer as olayer
    from oracle import norm as onorm
    torch.set_num_threads(os.cpu_count() or 1)
    W8, s = synthetic.weight_fp8(N, K, seed=0)
    x = synthetic.activations(M, K, seed=1)
    med = _time_cpu(lambda: ogemv.gemv_fp8_pern(x, W8, s), reps)
    # the same with the weights dequantised once up front (matmul + scale only)
    Wf = W8.to(torch.float16).float()
    xf = x.float()
    med_mm = _time_cpu(lambda: (xf @ Wf.T) * s.float(), reps)
    model, extra = _cpu_model()
    out = {"value": gemv_bytes(M, N, K) / med / 1e9, "unit": "GB/s", "cores": torch.get_num_threads(),
           "kind": "port",
           "sample": f"oracle gemv_fp8_pern (dequant fp8->fp16->fp32 + fp32 matmul + scale) on CPU, "
                     f"M={M} K={K} N={N}, median of {reps} after 2 warm-ups, {med * 1e3:.1f} ms/call; "
                     f"os.cpu_count()={os.cpu_count()}; cpu '{model}' ({extra})",
           "matmul_only": {"value": gemv_bytes(M, N, K) / med_mm / 1e9, "unit": "GB/s",
                           "ms_per_call": round(med_mm * 1e3, 2),
                           "sample": "same shape with W dequantised once before timing (fp32 matmul + scale)"}}
    # config 2: the batched GEMV at M = 16 on the headline weights
    x16 = synthetic.activations(16, K, seed=1)
    t = _time_cpu(lambda: ogemv.gemv_fp8_pern(x16, W8, s), reps)
    out["gemv_m16"] = {"value": round(gemv_bytes(16, N, K) / t / 1e9, 3), "unit": "GB/s",
                       "ms_per_call": round(t * 1e3, 2), "gpu_leg": "gemv_shapes M=16 K=4096 N=14336",
                       "sample": f"oracle gemv_fp8_pern, M=16 K={K} N={N}, median of {reps}"}
    del Wf
    # config 3: add+RMSNorm + per-token e4m3 quant, T = 64, H = 4096
    T, H = 64, 4096
    h = synthetic.activations(T, H, seed=T)
    r = synthetic.activations(T, H, seed=T + 1)
    w = synthetic.norm_weight(H, seed=H)
    t = _time_cpu(lambda: onorm.fused_add_rms_norm_quant(h, r, w, 1e-6), reps)
    out["norm_quant_t64"] = {"value": round(t * 1e6, 1), "unit": "us", "gpu_leg": "norm_quant_gemv T=64 H=4096 "
                             "norm_quant_us", "sample": f"oracle fused_add_rms_norm_quant, T={T} H={H}, median of {reps}"}
    # config 4: the a8w8 GEMM at the headline M = 2048, K = 4096, N = 6144
    Mg, Kg, Ng, greps = 2048, 4096, 6144, 3
    xa = synthetic.activations(Mg, Kg, seed=2).float()
    sa = torch.clamp(xa.abs().amax(dim=1) / 448.0, min=1.0 / (448.0 * 512.0))
    qa = (xa / sa[:, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8)
    Wg, sg = synthetic.weight_fp8(Ng, Kg, seed=3)
    Wg = Wg.view(torch.uint8)
    t = _time_cpu(lambda: ogemm.gemm_a8w8(qa, sa, Wg, sg), greps, warm=1)
    out["gemm_a8w8_m2048"] = {"value": round(2.0 * Mg * Ng * Kg / t / 1e12, 3), "unit": "TFLOP/s",
                              "ms_per_call": round(t * 1e3, 1), "gpu_leg": "gemm (a8w8 M=2048 K=4096 N=6144)",
                              "sample": f"oracle gemm_a8w8 (fp32 dequantise of both code matrices + fp32 matmul "
                                        f"+ scales), M={Mg} K={Kg} N={Ng}, median of {greps} after 1 warm-up"}
    del xa, qa, Wg
    # config 5: one decoder-layer step at M = 4
    p = synthetic.gemma_layer(seed=10)
    hl = synthetic.activations(4, p["hidden"], seed=20)
    rl = synthetic.activations(4, p["hidden"], seed=21)
    pos = synthetic.positions(4, seed=22)
    lreps = 3
    t = _time_cpu(lambda: olayer.decoder_step(p, hl, rl, pos), lreps, warm=1)
    out["layer_m4"] = {"value": round(t * 1e3, 1), "unit": "ms/step", "gpu_leg": "decoder_layer us_per_step",
                       "sample": f"oracle decoder_step (every GEMV dequantises its weights per call), M=4, "
                                 f"median of {lreps} after 1 warm-up"}
    return out


def main():
    global WARM_S
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-gemm", action="store_true")
    ap.add_argument("--no-layer", action="store_true")
    ap.add_argument("--no-parity", action="store_true", help="skip the post-timing parity counts against the oracle")
    ap.add_argument("--no-tables", action="store_true", help="skip the config-2 GEMV table and config-3 legs")
    ap.add_argument("--gemm-headline-only", action="store_true",
                    help="run only the headline a8w8 GEMM leg (M=2048, K=4096, N=6144) and print it (counter runs)")
    ap.add_argument("--small-ops-only", action="store_true",
                    help="run only the small-kernel leg (norm, quant, gelu_and_mul, QK-norm+RoPE) and print it")
    ap.add_argument("--warm-s", type=float, default=None,
                    help=f"seconds of untimed graph replays before each headline timing (default {WARM_S})")
    ap.add_argument("--copy-ref", action="store_true",
                    help="first run 10 plain device copies of N*K bytes (reference for HBM counter scaling)")
    a = ap.parse_args()
    if a.warm_s is not None:
        WARM_S = max(0.0, a.warm_s)
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {a.gpus} requested); the op pack has no "
              f"multi-GPU path. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    import esimd_learning_amd
    ops = esimd_learning_amd.ops()
    assert torch.cuda.is_available(), "no GPU visible"
    log(f"device: {torch.cuda.get_device_name(0)}")
    if a.copy_ref:
        src = torch.empty(14336 * 4096, dtype=torch.uint8, device="cuda:0").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy reference: 10 x {src.numel()} bytes")
        del src, dst
    if a.gemm_headline_only:
        print(json.dumps({"gemm": bench_gemm(ops, torch, max(10, a.steps // 20), max(3, a.warmup // 10))}), flush=True)
        return
    if a.small_ops_only:
        print(json.dumps({"small_ops": bench_small_ops(ops, torch, reps=max(20, a.steps // 2))}), flush=True)
        return

    g, (x, Wd, s, y) = bench_gemv(ops, torch, a.steps, a.warmup)
    log(f"gemv: read ceiling (one pass over the same weight bytes) {g['read_ceiling_us']:.2f} us")
    log(f"gemv: {g['avg_launch_us']:.2f} us/launch, {g['achieved']:.0f} GB/s; eager event median "
        f"{g['eager_event_us']['median']:.2f} us; wall {g['ms_per_step'] * 1e3:.2f} us/step")
    # spot check of the measured output
    from oracle import gemv as ogemv
    torch.cuda.synchronize()
    ref = ogemv.gemv_fp8_pern(x.cpu(), Wd.cpu(), s)
    err = (y.cpu().float() - ref).abs().max().item()
    assert err <= 1e-2 * ref.abs().max().item(), f"bench output check failed: {err}"

    out = {
        "metric": "fp8 GEMV HBM GB/s & %peak (M=1,K4096,N14336); fp8 GEMM TFLOPS M=2048",
        "value": round(g["value"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(g["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3 weights x fp16 activations, fp32 accumulate",
        "data": "synthetic (seeded N(0,0.02) weights quantised per row to e4m3; N(0,1) fp16 activations)",
        "config": {"workload": "esimd_gemv_fp8_pern decode GEMV, BASELINE config 2 headline shape",
                   "M": 1, "K": 4096, "N": 14336, "scale": "fp32 per output channel",
                   "weight_copies_rotated_GB": round(math.ceil(ROTATE_BYTES / (4096 * 14336)) * 4096 * 14336 / 1e9, 2),
                   "timing": "K launches captured in one HIP graph, replayed once"},
        "roofline": {"bound": "hbm", "achieved": round(g["achieved"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(g["achieved"] / HBM_PEAK_GBS, 4),
                     "traffic": load_traffic("gemv_dot_kernel_m1_k4096_n14336"),
                     "algorithmic_bytes": g["bytes"], "avg_launch_us": round(g["avg_launch_us"], 3),
                     "eager_event_us": g["eager_event_us"],
                     # the same weight bytes read once by cek_hbm_read_probe (no arithmetic):
                     # the practical one-pass ceiling at this size
                     "read_ceiling_us": round(g["read_ceiling_us"], 3),
                     "read_ceiling_GBps": round(4096 * 14336 / (g["read_ceiling_us"] * 1e-6) / 1e9, 1),
                     "frac_of_read_ceiling": round(g["read_ceiling_us"] / g["avg_launch_us"], 4)},
    }
    out["roofline"]["launch_floor_us"] = round(launch_floor_us(torch), 2)
    if not a.copy_ref:  # (counter runs keep the copy kernels to the reference copies)
        cbw = copy_bandwidth(torch)
        out["roofline"]["copy_GBps"] = round(cbw, 1)
        out["roofline"]["frac_of_copy"] = round(g["achieved"] / cbw, 4)
        log(f"device copy: {cbw:.0f} GB/s (read + write); GEMV at {g['achieved'] / cbw:.1%} of it")
    if not a.no_tables:
        out["gemv_scaling"] = bench_gemv_scaling(ops, torch)
        gs = out["gemv_scaling"]["fit"]
        log(f"gemv scaling: gemv fixed {gs['gemv']['fixed_us']} us + {gs['gemv']['marginal_TBps']} TB/s; probe fixed "
            f"{gs['probe']['fixed_us']} us + {gs['probe']['marginal_TBps']} TB/s")
        out["gemv_shapes"] = bench_gemv_table(ops, torch)
        log("gemv table: " + ", ".join(f"M{r['M']}/{r['K']}x{r['N']}={r['us']}us" for r in out["gemv_shapes"]))
        out["norm_quant_gemv"] = bench_norm_quant_gemv(ops, torch)
        log("norm+quant -> gemv: " + ", ".join(f"T{r['T']}/H{r['H']}={r['pair_us']}us" for r in out["norm_quant_gemv"]))
        out["small_ops"] = bench_small_ops(ops, torch)
        log("small ops: " + ", ".join(f"{r['op']}/T{r['T']}={r['us']}us" for r in out["small_ops"]))
    if not a.no_gemm:
        out["gemm"] = bench_gemm_all(ops, torch, max(10, a.steps // 20), max(3, a.warmup // 10))
        out["gemm"]["roofline"]["traffic"] = load_traffic("gemm_a8w8_pipe_b3_kernel_m2048_k4096_n6144")
        log(f"gemm: {out['gemm']['avg_launch_us']:.1f} us, {out['gemm']['tflops']:.0f} TFLOP/s")
        out["gemm_k_scaling"] = bench_gemm_k_scaling(ops, torch)
        gk = out["gemm_k_scaling"]
        log(f"gemm k scaling: fixed {gk['fixed_us']} us + {gk['per_step_us']} us per K step; 256x256 x 24 steps "
            f"{gk['equal_flops_256x256_24_steps_us']} us")
        out["gemm_pert"] = bench_gemm_pert(ops, torch, max(10, a.steps // 40), max(3, a.warmup // 10))
        log("gemm pert (w8a16): " + ", ".join(f"{r['config']}={r['avg_launch_us']}us/{r['tflops']}TF"
                                              for r in out["gemm_pert"]))
        out["gemm_pert_m_table"] = [r for Mx in (512, 2048, 4096)
                                    for r in bench_gemm_pert(ops, torch, max(10, a.steps // 40), 2, M=Mx, rotate=True)]
    if not a.no_layer:
        out["decoder_layer"] = bench_layer(torch, max(20, a.steps // 4))
        dl = out["decoder_layer"]
        log(f"layer: {dl['us_per_step']} us/step, {dl['weight_GBps']} GB/s; " +
            ", ".join(f"{k} {dl[k]}" for k in LAYER_VARIANTS if k != "us_per_step"))
    if not a.no_parity:
        log("parity against the oracle ...")
        out["parity"] = bench_parity(ops, torch)
        pt = out["parity"]["config3_norm_quant"]["totals"]
        pf = out["parity"]["config5_forward"]
        log(f"parity: quant mismatches {pt['quant_code_mismatches']} (ties {pt['quant_ties']}), fused code diffs "
            f"{pt['fused_code_diffs']} of {pt['elements']}; 8-layer forward err {pf['output_maxerr_over_maxref']}")
    if not a.no_cpu:
        log("cpu baseline ...")
        out["cpu_baseline"] = cpu_baseline(torch)
    out["host"] = platform.node()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
