"""Python wrappers of the ``torch.ops.custom_esimd_kernels_vllm`` ops.

The first four keep the reference's names, signatures and forwarding
(reference python/custom_esimd_kernels_vllm/ops.py:7-67); the docstrings
state this build's contract.  The rest wrap the new ops of the same
namespace.
"""

import torch

_ops = torch.ops.custom_esimd_kernels_vllm


def esimd_gemv_fp8_pern(
    input: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor,
    output: torch.Tensor,
    N: int, K: int,
) -> torch.Tensor:
    """fp8-weight GEMV with a per-output-channel scale, fp32 accumulation.

    input/output: [M, K]/[M, N] fp16 or bf16 of one dtype (every row is
    computed; the reference computes row 0); weight: [N, K] float8_e4m3fn or
    float8_e5m2; weight_scale: [N] fp16, bf16 or fp32.  Returns ``output``.
    """
    return _ops.esimd_gemv_fp8_pern(input, weight, weight_scale, output, N, K)


def esimd_gemv_fp8_pert(
    input: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor,
    output: torch.Tensor,
) -> torch.Tensor:
    """fp8-weight GEMV with a per-tensor fp32 scale (read on the device).

    N and K are taken from weight's shape.  Returns ``output``.
    """
    return _ops.esimd_gemv_fp8_pert(input, weight, weight_scale, output)


def esimd_fused_add_rms_norm_batched(
    hidden_states: torch.Tensor,
    residual: torch.Tensor,
    weight: torch.Tensor,
    eps: float,
) -> torch.Tensor:
    """Batched fused residual add + RMSNorm (Gemma-style), in place.

    residual = hidden_states + residual; hidden_states = rmsnorm(residual) *
    weight, with weight already shifted (w + 1.0).  Any number of rows.
    Returns ``hidden_states``.
    """
    return _ops.esimd_fused_add_rms_norm_batched(hidden_states, residual, weight, eps)


def esimd_gemm_fp8_pert(
    input: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor,
    output: torch.Tensor,
) -> torch.Tensor:
    """fp8-weight GEMM with a per-tensor fp32 scale, any M.

    input/output: [M, K]/[M, N] fp16 or bf16 of one dtype; weight [N, K] fp8.
    M <= 16 runs the decode GEMV kernels, larger M the MFMA GEMM.
    """
    return _ops.esimd_gemm_fp8_pert(input, weight, weight_scale, output)


# ---- new ops -------------------------------------------------------------

def esimd_gemv_fp8_pern_fused(input, weights, weight_scales, outputs) -> None:
    """Several per-channel-scale fp8 GEMVs sharing ``input`` in one launch.

    weights[i]: [N_i, K] fp8; weight_scales[i]: [N_i]; outputs[i]: [M, N_i].
    Each output equals esimd_gemv_fp8_pern on its own matrix.
    """
    _ops.esimd_gemv_fp8_pern_fused(input, list(weights), list(weight_scales), list(outputs))


def esimd_gemv_fp8_pert_fused(input, weights, weight_scales, outputs) -> None:
    """Several per-tensor-scale fp8 GEMVs sharing ``input`` in one launch."""
    _ops.esimd_gemv_fp8_pert_fused(input, list(weights), list(weight_scales), list(outputs))


def esimd_fused_add_rms_norm_quant_fp8(
    hidden_states: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float,
    out_q: torch.Tensor, out_scale: torch.Tensor,
) -> None:
    """residual += hidden_states (in place); per-token e4m3 codes of
    rmsnorm(residual) * weight into out_q [T, H] and fp32 scales into
    out_scale [T].  hidden_states is only read."""
    _ops.esimd_fused_add_rms_norm_quant_fp8(hidden_states, residual, weight, eps, out_q, out_scale)


def esimd_per_token_quant_fp8(input: torch.Tensor, out_q: torch.Tensor, out_scale: torch.Tensor) -> None:
    """Per-token e4m3 quantisation: out_scale[t] = max(amax_t / 448, 1/(448*512))."""
    _ops.esimd_per_token_quant_fp8(input, out_q, out_scale)


def esimd_gelu_and_mul(out: torch.Tensor, input: torch.Tensor) -> None:
    """out = gelu_tanh(input[..., :d]) * input[..., d:]."""
    _ops.esimd_gelu_and_mul(out, input)


def esimd_gemv_fp8_gelu_and_mul(
    input: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor, output: torch.Tensor,
) -> None:
    """Gate/up GEMV over a merged fp8 weight with gelu_and_mul fused.

    input [M, K] fp16/bf16; weight [2d, K] fp8 (gate rows, then up rows);
    weight_scale [2d] fp16/bf16/fp32; output [M, d] of input's dtype.
    output equals esimd_gemv_fp8_pern into [M, 2d] followed by
    esimd_gelu_and_mul, in one launch for decode batches.
    """
    _ops.esimd_gemv_fp8_gelu_and_mul(input, weight, weight_scale, output)


def esimd_fused_add_rms_norm_gemv_fp8(
    hidden_states: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float,
    residual_out: torch.Tensor, w: torch.Tensor, w_scale: torch.Tensor, output: torch.Tensor,
    gelu_and_mul: bool = False,
) -> None:
    """residual_out = hidden_states + residual; output = the fp8 GEMV of
    rmsnorm(residual_out) * weight (with ``gelu_and_mul``: w holds gate then up
    rows and output [M, d] is gelu_tanh(gate) * up).  One launch for up to
    four rows; the values equal esimd_fused_add_rms_norm_batched followed by
    the GEMV.  hidden_states and residual are only read."""
    _ops.esimd_fused_add_rms_norm_gemv_fp8(hidden_states, residual, weight, eps, residual_out, w, w_scale, output,
                                           gelu_and_mul)


def esimd_fused_add_rms_norm_quant_gemv_fp8(
    hidden_states: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float,
    residual_out: torch.Tensor, out_q: torch.Tensor, out_scale: torch.Tensor,
    b: torch.Tensor, b_scale: torch.Tensor, output: torch.Tensor, gelu_and_mul: bool = False,
) -> None:
    """esimd_fused_add_rms_norm_quant_fp8 (into residual_out, out_q, out_scale)
    followed by esimd_gemm_fp8_a8w8 (or its gelu_and_mul form), one launch
    for up to four rows."""
    _ops.esimd_fused_add_rms_norm_quant_gemv_fp8(hidden_states, residual, weight, eps, residual_out, out_q,
                                                 out_scale, b, b_scale, output, gelu_and_mul)


def esimd_qk_norm_rope(
    q: torch.Tensor, k: torch.Tensor, q_weight: torch.Tensor, k_weight: torch.Tensor,
    positions: torch.Tensor, eps: float, theta: float = 10000.0, is_neox: bool = True,
) -> None:
    """Per-head RMSNorm then rotary embedding of q and k, in place."""
    _ops.esimd_qk_norm_rope(q, k, q_weight, k_weight, positions, eps, theta, is_neox)


def gemv_tail_counters(n_q, n_k, device) -> torch.Tensor:
    """Zeroed arrival counters for esimd_gemv_fp8_qk_norm_rope (64 per head)."""
    return torch.zeros(64 * (n_q + n_k), dtype=torch.int32, device=device)


def esimd_gemv_fp8_qk_norm_rope(
    input: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor, output: torch.Tensor,
    q_weight: torch.Tensor, k_weight: torch.Tensor, positions: torch.Tensor, n_q: int, n_k: int,
    eps: float, theta: float, is_neox: bool, counters: torch.Tensor,
    q_out: torch.Tensor = None,
) -> None:
    """The QKV GEMV (esimd_gemv_fp8_pern into output [M, N]) followed by
    esimd_qk_norm_rope on its q columns [0, n_q hd) and k columns
    [n_q hd, (n_q + n_k) hd), in one launch for decode batches.  counters:
    int32 device tensor of >= 64 * (n_q + n_k) elements
    (``gemv_tail_counters``, allocated once by the caller, not per call, so
    that the call can be captured in a graph), zero before the first call and
    left zero by each.  q_out (optional, [M, n_q hd]) also receives the rotated q heads,
    as a copy of output's q columns would."""
    _ops.esimd_gemv_fp8_qk_norm_rope(input, weight, weight_scale, output, q_weight, k_weight, positions, n_q, n_k,
                                     eps, theta, is_neox, counters, q_out)


def esimd_gemv_fp8_add_rms_norm_defer_groups(N: int) -> int:
    """G, the number of partial sums of squares per row that
    esimd_gemv_fp8_add_rms_norm_defer writes for N output columns (N / 16,
    or N / 12 where that fills more CUs: N = 3072 -> 256); 0 if N is not a
    multiple of 16."""
    return _ops.esimd_gemv_fp8_add_rms_norm_defer_groups(N)


def esimd_defer_norm_shift(norm_weight: torch.Tensor) -> int:
    """The norm_shift E for esimd_gemv_fp8_add_rms_norm_defer with this norm
    weight: the smallest E with 2^E >= max|norm_weight| (so that the
    producer's output cannot overflow whatever the residual holds).  Reads
    the weight's maximum back to the host: call it once per weight, not per
    step."""
    return _ops.esimd_defer_norm_shift(float(norm_weight.float().abs().max()))


def esimd_gemv_fp8_add_rms_norm_defer(
    input: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor, residual: torch.Tensor,
    norm_weight: torch.Tensor, output: torch.Tensor, row_ss: torch.Tensor, norm_shift: int = 0,
) -> None:
    """The producer half of an add + RMSNorm deferred into the next GEMV
    (up to four rows, e4m3 weights): o = the GEMV's rounded output; residual
    += o in place; output = residual * norm_weight * 2^-norm_shift (rounded;
    the norm without its 1 / rms); row_ss [M, G] fp32, G =
    ``esimd_gemv_fp8_add_rms_norm_defer_groups(N)``, = the sums of squares of
    the unrounded (o + residual) * 2^-norm_shift over G equal runs of
    columns.  Feed output and row_ss to a ``*_rs`` op with eps *
    4^-norm_shift, which then applies 2^norm_shift / rms.  With norm_shift =
    ``esimd_defer_norm_shift(norm_weight)`` the output cannot overflow; with
    0 an fp16 output overflows where |residual * norm_weight| > 65504."""
    _ops.esimd_gemv_fp8_add_rms_norm_defer(input, weight, weight_scale, residual, norm_weight, output, row_ss,
                                           norm_shift)


def esimd_gemv_fp8_pern_rs(
    input: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor, output: torch.Tensor,
    row_ss: torch.Tensor, eps: float,
) -> None:
    """esimd_gemv_fp8_pern with each output row m scaled by
    rsqrt(sum(row_ss[m]) / K + eps) (the deferred norm's consumer)."""
    _ops.esimd_gemv_fp8_pern_rs(input, weight, weight_scale, output, row_ss, eps)


def esimd_gemv_fp8_gelu_and_mul_rs(
    input: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor, output: torch.Tensor,
    row_ss: torch.Tensor, eps: float,
) -> None:
    """esimd_gemv_fp8_gelu_and_mul with the gate and up rows scaled by the
    deferred norm's rsqrt(sum(row_ss[m]) / K + eps) before gelu_and_mul."""
    _ops.esimd_gemv_fp8_gelu_and_mul_rs(input, weight, weight_scale, output, row_ss, eps)


def esimd_gemv_fp8_qk_norm_rope_rs(
    input: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor, output: torch.Tensor,
    q_weight: torch.Tensor, k_weight: torch.Tensor, positions: torch.Tensor, n_q: int, n_k: int,
    eps: float, theta: float, is_neox: bool, counters: torch.Tensor, row_ss: torch.Tensor, row_eps: float,
    q_out: torch.Tensor = None,
) -> None:
    """esimd_gemv_fp8_qk_norm_rope with the GEMV's rows scaled by the
    deferred norm's rsqrt(sum(row_ss[m]) / K + row_eps) before QK-norm and
    RoPE."""
    _ops.esimd_gemv_fp8_qk_norm_rope_rs(input, weight, weight_scale, output, q_weight, k_weight, positions, n_q,
                                        n_k, eps, theta, is_neox, counters, row_ss, row_eps, q_out)


def esimd_gemm_fp8_a8w8(
    a: torch.Tensor, a_scale: torch.Tensor, b: torch.Tensor, b_scale: torch.Tensor,
    output: torch.Tensor,
) -> torch.Tensor:
    """output[m, n] = a_scale[m] * b_scale[n] * sum_k a[m, k] * b[n, k] (e4m3 x e4m3)."""
    return _ops.esimd_gemm_fp8_a8w8(a, a_scale, b, b_scale, output)


def esimd_gemm_fp8_a8w8_gelu_and_mul(
    a: torch.Tensor, a_scale: torch.Tensor, b: torch.Tensor, b_scale: torch.Tensor,
    output: torch.Tensor,
) -> None:
    """esimd_gemm_fp8_a8w8 over a merged [2d, K] gate/up weight, then
    gelu_and_mul, fused for M <= 16: output [M, d]."""
    _ops.esimd_gemm_fp8_a8w8_gelu_and_mul(a, a_scale, b, b_scale, output)
