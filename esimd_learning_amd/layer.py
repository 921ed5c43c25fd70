"""One Gemma-style decoder-layer decode step from the custom ops.

    h1, r1 = add_rmsnorm(hidden, residual, w_in)          esimd_fused_add_rms_norm_batched
    qkv    = h1 @ Wqkv^T * sqkv                           esimd_gemv_fp8_pern
                                   (the two as one launch: esimd_fused_add_rms_norm_gemv_fp8)
    q, k   = per-head RMSNorm + RoPE (in place in qkv)     esimd_qk_norm_rope
    a      = attention(q, k, v)        -- out of scope: a copy of q stands in for its output
    o      = a @ Wo^T * so                                esimd_gemv_fp8_pern
    h2, r2 = add_rmsnorm(o, r1, w_post)                   esimd_fused_add_rms_norm_batched
    g      = gelu_tanh(h2 @ Wg^T * sg) * (h2 @ Wu^T * su) esimd_gemv_fp8_gelu_and_mul
                                   (the two as one launch: esimd_fused_add_rms_norm_gemv_fp8)
    out    = g @ Wd^T * sd                                esimd_gemv_fp8_pern

The gate/up projection and gelu_and_mul run as one launch (Wgu = [Wg; Wu],
the GEMV's epilogue applies gelu_tanh(gate) * up to the rounded outputs);
``fuse_glu=False`` runs them as esimd_gemv_fp8_pern into [M, 2d] followed by
esimd_gelu_and_mul, which gives the same values.  With ``fuse_norm`` (up to
four rows) each add+RMSNorm runs in the prologue of the GEMV it feeds; r1 is
then kept in a buffer of the layer, hidden is only read, and residual
receives r2 as before.  It is off by default: every workgroup of the GEMV
then normalises the rows itself, which at M = 4 over the 768 and 1536
workgroups of QKV and gate/up costs more than the norm launch it saves.

With ``fuse_tails`` (the default; fp16/bf16 hand-offs, no ``fuse_norm``)
QK-norm+RoPE runs in the QKV GEMV (esimd_gemv_fp8_qk_norm_rope: per head,
the workgroup that finishes the head's rows last), which also writes the
rotated q heads into the attention stand-in's output -- two launches fewer
per step, the same values bit for bit.  Its arrival counters are allocated
(zeroed) once here and left zero by every call.

With ``act_fp8=True`` the two norm -> GEMV hand-offs carry e4m3 activations
instead of fp16: esimd_fused_add_rms_norm_quant_fp8 writes per-token codes
and scales, and esimd_gemm_fp8_a8w8 (esimd_gemm_fp8_a8w8_gelu_and_mul for
gate/up) consumes them (the hidden input is then
only read, not overwritten with the normed value).  Needs e4m3 weights.

With ``defer_norm`` (the default where it applies: up to four rows, e4m3
weights, fp16 hand-offs, ``fuse_tails`` and ``fuse_glu``, the shapes the
kernels take) each add+RMSNorm is split across the two
GEMVs around it instead of running as a launch of its own: the producer
GEMV (o_proj; in ``forward``, also the down projection of every layer but
the last, for the next layer's input norm) adds its output into the
residual, writes residual * w * 2^-shift and per-16-column sums of squares
(times 4^-shift), and the consumer (gate/up, the next layer's QKV) scales
its rows by the 2^shift / rms those sums give with eps * 4^-shift
(esimd_gemv_fp8_add_rms_norm_defer and the ``_rs`` ops).  The shift, the
smallest with 2^shift >= max|w|, bounds residual * w * 2^-shift by the
residual itself, so the hand-off cannot overflow fp16.
Two launches fewer per layer; the values match the unfused layer to within
the rounding of the moved 1 / rms, not bit for bit (``defer_norm=False``
gives the step that equals the separate ops bit for bit).

The intermediate buffers and counters are allocated once in the
constructor, so at decode sizes a step enqueues only kernels: it can be
captured in a HIP graph (``capture``) and replayed, which removes host launch
overhead from the latency-bound small kernels between the GEMVs.  (One
exception: with ``act_fp8`` at M = 64 the a8w8 op splits K and takes its
fp32 workspace from PyTorch's caching allocator on every call -- inside a
captured graph, from the graph's memory pool.)
"""

import torch


class GemmaDecodeLayer:
    def __init__(self, params, M, device="cuda:0", dtype=torch.float16, act_fp8=False, fuse_glu=True,
                 fuse_norm=False, fuse_tails=True, defer_norm=True):
        from . import ops as _load_ops
        self.ops = _load_ops()
        p = params
        self.M, self.dev, self.dtype = M, device, dtype
        self.hidden, self.hd, self.nq, self.nk = p["hidden"], p["head_dim"], p["n_q"], p["n_kv"]
        self.mlp, self.eps, self.theta = p["mlp"], p["eps"], p["theta"]
        t = lambda x: x.to(device)  # noqa: E731
        self.Wqkv, self.sqkv = t(p["Wqkv"]), t(p["sqkv"])
        self.Wo, self.so = t(p["Wo"]), t(p["so"])
        self.Wgu, self.sgu = t(p["Wgu"]), t(p["sgu"])
        self.Wd, self.sd = t(p["Wd"]), t(p["sd"])
        self.w_in, self.w_post = t(p["w_in"]).to(dtype), t(p["w_post"]).to(dtype)
        self.qw, self.kw = t(p["qw"]).to(dtype), t(p["kw"]).to(dtype)
        nqkv = self.Wqkv.shape[0]
        mk = lambda n: torch.empty(M, n, dtype=dtype, device=device)  # noqa: E731
        self.qkv = mk(nqkv)
        self.attn = mk(self.nq * self.hd)
        self.o = mk(self.hidden)
        self.gu = mk(2 * self.mlp)
        self.act = mk(self.mlp)
        self.out = mk(self.hidden)
        self.act_fp8 = act_fp8
        self.fuse_glu = fuse_glu
        self.fuse_norm = fuse_norm and M <= 4   # the fused launch covers up to four rows
        self.r_mid = mk(self.hidden)            # r1 between the two fused norms
        self.fuse_tails = fuse_tails and not act_fp8 and not self.fuse_norm
        self.cnt_rope = self.ops.gemv_tail_counters(self.nq, self.nk, device)
        e4m3 = all(w.dtype == torch.float8_e4m3fn for w in (self.Wqkv, self.Wo, self.Wgu, self.Wd))
        # the shapes the deferred-norm kernels take (else the unfused step)
        kib = lambda k: k % 1024 == 0 and k // 1024 in (2, 3, 4, 5, 14, 24)  # noqa: E731
        # (hidden: the QKV and gate/up K the consumers take, and at most 256
        # partial sums per row from the producers, N = hidden)
        shapes = (self.hidden in (3072, 4096) and kib(self.nq * self.hd) and kib(self.mlp)
                  and self.hd in (128, 256) and nqkv % 16 == 0 and self.mlp % 16 == 0)
        # fp16 only: in bf16 (8-bit mantissa) the moved rounding of x * w
        # against x * w / rms reached 1.1% of max|out| over two layers, above
        # the op pack's 1% bound (fp16: 0.14%)
        self.defer_norm = (defer_norm and dtype == torch.float16 and M <= 4 and e4m3 and self.fuse_tails and fuse_glu
                           and shapes)
        if self.defer_norm:
            # the producers write residual * w * 2^-shift with 2^shift >= max|w|,
            # which cannot overflow fp16 whatever the residual holds; the
            # consumers then take eps * 4^-shift (the weights are read back
            # once, here)
            self.shift_in = self.ops.esimd_defer_norm_shift(self.w_in)
            self.shift_post = self.ops.esimd_defer_norm_shift(self.w_post)
            groups = self.ops.esimd_gemv_fp8_add_rms_norm_defer_groups(self.hidden)
            ss = lambda: torch.empty(M, groups, dtype=torch.float32, device=device)  # noqa: E731
            self.ss_o, self.ss_d = ss(), ss()    # after o_proj; after down (the next layer's input norm)
        if act_fp8:
            if self.Wqkv.dtype != torch.float8_e4m3fn or self.Wgu.dtype != torch.float8_e4m3fn:
                raise ValueError("act_fp8 needs e4m3 weights")
            self.q8 = torch.empty(M, self.hidden, dtype=torch.float8_e4m3fn, device=device)
            self.s8 = torch.empty(M, dtype=torch.float32, device=device)
            self.Wqkv8, self.sqkv32 = self.Wqkv.view(torch.uint8), self.sqkv.float()
            self.Wgu8, self.sgu32 = self.Wgu.view(torch.uint8), self.sgu.float()
        self.graph = None

    def weight_bytes(self):
        return sum(w.numel() for w in (self.Wqkv, self.Wo, self.Wgu, self.Wd))

    def step(self, hidden, residual, positions, ss_in=None, next_norm=None):
        """hidden, residual: [M, hidden] (residual updated in place); returns out.

        defer_norm only: with ``ss_in`` (the previous layer's ss_d) hidden
        already holds residual * w_in * 2^-shift_in of the previous layer's
        deferred input norm of this layer and residual its sum; with
        ``next_norm`` (the next layer's (w_in, shift_in)) the down projection
        produces that for the next layer and ss_d."""
        o, hd, nq, nk = self.ops, self.hd, self.nq, self.nk
        if self.fuse_norm:
            return self._step_fused(hidden, residual, positions)
        if self.defer_norm:
            return self._step_defer(hidden, residual, positions, ss_in, next_norm)
        if ss_in is not None or next_norm is not None:
            raise ValueError("ss_in / next_norm need defer_norm")
        if self.act_fp8:
            o.esimd_fused_add_rms_norm_quant_fp8(hidden, residual, self.w_in, self.eps, self.q8, self.s8)
            o.esimd_gemm_fp8_a8w8(self.q8.view(torch.uint8), self.s8, self.Wqkv8, self.sqkv32, self.qkv)
        else:
            o.esimd_fused_add_rms_norm_batched(hidden, residual, self.w_in, self.eps)
            if self.fuse_tails:   # the tail also writes the attention stand-in's output
                o.esimd_gemv_fp8_qk_norm_rope(hidden, self.Wqkv, self.sqkv, self.qkv, self.qw, self.kw, positions,
                                              nq, nk, self.eps, self.theta, True, self.cnt_rope, self.attn)
            else:
                o.esimd_gemv_fp8_pern(hidden, self.Wqkv, self.sqkv, self.qkv, self.Wqkv.shape[0], self.hidden)
        if not self.fuse_tails:
            o.esimd_qk_norm_rope(self.qkv[:, : nq * hd], self.qkv[:, nq * hd:(nq + nk) * hd], self.qw, self.kw,
                                 positions, self.eps, self.theta, True)
            self.attn.copy_(self.qkv[:, : nq * hd])                # attention stand-in
        o.esimd_gemv_fp8_pern(self.attn, self.Wo, self.so, self.o, self.hidden, nq * hd)
        if self.act_fp8:
            o.esimd_fused_add_rms_norm_quant_fp8(self.o, residual, self.w_post, self.eps, self.q8, self.s8)
            if self.fuse_glu:
                o.esimd_gemm_fp8_a8w8_gelu_and_mul(self.q8.view(torch.uint8), self.s8, self.Wgu8, self.sgu32,
                                                   self.act)
            else:
                o.esimd_gemm_fp8_a8w8(self.q8.view(torch.uint8), self.s8, self.Wgu8, self.sgu32, self.gu)
        else:
            o.esimd_fused_add_rms_norm_batched(self.o, residual, self.w_post, self.eps)
            if self.fuse_glu:
                o.esimd_gemv_fp8_gelu_and_mul(self.o, self.Wgu, self.sgu, self.act)
            else:
                o.esimd_gemv_fp8_pern(self.o, self.Wgu, self.sgu, self.gu, 2 * self.mlp, self.hidden)
        if not self.fuse_glu:
            o.esimd_gelu_and_mul(self.act, self.gu)
        o.esimd_gemv_fp8_pern(self.act, self.Wd, self.sd, self.out, self.hidden, self.mlp)
        return self.out

    def _step_fused(self, hidden, residual, positions):
        o, hd, nq, nk = self.ops, self.hd, self.nq, self.nk
        if self.act_fp8:
            o.esimd_fused_add_rms_norm_quant_gemv_fp8(hidden, residual, self.w_in, self.eps, self.r_mid, self.q8,
                                                      self.s8, self.Wqkv8, self.sqkv32, self.qkv)
        else:
            o.esimd_fused_add_rms_norm_gemv_fp8(hidden, residual, self.w_in, self.eps, self.r_mid, self.Wqkv,
                                                self.sqkv, self.qkv)
        o.esimd_qk_norm_rope(self.qkv[:, : nq * hd], self.qkv[:, nq * hd:(nq + nk) * hd], self.qw, self.kw,
                             positions, self.eps, self.theta, True)
        self.attn.copy_(self.qkv[:, : nq * hd])                    # attention stand-in
        o.esimd_gemv_fp8_pern(self.attn, self.Wo, self.so, self.o, self.hidden, nq * hd)
        glu = self.fuse_glu
        y = self.act if glu else self.gu
        if self.act_fp8:
            o.esimd_fused_add_rms_norm_quant_gemv_fp8(self.o, self.r_mid, self.w_post, self.eps, residual, self.q8,
                                                      self.s8, self.Wgu8, self.sgu32, y, glu)
        else:
            o.esimd_fused_add_rms_norm_gemv_fp8(self.o, self.r_mid, self.w_post, self.eps, residual, self.Wgu,
                                                self.sgu, y, glu)
        if not glu:
            o.esimd_gelu_and_mul(self.act, self.gu)
        o.esimd_gemv_fp8_pern(self.act, self.Wd, self.sd, self.out, self.hidden, self.mlp)
        return self.out

    def _step_defer(self, hidden, residual, positions, ss_in, next_norm):
        o, hd, nq, nk, eps = self.ops, self.hd, self.nq, self.nk, self.eps
        if ss_in is None:
            o.esimd_fused_add_rms_norm_batched(hidden, residual, self.w_in, eps)
            o.esimd_gemv_fp8_qk_norm_rope(hidden, self.Wqkv, self.sqkv, self.qkv, self.qw, self.kw, positions,
                                          nq, nk, eps, self.theta, True, self.cnt_rope, self.attn)
        else:
            o.esimd_gemv_fp8_qk_norm_rope_rs(hidden, self.Wqkv, self.sqkv, self.qkv, self.qw, self.kw, positions,
                                             nq, nk, eps, self.theta, True, self.cnt_rope, ss_in,
                                             eps * 4.0 ** -self.shift_in, self.attn)
        o.esimd_gemv_fp8_add_rms_norm_defer(self.attn, self.Wo, self.so, residual, self.w_post, self.o, self.ss_o,
                                            self.shift_post)
        o.esimd_gemv_fp8_gelu_and_mul_rs(self.o, self.Wgu, self.sgu, self.act, self.ss_o,
                                         eps * 4.0 ** -self.shift_post)
        if next_norm is None:
            o.esimd_gemv_fp8_pern(self.act, self.Wd, self.sd, self.out, self.hidden, self.mlp)
        else:
            w_next, shift_next = next_norm
            o.esimd_gemv_fp8_add_rms_norm_defer(self.act, self.Wd, self.sd, residual, w_next, self.out, self.ss_d,
                                                shift_next)
        return self.out

    def capture(self, hidden, residual, positions, stream=None):
        """Capture one step on fixed input buffers in a HIP graph; replay with replay()."""
        s = stream or torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=s):
            self.step(hidden, residual, positions)
        torch.cuda.current_stream().wait_stream(s)
        return self.graph

    def replay(self):
        self.graph.replay()
        return self.out


def forward(layers, hidden, residual, positions):
    """A decode forward over `layers` in sequence: each layer's output buffer
    is the next layer's hidden state (which that layer's first norm
    overwrites), and the residual stream is updated in place by every layer.
    Between two ``defer_norm`` layers the next layer's input norm is
    deferred across the down projection and its QKV GEMV.  Returns the last
    layer's output buffer (for a deferred pair as for any other: the down
    projection's output is only the normed input of the next layer, the
    last layer's is the plain one)."""
    h, ss = hidden, None
    for i, layer in enumerate(layers):
        nxt = layers[i + 1] if i + 1 < len(layers) else None
        chain = nxt is not None and layer.defer_norm and nxt.defer_norm
        if layer.defer_norm:
            h = layer.step(h, residual, positions, ss_in=ss, next_norm=(nxt.w_in, nxt.shift_in) if chain else None)
        else:
            h = layer.step(h, residual, positions)
        ss = layer.ss_d if chain else None
    return h


def capture_forward(layers, hidden, residual, positions, stream=None):
    """forward() over `layers` captured in one HIP graph, as a serving loop
    captures a model's whole decode step (no launch gap between layers)."""
    s = stream or torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        forward(layers, hidden, residual, positions)
    torch.cuda.current_stream().wait_stream(s)
    return g
