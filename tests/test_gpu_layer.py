"""GPU parity of the Gemma-style decoder-layer step.

Compared with oracle.layer.decoder_step, which composes the oracle ops with
the same rounding to fp16 between steps.  Graph replays are checked against
the eager step, several replays in a row with eager work in between.
"""

import sys

import pytest
import torch

from conftest import assert_close_fp
from esimd_learning_amd import synthetic
from esimd_learning_amd.layer import GemmaDecodeLayer
from oracle import layer as olayer

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


SMALL = dict(hidden=512, n_q=4, n_kv=2, head_dim=64, mlp=1024)
CONFIG5 = dict(hidden=3072, n_q=16, n_kv=16, head_dim=256, mlp=24576)


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("act_fp8", [False, True])
@pytest.mark.parametrize("dims,M", [(SMALL, 3), (CONFIG5, 4), (SMALL, 6)])
def test_decoder_step_vs_oracle(ops, dev, dims, M, act_fp8, fused):
    _say(f"decoder step M={M} {dims} act_fp8={act_fp8} fused={fused}")
    p = synthetic.gemma_layer(seed=10, **dims)
    layer = GemmaDecodeLayer(p, M, dev, act_fp8=act_fp8, fuse_glu=fused, fuse_norm=fused)
    h = synthetic.activations(M, dims["hidden"], seed=20)
    r = synthetic.activations(M, dims["hidden"], seed=21)
    pos = synthetic.positions(M, seed=22)
    hd, rd = h.to(dev), r.to(dev)
    out = layer.step(hd, rd, pos.to(dev)).clone()
    torch.cuda.synchronize()
    ref_out, ref_r, _ = olayer.decoder_step(p, h, r, pos, act_fp8=act_fp8)
    assert_close_fp(rd.cpu(), ref_r.float(), "residual after the layer")
    assert_close_fp(out.cpu(), ref_out, "layer output")


@pytest.mark.parametrize("fuse_norm", [False, True])
@pytest.mark.parametrize("act_fp8", [False, True])
@pytest.mark.parametrize("dims", [SMALL, CONFIG5])
def test_decoder_step_graph_replays(ops, dev, act_fp8, fuse_norm, dims):
    M = 4
    p = synthetic.gemma_layer(seed=11, **dims)
    layer = GemmaDecodeLayer(p, M, dev, act_fp8=act_fp8, fuse_norm=fuse_norm)
    h0 = synthetic.activations(M, dims["hidden"], seed=30).to(dev)
    r0 = synthetic.activations(M, dims["hidden"], seed=31).to(dev)
    pos = synthetic.positions(M, seed=32).to(dev)
    # eager reference
    h, r = h0.clone(), r0.clone()
    ref = layer.step(h, r, pos).clone()
    ref_r = r.clone()
    # graph on fixed buffers, refreshed before each replay
    hb, rb = h0.clone(), r0.clone()
    layer.capture(hb, rb, pos)
    for _ in range(3):
        hb.copy_(h0)
        rb.copy_(r0)
        out = layer.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        assert torch.equal(rb, ref_r)
        torch.randn(1000, device=dev).sum().item()   # unrelated eager work between replays


@pytest.mark.parametrize("dims,M", [(CONFIG5, 4), (CONFIG5, 1), (SMALL, 3)])
def test_decoder_step_default_vs_oracle(ops, dev, dims, M):
    """The default step -- add+RMSNorms deferred across the GEMVs where the
    shapes allow (config 5 up to four rows), QK-norm+RoPE and the attention
    stand-in in the QKV GEMV's tail, gelu_and_mul in the gate/up epilogue --
    against the oracle."""
    _say(f"decoder step (default) M={M} {dims}")
    p = synthetic.gemma_layer(seed=16, **dims)
    layer = GemmaDecodeLayer(p, M, dev)
    assert layer.defer_norm == (dims is CONFIG5)
    h = synthetic.activations(M, dims["hidden"], seed=23)
    r = synthetic.activations(M, dims["hidden"], seed=24)
    pos = synthetic.positions(M, seed=25)
    hd, rd = h.to(dev), r.to(dev)
    out = layer.step(hd, rd, pos.to(dev)).clone()
    torch.cuda.synchronize()
    ref_out, ref_r, _ = olayer.decoder_step(p, h, r, pos)
    assert_close_fp(rd.cpu(), ref_r.float(), "residual after the layer")
    assert_close_fp(out.cpu(), ref_out, "layer output")
    nq = dims["n_q"] * dims["head_dim"]
    assert torch.equal(layer.attn, layer.qkv[:, :nq]), "attention stand-in = the rotated q heads"


def test_decoder_step_wide_hidden_runs_undeferred(ops, dev):
    """hidden = 5120 (320 partial sums per row, above what the deferred-norm
    consumers take): the layer keeps the norms as launches and steps
    correctly."""
    M, dims = 2, dict(hidden=5120, n_q=8, n_kv=4, head_dim=128, mlp=2048)
    p = synthetic.gemma_layer(seed=17, **dims)
    layer = GemmaDecodeLayer(p, M, dev)
    assert not layer.defer_norm
    h = synthetic.activations(M, dims["hidden"], seed=26)
    r = synthetic.activations(M, dims["hidden"], seed=27)
    pos = synthetic.positions(M, seed=28)
    hd, rd = h.to(dev), r.to(dev)
    out = layer.step(hd, rd, pos.to(dev)).clone()
    torch.cuda.synchronize()
    ref_out, ref_r, _ = olayer.decoder_step(p, h, r, pos)
    assert_close_fp(rd.cpu(), ref_r.float(), "residual after the layer")
    assert_close_fp(out.cpu(), ref_out, "layer output")


def test_decoder_step_tails_equal_separate_ops(ops, dev):
    """QK-norm+RoPE (and the attention stand-in's copy of q) in the QKV GEMV's
    last workgroup of each head gives the step the separate launches give,
    bit for bit; and the step matches the oracle."""
    M, dims = 4, CONFIG5
    p = synthetic.gemma_layer(seed=13, **dims)
    res = []
    for tails in (True, False):
        layer = GemmaDecodeLayer(p, M, dev, fuse_tails=tails, defer_norm=False)
        assert layer.fuse_tails == tails
        h = synthetic.activations(M, dims["hidden"], seed=50)
        r = synthetic.activations(M, dims["hidden"], seed=51)
        pos = synthetic.positions(M, seed=52)
        hd, rd = h.to(dev), r.to(dev)
        out = layer.step(hd, rd, pos.to(dev)).clone()
        res.append((out, rd.clone(), layer.qkv.clone(), layer.o.clone()))
        del layer
    torch.cuda.synchronize()
    for a, b in zip(*res):
        assert torch.equal(a, b)
    ref_out, ref_r, _ = olayer.decoder_step(p, h, r, pos)
    assert_close_fp(res[0][1].cpu(), ref_r.float(), "residual after the layer")
    assert_close_fp(res[0][0].cpu(), ref_out, "layer output")


@pytest.mark.parametrize("act_fp8", [False, True])
def test_decoder_step_fused_equals_unfused(ops, dev, act_fp8):
    """The fused launches (norm into the GEMV prologue, gelu into the gate/up
    epilogue) give the step the unfused ops give, bit for bit."""
    M, dims = 4, CONFIG5
    p = synthetic.gemma_layer(seed=12, **dims)
    outs = []
    for fuse in (True, False):
        layer = GemmaDecodeLayer(p, M, dev, act_fp8=act_fp8, fuse_glu=fuse, fuse_norm=fuse)
        h = synthetic.activations(M, dims["hidden"], seed=40).to(dev)
        r = synthetic.activations(M, dims["hidden"], seed=41).to(dev)
        outs.append((layer.step(h, r, synthetic.positions(M, seed=42).to(dev)).clone(), r.clone(),
                     layer.act.clone()))
        del layer
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_forward_chains_layers(ops, dev):
    """forward() over two layers (different weights) equals the two steps run
    by hand, the first layer's output feeding the second; capture_forward()
    replays equal the eager forward bit for bit (inputs refreshed before each
    replay, eager work between replays)."""
    from esimd_learning_amd.layer import capture_forward, forward
    M, dims = 4, SMALL
    stack = [GemmaDecodeLayer(synthetic.gemma_layer(seed=s, **dims), M, dev) for s in (14, 15)]
    h0 = synthetic.activations(M, dims["hidden"], seed=60).to(dev)
    r0 = synthetic.activations(M, dims["hidden"], seed=61).to(dev)
    pos = synthetic.positions(M, seed=62).to(dev)
    h, r = h0.clone(), r0.clone()
    ref = stack[1].step(stack[0].step(h, r, pos), r, pos).clone()
    ref_r = r.clone()
    h, r = h0.clone(), r0.clone()
    out = forward(stack, h, r, pos)
    torch.cuda.synchronize()
    assert out.data_ptr() == stack[1].out.data_ptr()
    assert torch.equal(out, ref) and torch.equal(r, ref_r)
    hb, rb = h0.clone(), r0.clone()
    g = capture_forward(stack, hb, rb, pos)
    for _ in range(3):
        hb.copy_(h0)
        rb.copy_(r0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(stack[1].out, ref)
        assert torch.equal(rb, ref_r)
        torch.randn(1000, device=dev).sum().item()
