"""Batch-1 GEMV parity on activations with outliers.

The int8-matrix-core GEMV writes each 16-element group of the activation
vector in block floating point relative to the group's largest magnitude M
(20-bit fixed point: every element carries an absolute error of at most
M * 2^-20), so an element next to an outlier keeps few of its own bits.
The bar stays the GEMV bar, 1e-4 normwise against the fp64 oracle: an
output's error is a sum of such per-element errors times weights, while
the output itself carries the outliers' contributions.

Inputs:
- synthetic: N(0, 1) with one element of every 16-group replaced by
  +-10^u, u uniform in [3, 4] (1e3..1e4 times the rest), at the config
  shapes of every weight type, plain, fused RMSNorm, fused silu * up and
  batched (4 token rows);
- from the model: gate/up of the last of 8 Phi-4-mini-shaped random-init
  layers (the hidden state grows by orders of magnitude layer by layer, to
  silu * up of order 1e7), through the Q4_K and Q6_K down GEMVs, plain and
  fused.
"""
import dataclasses

import numpy as np
import pytest

import oracle.oracle as orc
import rrr_hip
from rrr_hip import decode, synth

pytestmark = pytest.mark.gpu

TOL = 1e-4
THREADS = 16


def outliers(seed, n, lo=3.0, hi=4.0):
    """N(0, 1) with one element of every 16-group at +-10^U(lo, hi)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(n).astype(np.float32)
    g = n // 16
    pos = np.arange(g) * 16 + rng.integers(0, 16, g)
    x[pos] = (rng.choice([-1.0, 1.0], g) * 10.0 ** rng.uniform(lo, hi, g)).astype(np.float32)
    return x


SHAPES = [(12, 3072, 3072), (13, 3072, 5120), (14, 8192, 3072), (12, 8192, 3072), (12, 3072, 16384),
          (14, 3072, 200)]


@pytest.mark.parametrize("qtype,K,N", SHAPES)
def test_gemv_outlier_activations(ctx, qtype, K, N):
    raw = synth.weight(21, qtype, qtype, K, N)
    x = outliers(100 + qtype + K, K)
    W = ctx.weight_upload(qtype, K, N, raw)
    xb, yb = ctx.to_device(x), ctx.alloc(N * 4)
    ctx.gemv(xb, W, qtype, yb, K, N)
    ref = orc.gemv(qtype, raw, x, K, N, 1, THREADS, f64=True)[0]
    assert orc.normwise_err(ctx.download(yb), ref) < TOL
    # the outliers carry most of the output, but a kernel that lost the
    # small elements next to them would miss the bar: their share is above it
    xs = x.copy()
    xs[np.abs(xs) > 100] = 0
    ref_small = orc.gemv(qtype, raw, xs, K, N, 1, THREADS, f64=True)[0]
    assert np.max(np.abs(ref_small)) > 2 * TOL * np.max(np.abs(ref))
    W.free(); xb.free(); yb.free()


@pytest.mark.parametrize("qtype,K,N", [(13, 3072, 5120), (12, 3072, 16384), (14, 3072, 300)])
def test_gemv_rmsnorm_outliers(ctx, qtype, K, N):
    raw = synth.weight(22, qtype, qtype, K, N)
    x = outliers(200 + qtype, K)
    g = synth.normal_f32(22, 2, K, 1.0, 0.1)
    W = ctx.weight_upload(qtype, K, N, raw)
    xb, gb, yb = ctx.to_device(x), ctx.to_device(g), ctx.alloc(N * 4)
    ctx.gemv_rmsnorm(xb, gb, 1e-5, W, qtype, yb, K, N)
    ref = orc.gemv(qtype, raw, orc.rms_norm(x, g), K, N, 1, THREADS, f64=True)[0]
    assert orc.normwise_err(ctx.download(yb), ref) < TOL
    for b in (W, xb, gb, yb):
        b.free()


@pytest.mark.parametrize("qtype", [12, 14])
@pytest.mark.parametrize("where", ["gate", "up", "both"])
def test_gemv_silu_gate_outliers(ctx, qtype, where):
    F, N = 8192, 3072
    raw = synth.weight(23, qtype, qtype, F, N)
    rng = np.random.default_rng(300 + qtype)
    gate = outliers(301, F) if where in ("gate", "both") else rng.standard_normal(F).astype(np.float32)
    up = outliers(302, F) if where in ("up", "both") else rng.standard_normal(F).astype(np.float32)
    gu = np.concatenate([gate, up])
    h = synth.normal_f32(23, 3, N, 0.0, 10.0)
    W = ctx.weight_upload(qtype, F, N, raw)
    gub, hb = ctx.to_device(gu), ctx.to_device(h)
    ctx.gemv_residual(gub, rrr_hip.ACT_SILU_GATE, 0, W, qtype, hb, F, N)
    mid = orc.silu_gate(gu, F)
    ref = h.astype(np.float64) + orc.gemv(qtype, raw, mid, F, N, 1, THREADS, f64=True)[0]
    assert orc.normwise_err(ctx.download(hb), ref) < TOL
    for b in (W, gub, hb):
        b.free()


@pytest.mark.parametrize("qtype,K,N", [(12, 3072, 16384), (13, 3072, 5120)])
def test_batched_gemv_outliers(ctx, qtype, K, N):
    M = 4
    raw = synth.weight(24, qtype, qtype, K, N)
    X = np.concatenate([outliers(400 + m, K) for m in range(M)])
    W = ctx.weight_upload(qtype, K, N, raw)
    Xb, Yb = ctx.to_device(X), ctx.alloc(M * N * 4)
    ctx.gemv(Xb, W, qtype, Yb, K, N, M)
    Y = ctx.download(Yb).reshape(M, N)
    ref = orc.gemv(qtype, raw, X, K, N, M, THREADS, f64=True)
    for m in range(M):
        assert orc.normwise_err(Y[m], ref[m]) < TOL, m
    W.free(); Xb.free(); Yb.free()


@pytest.fixture(scope="module")
def deep_gate_up(ctx):
    """gate/up (f32, 2 x 8192) of layer 7 of an 8-layer Phi-4-mini-shaped
    random-init model after one token, and the final hidden state."""
    s = dataclasses.replace(decode.Phi4Shape(), n_layers=8, vocab=256, chunk=256)
    sw = decode.DecodeSweep(ctx, s, seed=3)
    sw.silu_fused = False   # keeps the 2F gate/up rows in sw.gate_up
    sw.record_token()
    ctx.sync()
    gu = ctx.download(sw.gate_up, np.float32, 2 * s.ffn_dim)
    hidden = ctx.download(sw.hidden, np.float32, s.d_model)
    del sw
    return gu, hidden


def test_deep_layer_activations_are_large(deep_gate_up):
    gu, hidden = deep_gate_up
    assert np.all(np.isfinite(gu)) and np.all(np.isfinite(hidden))
    mid = orc.silu_gate(gu, 8192)
    # the random-init hidden state drifts upward layer by layer: by layer 8
    # silu * up is of order 1e7 (a first layer's is of order 1)
    assert np.median(np.abs(mid)) > 1e5


@pytest.mark.parametrize("qtype", [12, 14])
def test_down_gemv_on_deep_layer_activations(ctx, deep_gate_up, qtype):
    gu, _ = deep_gate_up
    F, N = 8192, 3072
    raw = synth.weight(25, qtype, qtype, F, N)
    mid = orc.silu_gate(gu, F)
    W = ctx.weight_upload(qtype, F, N, raw)
    mb, yb = ctx.to_device(mid), ctx.alloc(N * 4)
    ctx.gemv(mb, W, qtype, yb, F, N)
    ref = orc.gemv(qtype, raw, mid, F, N, 1, THREADS, f64=True)[0]
    assert orc.normwise_err(ctx.download(yb), ref) < TOL
    # fused silu * up + residual on the raw gate/up
    gub, hb = ctx.to_device(gu), ctx.to_device(np.zeros(N, np.float32))
    ctx.gemv_residual(gub, rrr_hip.ACT_SILU_GATE, 0, W, qtype, hb, F, N)
    assert orc.normwise_err(ctx.download(hb), ref) < TOL
    for b in (W, mb, yb, gub, hb):
        b.free()
