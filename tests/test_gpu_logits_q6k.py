"""GPU parity of the logits on the raw Q6_K token_embd (RRR_LOGITS_Q6K)
against the oracle.

The reference builds its F32 logits matrix by dequantizing the tied
token_embd (phi4.rs:709, :866-893), so logits read from the raw Q6_K rows are
the same dot products over the same values: the bar is the GEMV bar, 1e-4
normwise relative error against the fp64 dot of x with dequant_q6_k of each
row (the oracle's Q6_K GEMV).  The F32 row layout over the oracle's
dequantized matrix is held to the same bar, and the two argmaxes agree when
the fp64 top two are farther apart than the tolerance.  RMSNorm folded into
the launch is bit-identical to rrr_rmsnorm followed by the unfused logits.
"""
import numpy as np
import pytest

import oracle.oracle as orc
import rrr_hip
from rrr_hip import synth

pytestmark = pytest.mark.gpu

TOL = 1e-4
THREADS = 16
K = 3072


def case(V, seed):
    raw = synth.weight(seed, 40, rrr_hip.Q6_K, K, V)
    x = synth.normal_f32(seed, 41, K)
    gamma = synth.normal_f32(seed, 42, K, 1.0, 0.1)
    return raw, x, gamma


def separated(ref):
    top2 = np.sort(ref)[-2:]
    return top2[1] - top2[0] > TOL * np.max(np.abs(ref))


@pytest.mark.parametrize("V", [16, 77, 1007, 20000])
def test_q6k_logits_parity(ctx, V):
    raw, x, gamma = case(V, 5)
    Eb = ctx.weight_upload(rrr_hip.Q6_K, K, V, raw)
    xb, gb, yb = ctx.to_device(x), ctx.to_device(gamma), ctx.alloc(V * 4)
    ctx.logits_f32(xb, Eb, yb, K, V, rrr_hip.LOGITS_Q6K, 0)
    ref = orc.gemv(rrr_hip.Q6_K, raw, x, K, V, 1, THREADS, f64=True)[0]
    assert orc.normwise_err(ctx.download(yb), ref) < TOL
    # fused RMSNorm: within the bar of the fp64 composition, and bitwise the
    # unfused rmsnorm -> logits sequence
    ctx.logits_rmsnorm(xb, gb, 1e-5, Eb, yb, K, V, rrr_hip.LOGITS_Q6K, 0)
    fused = ctx.download(yb)
    normed = orc.rms_norm(x, gamma, 1e-5)
    assert orc.normwise_err(fused, orc.gemv(rrr_hip.Q6_K, raw, normed, K, V, 1, THREADS, f64=True)[0]) < TOL
    nb = ctx.alloc(K * 4)
    ctx.rmsnorm(xb, gb, nb, 1, K, 1e-5)
    ctx.logits_f32(nb, Eb, yb, K, V, rrr_hip.LOGITS_Q6K, 0)
    assert np.array_equal(ctx.download(yb).view(np.uint32), fused.view(np.uint32))
    for b in (Eb, xb, gb, yb, nb):
        b.free()


def test_q6k_logits_equal_f32_logits_of_dequantized_matrix(ctx):
    """The same logits from the raw rows and from their F32 expansion (the
    reference's route): both within the bar, same argmax."""
    V = 8192
    raw, x, _ = case(V, 6)
    E = orc.dequant(rrr_hip.Q6_K, raw, V * K)                 # exact f32 values of dequant_q6_k
    ref = orc.gemv(rrr_hip.Q6_K, raw, x, K, V, 1, THREADS, f64=True)[0]
    Eq, Ef = ctx.weight_upload(rrr_hip.Q6_K, K, V, raw), ctx.to_device(E)
    xb, yq, yf = ctx.to_device(x), ctx.alloc(V * 4), ctx.alloc(V * 4)
    ctx.logits_f32(xb, Eq, yq, K, V, rrr_hip.LOGITS_Q6K, 0)
    ctx.logits_f32(xb, Ef, yf, K, V, rrr_hip.LOGITS_ROWS)
    q, f = ctx.download(yq), ctx.download(yf)
    assert orc.normwise_err(q, ref) < TOL and orc.normwise_err(f, ref) < TOL
    assert orc.normwise_err(q, f) < 2 * TOL
    if separated(ref):
        assert int(np.argmax(q)) == int(np.argmax(f)) == int(np.argmax(ref))
    for b in (Eq, Ef, xb, yq, yf):
        b.free()


def test_q6k_logits_full_vocab(ctx):
    """The Phi-4-mini vocabulary, 200,064 rows (504 MB of Q6_K): logits and
    the GPU argmax against the fp64 oracle."""
    V = 200064
    raw, x, gamma = case(V, 7)
    Eb = ctx.weight_upload(rrr_hip.Q6_K, K, V, raw)
    xb, gb, yb, ob = ctx.to_device(x), ctx.to_device(gamma), ctx.alloc(V * 4), ctx.alloc(4)
    ctx.logits_rmsnorm(xb, gb, 1e-5, Eb, yb, K, V, rrr_hip.LOGITS_Q6K, 0)
    ctx.argmax_f32(yb, V, ob)
    got = ctx.download(yb)
    ref = orc.gemv(rrr_hip.Q6_K, raw, orc.rms_norm(x, gamma, 1e-5), K, V, 1, THREADS, f64=True)[0]
    assert orc.normwise_err(got, ref) < TOL
    tok = int(ctx.download(ob, np.uint32, 1)[0])
    assert tok == int(np.argmax(got))
    if separated(ref):
        assert tok == int(np.argmax(ref))
    for b in (Eb, xb, gb, yb, ob):
        b.free()
