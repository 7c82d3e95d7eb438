"""GPU parity of the decode weight sweep (one token through the C ABI) against
the oracle composed in fp64, on a reduced Phi-4-mini shape: full layer
widths, 2 layers (one Q6_K and one Q4_K FFN-down), 20,000-entry vocab in
three transposed chunks (the last one partial).

Bars: logits and final hidden state within 1e-4 normwise relative error of
the fp64 composition (TOL); the GPU argmax is the first index of the maximum
of the GPU logits and agrees with the oracle's when the oracle's top two are
separated by more than the tolerance; graph replays are bitwise equal to the
eager run.
"""
import dataclasses

import numpy as np
import pytest

import oracle.oracle as orc
import rrr_hip
from rrr_hip import decode, synth
from decode_ref import gqa_gather, oracle_step, oracle_token

pytestmark = pytest.mark.gpu

TOL = 1e-4
THREADS = 16
SHAPE = dataclasses.replace(decode.Phi4Shape(), n_layers=2, vocab=20000)


@pytest.fixture(scope="module")
def sweep(ctx):
    sw = decode.DecodeSweep(ctx, SHAPE, seed=3, keep_host=True)
    sw.record_token()
    ctx.sync()
    yield sw


def test_decode_token_matches_oracle(sweep):
    logits, tok, hidden = sweep.results()
    ref_logits, ref_h = oracle_token(SHAPE, sweep.host)
    assert np.all(np.isfinite(logits))
    assert orc.normwise_err(hidden, ref_h) < TOL
    assert orc.normwise_err(logits, ref_logits) < TOL
    assert tok == int(np.argmax(logits))
    top2 = np.sort(ref_logits)[-2:]
    if top2[1] - top2[0] > TOL * np.max(np.abs(ref_logits)):
        assert tok == int(np.argmax(ref_logits))


def test_decode_token_q6k_logits_matches_oracle(ctx, sweep):
    """Logits from the raw Q6_K token_embd: the layers give the same bits as
    the F32-logits token, the logits match the fp64 dot over dequant_q6_k of
    the rows, and a graph of the token replays bitwise."""
    sw = decode.DecodeSweep(ctx, SHAPE, seed=3, keep_host=True, logits="q6k")
    sw.record_token()
    ctx.sync()
    logits, tok, hidden = sw.results()
    ref_logits, ref_h = oracle_token(SHAPE, sw.host, logits="q6k")
    assert np.array_equal(hidden.view(np.uint32), sweep.results()[2].view(np.uint32))
    assert np.all(np.isfinite(logits))
    assert orc.normwise_err(logits, ref_logits) < TOL
    assert tok == int(np.argmax(logits))
    top2 = np.sort(ref_logits)[-2:]
    if top2[1] - top2[0] > TOL * np.max(np.abs(ref_logits)):
        assert tok == int(np.argmax(ref_logits))
    g = sw.graph()
    for _ in range(2):
        ctx.fill_u32(sw.logits, 0)
        g.launch()
        ctx.sync()
        assert np.array_equal(sw.results()[0].view(np.uint32), logits.view(np.uint32))
    g.destroy()


def test_decode_silu_fused_is_bitwise_the_two_launch_form(ctx, sweep):
    """silu(gate) * up in the gate/up GEMV's epilogue (rrr_gemv_rmsnorm_silu,
    the default) and in the down GEMV's prologue (the 2F gate/up rows kept)
    give the same token bit for bit."""
    logits0, tok0, hidden0 = sweep.results()
    assert sweep.silu_fused
    sweep.silu_fused = False
    try:
        sweep.record_token()
        ctx.sync()
    finally:
        sweep.silu_fused = True
    logits, tok, hidden = sweep.results()
    assert tok == tok0
    assert np.array_equal(hidden.view(np.uint32), hidden0.view(np.uint32))
    assert np.array_equal(logits.view(np.uint32), logits0.view(np.uint32))


def test_decode_graph_replay_matches_eager(ctx, sweep):
    logits0, tok0, hidden0 = sweep.results()
    g = sweep.graph()
    for _ in range(3):
        g.launch()
        ctx.sync()
        logits, tok, hidden = sweep.results()
        assert tok == tok0
        assert np.array_equal(logits.view(np.uint32), logits0.view(np.uint32))
        assert np.array_equal(hidden.view(np.uint32), hidden0.view(np.uint32))
    g.destroy()


# ---- the full decode step with RoPE, the f16 KV caches and attention ----------

SHAPE_ATT = dataclasses.replace(SHAPE, max_seq=16)
ATT_POSITIONS = [0, 1, 2, 3, 4]


def test_decode_steps_with_attention_match_oracle(ctx):
    """Positions 0..4 in order: each step writes its cache row and attends
    over all rows so far, in the GPU sweep and in the oracle."""
    s = SHAPE_ATT
    sw = decode.DecodeSweep(ctx, s, seed=3, keep_host=True, attention=True)
    caches = [(np.zeros(s.max_seq * s.kv_stride, np.uint16), np.zeros(s.max_seq * s.kv_stride, np.uint16))
              for _ in range(s.n_layers)]
    for pos in ATT_POSITIONS:
        sw.record_token(pos)
        ctx.sync()
        logits, tok, hidden = sw.results()
        ref_logits, ref_h = oracle_step(s, sw.host, caches, pos)
        assert np.all(np.isfinite(logits))
        assert orc.normwise_err(hidden, ref_h) < TOL, pos
        assert orc.normwise_err(logits, ref_logits) < TOL, pos
        assert tok == int(np.argmax(logits))
    # the cache rows written so far hold each position's V (from the GEMV, so
    # equal to the oracle's within the tolerance and one f16 rounding)
    kc, vc = sw.kv[0]
    n = len(ATT_POSITIONS) * s.kv_stride
    vg = ctx.download(vc, np.uint16, n).view(np.float16).astype(np.float64)
    vo = caches[0][1][:n].view(np.float16).astype(np.float64)
    assert np.all(np.abs(vg - vo) <= TOL * np.max(np.abs(vo)) + np.abs(vo) * 2.0 ** -10)
    # a graph of the step at the last position replays bitwise (its cache
    # row is rewritten with the same values)
    logits0, tok0, hidden0 = sw.results()
    g = sw.graph(ATT_POSITIONS[-1])
    for _ in range(3):
        g.launch()
        ctx.sync()
        logits, tok, hidden = sw.results()
        assert np.array_equal(logits.view(np.uint32), logits0.view(np.uint32))
        assert np.array_equal(hidden.view(np.uint32), hidden0.view(np.uint32))
    g.destroy()
    # rope_kv_store in the QKV GEMV's epilogue (the default) and as its own
    # launch give the same step bit for bit
    assert sw.rope_fused
    sw.rope_fused = False
    try:
        sw.record_token(ATT_POSITIONS[-1])
        ctx.sync()
    finally:
        sw.rope_fused = True
    logits, tok, hidden = sw.results()
    assert np.array_equal(logits.view(np.uint32), logits0.view(np.uint32))
    assert np.array_equal(hidden.view(np.uint32), hidden0.view(np.uint32))
    with pytest.raises(ValueError):
        sw.record_token(s.max_seq)
