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
from decode_ref import oracle_step

pytestmark = pytest.mark.gpu

TOL = 1e-4
THREADS = 16
SHAPE = dataclasses.replace(decode.Phi4Shape(), n_layers=2, vocab=20000)


def gqa_gather(qkv, s):
    """Attention output at position 0: head h reads V of kv head h / hpk
    (phi4.rs attention with a single cached position)."""
    v = qkv[s.d_model + s.n_kv_heads * s.head_dim:].reshape(s.n_kv_heads, s.head_dim)
    return np.repeat(v, s.heads_per_kv, axis=0).reshape(-1)


def oracle_token(s, host, logits="f32"):
    d, F = s.d_model, s.ffn_dim
    h = host["x"].astype(np.float64)
    for i in range(s.n_layers):
        L = host[i]
        normed = orc.rms_norm(h.astype(np.float32), L["attn_norm"], s.eps)
        qkv = orc.gemv(rrr_hip.Q5_K, L["attn_qkv"], normed, d, s.qkv_dim, 1, THREADS, f64=True)[0]
        v = gqa_gather(qkv.astype(np.float32), s)
        h = h + orc.gemv(rrr_hip.Q4_K, L["attn_output"], v, d, d, 1, THREADS, f64=True)[0]
        normed = orc.rms_norm(h.astype(np.float32), L["ffn_norm"], s.eps)
        gu = orc.gemv(rrr_hip.Q4_K, L["ffn_up"], normed, d, 2 * F, 1, THREADS, f64=True)[0]
        mid = orc.silu_gate(gu.astype(np.float32), F)
        h = h + orc.gemv(s.down_type(i), L["ffn_down"], mid, F, d, 1, THREADS, f64=True)[0]
    normed = orc.rms_norm(h.astype(np.float32), host["out_norm"], s.eps)
    if logits == "q6k":
        out = orc.gemv(rrr_hip.Q6_K, host["emb_q6k"], normed, d, s.vocab, 1, THREADS, f64=True)[0]
    else:
        out = orc.logits(normed, host["emb"], d, s.vocab, 1, s.chunk, THREADS, f64=True)
    return out, h


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


def test_decode_sweep_persistent_matches_oracle(ctx, sweep):
    """The layers as one persistent launch (its own K split for the down
    GEMVs and its RMSNorm sums from the workgroups' completion records) are
    within the bar of the fp64 composition, the same bits on every run (the
    records' epochs carry over from run to run) and agree with the per-op
    token within the bar."""
    logits0, tok0, hidden0 = sweep.results()
    ref_logits, ref_h = oracle_token(SHAPE, sweep.host)
    sw = ctx.sweep(sweep.sweep_ops())
    try:
        first = None
        for _ in range(3):
            sweep.run_token_sweep(sw)
            sw.check()
            logits, tok, hidden = sweep.results()
            assert np.all(np.isfinite(logits))
            assert orc.normwise_err(hidden, ref_h) < TOL
            assert orc.normwise_err(logits, ref_logits) < TOL
            assert orc.normwise_err(hidden, hidden0.astype(np.float64)) < TOL
            assert tok == int(np.argmax(logits))
            if first is None:
                first = (logits, hidden)
            else:
                assert np.array_equal(logits.view(np.uint32), first[0].view(np.uint32))
                assert np.array_equal(hidden.view(np.uint32), first[1].view(np.uint32))
        # the token with the persistent sweep recorded as a graph: replays
        # (with eager work between them) give the eager bits
        ctx.graph_begin()
        sweep.run_token_sweep(sw)
        g = ctx.graph_end()
        for _ in range(3):
            ctx.fill_u32(sweep.logits, 0)
            ctx.fill_u32(sweep.hidden, 0x7FC00000)
            g.launch()
            ctx.sync()
            logits, tok, hidden = sweep.results()
            assert np.array_equal(logits.view(np.uint32), first[0].view(np.uint32))
            assert np.array_equal(hidden.view(np.uint32), first[1].view(np.uint32))
        g.destroy()
        sw.check()
    finally:
        sw.destroy()


def test_sweep_rejects_other_forms_and_runs_small_shapes(ctx):
    K, N = 3072, 64
    W = ctx.weight_upload(rrr_hip.Q6_K, K, N, synth.weight(1, 1, rrr_hip.Q6_K, K, N))
    W4 = ctx.weight_upload(rrr_hip.Q4_K, K, N, synth.weight(1, 2, rrr_hip.Q4_K, K, N))
    x, g, y = ctx.to_device(synth.normal_f32(1, 3, K)), ctx.to_device(synth.normal_f32(1, 4, K)), ctx.alloc(N * 4)
    try:
        # RMSNorm + Q6_K is not one of the decode layer's forms
        with pytest.raises(rrr_hip.RrrError) as e:
            ctx.sweep([("rmsnorm", x, g, 1e-5, W, rrr_hip.Q6_K, y, K, N)])
        assert e.value.code == rrr_hip.engine.ERR_UNSUPPORTED
        # an RMSNorm op that does not follow the op writing its input
        with pytest.raises(rrr_hip.RrrError) as e:
            ctx.sweep([("rmsnorm", x, g, 1e-5, W4, rrr_hip.Q4_K, y, K, N),
                       ("rmsnorm", x, g, 1e-5, W4, rrr_hip.Q4_K, y, K, N)])
        assert e.value.code == rrr_hip.engine.ERR_UNSUPPORTED
        # one op of 64 rows: one row on each of 64 workgroups, the rest idle
        sw = ctx.sweep([("rmsnorm", x, g, 1e-5, W4, rrr_hip.Q4_K, y, K, N)])
        ref = orc.gemv(rrr_hip.Q4_K, synth.weight(1, 2, rrr_hip.Q4_K, K, N),
                       orc.rms_norm(synth.normal_f32(1, 3, K), synth.normal_f32(1, 4, K), 1e-5), K, N, 1, THREADS,
                       f64=True)[0]
        for _ in range(2):
            ctx.fill_u32(y, 0x7FC00000)
            sw.run()
            sw.check()
            assert orc.normwise_err(ctx.download(y), ref) < TOL
        sw.destroy()
    finally:
        for b in (W, W4, x, g, y):
            b.free()


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
