"""GPU parity of the prefill path (forward_prefill_batched, phi4.rs:1200-1445,
with every step on the GPU) against the oracle.

Bars.
- RoPE + KV store of `rows` tokens: each row as the single-token op (V rows
  bit-exact, Q/K within the f32-angle bound of the decode tests), and the
  same bits as `rows` single-token launches.
- Causal prefill attention, f32 output, against the fp64 attention of each
  token over cache rows 0 .. pos0 + t: the matrix-core form (up to 4 query
  heads per KV head) at the MFMA bar, 2e-3 (measured with Q and P in f16
  hi + lo: median 4e-7 per token, worst 1.1e-4 at 2,029 rows, isolated
  elements), the VALU form (more heads per KV head) at 1e-4; the f16 output
  is the f32 result rounded to nearest even (bitwise).
- f16-activation GEMM: the MFMA bar, 2e-3 normwise against the fp64 product
  of the same f16 inputs with the exact dequantized weights (the kernel
  rounds the weights to f16 tiles), with and without K split over
  workgroups; the accumulate form adds its result to Y in f32 (bitwise Y0 +
  product); with inputs exact in both bf16 and f16 it gives the bits of the
  bf16-input GEMM.
- RMSNorm with f16 output: the f32 kernel's results rounded to nearest even
  (bitwise); silu_gate in f16 block floating point: the f32 kernel's results
  times the row's power of two 2^(15 - e) (max = f * 2^e), rounded to nearest
  even (bitwise), the row scale 2^(e - 15); the GEMM with row scales gives the
  unscaled GEMM's rows times them (bitwise).
- The composed prefill (2 layers, 20,000-entry vocab): the oracle composes
  the same steps in fp64 with the GEMM inputs rounded to f16 as the GPU does
  (the path's stated activation precision), so what is left is the MFMA
  kernels' f16 weight tiles: hidden rows, cached K/V and the last token's
  logits within the MFMA bar, 2e-3 normwise; a graph replay is bitwise the
  eager run.
"""
import dataclasses

import numpy as np
import pytest

import oracle.oracle as orc
import rrr_hip
from rrr_hip import decode, synth

pytestmark = pytest.mark.gpu

TOL, MFMA_TOL = 1e-4, 2e-3
THREADS = 16
NH, NKV, HD, RD = 24, 8, 128, 96
QD, KVS = NH * HD, NKV * HD
ROW = QD + 2 * KVS
MAX_SEQ = 2048
SHAPE = dataclasses.replace(decode.Phi4Shape(), n_layers=2, vocab=20000)


def f16r(x):
    """Round to f16 (nearest even) and back to f32."""
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def rope_bound(pos):
    return 4.0 * pos * 2.0 ** -24 + 1e-6


def factors(seed=3):
    return (1.0 + np.random.default_rng(seed).uniform(0.0, 3.0, RD // 2)).astype(np.float32)


@pytest.fixture(scope="module")
def caches(ctx):
    kc = ctx.alloc(MAX_SEQ * KVS * 2)
    vc = ctx.alloc(MAX_SEQ * KVS * 2)
    yield kc, vc
    kc.free(); vc.free()


@pytest.mark.parametrize("pos0,rows", [(0, 1), (0, 7), (100, 37), (2000, 48)])
def test_rope_kv_store_rows(ctx, caches, pos0, rows):
    kc, vc = caches
    rng = np.random.default_rng(pos0 + rows)
    qkv = rng.standard_normal((rows, ROW)).astype(np.float32)
    fac = factors()
    d_fac = ctx.to_device(fac)
    a = ctx.to_device(qkv)
    ctx.fill_u32(kc, 0x5A5A5A5A)
    ctx.fill_u32(vc, 0x5A5A5A5A)
    ctx.rope_kv_store_rows(a, rows, d_fac, RD // 2, kc, vc, pos0, NH, NKV, HD, RD, QD, KVS)
    got = ctx.download(a, np.float32, rows * ROW).reshape(rows, ROW)
    lo, hi = max(0, pos0 - 1), min(MAX_SEQ, pos0 + rows + 1)
    kg = ctx.download(kc, np.uint16, (hi - lo) * KVS, offset=lo * KVS * 2).reshape(hi - lo, KVS)
    vg = ctx.download(vc, np.uint16, (hi - lo) * KVS, offset=lo * KVS * 2).reshape(hi - lo, KVS)
    for t in range(rows):
        pos = pos0 + t
        ref, kref, vref = orc.rope_kv_store(qkv[t], np.zeros((pos + 1) * KVS, np.uint16),
                                            np.zeros((pos + 1) * KVS, np.uint16), pos, NH, NKV, HD, RD, factors=fac)
        r = pos - lo
        assert np.array_equal(vg[r], vref[pos * KVS:])
        assert np.array_equal(kg[r], orc.f32_to_f16_bits(got[t, QD:QD + KVS]))
        if pos == 0:
            assert np.array_equal(got[t], ref)
        else:
            assert orc.normwise_err(got[t, :QD], ref[:QD]) < rope_bound(pos)
            assert orc.normwise_err(got[t, QD:QD + KVS], ref[QD:QD + KVS]) < rope_bound(pos)
    for r in range(hi - lo):   # rows outside the prompt untouched
        if not pos0 <= lo + r < pos0 + rows:
            assert np.all(kg[r] == 0x5A5A) and np.all(vg[r] == 0x5A5A)
    # the same bits as one single-token launch per row
    b = ctx.to_device(qkv)
    for t in range(rows):
        v = ctx.view(b, t * ROW * 4, ROW * 4)
        ctx.rope_kv_store(v, d_fac, RD // 2, kc, vc, pos0 + t, NH, NKV, HD, RD, QD, KVS)
        v.free()
    assert np.array_equal(ctx.download(b, np.float32, rows * ROW).reshape(rows, ROW), got)
    kg2 = ctx.download(kc, np.uint16, (hi - lo) * KVS, offset=lo * KVS * 2).reshape(hi - lo, KVS)
    assert np.array_equal(kg2, kg)
    for buf in (a, b, d_fac):
        buf.free()


# (9, 40) and (25, 70): blocks of 32 cache rows that start past some of a
# workgroup's tokens (a wave whose first block holds none of a token's keys).
# Up to 256 workgroups of one query head each cover the short prompts; (0,
# 200, 8, 3), (7, 400, 8, 2) and (0, 300, 4, 4) take the grouped form (a
# workgroup per KV head's query heads)
@pytest.mark.parametrize("pos0,rows,nkv,hpk", [(0, 1, 8, 3), (0, 130, 8, 3), (100, 37, 8, 3), (2000, 48, 8, 3),
                                               (0, 64, 2, 8), (5, 20, 1, 1), (9, 40, 8, 3), (25, 70, 8, 3),
                                               (0, 200, 8, 3), (7, 400, 8, 2), (0, 300, 4, 4)])
def test_attention_prefill_parity(ctx, caches, pos0, rows, nkv, hpk):
    kc, vc = caches
    rng = np.random.default_rng(pos0 * 7 + rows + nkv * hpk)
    seq = pos0 + rows
    k = orc.f32_to_f16_bits(rng.standard_normal(seq * nkv * HD).astype(np.float32))
    v = orc.f32_to_f16_bits(rng.standard_normal(seq * nkv * HD).astype(np.float32))
    ctx.upload(kc, k)
    ctx.upload(vc, v)
    qd = nkv * hpk * HD
    row = qd + 2 * nkv * HD
    qkv = rng.standard_normal((rows, row)).astype(np.float32)
    dq = ctx.to_device(qkv)
    o32, o16 = ctx.alloc(rows * qd * 4), ctx.alloc(rows * qd * 2)
    ctx.attention_prefill(dq, rows, kc, vc, o32, pos0, nkv, hpk, HD)
    ctx.attention_prefill(dq, rows, kc, vc, o16, pos0, nkv, hpk, HD, out_type=rrr_hip.F16)
    got = ctx.download(o32, np.float32, rows * qd).reshape(rows, qd)
    bar = MFMA_TOL if hpk <= 4 else TOL
    errs = []
    for t in range(rows):
        ref = orc.attention_f64(qkv[t, :qd], k, v, pos0 + t + 1, nkv, hpk, HD)
        errs.append(orc.normwise_err(got[t], ref))
        assert errs[-1] < bar, t
    assert np.median(errs) < 1e-5
    h = ctx.download(o16, np.uint16, rows * qd).reshape(rows, qd)
    assert np.array_equal(h, got.astype(np.float16).view(np.uint16))
    for b in (dq, o32, o16):
        b.free()


# the last three split K (too few 256 x 128 tiles at a 512-token prompt)
def test_attention_prefill_large_queries(ctx, caches):
    """Queries of ~4e4 (a random-init model reaches 3.3e4 by its eighth
    layer): the matrix-core form scales each token's query by a power of two
    before its f16 split, so nothing overflows."""
    kc, vc = caches
    pos0, rows, nkv, hpk = 0, 40, 8, 3
    rng = np.random.default_rng(11)
    k = orc.f32_to_f16_bits((rng.standard_normal(rows * nkv * HD) * 0.01).astype(np.float32))
    v = orc.f32_to_f16_bits((rng.standard_normal(rows * nkv * HD) * 5e3).astype(np.float32))   # within f16
    ctx.upload(kc, k)
    ctx.upload(vc, v)
    qd = nkv * hpk * HD
    qkv = (rng.standard_normal((rows, qd + 2 * nkv * HD)) * 4e4).astype(np.float32)
    dq, o32 = ctx.to_device(qkv), ctx.alloc(rows * qd * 4)
    ctx.attention_prefill(dq, rows, kc, vc, o32, pos0, nkv, hpk, HD)
    got = ctx.download(o32, np.float32, rows * qd).reshape(rows, qd)
    assert np.all(np.isfinite(got))
    for t in range(rows):
        ref = orc.attention_f64(qkv[t, :qd], k, v, pos0 + t + 1, nkv, hpk, HD)
        assert orc.normwise_err(got[t], ref) < MFMA_TOL, t
    dq.free(); o32.free()


@pytest.mark.parametrize("qtype,K,N,M", [(rrr_hip.Q5_K, 3072, 5120, 128), (rrr_hip.Q4_K, 3072, 16384, 256),
                                         (rrr_hip.Q6_K, 8192, 3072, 128), (rrr_hip.Q4_K, 3072, 3072, 384),
                                         (rrr_hip.Q4_K, 3072, 3072, 512), (rrr_hip.Q5_K, 3072, 5120, 512),
                                         (rrr_hip.Q6_K, 8192, 3072, 512)])
def test_gemm_f16_parity(ctx, qtype, K, N, M):
    raw = synth.weight(4, 50 + qtype, qtype, K, N)
    X = f16r(synth.normal_f32(4, 51, M * K).reshape(M, K))
    Y0 = synth.normal_f32(4, 52, M * N).reshape(M, N)
    W = ctx.weight_upload(qtype, K, N, raw)
    xb = ctx.to_device(X.astype(np.float16).view(np.uint16))
    yb, ya = ctx.alloc(M * N * 4), ctx.to_device(Y0)
    ctx.gemm_f16(xb, W, qtype, yb, K, N, M)
    ctx.gemm_f16(xb, W, qtype, ya, K, N, M, accumulate=True)
    got = ctx.download(yb, np.float32, M * N).reshape(M, N)
    ref = orc.gemv(qtype, raw, X, K, N, M, THREADS, f64=True)
    assert orc.normwise_err(got, ref) < MFMA_TOL
    assert max(orc.normwise_err(got[m], ref[m]) for m in range(M)) < 4 * MFMA_TOL
    acc = ctx.download(ya, np.float32, M * N).reshape(M, N)
    assert np.array_equal(acc.view(np.uint32), (Y0 + got).view(np.uint32))
    for b in (W, xb, yb, ya):
        b.free()


def test_gemm_f16_equals_bf16_on_common_values(ctx):
    """Inputs exact in both bf16 and f16 (8 significant bits, exponents
    inside f16's normal range) reach the MFMA as the same f16 tiles."""
    qtype, K, N, M = rrr_hip.Q4_K, 3072, 3072, 128
    raw = synth.weight(5, 60, qtype, K, N)
    X = synth.normal_f32(5, 61, M * K).reshape(M, K)
    X = (X.view(np.uint32) & 0xFFFF0000).view(np.float32)              # bf16 values
    X[np.abs(X) < 2.0 ** -14] = 0.0
    assert np.array_equal(X.astype(np.float16).astype(np.float32), X)
    W = ctx.weight_upload(qtype, K, N, raw)
    xh = ctx.to_device(X.astype(np.float16).view(np.uint16))
    xbf = ctx.to_device((X.view(np.uint32) >> 16).astype(np.uint16))
    y1, y2 = ctx.alloc(M * N * 4), ctx.alloc(M * N * 4)
    ctx.gemm_f16(xh, W, qtype, y1, K, N, M)
    ctx.gemm_bf16(xbf, W, qtype, y2, K, N, M)
    assert np.array_equal(ctx.download(y1, np.uint32, M * N), ctx.download(y2, np.uint32, M * N))
    for b in (W, xh, xbf, y1, y2):
        b.free()


def block_f16(v):
    """Rows of f32 values in f16 block floating point: (f16 values of v * 2^(15 - e),
    row scales 2^(e - 15)) with max|v| = f * 2^e, f in [0.5, 1)."""
    v = np.asarray(v, np.float32)
    m = np.max(np.abs(v), axis=1)
    e = np.where((m > 0) & np.isfinite(m), np.frexp(m)[1], 15)
    sc = np.ldexp(np.float32(1.0), 15 - e).astype(np.float32)
    return (v * sc[:, None]).astype(np.float16), np.ldexp(np.float32(1.0), e - 15).astype(np.float32)


@pytest.mark.parametrize("rows,F", [(130, 8192), (12, 1000), (12, 1002), (12, 9000)])
def test_rmsnorm_and_silu_gate_f16(ctx, rows, F):
    """F = 8192 and 1000: the register form with 16-byte loads (a partial
    last pass at 1000); 1002 and 9000: the general form."""
    d = 3072
    x = synth.normal_f32(6, 70, rows * d)
    g = synth.normal_f32(6, 71, d, 1.0, 0.1)
    gu = synth.normal_f32(6, 72, rows * 2 * F, 0.0, 2.0)
    gu[2 * F * 7:2 * F * 8] *= 1e4                 # a row far past f16's range
    gu[2 * F * 9:2 * F * 10] = 0.0                 # and an all-zero row
    xb, gb, gub = ctx.to_device(x), ctx.to_device(g), ctx.to_device(gu)
    y32, y16 = ctx.alloc(rows * d * 4), ctx.alloc(rows * d * 2)
    m32, m16, rs = ctx.alloc(rows * F * 4), ctx.alloc(rows * F * 2), ctx.alloc(rows * 4)
    ctx.rmsnorm(xb, gb, y32, rows, d, 1e-5)
    ctx.rmsnorm_f16(xb, gb, y16, rows, d, 1e-5)
    ctx.silu_gate(gub, m32, rows, F)
    ctx.silu_gate_f16(gub, m16, rs, rows, F)
    assert np.array_equal(ctx.download(y16, np.uint16, rows * d),
                          ctx.download(y32, np.float32, rows * d).astype(np.float16).view(np.uint16))
    h, scale = block_f16(ctx.download(m32, np.float32, rows * F).reshape(rows, F))
    assert np.array_equal(ctx.download(m16, np.uint16, rows * F).reshape(rows, F), h.view(np.uint16))
    assert np.array_equal(ctx.download(rs, np.float32, rows), scale)
    assert np.all(np.isfinite(h.astype(np.float32)))
    for b in (xb, gb, gub, y32, y16, m32, m16, rs):
        b.free()


@pytest.mark.parametrize("M", [128, 512])
def test_gemm_f16_row_scale(ctx, M):
    qtype, K, N = rrr_hip.Q6_K, 8192, 3072
    raw = synth.weight(7, 80, qtype, K, N)
    X = f16r(synth.normal_f32(7, 81, M * K).reshape(M, K))
    rs = np.ldexp(np.float32(1.0), np.random.default_rng(7).integers(-20, 20, M)).astype(np.float32)
    W = ctx.weight_upload(qtype, K, N, raw)
    xb, rb = ctx.to_device(X.astype(np.float16).view(np.uint16)), ctx.to_device(rs)
    y1, y2 = ctx.alloc(M * N * 4), ctx.alloc(M * N * 4)
    ctx.gemm_f16(xb, W, qtype, y1, K, N, M)
    ctx.gemm_f16(xb, W, qtype, y2, K, N, M, row_scale=rb)
    a = ctx.download(y1, np.float32, M * N).reshape(M, N)
    assert np.array_equal(ctx.download(y2, np.float32, M * N).reshape(M, N).view(np.uint32),
                          (a * rs[:, None]).view(np.uint32))
    # and added to Y, as the prefill's down projection does
    Y0 = synth.normal_f32(7, 82, M * N).reshape(M, N)
    ctx.upload(y2, Y0)
    ctx.gemm_f16(xb, W, qtype, y2, K, N, M, accumulate=True, row_scale=rb)
    assert np.array_equal(ctx.download(y2, np.float32, M * N).reshape(M, N).view(np.uint32),
                          (Y0 + a * rs[:, None]).view(np.uint32))
    for b in (W, xb, rb, y1, y2):
        b.free()


# (K, N, M): split K (O-proj 4 ways, the down shape 4 ways, QKV 3 ways) and
# a 128-row prompt on 128 x 64 tiles (no split: the norm is its own launch)
@pytest.mark.parametrize("qtype,K,N,M,acc,scaled", [(rrr_hip.Q4_K, 3072, 3072, 512, True, False),
                                                    (rrr_hip.Q6_K, 8192, 3072, 512, True, True),
                                                    (rrr_hip.Q5_K, 3072, 5120, 512, False, False),
                                                    (rrr_hip.Q4_K, 3072, 3072, 128, True, False)])
def test_gemm_f16_rmsnorm_is_the_two_calls(ctx, qtype, K, N, M, acc, scaled):
    """rrr_gemm_f16_rmsnorm = rrr_gemm_f16 then rrr_rmsnorm_f16 of the rows,
    bit for bit: Y and the f16 norm rows."""
    raw = synth.weight(7, 90, qtype, K, N)
    X = f16r(synth.normal_f32(7, 91, M * K).reshape(M, K))
    rs = np.ldexp(np.float32(1.0), np.random.default_rng(9).integers(-8, 8, M)).astype(np.float32)
    Y0 = synth.normal_f32(7, 92, M * N, 0.0, 3.0)
    g = synth.normal_f32(7, 93, N, 1.0, 0.1)
    W = ctx.weight_upload(qtype, K, N, raw)
    xb, rb, gb = ctx.to_device(X.astype(np.float16).view(np.uint16)), ctx.to_device(rs), ctx.to_device(g)
    ya, yb = ctx.to_device(Y0), ctx.to_device(Y0)
    na, nb = ctx.alloc(M * N * 2), ctx.alloc(M * N * 2)
    rsb = rb if scaled else None
    ctx.gemm_f16(xb, W, qtype, ya, K, N, M, accumulate=acc, row_scale=rsb)
    ctx.rmsnorm_f16(ya, gb, na, M, N, 1e-5)
    ctx.gemm_f16_rmsnorm(xb, W, qtype, yb, K, N, M, gb, nb, 1e-5, accumulate=acc, row_scale=rsb)
    assert np.array_equal(ctx.download(yb, np.uint32, M * N), ctx.download(ya, np.uint32, M * N))
    assert np.array_equal(ctx.download(nb, np.uint16, M * N), ctx.download(na, np.uint16, M * N))
    for b in (W, xb, rb, gb, ya, yb, na, nb):
        b.free()


# (type, K, n_heads, n_kv_heads, head_dim, rope_dim, M, rows, pos0): the
# Phi-4-mini QKV (partial rotary) with K split 3 ways and padding rows, on
# 128 x 64 tiles (no split) and on 256 x 128 tiles without a split; full
# rotary with K split 8 ways; the kv_store form (rope_dim 0), K split 3 ways
@pytest.mark.parametrize("qtype,K,nh,nkv,hd,rd,M,rows,pos0", [
    (rrr_hip.Q5_K, 3072, 24, 8, 128, 96, 512, 500, 37),
    (rrr_hip.Q5_K, 3072, 24, 8, 128, 96, 128, 128, 0),
    (rrr_hip.Q4_K, 3072, 24, 8, 128, 96, 1024, 1000, 5),
    (rrr_hip.Q4_K, 2048, 8, 4, 64, 64, 512, 300, 11),
    (rrr_hip.Q6_K, 3072, 24, 8, 128, 0, 512, 512, 3)])
def test_gemm_f16_rope_kv_rows_is_the_two_calls(ctx, qtype, K, nh, nkv, hd, rd, M, rows, pos0):
    """rrr_gemm_f16_rope_kv_rows = rrr_gemm_f16 then rrr_rope_kv_store_rows,
    bit for bit: every qkv row (padding rows included) and both caches."""
    q_dim, kv = nh * hd, nkv * hd
    N = q_dim + 2 * kv
    raw = synth.weight(8, 40 + qtype, qtype, K, N)
    X = f16r(synth.normal_f32(8, 41, M * K).reshape(M, K))
    nf = rd // 2
    fac = (1.0 + np.abs(synth.normal_f32(8, 42, max(nf, 1)))).astype(np.float32)
    W = ctx.weight_upload(qtype, K, N, raw)
    xb, fb = ctx.to_device(X.astype(np.float16).view(np.uint16)), ctx.to_device(fac)
    crow = (pos0 + rows) * kv
    c0 = synth.normal_f32(8, 43, crow).astype(np.float16).view(np.uint16)
    qa, qb = ctx.alloc(M * N * 4), ctx.alloc(M * N * 4)
    ka, va, kb, vb = (ctx.to_device(c0) for _ in range(4))
    args = (fb if nf else None, nf)
    ctx.gemm_f16(xb, W, qtype, qa, K, N, M)
    ctx.rope_kv_store_rows(qa, rows, *args, ka, va, pos0, nh, nkv, hd, rd, q_dim, kv)
    ctx.gemm_f16_rope_kv_rows(xb, W, qtype, qb, K, M, rows, *args, kb, vb, pos0, nh, nkv, hd, rd, q_dim, kv)
    assert np.array_equal(ctx.download(qb, np.uint32, M * N), ctx.download(qa, np.uint32, M * N))
    assert np.array_equal(ctx.download(kb, np.uint16, crow), ctx.download(ka, np.uint16, crow))
    assert np.array_equal(ctx.download(vb, np.uint16, crow), ctx.download(va, np.uint16, crow))
    for b in (W, xb, fb, qa, qb, ka, va, kb, vb):
        b.free()


# (type, K, F, M, scale): the Phi-4-mini gate/up at 512 and 1024 rows, Q5_K /
# Q6_K weights, larger activations, 256 rows of a wider F
@pytest.mark.parametrize("qtype,K,F,M,xs", [(rrr_hip.Q4_K, 3072, 8192, 512, 1.0),
                                             (rrr_hip.Q4_K, 3072, 8192, 1024, 30.0),
                                             (rrr_hip.Q5_K, 2048, 8192, 512, 1.0),
                                             (rrr_hip.Q6_K, 1024, 16384, 256, 4.0)])
def test_gemm_f16_silu_gate_f16_is_the_two_calls(ctx, qtype, K, F, M, xs):
    """rrr_gemm_f16_silu_gate_f16 = rrr_gemm_f16 (N = 2F) then
    rrr_silu_gate_f16, bit for bit: the f16 rows and the row scales."""
    raw = synth.weight(9, 60 + qtype, qtype, K, 2 * F)
    X = f16r(synth.normal_f32(9, 61, M * K).reshape(M, K) * np.float32(xs))
    W = ctx.weight_upload(qtype, K, 2 * F, raw)
    xb = ctx.to_device(X.astype(np.float16).view(np.uint16))
    gu = ctx.alloc(M * 2 * F * 4)
    ma, mb = ctx.alloc(M * F * 2), ctx.alloc(M * F * 2)
    sa, sb = ctx.alloc(M * 4), ctx.alloc(M * 4)
    ctx.gemm_f16(xb, W, qtype, gu, K, 2 * F, M)
    ctx.silu_gate_f16(gu, ma, sa, M, F)
    ctx.gemm_f16_silu_gate_f16(xb, W, qtype, mb, sb, K, F, M)
    assert np.array_equal(ctx.download(mb, np.uint16, M * F), ctx.download(ma, np.uint16, M * F))
    assert np.array_equal(ctx.download(sb, np.uint32, M), ctx.download(sa, np.uint32, M))
    for b in (W, xb, gu, ma, mb, sa, sb):
        b.free()


def test_gemm_f16_silu_gate_f16_unsupported(ctx):
    """Shapes whose GEMM would split K or leave CUs idle are refused (the two
    calls do them)."""
    W = ctx.weight_upload(rrr_hip.Q4_K, 256, 256, synth.weight(9, 70, rrr_hip.Q4_K, 256, 256))
    xb, mb, sb = ctx.alloc(256 * 256 * 2), ctx.alloc(256 * 128 * 2), ctx.alloc(256 * 4)
    with pytest.raises(rrr_hip.RrrError):
        ctx.gemm_f16_silu_gate_f16(xb, W, rrr_hip.Q4_K, mb, sb, 256, 128, 256)
    for b in (W, xb, mb, sb):
        b.free()


def oracle_prefill(s, host, prompt, pos0, caches):
    """The prefill composed in the oracle: fp64 GEMMs and attention, the f32
    restatement of RoPE and the f16 cache store, the GEMM inputs rounded to
    f16 at the same points as the GPU path."""
    d, F, M = s.d_model, s.ffn_dim, prompt.shape[0]
    H = prompt.astype(np.float64)
    for i in range(s.n_layers):
        L = host[i]
        n = f16r(orc.rms_norm(H.astype(np.float32), L["attn_norm"], s.eps))
        qkv = orc.gemv(rrr_hip.Q5_K, L["attn_qkv"], n, d, s.qkv_dim, M, THREADS, f64=True).astype(np.float32)
        kc, vc = caches[i]
        for t in range(M):
            qkv[t], kc, vc = orc.rope_kv_store(qkv[t], kc, vc, pos0 + t, s.n_heads, s.n_kv_heads, s.head_dim,
                                               s.rope_dim, factors=host["rope_factors"], theta=s.rope_theta,
                                               attn_factor=s.rope_attn_factor)
        caches[i] = (kc, vc)
        att = np.stack([orc.attention_f64(qkv[t, :d], kc, vc, pos0 + t + 1, s.n_kv_heads, s.heads_per_kv,
                                          s.head_dim) for t in range(M)])
        H = H + orc.gemv(rrr_hip.Q4_K, L["attn_output"], f16r(att), d, d, M, THREADS, f64=True)
        n = f16r(orc.rms_norm(H.astype(np.float32), L["ffn_norm"], s.eps))
        gu = orc.gemv(rrr_hip.Q4_K, L["ffn_up"], n, d, 2 * F, M, THREADS, f64=True)
        mid, scale = block_f16(orc.silu_gate(gu.astype(np.float32), F).reshape(M, F))
        H = H + orc.gemv(s.down_type(i), L["ffn_down"], mid.astype(np.float32), F, d, M, THREADS,
                         f64=True) * scale[:, None].astype(np.float64)
    normed = orc.rms_norm(H[-1].astype(np.float32), host["out_norm"], s.eps)
    logits = orc.logits(normed, host["emb"], d, s.vocab, 1, s.chunk, THREADS, f64=True)
    return logits, H


@pytest.fixture(scope="module")
def sweep(ctx):
    sw = decode.DecodeSweep(ctx, SHAPE, seed=3, keep_host=True, attention=True)
    for kc, vc in sw.kv:
        ctx.fill_u32(kc, 0)
        ctx.fill_u32(vc, 0)
    return sw


@pytest.mark.parametrize("M,pos0", [(5, 0), (130, 0), (40, 9)])
def test_prefill_matches_oracle_composition(ctx, sweep, M, pos0):
    s = SHAPE
    prompt = decode.prompt_host(3, s, M)
    caches = [(np.zeros(s.max_seq * s.kv_stride, np.uint16), np.zeros(s.max_seq * s.kv_stride, np.uint16))
              for _ in range(s.n_layers)]
    if pos0:   # earlier cache rows: whatever the GPU caches hold there, copied to the oracle's
        for i, (kc, vc) in enumerate(sweep.kv):
            caches[i][0][:pos0 * s.kv_stride] = ctx.download(kc, np.uint16, pos0 * s.kv_stride)
            caches[i][1][:pos0 * s.kv_stride] = ctx.download(vc, np.uint16, pos0 * s.kv_stride)
    sweep.load_prompt(prompt)
    sweep.record_prefill(M, pos0)
    ctx.sync()
    logits, tok, hid = sweep.prefill_results(M)
    ref_logits, ref_h = oracle_prefill(s, sweep.host, prompt, pos0, caches)
    assert np.all(np.isfinite(hid)) and np.all(np.isfinite(logits))
    assert orc.normwise_err(hid, ref_h) < MFMA_TOL
    assert orc.normwise_err(logits, ref_logits) < MFMA_TOL
    assert tok == int(np.argmax(logits))
    for i, (kc, vc) in enumerate(sweep.kv):
        n = (pos0 + M) * s.kv_stride
        kg = ctx.download(kc, np.uint16, n).view(np.float16).astype(np.float64)
        vg = ctx.download(vc, np.uint16, n).view(np.float16).astype(np.float64)
        kr = caches[i][0][:n].view(np.float16).astype(np.float64)
        vr = caches[i][1][:n].view(np.float16).astype(np.float64)
        assert orc.normwise_err(kg, kr) < MFMA_TOL and orc.normwise_err(vg, vr) < MFMA_TOL


def test_prefill_graph_replay_matches_eager(ctx, sweep):
    M = 70
    prompt = decode.prompt_host(4, SHAPE, M)
    sweep.load_prompt(prompt)
    sweep.record_prefill(M, 0)
    ctx.sync()
    logits0, tok0, hid0 = sweep.prefill_results(M)
    ctx.graph_begin()
    sweep.record_prefill(M, 0)
    g = ctx.graph_end()
    for _ in range(2):
        sweep.load_prompt(prompt)
        ctx.fill_u32(sweep.logits, 0)
        g.launch()
        ctx.sync()
        logits, tok, hid = sweep.prefill_results(M)
        assert tok == tok0
        assert np.array_equal(hid.view(np.uint32), hid0.view(np.uint32))
        assert np.array_equal(logits.view(np.uint32), logits0.view(np.uint32))
    g.destroy()


def test_prefill_fused_norms_are_the_separate_calls(ctx, sweep):
    """record_prefill with its fused steps equals the separate calls bit for
    bit (hidden rows, logits and the cached K/V): the O-proj / FFN-down GEMMs
    writing the next norm (rrr_gemm_f16_rmsnorm), the QKV GEMM's split
    reduction doing the RoPE + KV store (rrr_gemm_f16_rope_kv_rows) and the
    gate/up GEMM writing silu * up (rrr_gemm_f16_silu_gate_f16).  130 tokens
    pad to 256 rows: every GEMM but gate/up splits K, and gate/up's 128 tiles
    are the fewest its fused form takes."""
    s, M = SHAPE, 130
    prompt = decode.prompt_host(5, s, M)
    out = []
    for fused in (False, True):
        sweep.prefill_fused = fused
        sweep.load_prompt(prompt)
        sweep.record_prefill(M, 0)
        ctx.sync()
        logits, tok, hid = sweep.prefill_results(M)
        kv = [ctx.download(kc, np.uint16, M * s.kv_stride) for kc, _ in sweep.kv]
        out.append((logits, tok, hid, kv))
    sweep.prefill_fused = True
    (l0, t0, h0, kv0), (l1, t1, h1, kv1) = out
    assert t0 == t1
    assert np.array_equal(h0.view(np.uint32), h1.view(np.uint32))
    assert np.array_equal(l0.view(np.uint32), l1.view(np.uint32))
    assert all(np.array_equal(a, b) for a, b in zip(kv0, kv1))
