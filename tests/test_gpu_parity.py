"""GPU parity of the HIP decode path against the CPU oracle.

Bars: dequantized weights bit-exact; GEMV / batched GEMV / RMSNorm / logits
within 1e-4 normwise relative error max|got - ref| / max|ref| against the
oracle evaluated in fp64 (TOL below), MFMA shapes (prefill GEMM, batched
GEMV above 16 rows) within 2e-3; fused kernels bit-identical to the unfused
sequence they replace.
"""
import os

import numpy as np
import pytest

import oracle.oracle as orc
import rrr_hip
from rrr_hip import synth

pytestmark = pytest.mark.gpu

TOL = 1e-4
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
THREADS = 16


def err(got, ref):
    return orc.normwise_err(got, ref)


def same_bits_or_both_nan(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return bool(np.all(nan | (a.view(np.uint32) == b.view(np.uint32))))


def weights(qtype, K, N, seed=1, stream=0):
    if qtype == rrr_hip.F32:
        return synth.normal_f32(seed, stream, N * K, 0.0, 0.02).view(np.uint8)
    return synth.weight(seed, stream, qtype, K, N)


# ---- dequant: bit-exact -------------------------------------------------------

@pytest.mark.parametrize("name,qtype", [("q4k", 12), ("q5k", 13), ("q6k", 14)])
def test_dequant_known_answer_blocks(ctx, name, qtype):
    z = np.load(os.path.join(GOLDEN, f"kat_{name}.npz"))
    blocks, expected = z["blocks"], z["expected"]
    n = blocks.shape[0] * 256
    W = ctx.weight_upload(qtype, 256, blocks.shape[0], blocks.reshape(-1))
    out = ctx.alloc(n * 4)
    ctx.dequant(qtype, W, out, n)
    assert same_bits_or_both_nan(ctx.download(out).reshape(-1, 256), expected)
    W.free(); out.free()


@pytest.mark.parametrize("qtype,K,N", [(12, 3072, 3072), (13, 3072, 5120), (14, 8192, 3072), (14, 3072, 77)])
def test_dequant_seeded_bit_exact(ctx, qtype, K, N):
    raw = weights(qtype, K, N, seed=2)
    W = ctx.weight_upload(qtype, K, N, raw)
    out = ctx.alloc(K * N * 4)
    ctx.dequant(qtype, W, out, K * N)
    assert same_bits_or_both_nan(ctx.download(out), orc.dequant(qtype, raw, K * N))
    W.free(); out.free()


# ---- GEMV (M = 1) ---------------------------------------------------------------

GEMV_SHAPES = [
    (12, 3072, 3072),   # config 1 / O-proj
    (13, 3072, 5120),   # QKV
    (14, 8192, 3072),   # down, Q6_K
    (12, 8192, 3072),   # down, Q4_K layers
    (12, 3072, 16384),  # gate+up
    (0, 3072, 4096),    # F32 rows
    # ragged and edge shapes
    (12, 256, 1), (13, 256, 3), (14, 256, 5), (0, 256, 7),
    (12, 768, 17), (13, 1280, 33), (14, 3072, 1001), (14, 2560, 9),
    (12, 12288, 64), (14, 16384, 40), (0, 12288, 9),
]


@pytest.mark.parametrize("qtype,K,N", GEMV_SHAPES)
def test_gemv_parity(ctx, qtype, K, N):
    raw = weights(qtype, K, N, seed=3, stream=qtype)
    x = synth.normal_f32(3, 100 + qtype, K)
    W = ctx.weight_upload(qtype, K, N, raw)
    xb = ctx.to_device(x)
    yb = ctx.alloc(N * 4)
    ctx.gemv(xb, W, qtype, yb, K, N)
    y = ctx.download(yb)
    ref = orc.gemv(qtype, raw, x, K, N, 1, THREADS, f64=True)[0]
    e = err(y, ref)
    assert e < TOL, e
    # the oracle's own f32 path sits inside the same bar
    assert err(orc.gemv(qtype, raw, x, K, N, 1, THREADS)[0], ref) < TOL
    W.free(); xb.free(); yb.free()


@pytest.mark.parametrize("qtype", [12, 13, 14, 0])
def test_gemv_one_hot_is_bit_exact_column(ctx, qtype):
    K, N = 1024, 96
    raw = weights(qtype, K, N, seed=4, stream=qtype)
    deq = (orc.dequant(qtype, raw, K * N) if qtype else raw.view(np.float32)).reshape(N, K)
    W = ctx.weight_upload(qtype, K, N, raw)
    xb, yb = ctx.alloc(K * 4), ctx.alloc(N * 4)
    for k in (0, 15, 16, 31, 32, 200, 255, 256, 513, 1023):
        x = np.zeros(K, np.float32)
        x[k] = 1.0
        ctx.upload(xb, x)
        ctx.gemv(xb, W, qtype, yb, K, N)
        # equal values (a -0.0 weight cannot survive as -0.0 through a sum)
        assert np.array_equal(ctx.download(yb), deq[:, k]), k
    W.free(); xb.free(); yb.free()


def test_matmul_kquant_helper_and_dispatch_names(ctx):
    # gpu_matmul_kquant (phi4.rs:631-658) and the name-keyed shaders
    K, N = 3072, 640
    for qtype, names in ((12, ("matmul_q4k", "matmul_gpuq4")), (13, ("matmul_q5k", "matmul_gpuq5")),
                         (14, ("matmul_q6k", "matmul_gpuq6"))):
        KK = 8192 if qtype == 14 else K
        raw = weights(qtype, KK, N, seed=5, stream=qtype)
        x = synth.normal_f32(5, qtype, KK)
        W = ctx.weight_upload(qtype, KK, N, raw)
        a, c = ctx.alloc(KK * 4), ctx.alloc(N * 4)
        y = ctx.matmul_kquant(a, W, c, qtype, x, KK, N)
        ref = orc.gemv(qtype, raw, x, KK, N, 1, THREADS, f64=True)[0]
        assert err(y, ref) < TOL
        for nm in names:
            ctx.fill_u32(c, 0x7FC00000)
            ctx.dispatch(nm, [a, W, c], [KK, N], [N, 1, 1])
            assert np.array_equal(ctx.download(c), y)
        W.free(); a.free(); c.free()


# ---- batched GEMV / skinny ----------------------------------------------------------

# Batched K-quant rows on the matrix cores: Q4_K / Q5_K at 2 <= M <= 32 with
# K <= 3072 on the skinny kernel (up to 16 rows with hi/lo-split activations,
# the GEMV bar; above that hi only, the MFMA bar), and every K-quant shape
# above 16 rows that the skinny kernel does not take (more than 32 rows,
# Q6_K, K > 3072) on the prefill GEMM with f16 block-floating-point rows
# (N % 64 == 0; the MFMA bar).  The rest runs on the VALU kernels (GEMV bar).
MFMA_TOL = 2e-3


def batched_tol(qtype, K, N, M):
    if qtype == 0 or M <= 16:
        return TOL
    if qtype in (12, 13) and M <= 32 and K <= 3072:
        return MFMA_TOL
    return MFMA_TOL if N % 64 == 0 else TOL


BATCH_NAME = {12: "matmul_gpuq4_batch", 13: "matmul_gpuq5_batch", 14: "matmul_gpuq6_batch"}


def check_batched(ctx, qtype, K, N, M, seed=6):
    raw = weights(qtype, K, N, seed=seed, stream=qtype)
    X = synth.normal_f32(seed, 50 + M, M * K)
    W = ctx.weight_upload(qtype, K, N, raw)
    Xb, Yb = ctx.to_device(X), ctx.alloc(M * N * 4)
    ctx.gemv(Xb, W, qtype, Yb, K, N, M)
    Y = ctx.download(Yb).reshape(M, N)
    ref = orc.gemv(qtype, raw, X, K, N, M, THREADS, f64=True)
    tol = batched_tol(qtype, K, N, M)
    assert np.all(np.isfinite(Y))
    for m in range(M):
        assert err(Y[m], ref[m]) < tol, m
    if qtype:
        # the reference's batch pipeline (push [K, N, M], grid [N, M, 1]) is the same call
        ctx.fill_u32(Yb, 0)
        ctx.dispatch(BATCH_NAME[qtype], [Xb, W, Yb], [K, N, M], [N, M, 1])
        assert np.array_equal(ctx.download(Yb).reshape(M, N), Y)
    W.free(); Xb.free(); Yb.free()


@pytest.mark.parametrize("qtype,K,N", [(12, 3072, 16384), (13, 3072, 5120), (12, 3072, 3072), (14, 8192, 3072),
                                       (0, 3072, 2048), (12, 512, 37), (13, 4096, 300)])
@pytest.mark.parametrize("M", [2, 3, 4, 8, 13, 16, 17, 32])
def test_batched_gemv_parity(ctx, qtype, K, N, M):
    check_batched(ctx, qtype, K, N, M)


# The reference's prefill calls these pipelines with M = the prompt length
# (forward_prefill_batched: QKV phi4.rs:1257-1268, gate/up :1346-1357, down
# :1380-1391): QKV Q5_K 5120x3072, gate/up Q4_K 16384x3072, down Q6_K and
# Q4_K 3072x8192, at prompt lengths that are and are not multiples of 128.
@pytest.mark.parametrize("qtype,K,N", [(13, 3072, 5120), (12, 3072, 16384), (14, 8192, 3072), (12, 8192, 3072)])
@pytest.mark.parametrize("M", [33, 100, 130, 512])
def test_batched_prompt_rows_parity(ctx, qtype, K, N, M):
    check_batched(ctx, qtype, K, N, M, seed=16)


def test_batched_rows_in_chunks(ctx):
    """1,600 rows of K = 8192: their f16 copy (26 MB) exceeds half of the
    48 MB workspace, so the rows go through in chunks of 1,536 and 64 (the
    last padded to 128 rows, which are computed and not stored)."""
    check_batched(ctx, 14, 8192, 512, 1600, seed=17)


def test_batched_rows_extreme_scales(ctx):
    """Rows of the f16 route are scaled by powers of two: a row of ~1e30, a
    row of ~1e-30 and a zero row come out as the unscaled rows would, a row
    holding inf or NaN makes only its own outputs non-finite."""
    qtype, K, N, M = 12, 3072, 1024, 40
    raw = weights(qtype, K, N, seed=18, stream=1)
    X = synth.normal_f32(18, 2, M * K).reshape(M, K)
    X[3] *= np.float32(1e30)
    X[4] *= np.float32(1e-30)
    X[5] = 0.0
    X[6, 17] = np.inf
    X[7, 1000] = np.nan
    W = ctx.weight_upload(qtype, K, N, raw)
    Xb, Yb = ctx.to_device(X.reshape(-1)), ctx.alloc(M * N * 4)
    ctx.gemv(Xb, W, qtype, Yb, K, N, M)
    Y = ctx.download(Yb).reshape(M, N)
    fin = [m for m in range(M) if m not in (6, 7)]
    ref = orc.gemv(qtype, raw, np.ascontiguousarray(X[fin]).reshape(-1), K, N, len(fin), THREADS, f64=True)
    for i, m in enumerate(fin):
        if m == 5:
            assert np.all(Y[m] == 0.0)
        else:
            assert err(Y[m], ref[i]) < MFMA_TOL, m
    assert not np.any(np.isfinite(Y[6])) and not np.any(np.isfinite(Y[7]))
    W.free(); Xb.free(); Yb.free()


@pytest.mark.parametrize("qtype,K,N,M", [(12, 3072, 1024, 4), (13, 3072, 640, 3), (14, 3072, 512, 2), (12, 3072, 1024, 8)])
def test_batched_small_rows_extreme_values(ctx, qtype, K, N, M):
    """A few rows on the matrix cores (2 to 4 on the int8 GEMV's multi-token
    form, 8 on the skinny kernel): a row of ~1e30, a zero row and a row
    holding inf keep to themselves; the others match the oracle at the GEMV
    bar."""
    raw = weights(qtype, K, N, seed=19, stream=2)
    X = synth.normal_f32(19, 3 + M, M * K).reshape(M, K)
    X[0] *= np.float32(1e30)
    X[1] = 0.0
    X[M - 1, 100] = np.inf
    W = ctx.weight_upload(qtype, K, N, raw)
    Xb, Yb = ctx.to_device(X.reshape(-1)), ctx.alloc(M * N * 4)
    ctx.gemv(Xb, W, qtype, Yb, K, N, M)
    Y = ctx.download(Yb).reshape(M, N)
    fin = list(range(M - 1))
    ref = orc.gemv(qtype, raw, np.ascontiguousarray(X[fin]).reshape(-1), K, N, len(fin), THREADS, f64=True)
    for i, m in enumerate(fin):
        if m == 1:
            assert np.all(Y[m] == 0.0)
        else:
            assert err(Y[m], ref[i]) < TOL, m
    assert not np.any(np.isfinite(Y[M - 1]))
    W.free(); Xb.free(); Yb.free()


# ---- RMSNorm, SwiGLU glue, residual ---------------------------------------------

@pytest.mark.parametrize("rows,d", [(1, 3072), (5, 3072), (1, 8192), (3, 1000), (1, 1)])
def test_rmsnorm_parity(ctx, rows, d):
    x = synth.normal_f32(7, rows, rows * d)
    g = synth.normal_f32(7, 100 + rows, d, 1.0, 0.1)
    xb, gb, yb = ctx.to_device(x), ctx.to_device(g), ctx.alloc(rows * d * 4)
    ctx.rmsnorm(xb, gb, yb, rows, d, 1e-5)
    y = ctx.download(yb).reshape(rows, d)
    xd = x.reshape(rows, d).astype(np.float64)
    ref = g * xd / np.sqrt(np.mean(xd * xd, axis=1, keepdims=True) + 1e-5)
    for r in range(rows):
        assert err(y[r], ref[r]) < TOL
    assert err(y, orc.rms_norm(x, g).reshape(rows, d)) < TOL
    if rows == 1:
        ctx.fill_u32(yb, 0)
        ctx.dispatch("rmsnorm", [xb, gb, yb], [1, d], [1, 1, 1])
        assert np.array_equal(ctx.download(yb), y[0])
    xb.free(); gb.free(); yb.free()


def test_silu_gate_and_residual(ctx):
    F, rows = 8192, 3
    gu = synth.normal_f32(8, 0, rows * 2 * F, 0.0, 3.0)
    gub, mid = ctx.to_device(gu), ctx.alloc(rows * F * 4)
    ctx.silu_gate(gub, mid, rows, F)
    assert err(ctx.download(mid), orc.silu_gate(gu, F)) < 1e-6
    a = synth.normal_f32(8, 1, 3072)
    b = synth.normal_f32(8, 2, 3072)
    ab, bb = ctx.to_device(a), ctx.to_device(b)
    ctx.residual_add(ab, bb, ab, 3072)  # in place, as the reference does on gpu_hidden
    assert np.array_equal(ctx.download(ab), orc.residual_add(a, b))
    ctx.dispatch("residual_add", [ab, bb, ab], [3072], [12, 1, 1])
    assert np.array_equal(ctx.download(ab), (a + b) + b)
    one = ctx.alloc(F * 4)
    ctx.dispatch("silu_gate", [gub, one], [F], [32, 1, 1])
    assert np.array_equal(ctx.download(one), ctx.download(mid, count=F))
    for bb_ in (gub, mid, ab, bb, one):
        bb_.free()


# ---- fused kernels are bit-identical to the unfused sequence ------------------------

@pytest.mark.parametrize("qtype,K,N", [(13, 3072, 5120), (12, 3072, 16384), (14, 3072, 300), (0, 3072, 2000)])
def test_gemv_rmsnorm_fused_bitwise(ctx, qtype, K, N):
    raw = weights(qtype, K, N, seed=9, stream=qtype)
    x = synth.normal_f32(9, 1, K)
    g = synth.normal_f32(9, 2, K, 1.0, 0.1)
    W = ctx.weight_upload(qtype, K, N, raw)
    xb, gb, nb = ctx.to_device(x), ctx.to_device(g), ctx.alloc(K * 4)
    y1, y2 = ctx.alloc(N * 4), ctx.alloc(N * 4)
    ctx.rmsnorm(xb, gb, nb, 1, K, 1e-5)
    ctx.gemv(nb, W, qtype, y1, K, N)
    ctx.gemv_rmsnorm(xb, gb, 1e-5, W, qtype, y2, K, N)
    a, b = ctx.download(y1), ctx.download(y2)
    assert np.array_equal(a, b)
    ref = orc.gemv(qtype, raw, orc.rms_norm(x, g), K, N, 1, THREADS, f64=True)[0]
    assert err(b, ref) < TOL
    for t in (W, xb, gb, nb, y1, y2):
        t.free()


@pytest.mark.parametrize("qtype,K,F", [(12, 3072, 8192), (13, 3072, 300), (14, 8192, 1000), (12, 1024, 13),
                                       (13, 1024, 20000)])
def test_gemv_rmsnorm_silu(ctx, qtype, K, F):
    """silu(gate) * up fused into the gate/up GEMV: against the oracle, and
    bitwise the activation the down GEMV's silu prologue builds from the 2F
    gate/up rows (a down GEMV on either gives the same result)."""
    raw = weights(qtype, K, 2 * F, seed=11, stream=qtype)
    x = synth.normal_f32(11, 1, K)
    g = synth.normal_f32(11, 2, K, 1.0, 0.1)
    W = ctx.weight_upload(qtype, K, 2 * F, raw)
    xb, gb = ctx.to_device(x), ctx.to_device(g)
    mid, gu = ctx.alloc(F * 4), ctx.alloc(2 * F * 4)
    ctx.gemv_rmsnorm_silu(xb, gb, 1e-5, W, qtype, mid, K, F)
    ctx.gemv_rmsnorm(xb, gb, 1e-5, W, qtype, gu, K, 2 * F)
    ref_gu = orc.gemv(qtype, raw, orc.rms_norm(x, g), K, 2 * F, 1, THREADS, f64=True)[0]
    ref = ref_gu[:F] / (1.0 + np.exp(-ref_gu[:F])) * ref_gu[F:]
    y = ctx.download(mid)
    assert err(y, ref) < TOL
    # a down GEMV (N = 64 rows of K = F) on the fused output and, with the
    # silu prologue, on the 2F rows: the same activation values give the
    # same sums
    if F % 256 == 0:
        N = 64
        rawd = weights(12, F, N, seed=11, stream=40)
        Wd = ctx.weight_upload(12, F, N, rawd)
        y1, y2 = ctx.to_device(np.zeros(N, np.float32)), ctx.to_device(np.zeros(N, np.float32))
        ctx.gemv_residual(mid, rrr_hip.ACT_IDENTITY, 0, Wd, 12, y1, F, N)
        ctx.gemv_residual(gu, rrr_hip.ACT_SILU_GATE, 0, Wd, 12, y2, F, N)
        assert np.array_equal(ctx.download(y1), ctx.download(y2))
        for t in (Wd, y1, y2):
            t.free()
    for t in (W, xb, gb, mid, gu):
        t.free()


def test_gemv_residual_kinds(ctx):
    K, N = 3072, 3072
    # identity: O-proj + residual
    raw = weights(12, K, N, seed=10, stream=1)
    W = ctx.weight_upload(12, K, N, raw)
    x = synth.normal_f32(10, 2, K)
    h = synth.normal_f32(10, 3, N, 0.0, 100.0)
    xb, hb = ctx.to_device(x), ctx.to_device(h)
    ctx.gemv_residual(xb, rrr_hip.ACT_IDENTITY, 0, W, 12, hb, K, N)
    ref = h.astype(np.float64) + orc.gemv(12, raw, x, K, N, 1, THREADS, f64=True)[0]
    assert err(ctx.download(hb), ref) < TOL
    # silu_gate + down (Q6_K) + residual
    F = 8192
    raw6 = weights(14, F, N, seed=10, stream=4)
    W6 = ctx.weight_upload(14, F, N, raw6)
    gu = synth.normal_f32(10, 5, 2 * F, 0.0, 2.0)
    gub = ctx.to_device(gu)
    ctx.upload(hb, h)
    ctx.gemv_residual(gub, rrr_hip.ACT_SILU_GATE, 0, W6, 14, hb, F, N)
    mid = orc.silu_gate(gu, F)
    ref = h.astype(np.float64) + orc.gemv(14, raw6, mid, F, N, 1, THREADS, f64=True)[0]
    assert err(ctx.download(hb), ref) < TOL
    # position-0 GQA attention output (V gathered per kv head) + O-proj + residual
    hd, hpk = 128, 3
    qkv = synth.normal_f32(10, 6, K + 2 * (K // hpk))
    qb = ctx.to_device(qkv)
    ctx.upload(hb, h)
    ctx.gemv_residual(qb, rrr_hip.ACT_GQA_V, hd | (hpk << 16), W, 12, hb, K, N)
    v = qkv[K + K // hpk:]
    attn = np.concatenate([v[(hh // hpk) * hd:(hh // hpk + 1) * hd] for hh in range(K // hd)])
    ref = h.astype(np.float64) + orc.gemv(12, raw, attn, K, N, 1, THREADS, f64=True)[0]
    assert err(ctx.download(hb), ref) < TOL
    for t in (W, W6, xb, hb, gub, qb):
        t.free()


# ---- logits and argmax -------------------------------------------------------------

@pytest.mark.parametrize("V,chunk", [(20000, 8192), (8192, 8192), (3456, 8192), (1000, 256), (700, 700), (8195, 4096)])
def test_logits_parity_both_layouts(ctx, V, chunk):
    K = 3072
    E = synth.normal_f32(11, V, V * K, 0.0, 0.02)
    x = synth.normal_f32(11, 1, K)
    ref = orc.logits(x, E, K, V, threads=THREADS, f64=True)
    xb, yb = ctx.to_device(x), ctx.alloc(V * 4)
    Eb = ctx.to_device(E)
    ctx.logits_f32(xb, Eb, yb, K, V, rrr_hip.LOGITS_ROWS)
    y_rows = ctx.download(yb)
    assert err(y_rows, ref) < TOL
    Ec = orc.logits_chunk_build(E, K, V, chunk)
    ctx.upload(Eb, Ec)
    ctx.fill_u32(yb, 0)
    ctx.logits_f32(xb, Eb, yb, K, V, rrr_hip.LOGITS_CHUNKED, chunk)
    y_chunk = ctx.download(yb)
    assert err(y_chunk, ref) < TOL
    if V <= chunk:  # one chunk: the reference's matmul_tiled call shape
        ctx.fill_u32(yb, 0)
        ctx.dispatch("matmul_tiled", [xb, Eb, yb], [1, K, V], [(V + 15) // 16, 1, 1])
        assert np.array_equal(ctx.download(yb), y_chunk)
    xb.free(); yb.free(); Eb.free()


def test_logits_full_vocab_both_layouts(ctx):
    """The full 200,064-entry vocabulary (2.46 GB of F32 weights) in both
    layouts: rows, and the reference's 25 transposed 8192-entry chunks
    (phi4.rs:874-893), whose last three start past 2 GiB of the buffer."""
    K, V, chunk = 3072, 200064, 8192
    E = synth.normal_f32(11, V, V * K, 0.0, 0.02)
    x = synth.normal_f32(11, 1, K)
    ref = orc.logits(x, E, K, V, threads=THREADS, f64=True)
    xb, yb = ctx.to_device(x), ctx.alloc(V * 4)
    Eb = ctx.to_device(E)
    ctx.fill_u32(yb, 0x7FC00000)
    ctx.logits_f32(xb, Eb, yb, K, V, rrr_hip.LOGITS_ROWS)
    y_rows = ctx.download(yb)
    assert np.all(np.isfinite(y_rows))
    assert err(y_rows, ref) < TOL
    Ec = orc.logits_chunk_build(E, K, V, chunk)
    del E
    ctx.upload(Eb, Ec)
    del Ec
    ctx.fill_u32(yb, 0x7FC00000)
    ctx.logits_f32(xb, Eb, yb, K, V, rrr_hip.LOGITS_CHUNKED, chunk)
    y_chunk = ctx.download(yb)
    assert np.all(np.isfinite(y_chunk))
    assert err(y_chunk, ref) < TOL
    # every chunk on its own, the ones past 2 GiB included
    for c in range(0, V, chunk):
        n = min(chunk, V - c)
        assert err(y_chunk[c:c + n], ref[c:c + n]) < 4 * TOL, c // chunk
    # fused RMSNorm over the chunks equals RMSNorm then the chunked logits
    g = synth.normal_f32(11, 2, K, 1.0, 0.1)
    gb, nb, y2 = ctx.to_device(g), ctx.alloc(K * 4), ctx.alloc(V * 4)
    ctx.rmsnorm(xb, gb, nb, 1, K, 1e-5)
    ctx.logits_f32(nb, Eb, yb, K, V, rrr_hip.LOGITS_CHUNKED, chunk)
    ctx.logits_rmsnorm(xb, gb, 1e-5, Eb, y2, K, V, rrr_hip.LOGITS_CHUNKED, chunk)
    assert np.array_equal(ctx.download(yb), ctx.download(y2))
    for b in (xb, yb, Eb, gb, nb, y2):
        b.free()


def ref_argmax(v):
    """The sequential loop of phi4.rs:1172-1183."""
    best_val, best_id = -np.inf, 0
    for j, x in enumerate(v):
        if x > best_val:
            best_val, best_id = x, j
    return best_id


@pytest.mark.parametrize("case", ["random", "ties", "nan", "all_neg_inf", "last", "single"])
def test_argmax_semantics(ctx, case):
    V = 200064
    v = synth.normal_f32(12, 0, V)
    if case == "ties":
        v[[5, 77777, 199999]] = 9.0
    elif case == "nan":
        v[[0, 10]] = np.nan
        v[123456] = 7.5
    elif case == "all_neg_inf":
        v[:] = -np.inf
        v[3] = np.nan
    elif case == "last":
        v[-1] = 100.0
    elif case == "single":
        v = v[:1]
        V = 1
    vb, ob = ctx.to_device(v), ctx.alloc(4)
    ctx.argmax_f32(vb, V, ob)
    got = int(ctx.download(ob, np.uint32)[0])
    exp = ref_argmax(v) if case in ("nan", "all_neg_inf", "single") else int(np.argmax(v))
    assert got == exp
    vb.free(); ob.free()


# ---- graphs --------------------------------------------------------------------------

def test_graph_replay_matches_eager(ctx):
    K, N = 3072, 5120
    raw = weights(13, K, N, seed=13)
    W = ctx.weight_upload(13, K, N, raw)
    x = synth.normal_f32(13, 1, K)
    g = synth.normal_f32(13, 2, K, 1.0, 0.1)
    xb, gb, yb, ob = ctx.to_device(x), ctx.to_device(g), ctx.alloc(N * 4), ctx.alloc(4)
    ctx.gemv_rmsnorm(xb, gb, 1e-5, W, 13, yb, K, N)
    ctx.argmax_f32(yb, N, ob)
    eager_y, eager_i = ctx.download(yb), ctx.download(ob, np.uint32)
    ctx.graph_begin()
    ctx.fill_u32(yb, 0)
    ctx.gemv_rmsnorm(xb, gb, 1e-5, W, 13, yb, K, N)
    ctx.argmax_f32(yb, N, ob)
    graph = ctx.graph_end()
    for rep in range(5):
        ctx.fill_u32(yb, 0x7FC00000)          # eager work between replays
        ctx.fill_u32(ob, 0xFFFFFFFF)
        graph.launch()
        assert np.array_equal(ctx.download(yb), eager_y), rep
        assert np.array_equal(ctx.download(ob, np.uint32), eager_i), rep
    graph.destroy()
    for t in (W, xb, gb, yb, ob):
        t.free()


# ---- prefill dequant-GEMM (fp16 MFMA, fp32 accumulate): 2e-3 ------------------

GEMM_TOL = 2e-3


def bf16_to_f32(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("qtype,K,N,M", [(12, 3072, 16384, 128), (14, 8192, 192, 128), (13, 3072, 256, 256),
                                         (12, 512, 128, 384), (14, 256, 64, 128),
                                         # rows padded inside the library: M not a multiple of 128, and
                                         # 2,048 rows of K = 8192 whose f16 copy goes through the
                                         # workspace in chunks of 1,536 and 512 rows
                                         (12, 3072, 3072, 100), (13, 512, 320, 1), (14, 8192, 1024, 2048),
                                         # 256 x 128 workgroup tiles
                                         (12, 512, 16384, 256), (14, 768, 16384, 256), (13, 256, 16384, 256),
                                         # config 5 as benchmarked (512-token prompt): gate+up in one round of
                                         # 256 x 128 tiles; down (48 tiles) with K split 5 ways, 7/7/6/6/6
                                         # super-blocks a split; Q4_K down and Q5_K QKV (80 tiles, split 3 ways)
                                         (12, 3072, 16384, 512), (14, 8192, 3072, 512), (12, 8192, 3072, 512),
                                         (13, 3072, 5120, 512)])
def test_gemm_bf16_parity(ctx, qtype, K, N, M):
    raw = weights(qtype, K, N, seed=11, stream=qtype)
    xb = synth.normal_bf16(11, 50 + qtype, M * K)
    W = ctx.weight_upload(qtype, K, N, raw)
    Xd, Yd = ctx.to_device(xb), ctx.alloc(M * N * 4)
    ctx.gemm_bf16(Xd, W, qtype, Yd, K, N, M)
    got = ctx.download(Yd, np.float32, M * N).reshape(M, N)
    ref = orc.gemv(qtype, raw, bf16_to_f32(xb), K, N, M, THREADS, f64=True).reshape(M, N)
    assert np.all(np.isfinite(got))
    assert err(got, ref) < GEMM_TOL
    # every row meets the bar on its own, so no tile is silently wrong
    row_err = np.max(np.abs(got - ref), axis=1) / np.max(np.abs(ref), axis=1)
    assert np.max(row_err) < 4 * GEMM_TOL
    W.free(); Xd.free(); Yd.free()


def test_gemm_bf16_unsupported_shapes(ctx):
    W = ctx.weight_upload(12, 256, 96, weights(12, 256, 96))
    X, Y = ctx.alloc(100 * 256 * 2), ctx.alloc(100 * 96 * 4)
    with pytest.raises(rrr_hip.RrrError) as ei:
        ctx.gemm_bf16(X, W, 12, Y, 256, 96, 100)      # N not a multiple of 64
    assert ei.value.code == rrr_hip.engine.ERR_UNSUPPORTED
    W.free(); X.free(); Y.free()
