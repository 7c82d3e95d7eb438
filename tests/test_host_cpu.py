"""CPU tests of the host side: the input generator, the C ABI's exports and
its argument validation (through a validation-only context, no GPU), and the
ComputeEngine mirror of the reference engine surface."""
import ctypes
import os
import re

import numpy as np
import pytest

import rrr_hip
from rrr_hip import _lib, synth
from rrr_hip.engine import (ERR_BAD_SHAPE, ERR_BAD_TYPE, ERR_INVALID_ARG, ERR_NO_DEVICE, ERR_NULL,
                            ERR_SHORT_BUFFER, ERR_STALE, ERR_STATE, ERR_UNSUPPORTED)

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(REPO, "include", h) for h in sorted(os.listdir(os.path.join(REPO, "include")))
           if h.endswith(".h")]


def header_symbols():
    text = "".join(open(h).read() for h in HEADERS)
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rrr_[a-z0-9_]+)\s*\(", text)))


# ---- generator ----------------------------------------------------------------

def test_f32_to_f16_matches_numpy_rne():
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504.0, 65520.0, 65519.99, 1e-8, 5.96e-8, 2.98e-8, 6.1e-5, np.inf, -np.inf],
                 np.float32),
    ]).astype(np.float32)
    # every f16 value and the midpoints between neighbours (ties to even)
    allh = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = ((allh[:-1] + allh[1:]) / 2).astype(np.float32)
    vals = np.concatenate([vals, allh.astype(np.float32), mids, -mids])
    ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([synth.f32_to_f16_bits(v) for v in vals], np.uint16)
    assert np.array_equal(got, ref)


def test_generator_is_deterministic_and_thread_independent():
    a = synth.weight(1, 5, 12, 3072, 64, threads=1)
    b = synth.weight(1, 5, 12, 3072, 64, threads=7)
    assert np.array_equal(a, b)
    n1 = synth.normal_f32(1, 9, 10001, threads=1)
    n2 = synth.normal_f32(1, 9, 10001, threads=6)
    assert np.array_equal(n1, n2)
    assert not np.array_equal(synth.weight(1, 6, 12, 3072, 4), synth.weight(1, 5, 12, 3072, 4))


def test_generator_recipes():
    # Q4_K/Q5_K: d = f16(|N|*0.01), dmin = f16(|N|*0.005), finite and >= 0
    for qt, bs in ((12, 144), (13, 176)):
        b = synth.weight(2, qt, qt, 256 * 4000, 1).reshape(-1, bs)
        d = b[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0]
        dmin = b[:, 2:4].copy().view(np.float16).astype(np.float64)[:, 0]
        assert np.all(np.isfinite(d)) and np.all(d >= 0) and np.all(dmin >= 0)
        assert 0.006 < d.mean() < 0.010 and 0.003 < dmin.mean() < 0.005  # E|N| = 0.798
        # packed 6-bit fields are uniform: mean of all 16 fields ~ 31.5
        assert 30.0 < b[:, 4:16].astype(np.float64).mean() < 133.0
    b = synth.weight(2, 14, 14, 256 * 4000, 1).reshape(-1, 210)
    sc = b[:, 192:208].view(np.int8)
    assert sc.min() == -32 and sc.max() == 31
    d = b[:, 208:210].copy().view(np.float16).astype(np.float64)[:, 0]
    assert 0.003 < d.mean() < 0.005
    x = synth.normal_f32(3, 0, 200000, 1.0, 0.1)
    assert abs(x.mean() - 1.0) < 2e-3 and abs(x.std() - 0.1) < 2e-3
    xb = synth.normal_bf16(3, 0, 1000)
    xf = (xb.astype(np.uint32) << 16).view(np.float32)
    assert np.allclose(xf, synth.normal_f32(3, 0, 1000), rtol=1 / 128)


# ---- C ABI exports ------------------------------------------------------------

def test_library_exports_every_header_symbol():
    lib = ctypes.CDLL(_lib.HIP_LIB)
    syms = header_symbols()
    assert len(syms) >= 30
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing
    # the Python binding declares a signature for each of them
    assert sorted(_lib.SIGNATURES) == syms


def test_abi_version_and_no_device_here():
    lib = _lib.hip()
    assert lib.rrr_abi_version() == 1
    assert lib.rrr_device_count() >= 0
    assert lib.rrr_tensor_bytes(12, 3072, 3072) == 5308416
    assert lib.rrr_tensor_bytes(13, 3072, 5120) == 10813440
    assert lib.rrr_tensor_bytes(14, 8192, 3072) == 20643840
    assert lib.rrr_tensor_bytes(0, 3072, 200064) == 2458386432
    assert lib.rrr_tensor_bytes(12, 3000, 1) == 0
    assert lib.rrr_tensor_bytes(7, 256, 1) == 0


# ---- validation (validation-only context) ----------------------------------------

@pytest.fixture
def vctx():
    c = rrr_hip.Context(rrr_hip.DEVICE_NONE)
    yield c
    c.close()


def code_of(fn, *args, **kw):
    with pytest.raises(rrr_hip.RrrError) as ei:
        fn(*args, **kw)
    return ei.value.code


def test_gemv_validation(vctx):
    K, N = 3072, 64
    x = vctx.alloc(K * 4)
    y = vctx.alloc(N * 4)
    W = vctx.alloc(rrr_hip.tensor_bytes(12, K, N))
    assert code_of(vctx.gemv, x, W, 12, y, K, N) == ERR_NO_DEVICE          # valid call, no GPU
    assert code_of(vctx.gemv, x, W, 11, y, K, N) == ERR_BAD_TYPE
    assert code_of(vctx.gemv, x, W, 12, y, 3000, N) == ERR_BAD_SHAPE
    assert code_of(vctx.gemv, x, W, 12, y, K, 0) == ERR_BAD_SHAPE
    assert code_of(vctx.gemv, x, W, 12, y, K, N, 0) == ERR_BAD_SHAPE
    assert code_of(vctx.gemv, x, W, 12, y, K, N + 1) == ERR_SHORT_BUFFER   # W too short
    assert code_of(vctx.gemv, x, W, 13, y, K, N) == ERR_SHORT_BUFFER       # Q5_K needs more bytes
    assert code_of(vctx.gemv, x, W, 12, y, K, N, 2) == ERR_SHORT_BUFFER    # X too short for M=2
    small_y = vctx.alloc(N * 4 - 4)
    assert code_of(vctx.gemv, x, W, 12, small_y, K, N) == ERR_SHORT_BUFFER
    nullbuf = rrr_hip.Buffer(vctx, None, 0)
    assert code_of(vctx.gemv, nullbuf, W, 12, y, K, N) == ERR_NULL
    assert code_of(vctx.gemv, x, W, 12, y, 65536 + 256, N) in (ERR_UNSUPPORTED, ERR_SHORT_BUFFER)


def test_stale_handles(vctx):
    b = vctx.alloc(64)
    h = b.handle
    b.free()
    stale = rrr_hip.Buffer(vctx, h, 64)
    assert code_of(vctx.upload, stale, np.zeros(4, np.float32)) in (ERR_STALE,)
    other = rrr_hip.Context(rrr_hip.DEVICE_NONE)
    ob = other.alloc(64)
    foreign = rrr_hip.Buffer(vctx, ob.handle, 64)
    assert code_of(vctx.upload, foreign, np.zeros(4, np.float32)) == ERR_STALE
    other.close()
    # a destroyed context is rejected
    lib = _lib.hip()
    assert lib.rrr_buf_size(None) == 0
    assert lib.rrr_sync(ctypes.c_void_p(other.handle or 0)) in (ERR_NULL,)


def test_views_and_ranges(vctx):
    b = vctx.alloc(4096)
    v = vctx.view(b, 1024, 1024)
    assert v.nbytes == 1024
    assert code_of(vctx.view, b, 4000, 200) == ERR_INVALID_ARG
    assert code_of(vctx.view, b, 2, 16) == ERR_INVALID_ARG
    assert code_of(b.free) == ERR_STATE  # views first
    v.free()
    assert code_of(vctx.upload, b, np.zeros(2000, np.float32)) == ERR_SHORT_BUFFER
    assert code_of(vctx.upload, b, np.zeros(16, np.float32)) == ERR_NO_DEVICE
    assert code_of(vctx.fill_u32, b, 0, 2, 8) == ERR_INVALID_ARG
    b.free()


def test_weight_upload_validation(vctx):
    raw = np.zeros(rrr_hip.tensor_bytes(14, 8192, 2), np.uint8)
    assert code_of(vctx.weight_upload, 14, 8192, 2, raw) == ERR_NO_DEVICE
    assert code_of(vctx.weight_upload, 14, 8192, 3, raw) == ERR_SHORT_BUFFER
    assert code_of(vctx.weight_upload, 9, 8192, 2, raw) == ERR_BAD_TYPE
    assert code_of(vctx.weight_upload, 14, 8000, 2, raw) == ERR_BAD_SHAPE


def test_elementwise_and_logits_validation(vctx):
    d = 3072
    x, g, y = vctx.alloc(d * 4), vctx.alloc(d * 4), vctx.alloc(d * 4)
    assert code_of(vctx.rmsnorm, x, g, y, 1, d) == ERR_NO_DEVICE
    assert code_of(vctx.rmsnorm, x, g, y, 2, d) == ERR_SHORT_BUFFER
    assert code_of(vctx.rmsnorm, x, g, y, 1, d, float("nan")) == ERR_INVALID_ARG
    assert code_of(vctx.silu_gate, x, y, 1, d) == ERR_SHORT_BUFFER
    assert code_of(vctx.residual_add, x, g, y, d + 1) == ERR_SHORT_BUFFER
    V, K = 1000, 256
    E = vctx.alloc(V * K * 4)
    lg = vctx.alloc(V * 4)
    xk = vctx.alloc(K * 4)
    assert code_of(vctx.logits_f32, xk, E, lg, K, V, rrr_hip.LOGITS_ROWS) == ERR_NO_DEVICE
    assert code_of(vctx.logits_f32, xk, E, lg, K, V, rrr_hip.LOGITS_CHUNKED, 300) == ERR_UNSUPPORTED
    assert code_of(vctx.logits_f32, xk, E, lg, K, V, 3) == ERR_INVALID_ARG
    assert code_of(vctx.logits_f32, xk, E, lg, K, V + 1, rrr_hip.LOGITS_ROWS) == ERR_SHORT_BUFFER
    # raw Q6_K token_embd rows: K % 256, the Q6_K tensor size
    E6 = vctx.alloc(rrr_hip.tensor_bytes(rrr_hip.Q6_K, K, V))
    lg2 = vctx.alloc((V + 16) * 4)
    assert code_of(vctx.logits_f32, xk, E6, lg, K, V, rrr_hip.LOGITS_Q6K, 0) == ERR_NO_DEVICE
    assert code_of(vctx.logits_f32, xk, E6, lg, K, V, rrr_hip.LOGITS_ROWS) == ERR_SHORT_BUFFER
    assert code_of(vctx.logits_f32, xk, E6, lg, 250, V, rrr_hip.LOGITS_Q6K, 0) == ERR_BAD_SHAPE
    assert code_of(vctx.logits_f32, xk, E6, lg2, K, V + 16, rrr_hip.LOGITS_Q6K, 0) == ERR_SHORT_BUFFER
    out = vctx.alloc(4)
    assert code_of(vctx.argmax_f32, lg, V, out) == ERR_NO_DEVICE
    assert code_of(vctx.argmax_f32, lg, V + 1, out) == ERR_SHORT_BUFFER
    # the logits with their argmax in one call: the logits' checks plus the index buffer
    gk = vctx.alloc(K * 4)
    assert code_of(vctx.logits_rmsnorm_argmax, xk, gk, 1e-5, E, lg, K, V, out, rrr_hip.LOGITS_ROWS) == ERR_NO_DEVICE
    assert code_of(vctx.logits_rmsnorm_argmax, xk, gk, 1e-5, E, lg, K, V, out, rrr_hip.LOGITS_CHUNKED, 256) == \
        ERR_NO_DEVICE
    assert code_of(vctx.logits_rmsnorm_argmax, xk, gk, 1e-5, E, lg, K, V + 1, out, rrr_hip.LOGITS_ROWS) == \
        ERR_SHORT_BUFFER
    short = vctx.alloc(2)
    assert code_of(vctx.logits_rmsnorm_argmax, xk, gk, 1e-5, E, lg, K, V, short, rrr_hip.LOGITS_ROWS) == \
        ERR_SHORT_BUFFER
    lib = _lib.hip()
    assert lib.rrr_logits_rmsnorm_argmax(vctx._h, xk._h, gk._h, 1e-5, E._h, lg._h, K, V, rrr_hip.LOGITS_ROWS, 0,
                                         None) == ERR_NULL


def test_fused_validation(vctx):
    K = 3072
    qkv = vctx.alloc((K + 2048) * 4)
    hid = vctx.alloc(K * 4)
    W = vctx.alloc(rrr_hip.tensor_bytes(12, K, K))
    param = 128 | (3 << 16)
    assert code_of(vctx.gemv_residual, qkv, rrr_hip.ACT_GQA_V, param, W, 12, hid, K, K) == ERR_NO_DEVICE
    assert code_of(vctx.gemv_residual, qkv, rrr_hip.ACT_GQA_V, 100 | (3 << 16), W, 12, hid, K, K) == ERR_INVALID_ARG
    assert code_of(vctx.gemv_residual, qkv, 7, 0, W, 12, hid, K, K) == ERR_INVALID_ARG
    assert code_of(vctx.gemv_residual, hid, rrr_hip.ACT_SILU_GATE, 0, W, 12, hid, K, K) == ERR_SHORT_BUFFER


def test_gemv_rmsnorm_silu_validation(vctx):
    K, F = 3072, 64
    x, g = vctx.alloc(K * 4), vctx.alloc(K * 4)
    W = vctx.alloc(rrr_hip.tensor_bytes(12, K, 2 * F))
    y = vctx.alloc(F * 4)                    # F outputs, not 2F
    assert code_of(vctx.gemv_rmsnorm_silu, x, g, 1e-5, W, 12, y, K, F) == ERR_NO_DEVICE   # valid call, no GPU
    assert code_of(vctx.gemv_rmsnorm_silu, x, g, 1e-5, W, 12, y, K, F + 1) == ERR_SHORT_BUFFER   # W holds 2F rows
    assert code_of(vctx.gemv_rmsnorm_silu, x, g, 1e-5, W, 12, vctx.alloc(F * 4 - 4), K, F) == ERR_SHORT_BUFFER
    assert code_of(vctx.gemv_rmsnorm_silu, x, g, 1e-5, W, 12, y, K, 0) == ERR_BAD_SHAPE
    assert code_of(vctx.gemv_rmsnorm_silu, x, g, 1e-5, W, 0, y, K, F) == ERR_UNSUPPORTED       # F32 rows
    assert code_of(vctx.gemv_rmsnorm_silu, x, g, float("nan"), W, 12, y, K, F) == ERR_INVALID_ARG
    nullbuf = rrr_hip.Buffer(vctx, None, 0)
    assert code_of(vctx.gemv_rmsnorm_silu, x, nullbuf, 1e-5, W, 12, y, K, F) == ERR_NULL


def test_dispatch_shim_validation(vctx):
    K, N = 3072, 16
    x, y = vctx.alloc(K * 4), vctx.alloc(N * 4)
    W = vctx.alloc(rrr_hip.tensor_bytes(13, K, N))
    assert code_of(vctx.dispatch, "matmul_q5k", [x, W, y], [K, N], [N, 1, 1]) == ERR_NO_DEVICE
    assert code_of(vctx.dispatch, "matmul_gpuq5", [x, W, y], [K, N], [N, 1, 1]) == ERR_NO_DEVICE
    assert code_of(vctx.dispatch, "matmul_q5k", [x, W, y], [K, N], [N + 1, 1, 1]) == ERR_INVALID_ARG
    assert code_of(vctx.dispatch, "matmul_q5k", [x, W], [K, N], [N, 1, 1]) == ERR_INVALID_ARG
    assert code_of(vctx.dispatch, "matmul_q5k", [x, W, y], [K], [N, 1, 1]) == ERR_INVALID_ARG
    assert code_of(vctx.dispatch, "attention", [x, W, y, x], [1, 8, 3, 128], [24, 1, 1]) == ERR_SHORT_BUFFER
    assert code_of(vctx.dispatch, "attention", [x, W, W, x], [1, 8, 3, 128], [24, 1, 1]) == ERR_NO_DEVICE
    assert code_of(vctx.dispatch, "attention", [x, W, W, x], [1, 8, 3, 128], [8, 1, 1]) == ERR_INVALID_ARG
    assert code_of(vctx.dispatch, "rope", [x, x], [0] * 5, [1, 1, 1]) == ERR_UNSUPPORTED
    assert code_of(vctx.dispatch, "no_such_shader", [x], [1], [1, 1, 1]) == ERR_UNSUPPORTED
    assert code_of(vctx.dispatch, "rmsnorm", [x, x, x], [1, K], [1, 1, 1]) == ERR_NO_DEVICE
    # batch: failing entry is named
    with pytest.raises(rrr_hip.RrrError) as ei:
        vctx.dispatch_batch([("matmul_q5k", [x, W, y], [K, N], [N, 1, 1], True),
                             ("rope", [x, x], [0] * 5, [1, 1, 1], True)])
    assert "entry 0" in ei.value.msg or ei.value.code == ERR_NO_DEVICE


def test_rope_kv_store_and_attention_validation(vctx):
    nh, nkv, hd, rd = 24, 8, 128, 96
    qd, kvs = nh * hd, nkv * hd
    qkv = vctx.alloc((qd + 2 * kvs) * 4)
    fac = vctx.alloc(48 * 4)
    kc, vc = vctx.alloc(16 * kvs * 2), vctx.alloc(16 * kvs * 2)
    rk = vctx.rope_kv_store
    assert code_of(rk, qkv, fac, 48, kc, vc, 15, nh, nkv, hd, rd, qd, kvs) == ERR_NO_DEVICE
    assert code_of(rk, qkv, fac, 48, kc, vc, 16, nh, nkv, hd, rd, qd, kvs) == ERR_SHORT_BUFFER   # row 16 of 16
    assert code_of(rk, qkv, fac, 49, kc, vc, 0, nh, nkv, hd, rd, qd, kvs) == ERR_SHORT_BUFFER    # factors
    assert code_of(rk, qkv, fac, 48, kc, vc, 0, nh, nkv, hd, 130, qd, kvs) == ERR_BAD_SHAPE      # rope_dim > hd
    assert code_of(rk, qkv, fac, 48, kc, vc, 0, nh, nkv, hd, 95, qd, kvs) == ERR_BAD_SHAPE       # odd rope_dim
    assert code_of(rk, qkv, fac, 48, kc, vc, 0, nh, nkv, hd, rd, qd, kvs + 2) == ERR_BAD_SHAPE   # kv_stride
    assert code_of(rk, qkv, fac, 48, kc, vc, 0, nh + 1, nkv, hd, rd, qd, kvs) == ERR_BAD_SHAPE   # q heads
    assert code_of(rk, qkv, None, 0, kc, vc, 0, 0, 0, 0, 0, qd, kvs) == ERR_NO_DEVICE           # kv_store form
    at = vctx.attention
    q, out = vctx.alloc(qd * 4), vctx.alloc(qd * 4)
    assert code_of(at, q, kc, vc, out, 16, nkv, 3, hd) == ERR_NO_DEVICE
    assert code_of(at, q, kc, vc, out, 17, nkv, 3, hd) == ERR_SHORT_BUFFER
    assert code_of(at, q, kc, vc, out, 0, nkv, 3, hd) == ERR_BAD_SHAPE
    assert code_of(at, q, kc, vc, out, 4, nkv, 3, 64) == ERR_UNSUPPORTED
    assert code_of(at, q, kc, vc, out, 2049, nkv, 3, hd) == ERR_UNSUPPORTED     # beyond 2048 cache rows
    assert code_of(at, q, kc, vc, out, 4, 8, 9, hd) == ERR_UNSUPPORTED
    assert code_of(at, q, kc, vc, out, 4, 16, 4, hd) in (ERR_UNSUPPORTED, ERR_SHORT_BUFFER)


def test_attention_noalloc_validation():
    # argument checks run before any HIP call (the pointers are never touched)
    lib = _lib.hip()
    p = 0x10000
    na = lib.rrr_attention_noalloc
    assert na(None, p, p, p, 16, 8, 3, 128, None) == ERR_NULL
    assert na(p, p, p, None, 16, 8, 3, 128, None) == ERR_NULL
    assert na(p, p, p, p, 16, 8, 3, 64, None) == ERR_UNSUPPORTED                # head_dim
    assert na(p, p, p, p, 0, 8, 3, 128, None) == ERR_BAD_SHAPE
    assert na(p, p, p, p, 2049, 8, 3, 128, None) == ERR_UNSUPPORTED             # the scratch array's rows
    assert b"2048" in lib.rrr_last_error()
    assert na(p, p, p, p, 16, 16, 8, 128, None) == ERR_UNSUPPORTED              # 128 query heads
    assert na(p, p, p, p, 16, 2, 9, 128, None) == ERR_UNSUPPORTED               # 9 per KV head
    assert na(p + 4, p, p, p, 16, 8, 3, 128, None) == ERR_INVALID_ARG           # alignment


def test_prefill_validation(vctx):
    nh, nkv, hd, rd = 24, 8, 128, 96
    qd, kvs = nh * hd, nkv * hd
    row = qd + 2 * kvs
    rows = 4
    qkv = vctx.alloc(rows * row * 4)
    fac = vctx.alloc(48 * 4)
    kc, vc = vctx.alloc(16 * kvs * 2), vctx.alloc(16 * kvs * 2)
    rr = vctx.rope_kv_store_rows
    assert code_of(rr, qkv, rows, fac, 48, kc, vc, 12, nh, nkv, hd, rd, qd, kvs) == ERR_NO_DEVICE
    assert code_of(rr, qkv, rows, fac, 48, kc, vc, 13, nh, nkv, hd, rd, qd, kvs) == ERR_SHORT_BUFFER   # rows 13..16
    assert code_of(rr, qkv, rows + 1, fac, 48, kc, vc, 0, nh, nkv, hd, rd, qd, kvs) == ERR_SHORT_BUFFER  # qkv
    assert code_of(rr, qkv, 0, fac, 48, kc, vc, 0, nh, nkv, hd, rd, qd, kvs) == ERR_BAD_SHAPE
    ap = vctx.attention_prefill
    o32, o16 = vctx.alloc(rows * qd * 4), vctx.alloc(rows * qd * 2)
    assert code_of(ap, qkv, rows, kc, vc, o32, 12, nkv, 3, hd) == ERR_NO_DEVICE
    assert code_of(ap, qkv, rows, kc, vc, o16, 12, nkv, 3, hd, out_type=rrr_hip.F16) == ERR_NO_DEVICE
    assert code_of(ap, qkv, rows, kc, vc, o16, 12, nkv, 3, hd) == ERR_SHORT_BUFFER          # f32 out in 2-byte room
    assert code_of(ap, qkv, rows, kc, vc, o32, 13, nkv, 3, hd) == ERR_SHORT_BUFFER          # caches
    assert code_of(ap, qkv, rows, kc, vc, o32, 12, nkv, 3, hd, out_type=14) == ERR_BAD_TYPE
    assert code_of(ap, qkv, rows, kc, vc, o32, 2046, nkv, 3, hd) == ERR_UNSUPPORTED        # past 2048 rows
    assert code_of(ap, qkv, rows, kc, vc, o32, 0, nkv, 3, 64) == ERR_UNSUPPORTED
    assert code_of(ap, qkv, 0, kc, vc, o32, 0, nkv, 3, hd) == ERR_BAD_SHAPE
    K, N, M = 3072, 3072, 128
    W = vctx.alloc(rrr_hip.tensor_bytes(12, K, N))
    X = vctx.alloc(M * K * 2)
    Y = vctx.alloc(M * N * 4)
    g = vctx.gemm_f16
    assert code_of(g, X, W, 12, Y, K, N, M) == ERR_NO_DEVICE
    assert code_of(g, X, W, 12, Y, K, N, M, accumulate=True) == ERR_NO_DEVICE
    assert code_of(g, X, W, 12, Y, K, N, 100) == ERR_UNSUPPORTED        # M % 128
    assert code_of(g, X, W, 12, Y, K, N - 64, M) == ERR_NO_DEVICE
    assert code_of(g, X, W, 12, Y, K, N, 2 * M) == ERR_SHORT_BUFFER
    assert code_of(g, X, W, 0, Y, K, N, M) == ERR_UNSUPPORTED
    x, gm = vctx.alloc(M * K * 4), vctx.alloc(K * 4)
    y16 = vctx.alloc(M * K * 2)
    assert code_of(vctx.rmsnorm_f16, x, gm, y16, M, K) == ERR_NO_DEVICE
    assert code_of(vctx.rmsnorm_f16, x, gm, y16, M + 1, K) == ERR_SHORT_BUFFER
    rs = vctx.alloc(M * 4)
    assert code_of(vctx.silu_gate_f16, x, y16, rs, M, K // 2) == ERR_NO_DEVICE
    assert code_of(vctx.silu_gate_f16, x, y16, rs, M, K) == ERR_SHORT_BUFFER
    assert code_of(vctx.silu_gate_f16, x, y16, rs, 2 * M, K // 4) == ERR_SHORT_BUFFER     # row scales
    assert code_of(g, X, W, 12, Y, K, N, M, row_scale=rs) == ERR_NO_DEVICE
    assert code_of(g, X, W, 12, Y, K, N, M, row_scale=vctx.alloc(4)) == ERR_SHORT_BUFFER
    # the gate/up GEMM with silu * up in its epilogue: shapes it takes reach
    # the device check, the rest are refused before it
    Ws = vctx.alloc(rrr_hip.tensor_bytes(12, K, 2 * 8192))
    Xs, ms, rss = vctx.alloc(512 * K * 2), vctx.alloc(512 * 8192 * 2), vctx.alloc(512 * 4)
    gs = vctx.gemm_f16_silu_gate_f16
    assert code_of(gs, Xs, Ws, 12, ms, rss, K, 8192, 512) == ERR_NO_DEVICE
    assert code_of(gs, Xs, Ws, 12, ms, rss, K, 8192, 256) == ERR_NO_DEVICE   # 128 tiles
    assert code_of(gs, Xs, Ws, 12, ms, rss, K, 8192, 128) == ERR_UNSUPPORTED  # M % 256
    assert code_of(gs, Xs, Ws, 12, ms, rss, K, 4096, 256) == ERR_UNSUPPORTED  # 64 tiles: K would split
    assert code_of(gs, Xs, Ws, 12, ms, rss, K, 8192, 1024) == ERR_SHORT_BUFFER
    assert code_of(gs, Xs, Ws, 0, ms, rss, K, 8192, 512) == ERR_UNSUPPORTED
    # the QKV GEMM with the RoPE + KV store of its rows
    qk = vctx.alloc(M * (qd + 2 * kvs) * 4)
    rk = vctx.gemm_f16_rope_kv_rows
    Wq = vctx.alloc(rrr_hip.tensor_bytes(12, 256, qd + 2 * kvs))
    Xq = vctx.alloc(M * 256 * 2)
    assert code_of(rk, Xq, Wq, 12, qk, 256, M, rows, fac, 48, kc, vc, 12, nh, nkv, hd, rd, qd, kvs) == ERR_NO_DEVICE
    assert code_of(rk, Xq, Wq, 12, qk, 256, M, M + 1, fac, 48, kc, vc, 0, nh, nkv, hd, rd, qd, kvs) == ERR_BAD_SHAPE
    assert code_of(rk, Xq, Wq, 12, qk, 256, M, rows, fac, 48, kc, vc, 13, nh, nkv, hd, rd, qd, kvs) == ERR_SHORT_BUFFER
    assert code_of(rk, Xq, Wq, 12, qk, 256, 2 * M, rows, fac, 48, kc, vc, 12, nh, nkv, hd, rd, qd,
                   kvs) == ERR_SHORT_BUFFER   # X and qkv hold M rows
    assert code_of(rk, Xq, Wq, 12, qk, 256, 100, rows, fac, 48, kc, vc, 12, nh, nkv, hd, rd, qd, kvs) == ERR_UNSUPPORTED


def test_graph_state_rules(vctx):
    assert code_of(vctx.graph_end) == ERR_STATE
    assert code_of(vctx.graph_begin) == ERR_NO_DEVICE
    assert code_of(vctx.timer_stop) == ERR_STATE


def test_compute_engine_mirror_requires_registration(monkeypatch):
    # ComputeEngine on a validation-only context: pipelines must be registered
    # (engine.rs:142 before engine.rs:476), buffer counts must match.
    eng = rrr_hip.ComputeEngine.__new__(rrr_hip.ComputeEngine)
    eng.ctx = rrr_hip.Context(rrr_hip.DEVICE_NONE)
    eng.pipeline_cache, eng.persistent_desc_sets = {}, []
    a = eng.alloc_buffer(3072 * 4)
    assert a.capacity == 3072 * 4
    with pytest.raises(rrr_hip.RrrError):
        eng.dispatch_by_name("rmsnorm", [a, a, a], [a.capacity] * 3, b"\x01\0\0\0\0\x0c\0\0", [1, 1, 1])
    eng.get_pipeline("rmsnorm", 3, 8)
    with pytest.raises(rrr_hip.RrrError) as ei:
        eng.dispatch_by_name("rmsnorm", [a, a, a], [a.capacity] * 3, b"\x01\0\0\0\0\x0c\0\0", [1, 1, 1])
    assert ei.value.code == ERR_NO_DEVICE
    h = eng.pre_allocate_desc_set("rmsnorm", [a, a, a], [a.capacity] * 3)
    with pytest.raises(rrr_hip.RrrError) as ei:
        eng.dispatch_batch_persistent_v2([("matmul_q4k", h, b"", [1, 1, 1], True)])
    assert ei.value.code == ERR_INVALID_ARG
    eng.close()


def test_decode_sweep_shape_and_bytes():
    # Phi-4-mini shape of the sweep and its per-token byte count, summed here
    # from the per-op algorithmic bytes (raw weights + activations once).
    from rrr_hip import decode
    s = decode.Phi4Shape()
    assert (s.qkv_dim, s.heads_per_kv, s.vocab % s.chunk) == (5120, 3, 3456)
    assert [s.down_type(i) for i in range(4)] == [rrr_hip.Q6_K, rrr_hip.Q4_K, rrr_hip.Q6_K, rrr_hip.Q4_K]
    norm2, qkv, o, up = 73_728, 10_846_208, 5_332_992, 28_389_376
    down_q6, down_q4 = 20_688_896, 14_200_832
    layers = 16 * (norm2 + qkv + o + up + down_q6) + 16 * (norm2 + qkv + o + up + down_q4)
    logits = 2_458_386_432 + 12_288 + 800_256
    assert s.bytes_per_token() == layers + 36_864 + logits == 4_446_025_216


def test_decode_host_tensors_are_reproducible():
    import dataclasses
    from rrr_hip import decode
    s = dataclasses.replace(decode.Phi4Shape(), n_layers=2, vocab=300, d_model=512, ffn_dim=1024,
                            n_heads=4, n_kv_heads=2, head_dim=128)
    a, b = decode.layer_host(3, s, 1), decode.layer_host(3, s, 1)
    for k in a:
        assert np.array_equal(a[k], b[k])
    assert a["ffn_down"].size == rrr_hip.tensor_bytes(rrr_hip.Q4_K, 1024, 512)
    assert decode.layer_host(3, s, 0)["ffn_down"].size == rrr_hip.tensor_bytes(rrr_hip.Q6_K, 1024, 512)
    assert not np.array_equal(decode.layer_host(3, s, 0)["attn_qkv"], a["attn_qkv"])
    emb = decode.embedding_chunks_host(3, s)
    assert emb.size == 300 * 512 and abs(float(emb.std()) - 0.02) < 0.002
