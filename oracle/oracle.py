"""ctypes wrapper of liboracle.so -- TEST INFRASTRUCTURE ONLY.

The CPU oracle restates the reference's CPU formulas (src/model/phi4.rs);
see rrr_oracle.h for the function-by-function citations and the checks that
pin each function.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module, and only to check results against
(or, for the cpu_baseline, to time the CPU formulas).
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")

_u8p = ctypes.POINTER(ctypes.c_uint8)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_u32 = ctypes.c_uint32
_sz = ctypes.c_size_t

_SIG = {
    "rrr_o_block_bytes": (_u32, [_u32]),
    "rrr_o_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "rrr_o_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "rrr_o_scale_min_k4": (None, [ctypes.c_int, _u8p, _u8p, _u8p]),
    "rrr_o_dequant": (ctypes.c_int, [_u32, _u8p, _sz, _f32p]),
    "rrr_o_repack_q4k": (None, [_u8p, _sz, _u8p]),
    "rrr_o_repack_q5k": (None, [_u8p, _sz, _u8p]),
    "rrr_o_repack_q6k": (None, [_u8p, _sz, _u8p]),
    "rrr_o_dequant_gpuq4": (None, [_u8p, _sz, _f32p]),
    "rrr_o_dequant_gpuq5": (None, [_u8p, _sz, _f32p]),
    "rrr_o_dequant_gpuq6": (None, [_u8p, _sz, _f32p]),
    "rrr_o_rms_norm_rows": (None, [_f32p, _f32p, _f32p, _sz, _sz, ctypes.c_float]),
    "rrr_o_silu_gate": (None, [_f32p, _f32p, _sz, _sz]),
    "rrr_o_residual_add": (None, [_f32p, _f32p, _f32p, _sz]),
    "rrr_o_gemv": (ctypes.c_int, [_u32, _u8p, _f32p, _f32p, _u32, _u32, _u32, ctypes.c_int]),
    "rrr_o_gemv_f64": (ctypes.c_int, [_u32, _u8p, _f32p, _f64p, _u32, _u32, _u32, ctypes.c_int]),
    "rrr_o_logits_f32": (ctypes.c_int, [_f32p, _f32p, _f32p, _u32, _u32, _u32, _u32, ctypes.c_int]),
    "rrr_o_logits_f64": (ctypes.c_int, [_f32p, _f32p, _f64p, _u32, _u32, _u32, _u32, ctypes.c_int]),
    "rrr_o_logits_chunk_build": (None, [_f32p, _u32, _u32, _u32, _f32p]),
    "rrr_o_f32_to_f16_n": (None, [_f32p, _u16p, _sz]),
    "rrr_o_rope": (None, [_f32p, _u32, _u32, _u32, _u32, ctypes.c_float, ctypes.c_float, _f32p, _u32]),
    "rrr_o_rope_kv_store": (None, [_f32p, _f32p, _u32, _u16p, _u16p, _u32, _u32, _u32, _u32, _u32, _u32, _u32,
                                   ctypes.c_float, ctypes.c_float]),
    "rrr_o_attention_f64": (None, [_f32p, _u16p, _u16p, _f64p, _u32, _u32, _u32, _u32]),
}

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        l = ctypes.CDLL(LIB)
        for name, (res, args) in _SIG.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def _p(a, t):
    return a.ctypes.data_as(t)


def block_bytes(qtype):
    return int(lib().rrr_o_block_bytes(qtype))


def f16_to_f32(bits):
    return lib().rrr_o_f16_to_f32(int(bits))


def scale_min_k4(j, q12):
    q = np.ascontiguousarray(q12, dtype=np.uint8)
    sc, mn = ctypes.c_uint8(), ctypes.c_uint8()
    lib().rrr_o_scale_min_k4(j, _p(q, _u8p), ctypes.byref(sc), ctypes.byref(mn))
    return sc.value, mn.value


def dequant(qtype, raw, n):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    if lib().rrr_o_dequant(qtype, _p(raw, _u8p), n, _p(out, _f32p)) != 0:
        raise ValueError(f"type {qtype}")
    return out


_REPACK = {12: ("rrr_o_repack_q4k", "rrr_o_dequant_gpuq4", 192),
           13: ("rrr_o_repack_q5k", "rrr_o_dequant_gpuq5", 320),
           14: ("rrr_o_repack_q6k", "rrr_o_dequant_gpuq6", 320)}


def dequant_via_repack(qtype, raw, n):
    """Dequantize through the reference's repacked GPU layout (phi4.rs:278-436)."""
    rp, rd, bs = _REPACK[qtype]
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    rep = np.zeros(n // 256 * bs, dtype=np.uint8)
    getattr(lib(), rp)(_p(raw, _u8p), n, _p(rep, _u8p))
    out = np.empty(n, dtype=np.float32)
    getattr(lib(), rd)(_p(rep, _u8p), n, _p(out, _f32p))
    return out


def rms_norm(x, w, eps=1e-5):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    d = w.shape[0]
    out = np.empty_like(x)
    lib().rrr_o_rms_norm_rows(_p(x, _f32p), _p(w, _f32p), _p(out, _f32p), x.size // d, d, eps)
    return out


def silu_gate(gu, F):
    gu = np.ascontiguousarray(gu, dtype=np.float32)
    rows = gu.size // (2 * F)
    out = np.empty(rows * F, dtype=np.float32)
    lib().rrr_o_silu_gate(_p(gu, _f32p), _p(out, _f32p), rows, F)
    return out


def residual_add(a, b):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    out = np.empty_like(a)
    lib().rrr_o_residual_add(_p(a, _f32p), _p(b, _f32p), _p(out, _f32p), a.size)
    return out


MAX_M = 1024   # token rows of one rrr_o_gemv call (rrr_oracle.c)


def gemv(qtype, W, X, K, N, M=1, threads=1, f64=False):
    """Y[M, N] from raw W (N x K of qtype) and X[M, K]; more than MAX_M rows
    go through in calls of MAX_M (every row is computed on its own)."""
    W = np.ascontiguousarray(W).view(np.uint8)
    X = np.ascontiguousarray(X, dtype=np.float32).reshape(-1)
    Y = np.empty(M * N, dtype=np.float64 if f64 else np.float32)
    for m0 in range(0, M, MAX_M):
        mc = min(MAX_M, M - m0)
        x = X[m0 * K:(m0 + mc) * K]
        y = Y[m0 * N:(m0 + mc) * N]
        if f64:
            rc = lib().rrr_o_gemv_f64(qtype, _p(W, _u8p), _p(x, _f32p), _p(y, _f64p), K, N, mc, threads)
        else:
            rc = lib().rrr_o_gemv(qtype, _p(W, _u8p), _p(x, _f32p), _p(y, _f32p), K, N, mc, threads)
        if rc != 0:
            raise ValueError("oracle gemv rejected its arguments")
    return Y.reshape(M, N)


def logits(x, E, K, V, layout=0, chunk=8192, threads=1, f64=False):
    x = np.ascontiguousarray(x, dtype=np.float32)
    E = np.ascontiguousarray(E, dtype=np.float32)
    if f64:
        y = np.empty(V, dtype=np.float64)
        rc = lib().rrr_o_logits_f64(_p(x, _f32p), _p(E, _f32p), _p(y, _f64p), K, V, layout, chunk, threads)
    else:
        y = np.empty(V, dtype=np.float32)
        rc = lib().rrr_o_logits_f32(_p(x, _f32p), _p(E, _f32p), _p(y, _f32p), K, V, layout, chunk, threads)
    if rc != 0:
        raise ValueError("oracle logits rejected its arguments")
    return y


def logits_chunk_build(E, K, V, chunk=8192):
    E = np.ascontiguousarray(E, dtype=np.float32)
    out = np.empty(V * K, dtype=np.float32)
    lib().rrr_o_logits_chunk_build(_p(E, _f32p), K, V, chunk, _p(out, _f32p))
    return out


def normwise_err(got, ref):
    """max_i |got_i - ref_i| / max_i |ref_i| (the tolerance metric)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.max(np.abs(ref))
    return float(np.max(np.abs(got - ref)) / (den if den > 0 else 1.0))


# ---- decode glue: RoPE, the f16 KV-cache store, decode attention ----

# the reference's legacy Phi-4-mini constants (phi4.rs:114-116)
ROPE_DIM, ROPE_THETA, ROPE_ATTN_FACTOR = 96, 10000.0, 1.190238


def f32_to_f16_bits(x):
    """binary32 -> binary16 bit patterns, round to nearest even."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.size, dtype=np.uint16)
    lib().rrr_o_f32_to_f16_n(_p(x, _f32p), _p(out, _u16p), x.size)
    return out.reshape(x.shape)


def rope(x, pos, n_heads, head_dim, rope_dim=ROPE_DIM, theta=ROPE_THETA, attn_factor=ROPE_ATTN_FACTOR,
         factors=None):
    """apply_rope_cfg (phi4.rs:238-256) on a copy of x (n_heads x head_dim)."""
    x = np.array(x, dtype=np.float32, copy=True).ravel()
    f = np.ascontiguousarray(factors if factors is not None else np.ones(1, np.float32), dtype=np.float32)
    nf = 0 if factors is None else f.size
    lib().rrr_o_rope(_p(x, _f32p), pos, n_heads, head_dim, rope_dim, theta, attn_factor, _p(f, _f32p), nf)
    return x


def rope_kv_store(qkv, k_cache, v_cache, pos, n_heads, n_kv_heads, head_dim, rope_dim=ROPE_DIM, factors=None,
                  theta=ROPE_THETA, attn_factor=ROPE_ATTN_FACTOR):
    """The rope_kv_store pipeline: returns (qkv after RoPE, k_cache, v_cache)
    with row pos of the (uint16) caches written; the inputs are not changed."""
    qkv = np.array(qkv, dtype=np.float32, copy=True).ravel()
    kc = np.array(k_cache, dtype=np.uint16, copy=True).ravel()
    vc = np.array(v_cache, dtype=np.uint16, copy=True).ravel()
    f = np.ascontiguousarray(factors if factors is not None else np.ones(1, np.float32), dtype=np.float32)
    nf = 0 if factors is None else f.size
    q_dim, kv_stride = n_heads * head_dim, n_kv_heads * head_dim
    assert qkv.size >= q_dim + 2 * kv_stride and kc.size >= (pos + 1) * kv_stride and vc.size == kc.size
    lib().rrr_o_rope_kv_store(_p(qkv, _f32p), _p(f, _f32p), nf, _p(kc, _u16p), _p(vc, _u16p), pos, n_heads,
                              n_kv_heads, head_dim, rope_dim, q_dim, kv_stride, theta, attn_factor)
    return qkv, kc, vc


def attention_f64(q, k_cache, v_cache, seq_len, n_kv_heads, heads_per_kv, head_dim):
    """Decode attention over cache rows [0, seq_len) in double."""
    q = np.ascontiguousarray(q, dtype=np.float32).ravel()
    kc = np.ascontiguousarray(k_cache, dtype=np.uint16).ravel()
    vc = np.ascontiguousarray(v_cache, dtype=np.uint16).ravel()
    assert q.size >= n_kv_heads * heads_per_kv * head_dim and kc.size >= seq_len * n_kv_heads * head_dim
    out = np.empty(n_kv_heads * heads_per_kv * head_dim, dtype=np.float64)
    lib().rrr_o_attention_f64(_p(q, _f32p), _p(kc, _u16p), _p(vc, _u16p), _p(out, _f64p), seq_len, n_kv_heads,
                              heads_per_kv, head_dim)
    return out
