"""Pins of the CPU oracle (oracle/rrr_oracle.c) by checks independent of it.

The reference holds no tests or fixtures for this path, so each oracle
function is pinned by something that does not share its code: exhaustive
comparison with numpy's IEEE conversion, a bijection over all inputs,
known-answer blocks packed element-major from intended values
(tests/golden/make_golden.py), the reference's second statement of the
layouts (the repackers, phi4.rs:278-436), fp64 closed forms and invariants.
"""
import os

import numpy as np
import pytest

import oracle.oracle as orc
import rrr_hip.synth as syn

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def same_bits_or_both_nan(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return np.all(nan | (a.view(np.uint32) == b.view(np.uint32)))


# ---- a1: f16 -> f32 (phi4.rs:442, half 2.7.1) ------------------------------

def test_f16_exhaustive_vs_numpy():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([orc.f16_to_f32(int(b)) for b in bits], np.float32)
    isnan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), isnan)
    assert np.array_equal(got[~isnan].view(np.uint32), ref[~isnan].view(np.uint32))
    # NaNs come back quiet with the payload in the top mantissa bits, sign kept
    g = got[isnan].view(np.uint32)
    assert np.all(g & 0x00400000)
    assert np.array_equal((g >> 31).astype(np.uint16), (bits[isnan] >> 15))


# ---- a2: 6-bit scale/min unpack (phi4.rs:492-498) -------------------------

def test_scale_min_bijection_exhaustive():
    # Each of the 16 fields reads at most 3 bytes; enumerate every value of the
    # bytes each field depends on and require the 96 bits <-> 16 fields map to
    # be a bijection (each field is a 6-bit value and every input bit is used
    # by exactly one field).
    rng = np.random.default_rng(1)
    owner = {}
    for j in range(8):
        for bit in range(96):
            q = np.zeros(12, np.uint8)
            q[bit // 8] = 1 << (bit % 8)
            sc, mn = orc.scale_min_k4(j, q)
            base_sc, base_mn = orc.scale_min_k4(j, np.zeros(12, np.uint8))
            assert base_sc == 0 and base_mn == 0
            for name, v in (("sc", sc), ("mn", mn)):
                if v:
                    assert v & (v - 1) == 0, "a single input bit must map to a single output bit"
                    key = bit
                    assert key not in owner, f"bit {bit} used by {owner.get(key)} and ({name},{j})"
                    owner[key] = (name, j, v.bit_length() - 1)
    assert sorted(owner) == list(range(96))
    # field values cover 0..63 exactly once per field position
    for (name, j) in {(n, j) for n, j, _ in owner.values()}:
        assert sorted(b for n2, j2, b in owner.values() if (n2, j2) == (name, j)) == list(range(6))
    # random round trip against the element-major packer of the fixture script
    from tests.golden.make_golden import pack_scales_k4
    for _ in range(2000):
        sc = rng.integers(0, 64, 8)
        mn = rng.integers(0, 64, 8)
        q = pack_scales_k4(sc, mn)
        for j in range(8):
            assert orc.scale_min_k4(j, q) == (sc[j], mn[j])


# ---- a3/a4/a5: dequant known-answer blocks --------------------------------

@pytest.mark.parametrize("name,qtype,bs", [("q4k", 12, 144), ("q5k", 13, 176), ("q6k", 14, 210)])
def test_dequant_known_answer_blocks(name, qtype, bs):
    z = np.load(os.path.join(GOLDEN, f"kat_{name}.npz"))
    blocks, expected = z["blocks"], z["expected"]
    assert blocks.shape[1] == bs
    got = orc.dequant(qtype, blocks.reshape(-1), blocks.shape[0] * 256).reshape(-1, 256)
    assert same_bits_or_both_nan(got, expected)


def test_q6k_scale_index_rule():
    # Block with 16 distinct scales and all quants at -32: element e must use
    # scale e // 16, which is is = g*8 + l/16 (+2 per quad) of phi4.rs:463.
    z = np.load(os.path.join(GOLDEN, "kat_q6k.npz"))
    got = orc.dequant(14, z["blocks"][0], 256)
    used = np.rint(-got / 32.0).astype(int)
    for e in range(256):
        g, r = divmod(e, 128)
        u, l = divmod(r, 32)
        assert used[e] == (g * 8 + l // 16 + 2 * u) + 1


@pytest.mark.parametrize("qtype", [12, 13, 14])
def test_dequant_matches_reference_repack_layout(qtype):
    # The reference states each layout twice: dequant_q*_k (phi4.rs:444-542)
    # and repack_q*k (phi4.rs:278-436).  Both readings must agree bit for bit.
    raw = syn.weight(11, qtype, qtype, 256 * 64, 1)
    n = 256 * 64
    assert same_bits_or_both_nan(orc.dequant(qtype, raw, n), orc.dequant_via_repack(qtype, raw, n))


@pytest.mark.parametrize("qtype", [12, 13, 14])
def test_dequant_value_ranges(qtype):
    # Closed-form bounds of the formulas: Q4_K/Q5_K w in [-dmin*63, d*63*qmax],
    # Q6_K |w| <= d*128*32, on the seeded generator's blocks.
    raw = syn.weight(12, qtype, qtype, 256 * 200, 1)
    w = orc.dequant(qtype, raw, 256 * 200).reshape(-1, 256)
    blocks = raw.reshape(-1, {12: 144, 13: 176, 14: 210}[qtype])
    if qtype == 14:
        d = blocks[:, 208:210].copy().view(np.float16).astype(np.float64)[:, 0]
        assert np.all(np.abs(w) <= d[:, None] * 128 * 32 + 1e-30)
    else:
        d = blocks[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0]
        dmin = blocks[:, 2:4].copy().view(np.float16).astype(np.float64)[:, 0]
        qmax = 15 if qtype == 12 else 31
        assert np.all(w >= -dmin[:, None] * 63 - 1e-30)
        assert np.all(w <= d[:, None] * 63 * qmax + 1e-30)


# ---- a10: RMSNorm (phi4.rs:593-599) ----------------------------------------

def test_rmsnorm_closed_form_and_invariants():
    x = syn.normal_f32(3, 1, 3072)
    g = syn.normal_f32(3, 2, 3072, 1.0, 0.1)
    y = orc.rms_norm(x, g)
    xd = x.astype(np.float64)
    ref = g.astype(np.float64) * xd / np.sqrt(np.mean(xd * xd) + 1e-5)
    assert orc.normwise_err(y, ref) < 1e-6
    # gamma = 1: unit RMS (up to eps); scaling x by c leaves y unchanged
    y1 = orc.rms_norm(x, np.ones(3072, np.float32))
    assert abs(np.sqrt(np.mean(y1.astype(np.float64) ** 2)) - 1.0) < 1e-4
    y4 = orc.rms_norm(4.0 * x, g)
    assert orc.normwise_err(y4, y) < 1e-5
    # eps matters for tiny inputs exactly as the closed form says
    xs = np.full(8, 1e-4, np.float32)
    ys = orc.rms_norm(xs, np.ones(8, np.float32))
    assert np.allclose(ys, 1e-4 / np.sqrt(1e-8 + 1e-5), rtol=1e-6)


def test_silu_gate_closed_form():
    gu = syn.normal_f32(3, 3, 2 * 1000, 0.0, 4.0)
    mid = orc.silu_gate(gu, 1000)
    g = gu[:1000].astype(np.float64)
    ref = g / (1.0 + np.exp(-g)) * gu[1000:].astype(np.float64)
    assert orc.normwise_err(mid, ref) < 1e-6


def test_residual_add():
    a = syn.normal_f32(3, 4, 3072)
    b = syn.normal_f32(3, 5, 3072)
    assert np.array_equal(orc.residual_add(a, b), a + b)


# ---- a6/a8: GEMV --------------------------------------------------------------

@pytest.mark.parametrize("qtype", [12, 13, 14])
def test_gemv_one_hot_gives_dequantized_column(qtype):
    K, N = 512, 16
    W = syn.weight(5, qtype, qtype, K, N)
    deq = orc.dequant(qtype, W, K * N).reshape(N, K)
    for k in (0, 1, 31, 32, 255, 256, 300, 511):
        x = np.zeros(K, np.float32)
        x[k] = 1.0
        y = orc.gemv(qtype, W, x, K, N)[0]
        assert np.array_equal(y, deq[:, k])


@pytest.mark.parametrize("qtype", [0, 12, 13, 14])
def test_gemv_against_fp64_numpy(qtype):
    K, N, M = 1024, 24, 3
    if qtype == 0:
        W = syn.normal_f32(6, 0, N * K).view(np.uint8)
        deq = W.view(np.float32).reshape(N, K).astype(np.float64)
    else:
        W = syn.weight(6, qtype, qtype, K, N)
        deq = orc.dequant(qtype, W, K * N).reshape(N, K).astype(np.float64)
    X = syn.normal_f32(6, 1, M * K).reshape(M, K)
    ref = X.astype(np.float64) @ deq.T
    y32 = orc.gemv(qtype, W, X, K, N, M)
    y64 = orc.gemv(qtype, W, X, K, N, M, f64=True)
    assert orc.normwise_err(y64, ref) < 1e-12
    assert orc.normwise_err(y32, ref) < 1e-5
    # all-ones activation gives row sums
    ones = np.ones(K, np.float32)
    assert orc.normwise_err(orc.gemv(qtype, W, ones, K, N, 1, f64=True)[0], deq.sum(axis=1)) < 1e-12


def test_gemv_thread_count_does_not_change_result():
    K, N = 768, 33
    W = syn.weight(8, 13, 13, K, N)
    x = syn.normal_f32(8, 1, K)
    assert np.array_equal(orc.gemv(13, W, x, K, N, threads=1), orc.gemv(13, W, x, K, N, threads=5))


# ---- a11: logits chunk layout (phi4.rs:874-893) ----------------------------

def test_logits_chunk_layout_and_equivalence():
    K, V, chunk = 64, 300, 128
    E = syn.normal_f32(9, 0, V * K, 0.0, 0.02)
    Em = E.reshape(V, K)
    chunks = orc.logits_chunk_build(E, K, V, chunk)
    # independent construction: transpose each vocab slice
    ref = np.concatenate([Em[s:s + chunk].T.reshape(-1) for s in range(0, V, chunk)])
    assert np.array_equal(chunks, ref)
    x = syn.normal_f32(9, 1, K)
    y_rows = orc.logits(x, E, K, V, layout=0)
    y_chunk = orc.logits(x, chunks, K, V, layout=1, chunk=chunk)
    assert np.array_equal(y_rows, y_chunk)
    assert orc.normwise_err(y_rows, Em.astype(np.float64) @ x.astype(np.float64)) < 1e-5


# ---- committed regression record --------------------------------------------

def test_seeded_fixture_regression():
    z = np.load(os.path.join(GOLDEN, "seeded_small.npz"))
    for qt, (K, N) in {12: (512, 8), 13: (768, 6), 14: (1024, 4)}.items():
        W = z[f"w{qt}"]
        assert np.array_equal(W, syn.weight(7, 100 + qt, qt, K, N)), "generator drifted"
        assert np.array_equal(orc.dequant(qt, W, K * N), z[f"deq{qt}"])
        assert np.array_equal(orc.gemv(qt, W, z[f"x{qt}"], K, N, 4), z[f"y{qt}"])
    assert np.array_equal(orc.rms_norm(z["norm_x"], z["norm_g"]), z["norm_y"])
    assert np.array_equal(orc.silu_gate(z["silu_gu"], 512), z["silu_mid"])
    assert np.array_equal(orc.logits(z["lg_x"], z["lg_E"], 256, 120), z["lg_y"])


# ---- decode glue: f16 store, RoPE, attention ------------------------------------

def test_f32_to_f16_matches_ieee_rne():
    # every binary16 value (as f32), every midpoint between neighbours (ties to
    # even), the overflow / subnormal edges, NaN and 2^20 random floats
    h = np.arange(0x10000, dtype=np.uint32).astype(np.uint16)
    f = h.view(np.float16).astype(np.float32)
    finite = np.isfinite(f)
    got = orc.f32_to_f16_bits(f[finite])
    assert np.array_equal(got, f[finite].astype(np.float16).view(np.uint16))
    pos = np.arange(0x7BFF, dtype=np.uint32).astype(np.uint16)
    lo = pos.view(np.float16).astype(np.float64)
    hi = (pos + 1).view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)               # exact in f32
    assert np.array_equal(orc.f32_to_f16_bits(mid), mid.astype(np.float16).view(np.uint16))
    assert np.array_equal(orc.f32_to_f16_bits(-mid), (-mid).astype(np.float16).view(np.uint16))
    rng = np.random.default_rng(5)
    r = (rng.standard_normal(1 << 20) * np.exp2(rng.uniform(-30, 20, 1 << 20))).astype(np.float32)
    with np.errstate(over="ignore"):
        want = r.astype(np.float16).view(np.uint16)
    assert np.array_equal(orc.f32_to_f16_bits(r), want)
    edge = np.array([65504.0, 65519.99, 65520.0, 1e9, 2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0001, 2.0 ** -26,
                     6.1e-5, np.inf, -np.inf, 0.0, -0.0], np.float32)
    with np.errstate(over="ignore"):
        assert np.array_equal(orc.f32_to_f16_bits(edge), edge.astype(np.float16).view(np.uint16))
    nan = orc.f32_to_f16_bits(np.array([np.nan], np.float32))[0]
    assert (nan & 0x7C00) == 0x7C00 and (nan & 0x3FF) != 0


def _rope_f64(x, pos, n_heads, hd, rd, theta, attn, factors):
    """apply_rope_cfg's rotation as a complex product in double."""
    y = np.array(x, np.float64).reshape(n_heads, hd)
    i = np.arange(rd // 2)
    f = np.ones(rd // 2) if factors is None else np.concatenate([factors, np.ones(max(0, rd // 2 - len(factors)))])[:rd // 2]
    ang = pos * (theta ** (-2.0 * i / rd)) / f
    z = (y[:, 0:rd:2] + 1j * y[:, 1:rd:2]) * np.exp(1j * ang) * attn
    y[:, 0:rd:2], y[:, 1:rd:2] = z.real, z.imag
    return y.ravel()


def test_rope_pins():
    rng = np.random.default_rng(11)
    nh, hd, rd = 3, 128, 96
    x = rng.standard_normal(nh * hd).astype(np.float32)
    fac = (1.0 + rng.uniform(0, 3, rd // 2)).astype(np.float32)
    # pos 0: cos 0 = 1 and sin 0 = 0 exactly, so the rotated dims are scaled
    # by the attention factor (one f32 product each) and the rest untouched
    y0 = orc.rope(x, 0, nh, hd, rd, factors=fac).reshape(nh, hd)
    xs = x.reshape(nh, hd)
    a = np.float32(orc.ROPE_ATTN_FACTOR)
    assert np.array_equal(y0[:, :rd], xs[:, :rd] * a)
    assert np.array_equal(y0[:, rd:], xs[:, rd:])
    for pos in (1, 7, 300, 2047):
        y = orc.rope(x, pos, nh, hd, rd, factors=fac)
        ref = _rope_f64(x, pos, nh, hd, rd, orc.ROPE_THETA, orc.ROPE_ATTN_FACTOR, fac)
        # f32 angle = pos * freq carries a relative error ~2^-24: |angle| <= 2047
        assert np.max(np.abs(y - ref)) < 2e-4 * np.max(np.abs(ref))
        yy = y.reshape(nh, hd)
        # each pair's norm is scaled by the attention factor
        n0 = np.hypot(xs[:, 0:rd:2].astype(np.float64), xs[:, 1:rd:2])
        n1 = np.hypot(yy[:, 0:rd:2].astype(np.float64), yy[:, 1:rd:2])
        assert np.allclose(n1, n0 * orc.ROPE_ATTN_FACTOR, rtol=1e-5, atol=1e-6)
        assert np.array_equal(yy[:, rd:], xs[:, rd:])
    # rotations compose: pos a then pos b equals pos a + b (with attn^2)
    ab = orc.rope(orc.rope(x, 5, nh, hd, rd, attn_factor=1.0), 9, nh, hd, rd, attn_factor=1.0)
    c = orc.rope(x, 14, nh, hd, rd, attn_factor=1.0)
    assert np.max(np.abs(ab - c)) < 1e-5 * np.max(np.abs(c))
    # factors past the list are 1 (no factors at all = plain RoPE)
    p1 = orc.rope(x, 33, nh, hd, rd, factors=np.ones(1, np.float32))
    p0 = orc.rope(x, 33, nh, hd, rd)
    assert np.array_equal(p1, p0)


def test_rope_kv_store_layout():
    rng = np.random.default_rng(12)
    nh, nkv, hd, rd = 6, 2, 128, 96
    qd, kvs = nh * hd, nkv * hd
    qkv = rng.standard_normal(qd + 2 * kvs).astype(np.float32)
    kc = np.zeros(4 * kvs, np.uint16)
    vc = np.zeros(4 * kvs, np.uint16)
    out, k2, v2 = orc.rope_kv_store(qkv, kc, vc, 2, nh, nkv, hd, rd)
    assert np.array_equal(out[:qd], orc.rope(qkv[:qd], 2, nh, hd, rd))
    assert np.array_equal(out[qd:qd + kvs], orc.rope(qkv[qd:qd + kvs], 2, nkv, hd, rd))
    assert np.array_equal(out[qd + kvs:], qkv[qd + kvs:])                     # V is not rotated
    assert np.array_equal(k2[2 * kvs:3 * kvs], orc.f32_to_f16_bits(out[qd:qd + kvs]))
    assert np.array_equal(v2[2 * kvs:3 * kvs], orc.f32_to_f16_bits(qkv[qd + kvs:]))
    assert not k2[:2 * kvs].any() and not k2[3 * kvs:].any() and not v2[3 * kvs:].any()
    # rope_dim = 0 (kv_store): no rotation
    out0, k0, _ = orc.rope_kv_store(qkv, kc, vc, 1, nh, nkv, hd, 0)
    assert np.array_equal(out0, qkv)
    assert np.array_equal(k0[kvs:2 * kvs], orc.f32_to_f16_bits(qkv[qd:qd + kvs]))


def test_attention_closed_forms():
    rng = np.random.default_rng(13)
    nkv, hpk, hd = 2, 3, 128
    nh, kvs = nkv * hpk, nkv * hd
    q = rng.standard_normal(nh * hd).astype(np.float32)
    S = 9
    kc = orc.f32_to_f16_bits(rng.standard_normal(S * kvs).astype(np.float32))
    vc = orc.f32_to_f16_bits(rng.standard_normal(S * kvs).astype(np.float32))
    vf = vc.view(np.float16).astype(np.float64).reshape(S, nkv, hd)   # exact widening (pinned above)
    # one position: the softmax is 1, the output is that V row
    o1 = orc.attention_f64(q, kc, vc, 1, nkv, hpk, hd).reshape(nh, hd)
    for h in range(nh):
        assert np.array_equal(o1[h], vf[0, h // hpk])
    # equal keys: uniform weights, the mean of V
    keq = np.tile(kc[:kvs], S)
    om = orc.attention_f64(q, keq, vc, S, nkv, hpk, hd).reshape(nh, hd)
    for h in range(nh):
        assert np.allclose(om[h], vf[:, h // hpk].mean(axis=0), rtol=0, atol=1e-12)
    # one dominant key: its V
    kd = np.zeros(S * kvs, np.uint16)
    qd = np.zeros(nh * hd, np.float32)
    qd[:] = 1.0
    big = orc.f32_to_f16_bits(np.full(hd, 30.0, np.float32))
    for g in range(nkv):
        kd[4 * kvs + g * hd:4 * kvs + (g + 1) * hd] = big
    od = orc.attention_f64(qd, kd, vc, S, nkv, hpk, hd).reshape(nh, hd)
    for h in range(nh):
        assert np.allclose(od[h], vf[4, h // hpk], rtol=0, atol=1e-9)
    # query heads of one KV group with the same query agree
    qs = np.tile(q[:hd], nh)
    os_ = orc.attention_f64(qs, kc, vc, S, nkv, hpk, hd).reshape(nh, hd)
    assert np.array_equal(os_[0], os_[1]) and np.array_equal(os_[0], os_[2])
