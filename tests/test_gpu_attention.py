"""GPU parity of the decode glue: RoPE + the f16 KV-cache store
(rope_kv_store / kv_store) and decode attention, against the CPU oracle.

Bars.  V rows of the cache are bit-exact (no arithmetic before the f16
rounding).  RoPE computes its angle pos * freq in f32 as the reference does,
so the angle itself carries a relative error near 2^-24 and the rotated
values may differ from the oracle by up to about pos * 2^-22 of their size
(the GPU's powf / sincos and the host libm may round freq differently);
the bound used is 4 * pos * 2^-24 + 1e-6 normwise, and K rows of the cache
are within that plus one f16 rounding (and equal the f16 rounding of the
GPU's own rotated K).  At pos 0 the rotation is an exact scaling,
so Q, K and the cache are bit-exact there.  Attention is within 1e-4
normwise of the fp64 oracle; one cached row gives that V row exactly.
"""
import numpy as np
import pytest

import oracle.oracle as orc
import rrr_hip

pytestmark = pytest.mark.gpu

NH, NKV, HD, RD = 24, 8, 128, 96
QD, KVS = NH * HD, NKV * HD
MAX_SEQ = 2048
TOL = 1e-4


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


@pytest.mark.parametrize("pos", [0, 1, 5, 333, 2047])
def test_rope_kv_store_parity(ctx, caches, pos):
    kc, vc = caches
    rng = np.random.default_rng(100 + pos)
    qkv = rng.standard_normal(QD + 2 * KVS).astype(np.float32)
    fac = factors()
    # a marker pattern in the rows around pos shows that only row pos is written
    lo, hi = max(0, pos - 2), min(MAX_SEQ, pos + 3)
    marker = np.full((hi - lo) * KVS, 0x5A5A, np.uint16)
    ctx.upload(kc, marker, offset=lo * KVS * 2)
    ctx.upload(vc, marker, offset=lo * KVS * 2)
    d_qkv = ctx.to_device(qkv)
    d_fac = ctx.to_device(fac)
    ctx.rope_kv_store(d_qkv, d_fac, RD // 2, kc, vc, pos, NH, NKV, HD, RD, QD, KVS)
    got = ctx.download(d_qkv, np.float32, QD + 2 * KVS)
    kg = ctx.download(kc, np.uint16, (hi - lo) * KVS, offset=lo * KVS * 2).reshape(hi - lo, KVS)
    vg = ctx.download(vc, np.uint16, (hi - lo) * KVS, offset=lo * KVS * 2).reshape(hi - lo, KVS)
    ref, kref, vref = orc.rope_kv_store(qkv, np.zeros((pos + 1) * KVS, np.uint16),
                                        np.zeros((pos + 1) * KVS, np.uint16), pos, NH, NKV, HD, RD, factors=fac)
    r = pos - lo
    assert np.array_equal(vg[r], vref[pos * KVS:])                              # V: bit-exact
    assert np.array_equal(got[QD + KVS:], qkv[QD + KVS:])                       # V not rotated
    if pos == 0:
        assert np.array_equal(got, ref)
        assert np.array_equal(kg[r], kref[:KVS])
    else:
        assert orc.normwise_err(got[:QD], ref[:QD]) < rope_bound(pos)
        assert orc.normwise_err(got[QD:QD + KVS], ref[QD:QD + KVS]) < rope_bound(pos)
        # the cached K is within the rotation bound plus one f16 rounding of
        # the oracle's rotated K
        kf = kg[r].view(np.float16).astype(np.float64)
        kr = ref[QD:QD + KVS].astype(np.float64)
        assert np.all(np.abs(kf - kr) <= rope_bound(pos) * np.max(np.abs(kr)) + np.abs(kr) * 2.0 ** -11 + 2.0 ** -25)
        # the cache holds the f16 rounding of the GPU's own rotated K
        assert np.array_equal(kg[r], orc.f32_to_f16_bits(got[QD:QD + KVS]))
    for rr in range(hi - lo):
        if rr != r:
            assert np.all(kg[rr] == 0x5A5A) and np.all(vg[rr] == 0x5A5A)
    d_qkv.free(); d_fac.free()


def test_rope_kv_store_dispatch_names(ctx, caches):
    """rope_kv_store and kv_store through rrr_dispatch with the reference's
    binding order and push layouts equal the typed entry point."""
    kc, vc = caches
    rng = np.random.default_rng(7)
    qkv = rng.standard_normal(QD + 2 * KVS).astype(np.float32)
    fac = factors()
    a, c = ctx.to_device(qkv), ctx.to_device(qkv)
    d_fac = ctx.to_device(fac)
    pos = 40
    ctx.rope_kv_store(a, d_fac, RD // 2, kc, vc, pos, NH, NKV, HD, RD, QD, KVS)
    k_typed = ctx.download(kc, np.uint16, KVS, offset=pos * KVS * 2)
    ctx.fill_u32(kc, 0)
    rp = (NH + NKV) * (RD // 2)
    ctx.dispatch("rope_kv_store", [c, d_fac, kc, vc], [pos, NH, NKV, HD, RD, QD, KVS],
                 [(max(rp, KVS // 2) + 63) // 64, 1, 1])
    assert np.array_equal(ctx.download(c, np.float32, QD + 2 * KVS), ctx.download(a, np.float32, QD + 2 * KVS))
    assert np.array_equal(ctx.download(kc, np.uint16, KVS, offset=pos * KVS * 2), k_typed)
    # kv_store: no rotation, K and V rounded to f16 into row pos
    d = ctx.to_device(qkv)
    ctx.dispatch("kv_store", [d, kc, vc], [pos, QD, KVS], [(KVS // 2 + 255) // 256, 1, 1])
    assert np.array_equal(ctx.download(d, np.float32, QD + 2 * KVS), qkv)
    assert np.array_equal(ctx.download(kc, np.uint16, KVS, offset=pos * KVS * 2),
                          orc.f32_to_f16_bits(qkv[QD:QD + KVS]))
    assert np.array_equal(ctx.download(vc, np.uint16, KVS, offset=pos * KVS * 2),
                          orc.f32_to_f16_bits(qkv[QD + KVS:]))
    for buf in (a, c, d, d_fac):
        buf.free()


def test_rope_kv_store_dispatch_placeholder_factor(ctx, caches):
    """A model without rope factors binds a one-float buffer that is never
    uploaded (phi4.rs:965-967); the shim reads it as no factors (factor 1,
    apply_rope_cfg's empty list, phi4.rs:243), whatever the float holds."""
    kc, vc = caches
    rng = np.random.default_rng(11)
    qkv = rng.standard_normal(QD + 2 * KVS).astype(np.float32)
    a, c = ctx.to_device(qkv), ctx.to_device(qkv)
    junk = ctx.to_device(np.array([7.25], np.float32))
    pos = 9
    ctx.rope_kv_store(a, None, 0, kc, vc, pos, NH, NKV, HD, RD, QD, KVS)
    k_typed = ctx.download(kc, np.uint16, KVS, offset=pos * KVS * 2)
    ctx.fill_u32(kc, 0)
    rp = (NH + NKV) * (RD // 2)
    ctx.dispatch("rope_kv_store", [c, junk, kc, vc], [pos, NH, NKV, HD, RD, QD, KVS],
                 [(max(rp, KVS // 2) + 63) // 64, 1, 1])
    assert np.array_equal(ctx.download(c, np.float32, QD + 2 * KVS), ctx.download(a, np.float32, QD + 2 * KVS))
    assert np.array_equal(ctx.download(kc, np.uint16, KVS, offset=pos * KVS * 2), k_typed)
    ref, _, _ = orc.rope_kv_store(qkv, np.zeros((pos + 1) * KVS, np.uint16), np.zeros((pos + 1) * KVS, np.uint16),
                                  pos, NH, NKV, HD, RD, factors=None)
    assert orc.normwise_err(ctx.download(c, np.float32, QD)[:QD], ref[:QD]) < rope_bound(pos)
    for buf in (a, c, junk):
        buf.free()


def _random_cache(rng, seq, nkv, scale=1.0):
    k = orc.f32_to_f16_bits((rng.standard_normal(seq * nkv * HD) * scale).astype(np.float32))
    v = orc.f32_to_f16_bits(rng.standard_normal(seq * nkv * HD).astype(np.float32))
    return k, v


@pytest.mark.parametrize("seq", [1, 2, 15, 16, 17, 100, 1000, 2047, 2048])
def test_attention_parity_phi4_shape(ctx, caches, seq):
    kc, vc = caches
    rng = np.random.default_rng(200 + seq)
    k, v = _random_cache(rng, seq, NKV)
    ctx.upload(kc, k)
    ctx.upload(vc, v)
    q = rng.standard_normal(QD).astype(np.float32)
    dq, out = ctx.to_device(q), ctx.alloc(QD * 4)
    ctx.attention(dq, kc, vc, out, seq, NKV, NH // NKV, HD)
    got = ctx.download(out, np.float32, QD)
    ref = orc.attention_f64(q, k, v, seq, NKV, NH // NKV, HD)
    assert np.all(np.isfinite(got))
    assert orc.normwise_err(got, ref) < TOL
    if seq == 1:
        vf = v.view(np.float16).astype(np.float32).reshape(NKV, HD)
        assert np.array_equal(got.reshape(NH, HD), np.repeat(vf, NH // NKV, axis=0))
    dq.free(); out.free()


@pytest.mark.parametrize("nkv,hpk,seq", [(1, 1, 300), (4, 2, 64), (2, 8, 513), (8, 4, 2048), (1, 5, 7)])
def test_attention_gqa_shapes(ctx, caches, nkv, hpk, seq):
    kc, vc = caches
    rng = np.random.default_rng(nkv * 1000 + hpk * 10 + seq)
    k, v = _random_cache(rng, seq, nkv, scale=2.0)
    ctx.upload(kc, k)
    ctx.upload(vc, v)
    q = (rng.standard_normal(nkv * hpk * HD) * 2.0).astype(np.float32)   # peaked softmax
    dq, out = ctx.to_device(q), ctx.alloc(nkv * hpk * HD * 4)
    ctx.attention(dq, kc, vc, out, seq, nkv, hpk, HD)
    got = ctx.download(out, np.float32, nkv * hpk * HD)
    ref = orc.attention_f64(q, k, v, seq, nkv, hpk, HD)
    assert orc.normwise_err(got, ref) < TOL
    dq.free(); out.free()


def test_attention_dispatch_name_and_graph_replay(ctx, caches):
    kc, vc = caches
    rng = np.random.default_rng(9)
    seq = 777
    k, v = _random_cache(rng, seq, NKV)
    ctx.upload(kc, k)
    ctx.upload(vc, v)
    q = rng.standard_normal(QD).astype(np.float32)
    dq, o1, o2 = ctx.to_device(q), ctx.alloc(QD * 4), ctx.alloc(QD * 4)
    ctx.attention(dq, kc, vc, o1, seq, NKV, NH // NKV, HD)
    ctx.dispatch("attention", [dq, kc, vc, o2], [seq, NKV, NH // NKV, HD], [NH, 1, 1])
    a = ctx.download(o1, np.float32, QD)
    assert np.array_equal(a, ctx.download(o2, np.float32, QD))
    ctx.graph_begin()
    ctx.attention(dq, kc, vc, o2, seq, NKV, NH // NKV, HD)
    g = ctx.graph_end()
    for _ in range(3):
        ctx.fill_u32(o2, 0)
        g.launch()
        ctx.sync()
        assert np.array_equal(ctx.download(o2, np.float32, QD), a)
    g.destroy()
    for b in (dq, o1, o2):
        b.free()


@pytest.mark.parametrize("pos,with_factors", [(0, True), (1, True), (77, False), (2047, True)])
def test_gemv_rmsnorm_rope_kv_is_the_two_launches(ctx, caches, pos, with_factors):
    """rrr_gemv_rmsnorm_rope_kv (rmsnorm -> QKV -> rope_kv_store in one
    launch, phi4.rs:1006-1017) leaves qkv and both cache rows bit for bit as
    rrr_gemv_rmsnorm followed by rrr_rope_kv_store, on the Phi-4-mini QKV
    shape (Q5_K 5120 x 3072: tiles of 10 rows, RoPE pairs inside a tile)."""
    from rrr_hip import synth
    kc, vc = caches
    K, N = QD, QD + 2 * KVS
    raw = synth.weight(7, 90 + pos, rrr_hip.Q5_K, K, N)
    W = ctx.weight_upload(rrr_hip.Q5_K, K, N, raw)
    x = ctx.to_device(synth.normal_f32(7, 91, K))
    g = ctx.to_device(synth.normal_f32(7, 92, K, 1.0, 0.1))
    fac = ctx.to_device(factors()) if with_factors else None
    nf = RD // 2 if with_factors else 0
    q1, q2 = ctx.alloc(N * 4), ctx.alloc(N * 4)
    rows = []
    for fused, q in ((False, q1), (True, q2)):
        ctx.fill_u32(kc, 0x5A5A5A5A, pos * KVS * 2, KVS * 2)
        ctx.fill_u32(vc, 0x5A5A5A5A, pos * KVS * 2, KVS * 2)
        if fused:
            ctx.gemv_rmsnorm_rope_kv(x, g, 1e-5, W, rrr_hip.Q5_K, q, K, fac, nf, kc, vc, pos, NH, NKV, HD, RD, QD, KVS)
        else:
            ctx.gemv_rmsnorm(x, g, 1e-5, W, rrr_hip.Q5_K, q, K, N)
            ctx.rope_kv_store(q, fac, nf, kc, vc, pos, NH, NKV, HD, RD, QD, KVS)
        rows.append((ctx.download(q, np.uint32, N), ctx.download(kc, np.uint16, KVS, offset=pos * KVS * 2),
                     ctx.download(vc, np.uint16, KVS, offset=pos * KVS * 2)))
    for a, b in zip(rows[0], rows[1]):
        assert np.array_equal(a, b)
    assert not np.all(rows[1][2] == 0x5A5A)   # the V row was written
    for b in (W, x, g, q1, q2) + ((fac,) if fac is not None else ()):
        b.free()


@pytest.mark.parametrize("qtype,K,nh,nkv,hd,rd,pos", [
    (rrr_hip.Q4_K, 3072, 24, 8, 128, 96, 5),       # Q4_K rows, tiles of 10
    (rrr_hip.Q6_K, 3072, 24, 8, 128, 96, 300),     # Q6_K rows
    (rrr_hip.Q5_K, 3072, 16, 8, 128, 128, 9),      # N = 4096: one tile of 16 rows per workgroup
    (rrr_hip.Q5_K, 3072, 64, 64, 128, 64, 33),     # N = 24,576: several tiles per workgroup
    (rrr_hip.Q4_K, 8192, 24, 8, 128, 96, 2),       # K = 8192: two super-blocks a wave
    (rrr_hip.Q5_K, 3072, 24, 8, 128, 0, 7),        # rope_dim 0: the kv_store form
    (rrr_hip.Q4_K, 512, 1, 1, 1024, 1024, 11),     # 512 rotation pairs on a 256-thread workgroup
])
def test_gemv_rope_kv_forms_are_the_two_launches(ctx, qtype, K, nh, nkv, hd, rd, pos):
    """The fused QKV + RoPE + KV-store GEMV on every tile plan and weight
    type it takes leaves qkv and both cache rows bit for bit as the GEMV
    followed by rrr_rope_kv_store."""
    from rrr_hip import synth
    qd, kvs = nh * hd, nkv * hd
    N = qd + 2 * kvs
    raw = synth.weight(8, 10 + qtype, qtype, K, N)
    W = ctx.weight_upload(qtype, K, N, raw)
    x = ctx.to_device(synth.normal_f32(8, 11, K))
    g = ctx.to_device(synth.normal_f32(8, 12, K, 1.0, 0.1))
    nf = rd // 2
    fac = ctx.to_device((1.0 + np.random.default_rng(rd).uniform(0.0, 3.0, nf)).astype(np.float32)) if nf else None
    kc, vc = ctx.alloc((pos + 1) * kvs * 2), ctx.alloc((pos + 1) * kvs * 2)
    q1, q2 = ctx.alloc(N * 4), ctx.alloc(N * 4)
    rows = []
    for fused, q in ((False, q1), (True, q2)):
        ctx.fill_u32(kc, 0x5A5A5A5A)
        ctx.fill_u32(vc, 0x5A5A5A5A)
        if fused:
            ctx.gemv_rmsnorm_rope_kv(x, g, 1e-5, W, qtype, q, K, fac, nf, kc, vc, pos, nh, nkv, hd, rd, qd, kvs)
        else:
            ctx.gemv_rmsnorm(x, g, 1e-5, W, qtype, q, K, N)
            ctx.rope_kv_store(q, fac, nf, kc, vc, pos, nh, nkv, hd, rd, qd, kvs)
        rows.append((ctx.download(q, np.uint32, N), ctx.download(kc, np.uint16, (pos + 1) * kvs),
                     ctx.download(vc, np.uint16, (pos + 1) * kvs)))
    for a, b in zip(rows[0], rows[1]):
        assert np.array_equal(a, b)
    assert not np.all(rows[1][2][pos * kvs:] == 0x5A5A)   # row pos of V was written
    assert np.all(rows[1][1][:pos * kvs] == 0x5A5A)       # and no other row
    for b in (W, x, g, kc, vc, q1, q2) + ((fac,) if fac is not None else ()):
        b.free()

