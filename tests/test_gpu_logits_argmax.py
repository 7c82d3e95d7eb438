"""The logits with their argmax in one call (rrr_logits_rmsnorm_argmax).

On the reference's transposed chunks the argmax runs inside the split-K
logits launch: the last workgroup of each 256-entry slab reduces the slab to
its (max, first index), and the last slab to finish reduces the slabs'
candidates.  Checked on the same inputs: the logits are bitwise those of
rrr_logits_rmsnorm, and the index is both rrr_argmax_f32's on those logits
and the sequential rule of phi4.rs:1172-1183 applied on the host (start from
(-inf, 0), replace only on strictly greater: the first maximal index wins,
NaN never wins) -- with ties planted across chunks and inside one slab, a row
whose logit is NaN and rows whose logit is +inf.  Repeated calls and graph
replays return the same index (the arrival counters return to zero).
"""
import numpy as np
import pytest

import oracle.oracle as orc
import rrr_hip
from rrr_hip import synth

pytestmark = pytest.mark.gpu

K = 3072


def host_argmax(v):
    """The sequential rule, vectorised: NaN never wins, the first maximum does."""
    ok = ~np.isnan(v)
    if not ok.any():
        return 0
    m = v[ok].max()
    if m == -np.inf:
        return 0
    return int(np.flatnonzero(ok & (v == m))[0])


def run(ctx, E, x, g, V, layout, chunk):
    """(fused logits, fused index, logits of rrr_logits_rmsnorm, index of rrr_argmax_f32 on them)."""
    Eh = orc.logits_chunk_build(E, K, V, chunk) if layout == rrr_hip.LOGITS_CHUNKED else E
    Eb, xb, gb = ctx.to_device(Eh), ctx.to_device(x), ctx.to_device(g)
    y1, y2, i1, i2 = ctx.alloc(V * 4), ctx.alloc(V * 4), ctx.alloc(4), ctx.alloc(4)
    ctx.logits_rmsnorm_argmax(xb, gb, 1e-5, Eb, y1, K, V, i1, layout, chunk)
    ctx.logits_rmsnorm(xb, gb, 1e-5, Eb, y2, K, V, layout, chunk)
    ctx.argmax_f32(y2, V, i2)
    out = (ctx.download(y1), int(ctx.download(i1, np.uint32, 1)[0]), ctx.download(y2),
           int(ctx.download(i2, np.uint32, 1)[0]))
    # again: the counters came back to zero
    ctx.fill_u32(i1, 0xFFFFFFFF)
    ctx.logits_rmsnorm_argmax(xb, gb, 1e-5, Eb, y1, K, V, i1, layout, chunk)
    assert int(ctx.download(i1, np.uint32, 1)[0]) == out[1]
    for b in (Eb, xb, gb, y1, y2, i1, i2):
        b.free()
    return out


def check(ctx, E, x, g, V, layout, chunk, expect=None):
    y, idx, y_ref, idx_ref = run(ctx, E, x, g, V, layout, chunk)
    assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32))
    assert idx == idx_ref == host_argmax(y_ref)
    if expect is not None:
        assert idx == expect
    return y


def inputs(V, seed):
    E = synth.normal_f32(seed, V, V * K, 0.0, 0.02).reshape(V, K)
    x = synth.normal_f32(seed, 1, K)
    g = synth.normal_f32(seed, 2, K, 1.0, 0.1)
    return E, x, g


@pytest.mark.parametrize("V,chunk", [(20000, 8192), (65659, 8192), (1000, 256), (8195, 4096), (300, 8192)])
def test_fused_argmax_matches(ctx, V, chunk):
    E, x, g = inputs(V, 21)
    check(ctx, E.reshape(-1), x, g, V, rrr_hip.LOGITS_CHUNKED, chunk)


def test_fused_argmax_rows_layout(ctx):
    E, x, g = inputs(5000, 22)
    check(ctx, E.reshape(-1), x, g, 5000, rrr_hip.LOGITS_ROWS, 0)


def test_fused_argmax_planted_ties_nan_inf(ctx):
    V, chunk = 20000, 8192
    E, x, g = inputs(V, 23)
    normed = orc.rms_norm(x, g, 1e-5)
    big = (0.01 * normed).astype(np.float32)      # a logit far above every random row's
    # a tie across chunks and slabs: rows 17000 (chunk 2) and 300 (chunk 0)
    E[17000] = big
    E[300] = big
    # a row whose logit is NaN (inf * mixed signs) never wins
    E[50] = np.inf
    check(ctx, E.reshape(-1), x, g, V, rrr_hip.LOGITS_CHUNKED, chunk, expect=300)
    # a tie inside one slab (entries 9000 and 9003 of chunk 1), above the first
    E[9003] = 2 * big
    E[9000] = 2 * big
    check(ctx, E.reshape(-1), x, g, V, rrr_hip.LOGITS_CHUNKED, chunk, expect=9000)
    # +inf logits (one infinite weight where the normed input is positive):
    # the first of them wins over every finite logit
    k0 = int(np.flatnonzero(normed > 0)[0])
    for r in (15000, 12345):
        E[r] = 0.0
        E[r, k0] = np.inf
    y = check(ctx, E.reshape(-1), x, g, V, rrr_hip.LOGITS_CHUNKED, chunk, expect=12345)
    assert np.isposinf(y[12345]) and np.isposinf(y[15000]) and np.isnan(y[50])


def test_fused_argmax_graph_replay(ctx):
    V, chunk = 20000, 8192
    E, x, g = inputs(V, 24)
    Eb = ctx.to_device(orc.logits_chunk_build(E.reshape(-1), K, V, chunk))
    xb, gb = ctx.to_device(x), ctx.to_device(g)
    y, i = ctx.alloc(V * 4), ctx.alloc(4)
    ctx.logits_rmsnorm_argmax(xb, gb, 1e-5, Eb, y, K, V, i, rrr_hip.LOGITS_CHUNKED, chunk)
    want_y, want_i = ctx.download(y), int(ctx.download(i, np.uint32, 1)[0])
    ctx.graph_begin()
    ctx.logits_rmsnorm_argmax(xb, gb, 1e-5, Eb, y, K, V, i, rrr_hip.LOGITS_CHUNKED, chunk)
    gr = ctx.graph_end()
    for _ in range(3):
        ctx.fill_u32(y, 0)
        ctx.fill_u32(i, 0xFFFFFFFF)
        gr.launch()
        ctx.sync()
        assert int(ctx.download(i, np.uint32, 1)[0]) == want_i
        assert np.array_equal(ctx.download(y).view(np.uint32), want_y.view(np.uint32))
    gr.destroy()
    for b in (Eb, xb, gb, y, i):
        b.free()
