"""GPU tests of the GGUF raw-upload path.

The seeded synthetic model exported with write_synthetic_gguf and loaded
through the reader (rrr_gguf_upload, DecodeSweep(gguf=...)) must run
bit-identically to the same weights uploaded from memory -- the decode sweep,
decode steps with attention, and a prefill -- and the input row that embed()
dequantizes on the device from the raw token_embd must equal the oracle's
dequantization of that row bit for bit.  A layout the export does not
produce (untied Q6_K output.weight, Q4_K token_embd, F16 norms, no rope
factors) is checked against the oracle's fp64 composition.
"""
import dataclasses

import numpy as np
import pytest

import oracle.oracle as orc
import rrr_hip
from rrr_hip import decode, synth
from rrr_hip import gguf as G

pytestmark = pytest.mark.gpu

SHAPE = dataclasses.replace(decode.Phi4Shape(), n_layers=2, vocab=20000, max_seq=128)


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    p = tmp_path_factory.mktemp("gguf") / "synthetic.gguf"
    decode.write_synthetic_gguf(p, SHAPE, seed=3, alignment=64)
    m = G.GGUFModel.load(p)
    yield m
    m.close()


def test_upload_holds_the_file_bytes(ctx, model):
    for name in ("blk.0.attn_qkv.weight", "blk.1.ffn_down.weight", "blk.0.ffn_up.weight", "token_embd.weight",
                 "output_norm.weight"):
        buf = model.upload(ctx, name)
        try:
            assert np.array_equal(ctx.download(buf, np.uint8), model.tensor_bytes(name)), name
        finally:
            buf.free()


def test_embed_is_the_dequantized_row(ctx, model):
    sw = decode.DecodeSweep(ctx, SHAPE, gguf=model, logits="q6k")
    d = SHAPE.d_model
    row_bytes = d // 256 * 210
    raw = model.tensor_bytes("token_embd.weight")
    for tok in (0, 1, 4097, SHAPE.vocab - 1):
        sw.embed(tok)
        got = ctx.download(sw.x_in, np.float32, d)
        ref = orc.dequant(rrr_hip.Q6_K, np.ascontiguousarray(raw[tok * row_bytes:(tok + 1) * row_bytes]), d)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), tok
    with pytest.raises(ValueError):
        sw.embed(SHAPE.vocab)


def same(a, b):
    la, ta, ha = a.results()
    lb, tb, hb = b.results()
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    assert np.array_equal(ha.view(np.uint32), hb.view(np.uint32))
    assert ta == tb
    return la, ta


def test_gguf_model_runs_bitwise_like_the_synthetic_one(ctx, model):
    a = decode.DecodeSweep(ctx, SHAPE, seed=3, gguf=model, logits="q6k", attention=True)
    b = decode.DecodeSweep(ctx, SHAPE, seed=3, logits="q6k", attention=True)
    assert [L["types"] for L in a.layers] == [L["types"] for L in b.layers]
    a.embed(777)
    ctx.upload(b.x_in, ctx.download(a.x_in, np.float32, SHAPE.d_model))
    for sw in (a, b):
        sw.record_token()
    ctx.sync()
    logits, tok = same(a, b)
    assert np.all(np.isfinite(logits)) and tok == int(np.argmax(logits))
    for pos in range(3):
        for sw in (a, b):
            sw.record_token(pos)
        ctx.sync()
        same(a, b)
    M, pos0 = 40, 3
    rows = decode.prompt_host(3, SHAPE, M)
    out = []
    for sw in (a, b):
        sw.load_prompt(rows)
        sw.record_prefill(M, pos0)
        ctx.sync()
        out.append(sw.prefill_results(M))
    (la, ta, ha), (lb, tb, hb) = out
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32)) and ta == tb
    assert np.array_equal(ha.view(np.uint32), hb.view(np.uint32))
    assert np.all(np.isfinite(ha))


def test_gguf_layout_errors(ctx, tmp_path):
    s = dataclasses.replace(SHAPE, n_layers=1, vocab=512)
    p = tmp_path / "bad.gguf"
    decode.write_synthetic_gguf(p, s, seed=1)
    with G.GGUFModel.load(p) as m:
        with pytest.raises(ValueError):
            decode.DecodeSweep(ctx, s, gguf=m, logits="f32")
    # a Qwen2-style layout (separate Q/K/V) is refused before any upload
    md = [("general.architecture", G.STRING, "qwen2"), ("qwen2.embedding_length", G.UINT32, 256),
          ("qwen2.attention.head_count", G.UINT32, 2), ("qwen2.block_count", G.UINT32, 1)]
    G.write_gguf(tmp_path / "qwen.gguf", md, [("blk.0.attn_q.weight", 0, (256, 256), np.zeros(65536, np.float32)),
                                               ("token_embd.weight", 14, (256, 8), np.zeros(8 * 210, np.uint8))])
    with G.GGUFModel.load(tmp_path / "qwen.gguf") as m:
        with pytest.raises(ValueError, match="Qwen2"):
            decode.DecodeSweep(ctx, s, gguf=m, logits="q6k")


def test_untied_output_f16_norms_without_rope_factors(ctx, tmp_path):
    """A GGUF layout the synthetic export does not produce: a Q4_K token_embd
    with a separate Q6_K output.weight, F16 norm weights, no rope factors.
    The position-0 token from embed(t) against the oracle composed in fp64
    over the file's own tensors (1e-4 normwise)."""
    s = dataclasses.replace(SHAPE, n_layers=1, vocab=2000)
    d, F = s.d_model, s.ffn_dim
    L = decode.layer_host(9, s, 0)
    f16 = lambda v: v.astype(np.float16)
    emb = synth.weight(9, 500, rrr_hip.Q4_K, d, s.vocab)
    outw = synth.weight(9, 501, rrr_hip.Q6_K, d, s.vocab)
    onorm = f16(decode.gamma_host(9, 502, d))
    md = [("general.architecture", G.STRING, "phi3"), ("phi3.embedding_length", G.UINT32, d),
          ("phi3.feed_forward_length", G.UINT32, F), ("phi3.block_count", G.UINT32, 1),
          ("phi3.attention.head_count", G.UINT32, s.n_heads),
          ("phi3.attention.head_count_kv", G.UINT32, s.n_kv_heads), ("phi3.rope.dimension_count", G.UINT32, s.rope_dim)]
    tensors = [("token_embd.weight", rrr_hip.Q4_K, (d, s.vocab), emb),
               ("output.weight", rrr_hip.Q6_K, (d, s.vocab), outw),
               ("output_norm.weight", rrr_hip.F16, (d,), onorm),
               ("blk.0.attn_norm.weight", rrr_hip.F16, (d,), f16(L["attn_norm"])),
               ("blk.0.ffn_norm.weight", rrr_hip.F16, (d,), f16(L["ffn_norm"]))]
    for name, qt, K, N in s.layer_tensors(0):
        tensors.append((f"blk.0.{name}.weight", qt, (K, N), L[name]))
    p = tmp_path / "untied.gguf"
    G.write_gguf(p, md, tensors)
    tok = 1234
    with G.GGUFModel.load(p) as m:
        cfg = G.ModelConfig.from_gguf(m)
        assert cfg.has_output_weight and not cfg.has_rope_factors
        sw = decode.DecodeSweep(ctx, s, gguf=m, logits="q6k")
        sw.embed(tok)
        sw.record_token()
        ctx.sync()
        logits, top, hidden = sw.results()
        del sw
    row = emb.reshape(s.vocab, -1)[tok]
    h = orc.dequant(rrr_hip.Q4_K, np.ascontiguousarray(row), d).astype(np.float64)
    g32 = lambda v: v.astype(np.float32)
    normed = orc.rms_norm(h.astype(np.float32), g32(f16(L["attn_norm"])), s.eps)
    qkv = orc.gemv(rrr_hip.Q5_K, L["attn_qkv"], normed, d, s.qkv_dim, 1, 16, f64=True)[0]
    v = qkv[d + s.n_kv_heads * s.head_dim:].reshape(s.n_kv_heads, s.head_dim)
    att = np.repeat(v, s.heads_per_kv, axis=0).reshape(-1).astype(np.float32)
    h = h + orc.gemv(rrr_hip.Q4_K, L["attn_output"], att, d, d, 1, 16, f64=True)[0]
    normed = orc.rms_norm(h.astype(np.float32), g32(f16(L["ffn_norm"])), s.eps)
    gu = orc.gemv(rrr_hip.Q4_K, L["ffn_up"], normed, d, 2 * F, 1, 16, f64=True)[0]
    mid = orc.silu_gate(gu.astype(np.float32), F)
    h = h + orc.gemv(s.down_type(0), L["ffn_down"], mid, F, d, 1, 16, f64=True)[0]
    normed = orc.rms_norm(h.astype(np.float32), g32(onorm), s.eps)
    ref = orc.gemv(rrr_hip.Q6_K, outw, normed, d, s.vocab, 1, 16, f64=True)[0]
    assert orc.normwise_err(hidden, h) < 1e-4
    assert orc.normwise_err(logits, ref) < 1e-4
    assert top == int(np.argmax(logits))
