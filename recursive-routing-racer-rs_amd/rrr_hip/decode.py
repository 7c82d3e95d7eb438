"""Phi-4-mini-shaped decode weight sweep, batch 1.

One token of the dispatch table that the reference builds once
(phi4.rs:972-1064) and replays per token (forward_gpu, phi4.rs:1099-1168),
issued through the C ABI and normally recorded as one graph.

Per layer (phi4.rs:1006-1033), with the reference's separate dispatches
fused where the numerics allow it:

    rmsnorm(attn_norm) -> QKV GEMV            rrr_gemv_rmsnorm          Q5_K 5120x3072
    rope_kv_store + attention                 (position 0: RoPE is the identity and
                                               softmax over one key is 1, so the
                                               attention output is V gathered per
                                               GQA head)
    O-proj GEMV -> residual_add               rrr_gemv_residual(GQA_V)  Q4_K 3072x3072
    rmsnorm(ffn_norm) -> gate+up GEMV         rrr_gemv_rmsnorm          Q4_K 16384x3072
    silu_gate -> down GEMV -> residual_add    rrr_gemv_residual(SILU)   Q6_K (even layers) /
                                                                        Q4_K (odd) 3072x8192

then rmsnorm(output_norm) -> F32 logits over the transposed 8192-entry vocab
chunks (phi4.rs:874-893, 1049-1064) as rrr_logits_rmsnorm, and the argmax
that the reference does on the host (phi4.rs:1172-1195) as rrr_argmax_f32.
The fused entry points are bitwise equal to their unfused sequences.

With attention=True the sweep also owns per-layer f16 KV caches and
record_token(pos) runs the full decode step at position pos (phi4.rs:1006-1033
with the attention rows in): rope_kv_store (RoPE on Q and K, K and V stored
in row pos) and attention over rows 0..pos replace the position-0 gather,
and the O-proj GEMV takes the attention output.

Weights are seeded synthetic tensors (the recipes of synth.py); each tensor
has its own stream id, so any subset can be regenerated on the host.
"""
from dataclasses import dataclass

import numpy as np

from . import engine as E
from . import synth


@dataclass(frozen=True)
class Phi4Shape:
    d_model: int = 3072
    n_layers: int = 32
    n_heads: int = 24
    n_kv_heads: int = 8
    head_dim: int = 128
    ffn_dim: int = 8192
    vocab: int = 200064
    eps: float = 1e-5
    chunk: int = 8192            # logits vocab chunk (phi4.rs:877)
    rope_dim: int = 96           # phi4.rs:114-116
    rope_theta: float = 10000.0
    rope_attn_factor: float = 1.190238
    max_seq: int = 2048          # KV-cache rows (MAX_SEQ, phi4.rs:181)

    @property
    def qkv_dim(self):
        return self.d_model + 2 * self.n_kv_heads * self.head_dim

    @property
    def heads_per_kv(self):
        return self.n_heads // self.n_kv_heads

    @property
    def kv_stride(self):
        return self.n_kv_heads * self.head_dim

    def down_type(self, layer):
        return E.Q6_K if layer % 2 == 0 else E.Q4_K

    def layer_tensors(self, layer):
        """(name, qtype, K, N) of the layer's four weight matrices."""
        d, f = self.d_model, self.ffn_dim
        return [("attn_qkv", E.Q5_K, d, self.qkv_dim), ("attn_output", E.Q4_K, d, d),
                ("ffn_up", E.Q4_K, d, 2 * f), ("ffn_down", self.down_type(layer), f, d)]

    def bytes_per_token(self, logits="f32"):
        """Algorithmic HBM bytes of one token: raw weight bytes plus every
        activation read or written once; logits from the F32 matrix or, with
        logits="q6k", from the raw Q6_K token_embd."""
        d, f = self.d_model, self.ffn_dim
        total = 0
        for i in range(self.n_layers):
            total += 2 * 3 * d * 4                                     # two RMSNorms (x, gamma, y)
            for _, qt, K, N in self.layer_tensors(i):
                total += E.tensor_bytes(qt, K, N) + K * 4 + N * 4
        total += 3 * d * 4                                             # output norm
        emb = E.tensor_bytes(E.Q6_K, d, self.vocab) if logits == "q6k" else self.vocab * d * 4
        total += emb + d * 4 + self.vocab * 4                          # logits
        return total


# stream ids of the synthetic tensors
def _stream(layer, slot):
    return 1000 + 16 * layer + slot


S_ATTN_NORM, S_QKV, S_O, S_FFN_NORM, S_UP, S_DOWN = range(6)
S_OUT_NORM, S_EMB, S_X, S_ROPE, S_EMB_Q6K, S_PROMPT = 10, 11, 12, 13, 14, 15


def gamma_host(seed, stream, d):
    return synth.normal_f32(seed, stream, d, 1.0, 0.1)


def layer_host(seed, shape, layer):
    """Host copies of one layer: dict of raw weight bytes and norm gammas."""
    out = {"attn_norm": gamma_host(seed, _stream(layer, S_ATTN_NORM), shape.d_model),
           "ffn_norm": gamma_host(seed, _stream(layer, S_FFN_NORM), shape.d_model)}
    slots = {"attn_qkv": S_QKV, "attn_output": S_O, "ffn_up": S_UP, "ffn_down": S_DOWN}
    for name, qt, K, N in shape.layer_tensors(layer):
        out[name] = synth.weight(seed, _stream(layer, slots[name]), qt, K, N)
    return out


def embedding_chunks_host(seed, shape):
    """The logits matrix E ~ N(0, 0.02) in the reference's transposed chunk
    layout, generated directly in storage order: chunk c (n entries) holds
    B_c[d * n + v] = E[c * chunk + v][d] (phi4.rs:886)."""
    return synth.normal_f32(seed, S_EMB, shape.vocab * shape.d_model, 0.0, 0.02)


def embedding_q6k_host(seed, shape):
    """The tied token_embd as raw Q6_K super-blocks (vocab rows of d_model /
    256 blocks), the tensor the reference dequantizes into its F32 logits
    matrix (phi4.rs:709, :866-893)."""
    return synth.weight(seed, S_EMB_Q6K, E.Q6_K, shape.d_model, shape.vocab)


def prompt_host(seed, shape, M):
    """The hidden states of M prompt tokens (stand in for their embedding
    rows), rows of d_model f32."""
    return synth.normal_f32(seed, S_PROMPT, M * shape.d_model).reshape(M, shape.d_model)


def prefill_flops(shape, M):
    """2 M N K over the layer GEMMs of an M-token prompt (the MFMA work)."""
    return sum(2 * M * N * K for i in range(shape.n_layers) for _, _, K, N in shape.layer_tensors(i))


def rope_factors_host(seed, shape):
    """LongRoPE divisors of the rope_dim / 2 frequency pairs (the model's
    rope_factors_short tensor, phi4.rs:711-712), synthetic: 1 + |N(0, 1)|."""
    return (1.0 + np.abs(synth.normal_f32(seed, S_ROPE, shape.rope_dim // 2))).astype(np.float32)


def x_host(seed, shape):
    """The token's input hidden state (stands in for the embedding row)."""
    return synth.normal_f32(seed, S_X, shape.d_model)


class DecodeSweep:
    """Device weights and activations of the sweep; record_token() issues one
    token's operations on the context's stream."""

    def __init__(self, ctx, shape=Phi4Shape(), seed=3, keep_host=False, attention=False, logits="f32"):
        """logits: "f32" (the F32 matrix in the reference's transposed
        chunks), "q6k" (a raw Q6_K token_embd read as stored) or "both"
        (both held; `logits_mode` picks the one a token uses)."""
        if logits not in ("f32", "q6k", "both"):
            raise ValueError(f"logits={logits!r}")
        self.ctx, self.shape, self.seed = ctx, shape, seed
        self.host = {} if keep_host else None
        d = shape.d_model
        self.layers = []
        for i in range(shape.n_layers):
            h = layer_host(seed, shape, i)
            dev = {"attn_norm": ctx.to_device(h["attn_norm"]), "ffn_norm": ctx.to_device(h["ffn_norm"])}
            for name, qt, K, N in shape.layer_tensors(i):
                dev[name] = ctx.weight_upload(qt, K, N, h[name])
            self.layers.append(dev)
            if keep_host:
                self.host[i] = h
        out_norm = gamma_host(seed, S_OUT_NORM, d)
        x = x_host(seed, shape)
        self.out_norm = ctx.to_device(out_norm)
        self.x_in = ctx.to_device(x)
        if keep_host:
            self.host.update(out_norm=out_norm, x=x)
        self.emb = self.emb_q6k = None
        if logits in ("f32", "both"):
            emb = embedding_chunks_host(seed, shape)
            self.emb = ctx.to_device(emb)
            if keep_host:
                self.host["emb"] = emb
            del emb
        if logits in ("q6k", "both"):
            raw = embedding_q6k_host(seed, shape)
            self.emb_q6k = ctx.weight_upload(E.Q6_K, d, shape.vocab, raw)
            if keep_host:
                self.host["emb_q6k"] = raw
            del raw
        self.logits_mode = "q6k" if logits == "q6k" else "f32"
        self.zero = ctx.to_device(np.zeros(d, np.float32))
        self.hidden = ctx.alloc(d * 4)
        self.qkv = ctx.alloc(shape.qkv_dim * 4)
        self.gate_up = ctx.alloc(2 * shape.ffn_dim * 4)
        self.logits = ctx.alloc(shape.vocab * 4)
        self.token = ctx.alloc(4)
        self.attention = attention
        if attention:
            fac = rope_factors_host(seed, shape)
            self.rope_factors = ctx.to_device(fac)
            if keep_host:
                self.host["rope_factors"] = fac
            cache_bytes = shape.max_seq * shape.kv_stride * 2
            self.kv = [(ctx.alloc(cache_bytes), ctx.alloc(cache_bytes)) for _ in range(shape.n_layers)]
            self.attn_out = ctx.alloc(d * 4)

    def record_token(self, pos=None):
        """One token: the position-0 weight sweep (pos None), or with
        attention=True the full decode step at position pos."""
        c, s = self.ctx, self.shape
        d = s.d_model
        gqa = s.head_dim | (s.heads_per_kv << 16)
        if pos is not None and not (self.attention and 0 <= pos < s.max_seq):
            raise ValueError("a position needs attention=True and pos < max_seq")
        c.residual_add(self.x_in, self.zero, self.hidden, d)       # hidden = embedding row
        for i, L in enumerate(self.layers):
            c.gemv_rmsnorm(self.hidden, L["attn_norm"], s.eps, L["attn_qkv"], E.Q5_K, self.qkv, d, s.qkv_dim)
            if pos is None:
                c.gemv_residual(self.qkv, E.ACT_GQA_V, gqa, L["attn_output"], E.Q4_K, self.hidden, d, d)
            else:
                kc, vc = self.kv[i]
                c.rope_kv_store(self.qkv, self.rope_factors, s.rope_dim // 2, kc, vc, pos, s.n_heads, s.n_kv_heads,
                                s.head_dim, s.rope_dim, d, s.kv_stride, s.rope_theta, s.rope_attn_factor)
                c.attention(self.qkv, kc, vc, self.attn_out, pos + 1, s.n_kv_heads, s.heads_per_kv, s.head_dim)
                c.gemv_residual(self.attn_out, E.ACT_IDENTITY, 0, L["attn_output"], E.Q4_K, self.hidden, d, d)
            c.gemv_rmsnorm(self.hidden, L["ffn_norm"], s.eps, L["ffn_up"], E.Q4_K, self.gate_up, d, 2 * s.ffn_dim)
            c.gemv_residual(self.gate_up, E.ACT_SILU_GATE, 0, L["ffn_down"], s.down_type(i), self.hidden,
                            s.ffn_dim, d)
        self.record_logits()

    def record_logits(self):
        """Final RMSNorm + logits (F32 chunks or raw Q6_K rows, by
        logits_mode) + argmax."""
        c, s = self.ctx, self.shape
        if self.logits_mode == "q6k":
            c.logits_rmsnorm(self.hidden, self.out_norm, s.eps, self.emb_q6k, self.logits, s.d_model, s.vocab,
                             E.LOGITS_Q6K, 0)
        else:
            c.logits_rmsnorm(self.hidden, self.out_norm, s.eps, self.emb, self.logits, s.d_model, s.vocab,
                             E.LOGITS_CHUNKED, s.chunk)
        c.argmax_f32(self.logits, s.vocab, self.token)

    # ---- prefill: the prompt's tokens through every layer at once ----------
    PREFILL_ROWS = 128   # the prefill GEMM's row block; prompts are padded to it with zero rows

    def prefill_buffers(self, M):
        """Activation rows of an M-token prompt, padded to a multiple of
        PREFILL_ROWS rows (allocated once for the largest prompt so far)."""
        s, c = self.shape, self.ctx
        Mp = -(-M // self.PREFILL_ROWS) * self.PREFILL_ROWS
        pf = getattr(self, "_pf", None)
        if pf is None or pf["Mp"] < Mp:
            if pf is not None:
                for v in pf["last"].values():
                    v.free()
                for k, b in pf.items():
                    if k not in ("Mp", "last"):
                        b.free()
            d, F = s.d_model, s.ffn_dim
            pf = {"Mp": Mp, "hid": c.alloc(Mp * d * 4), "n16": c.alloc(Mp * d * 2),
                  "qkv": c.alloc(Mp * s.qkv_dim * 4), "att16": c.alloc(Mp * d * 2),
                  "gu": c.alloc(Mp * 2 * F * 4), "mid16": c.alloc(Mp * F * 2), "mid_scale": c.alloc(Mp * 4)}
            for k, b in pf.items():
                if k != "Mp":
                    c.fill_u32(b, 0)
            pf["last"] = {}   # views of the last prompt row, by prompt length
            self._pf = pf
        return pf

    def record_prefill(self, M, pos0=0):
        """The prompt's M tokens at positions pos0 .. pos0 + M - 1 through
        every layer (forward_prefill_batched, phi4.rs:1200-1445, with every
        step on the GPU): per layer RMSNorm rows -> QKV GEMM -> RoPE + KV
        store of all rows -> causal attention -> O GEMM + residual -> RMSNorm
        rows -> gate/up GEMM -> silu * up -> down GEMM + residual; then the
        final RMSNorm, logits and argmax of the last token.  The GEMM inputs
        are f16 (nearest even; silu * up in per-row block floating point);
        the hidden states, qkv and gate/up stay f32.
        The token rows must be in prefill_buffers(M)["hid"] (rows >= M zero),
        e.g. from load_prompt().  Fills cache rows pos0 .. pos0 + M - 1."""
        if not self.attention:
            raise ValueError("prefill needs attention=True (the KV caches)")
        s, c = self.shape, self.ctx
        if M < 1 or pos0 + M > s.max_seq:
            raise ValueError(f"positions {pos0}..{pos0 + M - 1} outside the cache")
        pf = self.prefill_buffers(M)
        Mp, d, F = pf["Mp"], s.d_model, s.ffn_dim
        if M < Mp:   # rows past the prompt stay zero through every step
            c.fill_u32(pf["att16"], 0, M * d * 2, (Mp - M) * d * 2)
        for i, L in enumerate(self.layers):
            kc, vc = self.kv[i]
            c.rmsnorm_f16(pf["hid"], L["attn_norm"], pf["n16"], Mp, d, s.eps)
            c.gemm_f16(pf["n16"], L["attn_qkv"], E.Q5_K, pf["qkv"], d, s.qkv_dim, Mp)
            c.rope_kv_store_rows(pf["qkv"], M, self.rope_factors, s.rope_dim // 2, kc, vc, pos0, s.n_heads,
                                 s.n_kv_heads, s.head_dim, s.rope_dim, d, s.kv_stride, s.rope_theta,
                                 s.rope_attn_factor)
            c.attention_prefill(pf["qkv"], M, kc, vc, pf["att16"], pos0, s.n_kv_heads, s.heads_per_kv, s.head_dim,
                                out_type=E.F16)
            c.gemm_f16(pf["att16"], L["attn_output"], E.Q4_K, pf["hid"], d, d, Mp, accumulate=True)
            c.rmsnorm_f16(pf["hid"], L["ffn_norm"], pf["n16"], Mp, d, s.eps)
            c.gemm_f16(pf["n16"], L["ffn_up"], E.Q4_K, pf["gu"], d, 2 * F, Mp)
            c.silu_gate_f16(pf["gu"], pf["mid16"], pf["mid_scale"], Mp, F)
            c.gemm_f16(pf["mid16"], L["ffn_down"], s.down_type(i), pf["hid"], F, d, Mp, accumulate=True,
                       row_scale=pf["mid_scale"])
        if M not in pf["last"]:
            pf["last"][M] = c.view(pf["hid"], (M - 1) * d * 4, d * 4)
        hidden, self.hidden = self.hidden, pf["last"][M]
        try:
            self.record_logits()
        finally:
            self.hidden = hidden

    def load_prompt(self, rows):
        """Upload prompt hidden rows (M x d_model f32) into the prefill
        buffers, zeroing the padding rows."""
        M = rows.shape[0]
        pf = self.prefill_buffers(M)
        d = self.shape.d_model
        self.ctx.upload(pf["hid"], np.ascontiguousarray(rows, np.float32))
        if M < pf["Mp"]:
            self.ctx.fill_u32(pf["hid"], 0, M * d * 4, (pf["Mp"] - M) * d * 4)
        return pf

    def prefill_results(self, M):
        """(logits of the last token, argmax, hidden rows M x d_model)."""
        c, s = self.ctx, self.shape
        hid = c.download(self._pf["hid"], np.float32, M * s.d_model).reshape(M, s.d_model)
        return (c.download(self.logits, np.float32, s.vocab), int(c.download(self.token, np.uint32, 1)[0]), hid)

    def sweep_ops(self):
        """The 4 fused GEMVs of every layer as one persistent sweep's op list
        (the same calls record_token issues one by one)."""
        s = self.shape
        d = s.d_model
        gqa = s.head_dim | (s.heads_per_kv << 16)
        ops = []
        for i, L in enumerate(self.layers):
            ops += [("rmsnorm", self.hidden, L["attn_norm"], s.eps, L["attn_qkv"], E.Q5_K, self.qkv, d, s.qkv_dim),
                    ("residual", self.qkv, E.ACT_GQA_V, gqa, L["attn_output"], E.Q4_K, self.hidden, d, d),
                    ("rmsnorm", self.hidden, L["ffn_norm"], s.eps, L["ffn_up"], E.Q4_K, self.gate_up, d,
                     2 * s.ffn_dim),
                    ("residual", self.gate_up, E.ACT_SILU_GATE, 0, L["ffn_down"], s.down_type(i), self.hidden,
                     s.ffn_dim, d)]
        return ops

    def run_token_sweep(self, sweep):
        """One token with the layers as one persistent launch (`sweep` from
        ctx.sweep(self.sweep_ops())), the logits and argmax as before."""
        c, s = self.ctx, self.shape
        c.residual_add(self.x_in, self.zero, self.hidden, s.d_model)
        sweep.run()
        self.record_logits()

    def graph(self, pos=None, logits=None):
        """One token as a HIP graph; logits ("f32" / "q6k") overrides
        logits_mode for it."""
        mode = self.logits_mode
        if logits is not None:
            if (self.emb_q6k if logits == "q6k" else self.emb) is None:
                raise ValueError(f"no {logits} logits matrix was built")
            self.logits_mode = logits
        try:
            self.ctx.graph_begin()
            self.record_token(pos)
            return self.ctx.graph_end()
        finally:
            self.logits_mode = mode

    def results(self):
        """(logits f32[vocab], argmax index, final hidden state f32[d])."""
        c = self.ctx
        return (c.download(self.logits, np.float32, self.shape.vocab),
                int(c.download(self.token, np.uint32, 1)[0]),
                c.download(self.hidden, np.float32, self.shape.d_model))
