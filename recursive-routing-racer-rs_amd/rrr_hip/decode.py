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
    rmsnorm(ffn_norm) -> gate+up GEMV         rrr_gemv_rmsnorm_silu     Q4_K 16384x3072
      -> silu_gate                            (silu * up in its epilogue)
    down GEMV -> residual_add                 rrr_gemv_residual         Q6_K (even layers) /
                                                                        Q4_K (odd) 3072x8192
    (silu_fused False: rrr_gemv_rmsnorm into the 2F gate/up rows, then
    rrr_gemv_residual(SILU) with silu_gate in the down GEMV's prologue)

then rmsnorm(output_norm) -> F32 logits over the transposed 8192-entry vocab
chunks (phi4.rs:874-893, 1049-1064) as rrr_logits_rmsnorm, and the argmax
that the reference does on the host (phi4.rs:1172-1195) as rrr_argmax_f32.
The fused entry points are bitwise equal to their unfused sequences.

With attention=True the sweep also owns per-layer f16 KV caches and
record_token(pos) runs the full decode step at position pos (phi4.rs:1006-1033
with the attention rows in): rope_kv_store (RoPE on Q and K, K and V stored
in row pos; in the QKV GEMV's epilogue, rrr_gemv_rmsnorm_rope_kv) and
attention over rows 0..pos replace the position-0 gather, and the O-proj GEMV
takes the attention output.

Weights are seeded synthetic tensors (the recipes of synth.py; each tensor
has its own stream id, so any subset can be regenerated on the host), or a
GGUF model's tensors uploaded as stored (DecodeSweep(..., gguf=model)), the
weight types then read per tensor from the file.
"""
from dataclasses import dataclass

import numpy as np

from . import engine as E
from . import synth
from .gguf import ModelConfig


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


def shape_from_config(cfg, max_seq=2048, chunk=8192):
    """The decode shape of a model configuration read from GGUF metadata."""
    return Phi4Shape(d_model=cfg.d_model, n_layers=cfg.n_layers, n_heads=cfg.n_heads, n_kv_heads=cfg.n_kv_heads,
                     head_dim=cfg.head_dim, ffn_dim=cfg.ffn_dim, vocab=cfg.vocab_size, eps=cfg.rms_eps, chunk=chunk,
                     rope_dim=cfg.rope_dim, rope_theta=cfg.rope_theta, rope_attn_factor=cfg.rope_attn_factor,
                     max_seq=max_seq)


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


def write_synthetic_gguf(path, shape, seed=3, alignment=32):
    """Writes the seeded synthetic model of `shape` as a Phi-3-architecture
    GGUF file: the metadata keys ModelConfig.from_gguf reads, and the tensors
    DecodeSweep(gguf=...) loads under their GGUF names, holding the same bytes
    as the synthetic sweep of the same seed (the Q6_K token_embd tied to the
    output).  Returns the data section's file offset."""
    from . import gguf as G
    a = "phi3"
    md = [("general.architecture", G.STRING, a), ("general.name", G.STRING, f"synthetic seed {seed}"),
          (f"{a}.context_length", G.UINT32, shape.max_seq), (f"{a}.embedding_length", G.UINT32, shape.d_model),
          (f"{a}.feed_forward_length", G.UINT32, shape.ffn_dim), (f"{a}.block_count", G.UINT32, shape.n_layers),
          (f"{a}.attention.head_count", G.UINT32, shape.n_heads),
          (f"{a}.attention.head_count_kv", G.UINT32, shape.n_kv_heads),
          (f"{a}.attention.layer_norm_rms_epsilon", G.FLOAT32, shape.eps),
          (f"{a}.rope.dimension_count", G.UINT32, shape.rope_dim),
          (f"{a}.rope.freq_base", G.FLOAT32, shape.rope_theta),
          (f"{a}.rope.scaling.attn_factor", G.FLOAT32, shape.rope_attn_factor),
          ("general.file_type", G.UINT32, 15), ("general.quantization_version", G.UINT32, 2)]
    d = shape.d_model
    fac = rope_factors_host(seed, shape)
    tensors = [("token_embd.weight", E.Q6_K, (d, shape.vocab), embedding_q6k_host(seed, shape)),
               ("output_norm.weight", E.F32, (d,), gamma_host(seed, S_OUT_NORM, d)),
               ("rope_factors_long.weight", E.F32, (fac.size,), fac),
               ("rope_factors_short.weight", E.F32, (fac.size,), fac)]
    for i in range(shape.n_layers):
        h = layer_host(seed, shape, i)
        p = f"blk.{i}."
        tensors.append((p + "attn_norm.weight", E.F32, (d,), h["attn_norm"]))
        for name, qt, K, N in shape.layer_tensors(i):
            tensors.append((p + name + ".weight", qt, (K, N), h[name]))
            if name == "attn_output":
                tensors.append((p + "ffn_norm.weight", E.F32, (d,), h["ffn_norm"]))
    return G.write_gguf(path, md, tensors, alignment=alignment)


class DecodeSweep:
    """Device weights and activations of the sweep; record_token() issues one
    token's operations on the context's stream."""

    def __init__(self, ctx, shape=Phi4Shape(), seed=3, keep_host=False, attention=False, logits="f32", gguf=None):
        """logits: "f32" (the F32 matrix in the reference's transposed
        chunks), "q6k" (a raw Q6_K token_embd read as stored) or "both"
        (both held; `logits_mode` picks the one a token uses).

        gguf: a GGUFModel to take the shape (ModelConfig.from_gguf) and every
        weight from, uploaded as stored; `shape` then only gives max_seq and
        chunk, logits must be "q6k" (the raw Q6_K output matrix) and the
        token's input row comes from embed(token)."""
        if logits not in ("f32", "q6k", "both"):
            raise ValueError(f"logits={logits!r}")
        if gguf is not None:
            if logits != "q6k":
                raise ValueError("a GGUF model's logits read its raw Q6_K output matrix: use logits='q6k'")
            shape = shape_from_config(ModelConfig.from_gguf(gguf), max_seq=shape.max_seq, chunk=shape.chunk)
        self.ctx, self.shape, self.seed, self.gguf = ctx, shape, seed, gguf
        self.host = {} if keep_host else None
        d = shape.d_model
        self.emb = self.emb_q6k = self.tok_emb = None
        if gguf is None:
            self._load_synthetic(logits)
        else:
            self._load_gguf()
        self.logits_mode = "q6k" if logits == "q6k" else "f32"
        self.zero = ctx.to_device(np.zeros(d, np.float32))
        self.hidden = ctx.alloc(d * 4)
        self.qkv = ctx.alloc(shape.qkv_dim * 4)
        self.gate_up = ctx.alloc(2 * shape.ffn_dim * 4)
        self.ffn_mid = ctx.alloc(shape.ffn_dim * 4)
        # silu(gate) * up fused into the gate/up GEMV (rrr_gemv_rmsnorm_silu);
        # False: the GEMV into gate_up and silu in the down GEMV's prologue
        # (the same values bit for bit)
        self.silu_fused = True
        # at a position (attention=True): rmsnorm -> QKV -> rope_kv_store as
        # one launch (rrr_gemv_rmsnorm_rope_kv); False: the two launches
        # (the same values bit for bit)
        self.rope_fused = True
        # prefill: the O-proj and FFN-down GEMMs write the next RMSNorm's f16
        # rows in the same call (rrr_gemm_f16_rmsnorm); False: separate calls
        self.prefill_fused = True
        self.logits = ctx.alloc(shape.vocab * 4)
        self.token = ctx.alloc(4)
        self.attention = attention
        if attention:
            fac = self._rope_factors_host
            self.n_rope_factors = 0 if fac is None else fac.size
            self.rope_factors = ctx.to_device(np.ones(1, np.float32) if fac is None else fac)
            if keep_host:
                self.host["rope_factors"] = fac
            cache_bytes = shape.max_seq * shape.kv_stride * 2
            self.kv = [(ctx.alloc(cache_bytes), ctx.alloc(cache_bytes)) for _ in range(shape.n_layers)]
            self.attn_out = ctx.alloc(d * 4)

    def _load_synthetic(self, logits):
        ctx, shape, seed, keep_host = self.ctx, self.shape, self.seed, self.host is not None
        d = shape.d_model
        self.layers = []
        for i in range(shape.n_layers):
            h = layer_host(seed, shape, i)
            dev = {"attn_norm": ctx.to_device(h["attn_norm"]), "ffn_norm": ctx.to_device(h["ffn_norm"]),
                   "types": {}}
            for name, qt, K, N in shape.layer_tensors(i):
                dev[name] = ctx.weight_upload(qt, K, N, h[name])
                dev["types"][name] = qt
            self.layers.append(dev)
            if keep_host:
                self.host[i] = h
        out_norm = gamma_host(seed, S_OUT_NORM, d)
        x = x_host(seed, shape)
        self.out_norm = ctx.to_device(out_norm)
        self.x_in = ctx.to_device(x)
        if keep_host:
            self.host.update(out_norm=out_norm, x=x)
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
        self._rope_factors_host = rope_factors_host(seed, shape)

    def _gguf_vector(self, name, n):
        """A 1-D F32 or F16 tensor of n elements as float32 (norm weights,
        rope factors; dequant_tensor_f32, phi4.rs:572-587, for these types)."""
        g = self.gguf
        info = g.tensor_info(name)
        if info.n_elements != n or info.typ not in (E.F32, E.F16):
            raise ValueError(f"{name}: {info.n_elements} elements of ggml type {info.typ}; "
                             f"{n} elements of F32 or F16 expected")
        raw = g.tensor_bytes(name)
        return (raw.view(np.float32) if info.typ == E.F32 else raw.view(np.float16)).astype(np.float32)

    def _gguf_weight(self, name, K, N, types=(E.Q4_K, E.Q5_K, E.Q6_K)):
        info = self.gguf.tensor_info(name)
        if info.shape[:2] != (K, N) or info.n_elements != K * N:
            raise ValueError(f"{name}: shape {info.shape}, expected ({K}, {N})")
        if info.typ not in types:
            raise ValueError(f"{name}: ggml type {info.typ}; this path reads types {types}")
        return self.gguf.upload(self.ctx, name), info.typ

    def _load_gguf(self):
        """Weights of a Phi-3/4-layout GGUF (combined attn_qkv and ffn_up;
        load_from_gguf, phi4.rs:704-869), raw bytes uploaded unchanged."""
        g, s, keep_host = self.gguf, self.shape, self.host is not None
        cfg = ModelConfig.from_gguf(g)
        if cfg.separate_qkv or cfg.separate_gate_up or cfg.has_qkv_bias:
            raise ValueError("separate Q/K/V or gate/up tensors and QKV biases (the Qwen2 layout) are not on "
                             "this decode path")
        if s.n_heads * s.head_dim != s.d_model or s.head_dim != 128:
            raise ValueError(f"head_dim {s.head_dim} x {s.n_heads} heads: the attention kernels need "
                             "head_dim 128 and n_heads * head_dim = d_model")
        d, f = s.d_model, s.ffn_dim
        self.layers = []
        for i in range(s.n_layers):
            p = f"blk.{i}."
            dev = {"types": {}}
            h = {}
            for name in ("attn_norm", "ffn_norm"):
                h[name] = self._gguf_vector(p + name + ".weight", d)
                dev[name] = self.ctx.to_device(h[name])
            for name, K, N in (("attn_qkv", d, s.qkv_dim), ("attn_output", d, d), ("ffn_up", d, 2 * f),
                               ("ffn_down", f, d)):
                dev[name], dev["types"][name] = self._gguf_weight(p + name + ".weight", K, N)
                if keep_host:
                    h[name] = g.tensor_bytes(p + name + ".weight")
            self.layers.append(dev)
            if keep_host:
                self.host[i] = h
        out_norm = self._gguf_vector("output_norm.weight", d)
        self.out_norm = self.ctx.to_device(out_norm)
        out_name = "output.weight" if cfg.has_output_weight else "token_embd.weight"
        self.emb_q6k, _ = self._gguf_weight(out_name, d, s.vocab, (E.Q6_K,))
        if cfg.has_output_weight:
            self.tok_emb, self.tok_emb_type = self._gguf_weight("token_embd.weight", d, s.vocab,
                                                                (E.F32, E.Q4_K, E.Q5_K, E.Q6_K))
        else:
            self.tok_emb, self.tok_emb_type = self.emb_q6k, E.Q6_K
        self.tok_row_bytes = E.tensor_bytes(self.tok_emb_type, d, 1)
        self.x_in = self.ctx.alloc(d * 4)
        self.embed(0)
        if keep_host:
            self.host.update(out_norm=out_norm, emb_q6k=g.tensor_bytes(out_name))
        self._rope_factors_host = None
        if cfg.has_rope_factors:
            self._rope_factors_host = self._gguf_vector("rope_factors_short.weight", s.rope_dim // 2)

    def embed(self, token):
        """The step's input row: row `token` of token_embd dequantized on the
        device into x_in (Phi4Model::embed, phi4.rs:2085-2089; bit-exact with
        the reference's host-dequantized embedding).  GGUF models only."""
        if self.tok_emb is None:
            raise ValueError("embed() needs a model loaded from GGUF (the synthetic input row is fixed)")
        if not 0 <= token < self.shape.vocab:
            raise ValueError(f"token {token} outside the vocabulary of {self.shape.vocab}")
        row = self.ctx.view(self.tok_emb, token * self.tok_row_bytes, self.tok_row_bytes)
        try:
            self.ctx.dequant(self.tok_emb_type, row, self.x_in, self.shape.d_model)
        finally:
            row.free()

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
            T = L["types"]
            if pos is None:
                c.gemv_rmsnorm(self.hidden, L["attn_norm"], s.eps, L["attn_qkv"], T["attn_qkv"], self.qkv, d,
                               s.qkv_dim)
                c.gemv_residual(self.qkv, E.ACT_GQA_V, gqa, L["attn_output"], T["attn_output"], self.hidden, d, d)
            else:
                kc, vc = self.kv[i]
                if self.rope_fused:
                    # rmsnorm -> QKV -> rope_kv_store as one launch (bitwise the two)
                    c.gemv_rmsnorm_rope_kv(self.hidden, L["attn_norm"], s.eps, L["attn_qkv"], T["attn_qkv"], self.qkv,
                                           d, self.rope_factors, self.n_rope_factors, kc, vc, pos, s.n_heads,
                                           s.n_kv_heads, s.head_dim, s.rope_dim, d, s.kv_stride, s.rope_theta,
                                           s.rope_attn_factor)
                else:
                    c.gemv_rmsnorm(self.hidden, L["attn_norm"], s.eps, L["attn_qkv"], T["attn_qkv"], self.qkv, d,
                                   s.qkv_dim)
                    c.rope_kv_store(self.qkv, self.rope_factors, self.n_rope_factors, kc, vc, pos, s.n_heads,
                                    s.n_kv_heads, s.head_dim, s.rope_dim, d, s.kv_stride, s.rope_theta,
                                    s.rope_attn_factor)
                c.attention(self.qkv, kc, vc, self.attn_out, pos + 1, s.n_kv_heads, s.heads_per_kv, s.head_dim)
                c.gemv_residual(self.attn_out, E.ACT_IDENTITY, 0, L["attn_output"], T["attn_output"], self.hidden, d, d)
            if self.silu_fused and T["ffn_up"] in (E.Q4_K, E.Q5_K, E.Q6_K):
                # silu(gate) * up in the gate/up GEMV's epilogue: the down
                # GEMV reads F activations instead of 2F
                c.gemv_rmsnorm_silu(self.hidden, L["ffn_norm"], s.eps, L["ffn_up"], T["ffn_up"], self.ffn_mid, d,
                                    s.ffn_dim)
                c.gemv_residual(self.ffn_mid, E.ACT_IDENTITY, 0, L["ffn_down"], T["ffn_down"], self.hidden,
                                s.ffn_dim, d)
            else:
                c.gemv_rmsnorm(self.hidden, L["ffn_norm"], s.eps, L["ffn_up"], T["ffn_up"], self.gate_up, d,
                               2 * s.ffn_dim)
                c.gemv_residual(self.gate_up, E.ACT_SILU_GATE, 0, L["ffn_down"], T["ffn_down"], self.hidden,
                                s.ffn_dim, d)
        self.record_logits()

    def record_logits(self):
        """Final RMSNorm + logits (F32 chunks or raw Q6_K rows, by
        logits_mode) + argmax, one call (on the F32 chunks the argmax runs
        inside the logits launch)."""
        c, s = self.ctx, self.shape
        if self.logits_mode == "q6k":
            c.logits_rmsnorm_argmax(self.hidden, self.out_norm, s.eps, self.emb_q6k, self.logits, s.d_model, s.vocab,
                                    self.token, E.LOGITS_Q6K, 0)
        else:
            c.logits_rmsnorm_argmax(self.hidden, self.out_norm, s.eps, self.emb, self.logits, s.d_model, s.vocab,
                                    self.token, E.LOGITS_CHUNKED, s.chunk)

    # ---- prefill: the prompt's tokens through every layer at once ----------
    @staticmethod
    def _silu_gemm_ok(Mp, F):
        """The shapes rrr_gemm_f16_silu_gate_f16 takes (else the two calls)."""
        return Mp % 256 == 0 and F % 64 == 0 and (F // 64) * (Mp // 256) >= 128 and Mp * F * 4 <= (48 << 20)

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
        fused = self.prefill_fused
        for i, L in enumerate(self.layers):
            T = L["types"]
            kc, vc = self.kv[i]
            if i == 0 or not fused:   # else the previous layer's down GEMM wrote this norm
                c.rmsnorm_f16(pf["hid"], L["attn_norm"], pf["n16"], Mp, d, s.eps)
            if fused:   # the QKV GEMM's split reduction is the RoPE + KV store's first step
                c.gemm_f16_rope_kv_rows(pf["n16"], L["attn_qkv"], T["attn_qkv"], pf["qkv"], d, Mp, M,
                                        self.rope_factors, self.n_rope_factors, kc, vc, pos0, s.n_heads,
                                        s.n_kv_heads, s.head_dim, s.rope_dim, d, s.kv_stride, s.rope_theta,
                                        s.rope_attn_factor)
            else:
                c.gemm_f16(pf["n16"], L["attn_qkv"], T["attn_qkv"], pf["qkv"], d, s.qkv_dim, Mp)
                c.rope_kv_store_rows(pf["qkv"], M, self.rope_factors, self.n_rope_factors, kc, vc, pos0, s.n_heads,
                                     s.n_kv_heads, s.head_dim, s.rope_dim, d, s.kv_stride, s.rope_theta,
                                     s.rope_attn_factor)
            c.attention_prefill(pf["qkv"], M, kc, vc, pf["att16"], pos0, s.n_kv_heads, s.heads_per_kv, s.head_dim,
                                out_type=E.F16)
            if fused:
                c.gemm_f16_rmsnorm(pf["att16"], L["attn_output"], T["attn_output"], pf["hid"], d, d, Mp,
                                   L["ffn_norm"], pf["n16"], s.eps, accumulate=True)
            else:
                c.gemm_f16(pf["att16"], L["attn_output"], T["attn_output"], pf["hid"], d, d, Mp, accumulate=True)
                c.rmsnorm_f16(pf["hid"], L["ffn_norm"], pf["n16"], Mp, d, s.eps)
            if fused and self._silu_gemm_ok(Mp, F):   # silu(gate) * up in the gate/up GEMM's epilogue
                c.gemm_f16_silu_gate_f16(pf["n16"], L["ffn_up"], T["ffn_up"], pf["mid16"], pf["mid_scale"], d, F, Mp)
            else:
                c.gemm_f16(pf["n16"], L["ffn_up"], T["ffn_up"], pf["gu"], d, 2 * F, Mp)
                c.silu_gate_f16(pf["gu"], pf["mid16"], pf["mid_scale"], Mp, F)
            if fused and i + 1 < len(self.layers):   # the next layer's attention norm with it
                c.gemm_f16_rmsnorm(pf["mid16"], L["ffn_down"], T["ffn_down"], pf["hid"], F, d, Mp,
                                   self.layers[i + 1]["attn_norm"], pf["n16"], s.eps, accumulate=True,
                                   row_scale=pf["mid_scale"])
            else:
                c.gemm_f16(pf["mid16"], L["ffn_down"], T["ffn_down"], pf["hid"], F, d, Mp, accumulate=True,
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
