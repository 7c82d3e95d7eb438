"""The decode step composed in the oracle (test helper shared by the GPU
decode tests): fp64 GEMVs and attention, the f32 RoPE and f16 cache store."""
import numpy as np

import oracle.oracle as orc
import rrr_hip

THREADS = 16


def oracle_step(s, host, caches, pos):
    """One decode step at position pos in the oracle, layer by layer as
    phi4.rs:1006-1033: RMSNorm -> QKV -> rope_kv_store -> attention -> O-proj
    + residual -> RMSNorm -> gate/up -> silu * up -> down + residual.  The
    GEMVs and attention are fp64; RoPE and the f16 cache store are the f32
    restatement.  caches[i] = (k, v) uint16 arrays, updated in place."""
    d, F = s.d_model, s.ffn_dim
    h = host["x"].astype(np.float64)
    for i in range(s.n_layers):
        L = host[i]
        normed = orc.rms_norm(h.astype(np.float32), L["attn_norm"], s.eps)
        qkv = orc.gemv(rrr_hip.Q5_K, L["attn_qkv"], normed, d, s.qkv_dim, 1, THREADS, f64=True)[0].astype(np.float32)
        kc, vc = caches[i]
        qkv, kc, vc = orc.rope_kv_store(qkv, kc, vc, pos, s.n_heads, s.n_kv_heads, s.head_dim, s.rope_dim,
                                        factors=host["rope_factors"], theta=s.rope_theta,
                                        attn_factor=s.rope_attn_factor)
        caches[i] = (kc, vc)
        att = orc.attention_f64(qkv[:d], kc, vc, pos + 1, s.n_kv_heads, s.heads_per_kv, s.head_dim)
        h = h + orc.gemv(rrr_hip.Q4_K, L["attn_output"], att.astype(np.float32), d, d, 1, THREADS, f64=True)[0]
        normed = orc.rms_norm(h.astype(np.float32), L["ffn_norm"], s.eps)
        gu = orc.gemv(rrr_hip.Q4_K, L["ffn_up"], normed, d, 2 * F, 1, THREADS, f64=True)[0]
        mid = orc.silu_gate(gu.astype(np.float32), F)
        h = h + orc.gemv(s.down_type(i), L["ffn_down"], mid, F, d, 1, THREADS, f64=True)[0]
    normed = orc.rms_norm(h.astype(np.float32), host["out_norm"], s.eps)
    logits = orc.logits(normed, host["emb"], d, s.vocab, 1, s.chunk, THREADS, f64=True)
    return logits, h


def gqa_gather(qkv, s):
    """Attention output at position 0: head h reads V of kv head h / hpk
    (phi4.rs attention with a single cached position)."""
    v = qkv[s.d_model + s.n_kv_heads * s.head_dim:].reshape(s.n_kv_heads, s.head_dim)
    return np.repeat(v, s.heads_per_kv, axis=0).reshape(-1)


def oracle_token(s, host, logits="f32"):
    """One position-0 token of the weight sweep in the oracle: the GEMVs and
    the logits in fp64, attention over the one cached row as the GQA V
    gather; logits "f32" (the transposed chunks) or "q6k" (token_embd)."""
    d, F = s.d_model, s.ffn_dim
    h = host["x"].astype(np.float64)
    for i in range(s.n_layers):
        L = host[i]
        normed = orc.rms_norm(h.astype(np.float32), L["attn_norm"], s.eps)
        qkv = orc.gemv(rrr_hip.Q5_K, L["attn_qkv"], normed, d, s.qkv_dim, 1, THREADS, f64=True)[0]
        v = gqa_gather(qkv.astype(np.float32), s)
        h = h + orc.gemv(rrr_hip.Q4_K, L["attn_output"], v, d, d, 1, THREADS, f64=True)[0]
        normed = orc.rms_norm(h.astype(np.float32), L["ffn_norm"], s.eps)
        gu = orc.gemv(rrr_hip.Q4_K, L["ffn_up"], normed, d, 2 * F, 1, THREADS, f64=True)[0]
        mid = orc.silu_gate(gu.astype(np.float32), F)
        h = h + orc.gemv(s.down_type(i), L["ffn_down"], mid, F, d, 1, THREADS, f64=True)[0]
    normed = orc.rms_norm(h.astype(np.float32), host["out_norm"], s.eps)
    if logits == "q6k":
        out = orc.gemv(rrr_hip.Q6_K, host["emb_q6k"], normed, d, s.vocab, 1, THREADS, f64=True)[0]
    else:
        out = orc.logits(normed, host["emb"], d, s.vocab, 1, s.chunk, THREADS, f64=True)
    return out, h
