"""The reference's own per-token dispatch table, replayed on the GPU through
the name-keyed shim.

The reference builds its decode token once as a list of pre-bound
dispatches (phi4.rs:915-1064: 11 per layer -- rmsnorm, the QKV K-quant
shader, rope_kv_store, attention, the O-proj shader, residual_add, rmsnorm,
the gate/up shader, silu_gate, the down shader, residual_add -- then the
output rmsnorm and one matmul_tiled per 8192-entry vocab chunk) and replays
it per token with dispatch_batch_persistent_v2 (engine.rs:317-370), building
only the push constants per token (forward_gpu, phi4.rs:1099-1159).  Here
the same table is built against the ComputeEngine mirror
(pre_allocate_desc_set views over the reference's buffers, the same sizes,
names, push layouts and grids) and replayed through rrr_dispatch_batch at
positions 0..4; the logits are read back per chunk and the token is the
chunked argmax of phi4.rs:1172-1183.

Bars: hidden state and logits within 1e-4 normwise of the oracle step
(fp64 GEMVs and attention, the f32 RoPE and f16 cache store); the token
equals the first maximal index of the GPU logits and the oracle's when its
top two are apart by more than the tolerance.
"""
import dataclasses
import struct

import numpy as np
import pytest

import oracle.oracle as orc
import rrr_hip
from rrr_hip import decode
from decode_ref import oracle_step

pytestmark = pytest.mark.gpu

TOL = 1e-4
SHAPE = dataclasses.replace(decode.Phi4Shape(), n_layers=2, vocab=20000, max_seq=16)
POSITIONS = [0, 1, 2, 3, 4]

# repacked block sizes of the types load_weight_gpu returns (phi4.rs:146-151,
# :752-755); the table sizes the weight bindings with them
GPU_QTYPE = {rrr_hip.Q4_K: ("matmul_gpuq4", 192), rrr_hip.Q5_K: ("matmul_gpuq5", 320),
             rrr_hip.Q6_K: ("matmul_gpuq6", 320)}


def u32s(*v):
    return b"".join(struct.pack("<I", x) for x in v)


class ReferenceTable:
    """Phi4Model's GPU-resident buffers and mega dispatch list
    (phi4.rs:858-1064), bound to the ComputeEngine mirror."""

    def __init__(self, eng, s, seed=3):
        self.eng, self.s = eng, s
        d, F, qkv_dim = s.d_model, s.ffn_dim, s.qkv_dim
        gate_up_dim = 2 * F
        kv_stride = s.kv_stride
        # pipelines (get_pipeline name, bindings, push bytes)
        for name, nb, pb in (("rmsnorm", 3, 8), ("matmul_gpuq4", 3, 8), ("matmul_gpuq5", 3, 8),
                             ("matmul_gpuq6", 3, 8), ("rope_kv_store", 4, 28), ("attention", 4, 16),
                             ("residual_add", 3, 4), ("silu_gate", 2, 4), ("matmul_tiled", 3, 12)):
            eng.get_pipeline(name, nb, pb)
        ctx = eng.ctx
        self.host = {}
        self.layers = []
        for i in range(s.n_layers):
            h = decode.layer_host(seed, s, i)
            self.host[i] = h
            L = {"attn_norm": eng.alloc_buffer(d * 4), "ffn_norm": eng.alloc_buffer(d * 4)}
            eng.upload(L["attn_norm"], h["attn_norm"])
            eng.upload(L["ffn_norm"], h["ffn_norm"])
            for name, qt, K, N in s.layer_tensors(i):
                L[name] = (ctx.weight_upload(qt, K, N, h[name]), qt, K, N)
            self.layers.append(L)
        out_norm = decode.gamma_host(seed, decode.S_OUT_NORM, d)
        x = decode.x_host(seed, s)
        fac = decode.rope_factors_host(seed, s)
        emb = decode.embedding_chunks_host(seed, s)   # the transposed chunks, back to back
        self.host.update(out_norm=out_norm, x=x, rope_factors=fac, emb=emb)
        self.x = x
        # per-chunk embedding and logit buffers (phi4.rs:874-893, :907-912)
        self.emb_bufs, self.logit_out_bufs = [], []
        start = 0
        while start < s.vocab:
            n = min(s.chunk, s.vocab - start)
            b = eng.alloc_buffer(d * n * 4)
            eng.upload(b, emb[start * d:(start + n) * d])
            self.emb_bufs.append((b, n))
            self.logit_out_bufs.append(eng.alloc_buffer(n * 4))
            start += n
        attn_out_buf = eng.alloc_buffer(d * 4)
        kv_size = s.max_seq * kv_stride * 2
        self.kv_bufs = [(eng.alloc_buffer(kv_size), eng.alloc_buffer(kv_size)) for _ in range(s.n_layers)]
        for kb, vb in self.kv_bufs:
            ctx.fill_u32(kb, 0)
            ctx.fill_u32(vb, 0)
        self.gpu_hidden = eng.alloc_buffer(d * 4)
        gpu_normed = eng.alloc_buffer(d * 4)
        gpu_qkv = eng.alloc_buffer(qkv_dim * 4)
        gpu_gate_up = eng.alloc_buffer(gate_up_dim * 4)
        gpu_ffn_mid = eng.alloc_buffer(F * 4)
        gpu_tmp = eng.alloc_buffer(d * 4)
        rope_factor_len = fac.size if fac.size else 1
        gpu_rope_factors = eng.alloc_buffer(rope_factor_len * 4)
        eng.upload(gpu_rope_factors, fac)
        gpu_output_norm_w = eng.alloc_buffer(d * 4)
        eng.upload(gpu_output_norm_w, out_norm)

        d4 = d * 4
        kv_max_bytes = s.max_seq * kv_stride * 2
        self.mega = []   # (pipeline name, desc set, workgroups, needs_barrier)

        def pre(name, bufs, sizes, wg, barrier=True):
            self.mega.append((name, eng.pre_allocate_desc_set(name, bufs, sizes), wg, barrier))

        rope_pairs = (s.n_heads + s.n_kv_heads) * (s.rope_dim // 2)
        fused_wg = (max(rope_pairs, kv_stride // 2) + 63) // 64
        silu_wg = (F + 255) // 256
        resid_wg = (d + 255) // 256
        self.kq = []   # (K, N) of the 4 K-quant slots of each layer, for the push constants
        for i, L in enumerate(self.layers):
            kb, vb = self.kv_bufs[i]
            sh = {}
            for name in ("attn_qkv", "attn_output", "ffn_up", "ffn_down"):
                buf, qt, K, N = L[name]
                pname, bb = GPU_QTYPE[qt]
                sh[name] = (buf, pname, K, N, N * (K // 256) * bb)
            self.kq.append({k: (v[2], v[3]) for k, v in sh.items()})

            def kq(name, src, dst):
                buf, pname, K, N, wb = sh[name]
                pre(pname, [src, buf, dst], [K * 4, wb, N * 4], [N, 1, 1])

            pre("rmsnorm", [self.gpu_hidden, L["attn_norm"], gpu_normed], [d4, d4, d4], [1, 1, 1])
            kq("attn_qkv", gpu_normed, gpu_qkv)
            pre("rope_kv_store", [gpu_qkv, gpu_rope_factors, kb, vb],
                [qkv_dim * 4, rope_factor_len * 4, kv_max_bytes, kv_max_bytes], [fused_wg, 1, 1])
            pre("attention", [gpu_qkv, kb, vb, attn_out_buf], [d4, kv_max_bytes, kv_max_bytes, d4],
                [s.n_heads, 1, 1])
            kq("attn_output", attn_out_buf, gpu_tmp)
            pre("residual_add", [self.gpu_hidden, gpu_tmp, self.gpu_hidden], [d4, d4, d4], [resid_wg, 1, 1])
            pre("rmsnorm", [self.gpu_hidden, L["ffn_norm"], gpu_normed], [d4, d4, d4], [1, 1, 1])
            kq("ffn_up", gpu_normed, gpu_gate_up)
            pre("silu_gate", [gpu_gate_up, gpu_ffn_mid], [gate_up_dim * 4, F * 4], [silu_wg, 1, 1])
            kq("ffn_down", gpu_ffn_mid, gpu_tmp)
            pre("residual_add", [self.gpu_hidden, gpu_tmp, self.gpu_hidden], [d4, d4, d4], [resid_wg, 1, 1])
        pre("rmsnorm", [self.gpu_hidden, gpu_output_norm_w, gpu_normed], [d4, d4, d4], [1, 1, 1])
        for (emb_buf, n), lo in zip(self.emb_bufs, self.logit_out_bufs):
            pre("matmul_tiled", [gpu_normed, emb_buf, lo], [d * 4, d * n * 4, n * 4], [(n + 15) // 16, 1, 1],
                False)

    def forward(self, pos):
        """forward_gpu (phi4.rs:1099-1195): upload the hidden row, the push
        constants of every entry, one batch, then the chunked readback and
        argmax.  Returns (logits, token, final hidden state)."""
        s, eng = self.s, self.eng
        d = s.d_model
        eng.upload(self.gpu_hidden, self.x)
        norm = u32s(1, d)
        rope_kv = u32s(pos, s.n_heads, s.n_kv_heads, s.head_dim, s.rope_dim, s.n_heads * s.head_dim, s.kv_stride)
        attn = u32s(pos + 1, s.n_kv_heads, s.heads_per_kv, s.head_dim)
        silu, resid = u32s(s.ffn_dim), u32s(d)
        slots = [norm, "attn_qkv", rope_kv, attn, "attn_output", resid, norm, "ffn_up", silu, "ffn_down", resid]
        push = []
        for li in range(s.n_layers):
            for p in slots:
                push.append(u32s(*self.kq[li][p]) if isinstance(p, str) else p)
        push.append(norm)
        for _, n in self.emb_bufs:
            push.append(u32s(1, d, n))
        assert len(push) == len(self.mega) == 11 * s.n_layers + 1 + len(self.emb_bufs)
        eng.dispatch_batch_persistent_v2([(name, ds, p, wg, barrier)
                                          for (name, ds, wg, barrier), p in zip(self.mega, push)])
        # the chunked readback and CPU argmax of phi4.rs:1172-1195
        best_val, best_id, off = -np.inf, 0, 0
        chunks = []
        for (_, n), lo in zip(self.emb_bufs, self.logit_out_bufs):
            src = eng.download(lo, n)
            for j in range(n):
                if src[j] > best_val:
                    best_val, best_id = src[j], off + j
            chunks.append(src)
            off += n
        hidden = eng.download(self.gpu_hidden, d)
        return np.concatenate(chunks), best_id, hidden


@pytest.fixture(scope="module")
def table():
    eng = rrr_hip.ComputeEngine(device=0)
    t = ReferenceTable(eng, SHAPE)
    yield t
    eng.close()


def test_reference_dispatch_table_matches_oracle(table):
    s = SHAPE
    assert len(table.mega) == 11 * s.n_layers + 1 + 3      # 20,000 entries: chunks of 8192, 8192, 3616
    caches = [(np.zeros(s.max_seq * s.kv_stride, np.uint16), np.zeros(s.max_seq * s.kv_stride, np.uint16))
              for _ in range(s.n_layers)]
    for pos in POSITIONS:
        logits, tok, hidden = table.forward(pos)
        ref_logits, ref_h = oracle_step(s, table.host, caches, pos)
        assert np.all(np.isfinite(logits)), pos
        assert orc.normwise_err(hidden, ref_h) < TOL, pos
        assert orc.normwise_err(logits, ref_logits) < TOL, pos
        assert tok == int(np.argmax(logits)), pos
        top2 = np.sort(ref_logits)[-2:]
        if top2[1] - top2[0] > TOL * np.max(np.abs(ref_logits)):
            assert tok == int(np.argmax(ref_logits)), pos
    # the K cache rows written by rope_kv_store hold the oracle's rotated K
    # within one f16 rounding of the tolerance
    n = len(POSITIONS) * s.kv_stride
    kg = table.eng.download(table.kv_bufs[0][0], n, np.uint16).view(np.float16).astype(np.float64)
    ko = caches[0][0][:n].view(np.float16).astype(np.float64)
    assert np.all(np.abs(kg - ko) <= TOL * np.max(np.abs(ko)) + np.abs(ko) * 2.0 ** -10)


def test_reference_dispatch_table_matches_decode_sweep(ctx, table):
    """The shim's replay of the reference table and the fused decode step
    (DecodeSweep with attention) compute the same token at position 0..1."""
    s = SHAPE
    sw = decode.DecodeSweep(ctx, s, seed=3, attention=True)
    for b in sw.kv:
        ctx.fill_u32(b[0], 0)
        ctx.fill_u32(b[1], 0)
    for kb, vb in table.kv_bufs:
        table.eng.ctx.fill_u32(kb, 0)
        table.eng.ctx.fill_u32(vb, 0)
    for pos in (0, 1):
        logits_t, tok_t, hid_t = table.forward(pos)
        sw.record_token(pos)
        ctx.sync()
        logits_s, tok_s, hid_s = sw.results()
        assert orc.normwise_err(hid_t, hid_s.astype(np.float64)) < TOL, pos
        assert orc.normwise_err(logits_t, logits_s.astype(np.float64)) < TOL, pos
