"""Python host binding of librrr_hip.

`Context` is a thin, typed wrapper over the C ABI (include/rrr_hip.h).
`ComputeEngine`, `GpuBuffer` and `DescSetHandle` mirror the reference's
engine surface (src/gpu/engine.rs, re-exported by src/gpu/mod.rs:3) so that
code written against the reference's call shapes -- get_pipeline,
alloc_buffer, pre_allocate_desc_set, dispatch_by_name, dispatch_batch,
dispatch_batch_parallel, dispatch_batch_persistent_v2 -- runs unchanged on
MI355X.  Every method raises RrrError on a non-zero status instead of
panicking like the reference's `.unwrap()`s.
"""
import ctypes
import struct

import numpy as np

from . import _lib

OK = 0
ERR_INVALID_ARG = -1
ERR_BAD_TYPE = -2
ERR_BAD_SHAPE = -3
ERR_SHORT_BUFFER = -4
ERR_NULL = -5
ERR_HIP = -6
ERR_UNSUPPORTED = -7
ERR_NO_DEVICE = -8
ERR_STATE = -9
ERR_STALE = -10
ERR_FORMAT = -11
ERR_NOT_FOUND = -12
ERR_IO = -13

F32, F16, Q4_K, Q5_K, Q6_K = 0, 1, 12, 13, 14
LOGITS_ROWS, LOGITS_CHUNKED, LOGITS_Q6K = 0, 1, 2
ACT_IDENTITY, ACT_SILU_GATE, ACT_GQA_V = 0, 1, 2
PROBE_MFMA_F16_16X16X32, PROBE_MFMA_F16_32X32X16, PROBE_MFMA_I8_16X16X64 = 0, 1, 2
PHASES_PLAIN, PHASES_RMSNORM, PHASES_RESIDUAL, PHASES_RMSNORM_SILU = 0, 1, 2, 3
DEVICE_NONE = -1
BLOCK_BYTES = {Q4_K: 144, Q5_K: 176, Q6_K: 210, F32: 1024}


class RrrError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"[{code}] {msg}")
        self.code = code
        self.msg = msg


def _check(rc):
    if rc != OK:
        raise RrrError(rc, _lib.hip().rrr_last_error().decode())
    return rc


def tensor_bytes(qtype, K, N):
    return int(_lib.hip().rrr_tensor_bytes(qtype, K, N))


def device_count():
    return int(_lib.hip().rrr_device_count())


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


class Buffer:
    """A device buffer (or view) owned by a Context."""

    def __init__(self, ctx, handle, nbytes):
        self.ctx = ctx
        self.handle = handle
        self.nbytes = nbytes

    @property
    def _h(self):
        return ctypes.c_void_p(self.handle)

    def free(self):
        if self.handle:
            _check(_lib.hip().rrr_buf_free(self.ctx._h, self._h))
            self.handle = None


class Graph:
    def __init__(self, ctx, handle):
        self.ctx = ctx
        self.handle = handle

    def launch(self):
        _check(_lib.hip().rrr_graph_launch(self.ctx._h, ctypes.c_void_p(self.handle)))

    def destroy(self):
        if self.handle:
            _check(_lib.hip().rrr_graph_destroy(self.ctx._h, ctypes.c_void_p(self.handle)))
            self.handle = None


class Context:
    """One rrr_ctx: a HIP device plus one stream."""

    def __init__(self, device=0):
        self.lib = _lib.hip()
        h = ctypes.c_void_p()
        _check(self.lib.rrr_init(device, ctypes.byref(h)))
        self.handle = h.value
        self.device = device

    @property
    def _h(self):
        return ctypes.c_void_p(self.handle)

    def close(self):
        if self.handle:
            _check(self.lib.rrr_destroy(self._h))
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- buffers --
    def alloc(self, nbytes):
        h = ctypes.c_void_p()
        _check(self.lib.rrr_buf_alloc(self._h, nbytes, ctypes.byref(h)))
        return Buffer(self, h.value, nbytes)

    def view(self, buf, offset, nbytes):
        h = ctypes.c_void_p()
        _check(self.lib.rrr_buf_view(self._h, buf._h, offset, nbytes, ctypes.byref(h)))
        return Buffer(self, h.value, nbytes)

    def upload(self, buf, array, offset=0):
        a = np.ascontiguousarray(array)
        _check(self.lib.rrr_buf_upload(self._h, buf._h, offset, _ptr(a), a.nbytes))

    def download(self, buf, dtype=np.float32, count=None, offset=0):
        dt = np.dtype(dtype)
        if count is None:
            count = (buf.nbytes - offset) // dt.itemsize
        out = np.empty(count, dtype=dt)
        _check(self.lib.rrr_buf_download(self._h, buf._h, offset, _ptr(out), out.nbytes))
        return out

    def to_device(self, array):
        a = np.ascontiguousarray(array)
        b = self.alloc(max(a.nbytes, 4))
        self.upload(b, a)
        return b

    def fill_u32(self, buf, value, offset=0, nbytes=None):
        nbytes = buf.nbytes - offset if nbytes is None else nbytes
        _check(self.lib.rrr_buf_fill_u32(self._h, buf._h, offset, nbytes, value))

    def weight_upload(self, qtype, K, N, raw):
        a = np.ascontiguousarray(raw)
        h = ctypes.c_void_p()
        _check(self.lib.rrr_weight_upload(self._h, qtype, K, N, _ptr(a), a.nbytes, ctypes.byref(h)))
        return Buffer(self, h.value, tensor_bytes(qtype, K, N))

    # -- ops --
    def dequant(self, qtype, W, out, n):
        _check(self.lib.rrr_dequant(self._h, qtype, W._h, out._h, n))

    def gemv(self, X, W, qtype, Y, K, N, M=1):
        _check(self.lib.rrr_gemv(self._h, X._h, W._h, qtype, Y._h, K, N, M))

    def gemm_bf16(self, X, W, qtype, Y, K, N, M):
        _check(self.lib.rrr_gemm_bf16(self._h, X._h, W._h, qtype, Y._h, K, N, M))

    def rmsnorm(self, x, gamma, y, rows, d, eps=1e-5):
        _check(self.lib.rrr_rmsnorm(self._h, x._h, gamma._h, y._h, rows, d, eps))

    def silu_gate(self, gu, mid, rows, F):
        _check(self.lib.rrr_silu_gate(self._h, gu._h, mid._h, rows, F))

    def residual_add(self, a, b, out, n):
        _check(self.lib.rrr_residual_add(self._h, a._h, b._h, out._h, n))

    def logits_f32(self, x, E, y, K, V, layout=LOGITS_ROWS, chunk=8192):
        _check(self.lib.rrr_logits_f32(self._h, x._h, E._h, y._h, K, V, layout, chunk))

    def argmax_f32(self, logits, V, out_index):
        _check(self.lib.rrr_argmax_f32(self._h, logits._h, V, out_index._h))

    def gemv_rmsnorm(self, x, gamma, eps, W, qtype, Y, K, N):
        _check(self.lib.rrr_gemv_rmsnorm(self._h, x._h, gamma._h, eps, W._h, qtype, Y._h, K, N))

    def gemv_rmsnorm_silu(self, x, gamma, eps, W, qtype, Y, K, F):
        """Y[F] = silu(gate) * up of W (2F rows: gate, then up) . rmsnorm(x)."""
        _check(self.lib.rrr_gemv_rmsnorm_silu(self._h, x._h, gamma._h, eps, W._h, qtype, Y._h, K, F))

    def gemv_residual(self, x, act_kind, act_param, W, qtype, hidden, K, N):
        _check(self.lib.rrr_gemv_residual(self._h, x._h, act_kind, act_param, W._h, qtype, hidden._h, K, N))

    def logits_rmsnorm(self, x, gamma, eps, E, y, K, V, layout=LOGITS_ROWS, chunk=8192):
        _check(self.lib.rrr_logits_rmsnorm(self._h, x._h, gamma._h, eps, E._h, y._h, K, V, layout, chunk))

    def logits_rmsnorm_argmax(self, x, gamma, eps, E, y, K, V, index, layout=LOGITS_ROWS, chunk=8192):
        """rrr_logits_rmsnorm plus the argmax of the logits into `index` (u32)."""
        _check(self.lib.rrr_logits_rmsnorm_argmax(self._h, x._h, gamma._h, eps, E._h, y._h, K, V, layout, chunk,
                                                   index._h))

    def rope_kv_store(self, qkv, rope_factors, n_factors, k_cache, v_cache, pos, n_heads, n_kv_heads, head_dim,
                      rope_dim, q_dim, kv_stride, theta=10000.0, attn_factor=1.190238):
        _check(self.lib.rrr_rope_kv_store(self._h, qkv._h, rope_factors._h if rope_factors is not None else None,
                                          n_factors, k_cache._h, v_cache._h, pos, n_heads, n_kv_heads, head_dim,
                                          rope_dim, q_dim, kv_stride, theta, attn_factor))

    def gemv_rmsnorm_rope_kv(self, x, gamma, eps, W, qtype, qkv, K, rope_factors, n_factors, k_cache, v_cache, pos,
                             n_heads, n_kv_heads, head_dim, rope_dim, q_dim, kv_stride, theta=10000.0,
                             attn_factor=1.190238):
        _check(self.lib.rrr_gemv_rmsnorm_rope_kv(self._h, x._h, gamma._h, eps, W._h, qtype, qkv._h, K,
                                                 rope_factors._h if rope_factors is not None else None, n_factors,
                                                 k_cache._h, v_cache._h, pos, n_heads, n_kv_heads, head_dim, rope_dim,
                                                 q_dim, kv_stride, theta, attn_factor))

    def attention(self, q, k_cache, v_cache, out, seq_len, n_kv_heads, heads_per_kv, head_dim):
        _check(self.lib.rrr_attention(self._h, q._h, k_cache._h, v_cache._h, out._h, seq_len, n_kv_heads,
                                      heads_per_kv, head_dim))

    # ---- prefill -------------------------------------------------------
    def rope_kv_store_rows(self, qkv, rows, rope_factors, n_factors, k_cache, v_cache, pos0, n_heads, n_kv_heads,
                           head_dim, rope_dim, q_dim, kv_stride, theta=10000.0, attn_factor=1.190238):
        _check(self.lib.rrr_rope_kv_store_rows(self._h, qkv._h, rows,
                                               rope_factors._h if rope_factors is not None else None, n_factors,
                                               k_cache._h, v_cache._h, pos0, n_heads, n_kv_heads, head_dim, rope_dim,
                                               q_dim, kv_stride, theta, attn_factor))

    def attention_prefill(self, qkv, rows, k_cache, v_cache, out, pos0, n_kv_heads, heads_per_kv, head_dim,
                          out_type=F32):
        _check(self.lib.rrr_attention_prefill(self._h, qkv._h, rows, k_cache._h, v_cache._h, out._h, out_type, pos0,
                                              n_kv_heads, heads_per_kv, head_dim))

    def gemm_f16(self, X, W, qtype, Y, K, N, M, accumulate=False, row_scale=None):
        _check(self.lib.rrr_gemm_f16(self._h, X._h, row_scale._h if row_scale is not None else None, W._h, qtype,
                                     Y._h, K, N, M, 1 if accumulate else 0))

    def gemm_f16_rmsnorm(self, X, W, qtype, Y, K, N, M, gamma, y16, eps=1e-5, accumulate=False, row_scale=None):
        _check(self.lib.rrr_gemm_f16_rmsnorm(self._h, X._h, row_scale._h if row_scale is not None else None, W._h,
                                             qtype, Y._h, K, N, M, 1 if accumulate else 0, gamma._h, eps, y16._h))

    def gemm_f16_rope_kv_rows(self, X, W, qtype, qkv, K, M, rows, rope_factors, n_factors, k_cache, v_cache, pos0,
                              n_heads, n_kv_heads, head_dim, rope_dim, q_dim, kv_stride, theta=10000.0,
                              attn_factor=1.190238):
        _check(self.lib.rrr_gemm_f16_rope_kv_rows(self._h, X._h, W._h, qtype, qkv._h, K, M, rows,
                                                  rope_factors._h if rope_factors is not None else None, n_factors,
                                                  k_cache._h, v_cache._h, pos0, n_heads, n_kv_heads, head_dim,
                                                  rope_dim, q_dim, kv_stride, theta, attn_factor))

    def gemm_f16_silu_gate_f16(self, X, W, qtype, mid, row_scale, K, F, M):
        _check(self.lib.rrr_gemm_f16_silu_gate_f16(self._h, X._h, W._h, qtype, mid._h, row_scale._h, K, F, M))

    def rmsnorm_f16(self, x, gamma, y, rows, d, eps=1e-5):
        _check(self.lib.rrr_rmsnorm_f16(self._h, x._h, gamma._h, y._h, rows, d, eps))

    def silu_gate_f16(self, gate_up, mid, row_scale, rows, F):
        _check(self.lib.rrr_silu_gate_f16(self._h, gate_up._h, mid._h, row_scale._h, rows, F))

    def dispatch(self, name, bufs, push_u32, groups):
        arr = (ctypes.c_void_p * max(len(bufs), 1))(*[b.handle for b in bufs])
        pb = struct.pack("<%dI" % len(push_u32), *push_u32)
        g = (ctypes.c_uint32 * 3)(*groups)
        _check(self.lib.rrr_dispatch(self._h, name.encode(), arr, len(bufs), pb, len(pb), g))

    def dispatch_batch(self, entries):
        """entries: list of (name, bufs, push_u32, groups, barrier)."""
        keep = []
        descs = (_lib.DispatchDesc * max(len(entries), 1))()
        for i, (name, bufs, push, groups, barrier) in enumerate(entries):
            arr = (ctypes.c_void_p * max(len(bufs), 1))(*[b.handle for b in bufs])
            pb = ctypes.create_string_buffer(struct.pack("<%dI" % len(push), *push), 4 * len(push) or 1)
            nm = name.encode()
            keep += [arr, pb, nm]
            descs[i].name = nm
            descs[i].bufs = ctypes.cast(arr, ctypes.POINTER(ctypes.c_void_p))
            descs[i].n_bufs = len(bufs)
            descs[i].push = ctypes.cast(pb, ctypes.c_void_p)
            descs[i].push_bytes = 4 * len(push)
            descs[i].groups = (ctypes.c_uint32 * 3)(*groups)
            descs[i].barrier = 1 if barrier else 0
        _check(self.lib.rrr_dispatch_batch(self._h, descs, len(entries)))

    # -- graphs, sync, timing --
    def graph_begin(self):
        _check(self.lib.rrr_graph_begin(self._h))

    def graph_end(self):
        h = ctypes.c_void_p()
        _check(self.lib.rrr_graph_end(self._h, ctypes.byref(h)))
        return Graph(self, h.value)

    def set_async(self, flag):
        _check(self.lib.rrr_set_async(self._h, 1 if flag else 0))

    # ---- platform probes (include/rrr_probe.h) ---------------------------
    def probe_read(self, buf, nbytes, sink):
        _check(self.lib.rrr_probe_read(self._h, buf._h, nbytes, sink._h))

    def probe_read_shares(self, buf, nbytes, sink):
        _check(self.lib.rrr_probe_read_shares(self._h, buf._h, nbytes, sink._h))

    def probe_gemv_phases(self, op, x, W, qtype, y, K, N, stamps, gamma=None, eps=1e-5, act_kind=0, act_param=0):
        """One stamped GEMV launch (include/rrr_probe.h); returns (grid, waves)."""
        g, w = ctypes.c_uint32(), ctypes.c_uint32()
        _check(self.lib.rrr_probe_gemv_phases(self._h, op, act_kind, act_param, x._h,
                                              gamma._h if gamma is not None else None, eps, W._h, qtype, y._h, K, N,
                                              stamps._h, ctypes.byref(g), ctypes.byref(w)))
        return g.value, w.value

    def probe_mfma(self, kind, waves_per_cu, iters, sink):
        _check(self.lib.rrr_probe_mfma(self._h, kind, waves_per_cu, iters, sink._h))

    def probe_cus(self):
        return int(self.lib.rrr_probe_cus(self._h))

    def sync(self):
        _check(self.lib.rrr_sync(self._h))

    def timer_start(self):
        _check(self.lib.rrr_timer_start(self._h))

    def timer_stop(self):
        ms = ctypes.c_float()
        _check(self.lib.rrr_timer_stop(self._h, ctypes.byref(ms)))
        return ms.value

    def matmul_kquant(self, buf_a, weight_buf, buf_c, qtype, a, K, N):
        a = np.ascontiguousarray(a, dtype=np.float32)
        c = np.empty(N, dtype=np.float32)
        _check(self.lib.rrr_matmul_kquant(self._h, buf_a._h, weight_buf._h, buf_c._h, qtype, _ptr(a), _ptr(c), K, N))
        return c


# ---------------------------------------------------------------------------
# Mirror of the reference engine surface (src/gpu/engine.rs).

class GpuBuffer(Buffer):
    """GpuBuffer (engine.rs:38-43): `capacity` is the size in bytes.  There is
    no `.mapped` pointer: MI355X buffers live in HBM, so host access goes
    through upload()/download() (replacing phi4.rs:616-626)."""

    @property
    def capacity(self):
        return self.nbytes


class DescSetHandle(int):
    """DescSetHandle (engine.rs:11-13): index of a pre-allocated binding."""


class ComputeEngine:
    """ComputeEngine (engine.rs:15-29) over librrr_hip.

    `shader_dir` is accepted and ignored: the kernels are compiled into the
    library, there are no SPIR-V files to load (engine.rs:131-139)."""

    def __init__(self, shader_dir=None, device=0):
        self.ctx = Context(device)
        self.pipeline_cache = {}
        self.persistent_desc_sets = []

    def get_pipeline(self, name, num_buffers, push_size):
        """engine.rs:142-197.  Records the binding count and push size so
        dispatches can be checked against them."""
        self.pipeline_cache.setdefault(name, (num_buffers, push_size))
        return self.pipeline_cache[name]

    def alloc_buffer(self, size):
        """engine.rs:200-229 (device memory instead of host-coherent)."""
        b = self.ctx.alloc(size)
        return GpuBuffer(self.ctx, b.handle, b.nbytes)

    def upload(self, buf, data):
        self.ctx.upload(buf, data)

    def download(self, buf, count, dtype=np.float32):
        return self.ctx.download(buf, dtype, count)

    def _bound(self, bufs, sizes):
        """Binding i covers bytes [0, sizes[i]) of bufs[i] (engine.rs:257-259)."""
        out = []
        for b, s in zip(bufs, sizes):
            out.append(b if s >= b.nbytes else self.ctx.view(b, 0, s))
        return out

    def _free_views(self, bound, bufs):
        for v, b in zip(bound, bufs):
            if v is not b:
                v.free()

    def pre_allocate_desc_set(self, pipeline_name, buffers, buffer_sizes):
        """engine.rs:244-268."""
        if pipeline_name not in self.pipeline_cache:
            raise RrrError(ERR_STATE, f"pipeline '{pipeline_name}' was never registered with get_pipeline")
        self.persistent_desc_sets.append((pipeline_name, self._bound(buffers, buffer_sizes)))
        return DescSetHandle(len(self.persistent_desc_sets) - 1)

    @staticmethod
    def _push_words(push):
        if isinstance(push, (bytes, bytearray)):
            if len(push) % 4:
                raise RrrError(ERR_INVALID_ARG, "push constants must be whole u32 words")
            return list(struct.unpack("<%dI" % (len(push) // 4), push))
        return list(push)

    def _check_registered(self, name, n_bufs, push_words):
        if name not in self.pipeline_cache:
            raise RrrError(ERR_STATE, f"pipeline '{name}' was never registered with get_pipeline")
        nb, ps = self.pipeline_cache[name]
        if n_bufs != nb or 4 * len(push_words) > ps:
            raise RrrError(ERR_INVALID_ARG, f"pipeline '{name}' registered with {nb} buffers / {ps} push bytes")

    def dispatch_by_name(self, name, buffers, buffer_sizes, push_constants, groups):
        """engine.rs:476-486: one dispatch, then wait."""
        words = self._push_words(push_constants)
        self._check_registered(name, len(buffers), words)
        bound = self._bound(buffers, buffer_sizes)
        try:
            self.ctx.dispatch(name, bound, words, groups)
        finally:
            self._free_views(bound, buffers)

    def _batch(self, dispatches):
        entries, temps = [], []
        for name, bufs, sizes, push, groups in dispatches:
            words = self._push_words(push)
            self._check_registered(name, len(bufs), words)
            bound = self._bound(bufs, sizes)
            temps.append((bound, bufs))
            entries.append((name, bound, words, groups, True))
        try:
            self.ctx.dispatch_batch(entries)
        finally:
            for bound, bufs in temps:
                self._free_views(bound, bufs)

    def dispatch_batch(self, dispatches):
        """engine.rs:380-386: ordered launches, one wait."""
        self._batch(dispatches)

    def dispatch_batch_parallel(self, dispatches):
        """engine.rs:389-394: the reference drops the barriers; launches on one
        stream are ordered anyway, so this is the same call."""
        self._batch(dispatches)

    def dispatch_batch_persistent_v2(self, dispatches):
        """engine.rs:317-370: (name, DescSetHandle, push, groups, barrier)."""
        entries = []
        for name, handle, push, groups, barrier in dispatches:
            pname, bound = self.persistent_desc_sets[int(handle)]
            if pname != name:
                raise RrrError(ERR_INVALID_ARG, f"descriptor set {int(handle)} belongs to '{pname}', not '{name}'")
            words = self._push_words(push)
            self._check_registered(name, len(bound), words)
            entries.append((name, bound, words, groups, barrier))
        self.ctx.dispatch_batch(entries)

    def close(self):
        self.ctx.close()
