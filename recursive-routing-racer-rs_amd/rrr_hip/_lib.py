"""ctypes loader for librrr_hip.so and librrr_synth.so.

The product path is the HIP library: if it has not been built, loading raises
instead of falling back to anything else.
"""
import ctypes
import os

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_DIR = os.path.join(PKG_DIR, "lib")
HIP_LIB = os.path.join(LIB_DIR, "librrr_hip.so")
SYNTH_LIB = os.path.join(LIB_DIR, "librrr_synth.so")

c_ctx_p = ctypes.c_void_p
c_buf_p = ctypes.c_void_p
u32 = ctypes.c_uint32
u64 = ctypes.c_uint64
i32 = ctypes.c_int
f32 = ctypes.c_float
vp = ctypes.c_void_p


class DispatchDesc(ctypes.Structure):
    """rrr_dispatch_desc (include/rrr_hip.h)."""
    _fields_ = [
        ("name", ctypes.c_char_p),
        ("bufs", ctypes.POINTER(c_buf_p)),
        ("n_bufs", u32),
        ("push", vp),
        ("push_bytes", u32),
        ("groups", u32 * 3),
        ("barrier", u32),
    ]


class GgufKv(ctypes.Structure):
    """rrr_gguf_kv (include/rrr_gguf.h)."""
    _fields_ = [
        ("key", ctypes.c_char_p),
        ("key_len", u64),
        ("type", u32),
        ("elem_type", u32),
        ("count", u64),
        ("data", vp),
        ("bytes", u64),
    ]


class GgufTensor(ctypes.Structure):
    """rrr_gguf_tensor (include/rrr_gguf.h)."""
    _fields_ = [
        ("name", ctypes.c_char_p),
        ("name_len", u64),
        ("n_dims", u32),
        ("type", u32),
        ("dims", u64 * 4),
        ("offset", u64),
        ("n_elements", u64),
        ("bytes", u64),
        ("data", vp),
    ]


# name -> (restype, argtypes); every symbol include/rrr_hip.h and include/rrr_gguf.h declare.
SIGNATURES = {
    "rrr_init": (i32, [i32, ctypes.POINTER(c_ctx_p)]),
    "rrr_destroy": (i32, [c_ctx_p]),
    "rrr_last_error": (ctypes.c_char_p, []),
    "rrr_abi_version": (i32, []),
    "rrr_device_count": (i32, []),
    "rrr_buf_alloc": (i32, [c_ctx_p, u64, ctypes.POINTER(c_buf_p)]),
    "rrr_buf_view": (i32, [c_ctx_p, c_buf_p, u64, u64, ctypes.POINTER(c_buf_p)]),
    "rrr_buf_free": (i32, [c_ctx_p, c_buf_p]),
    "rrr_buf_size": (u64, [c_buf_p]),
    "rrr_buf_upload": (i32, [c_ctx_p, c_buf_p, u64, vp, u64]),
    "rrr_buf_download": (i32, [c_ctx_p, c_buf_p, u64, vp, u64]),
    "rrr_buf_fill_u32": (i32, [c_ctx_p, c_buf_p, u64, u64, u32]),
    "rrr_tensor_bytes": (u64, [u32, u32, u32]),
    "rrr_weight_upload": (i32, [c_ctx_p, u32, u32, u32, vp, u64, ctypes.POINTER(c_buf_p)]),
    "rrr_dequant": (i32, [c_ctx_p, u32, c_buf_p, c_buf_p, u64]),
    "rrr_gemv": (i32, [c_ctx_p, c_buf_p, c_buf_p, u32, c_buf_p, u32, u32, u32]),
    "rrr_gemm_bf16": (i32, [c_ctx_p, c_buf_p, c_buf_p, u32, c_buf_p, u32, u32, u32]),
    "rrr_rmsnorm": (i32, [c_ctx_p, c_buf_p, c_buf_p, c_buf_p, u32, u32, f32]),
    "rrr_silu_gate": (i32, [c_ctx_p, c_buf_p, c_buf_p, u32, u32]),
    "rrr_residual_add": (i32, [c_ctx_p, c_buf_p, c_buf_p, c_buf_p, u32]),
    "rrr_logits_f32": (i32, [c_ctx_p, c_buf_p, c_buf_p, c_buf_p, u32, u32, u32, u32]),
    "rrr_argmax_f32": (i32, [c_ctx_p, c_buf_p, u32, c_buf_p]),
    "rrr_gemv_rmsnorm": (i32, [c_ctx_p, c_buf_p, c_buf_p, f32, c_buf_p, u32, c_buf_p, u32, u32]),
    "rrr_gemv_rmsnorm_silu": (i32, [c_ctx_p, c_buf_p, c_buf_p, f32, c_buf_p, u32, c_buf_p, u32, u32]),
    "rrr_gemv_residual": (i32, [c_ctx_p, c_buf_p, u32, u32, c_buf_p, u32, c_buf_p, u32, u32]),
    "rrr_logits_rmsnorm": (i32, [c_ctx_p, c_buf_p, c_buf_p, f32, c_buf_p, c_buf_p, u32, u32, u32, u32]),
    "rrr_logits_rmsnorm_argmax": (i32, [c_ctx_p, c_buf_p, c_buf_p, f32, c_buf_p, c_buf_p, u32, u32, u32, u32, c_buf_p]),
    "rrr_rope_kv_store": (i32, [c_ctx_p, c_buf_p, c_buf_p, u32, c_buf_p, c_buf_p, u32, u32, u32, u32, u32, u32, u32,
                                f32, f32]),
    "rrr_gemv_rmsnorm_rope_kv": (i32, [c_ctx_p, c_buf_p, c_buf_p, f32, c_buf_p, u32, c_buf_p, u32, c_buf_p, u32,
                                       c_buf_p, c_buf_p, u32, u32, u32, u32, u32, u32, u32, f32, f32]),
    "rrr_attention": (i32, [c_ctx_p, c_buf_p, c_buf_p, c_buf_p, c_buf_p, u32, u32, u32, u32]),
    "rrr_attention_noalloc": (i32, [vp, vp, vp, vp, u32, u32, u32, u32, vp]),
    "rrr_probe_read": (i32, [c_ctx_p, c_buf_p, u64, c_buf_p]),
    "rrr_probe_read_shares": (i32, [c_ctx_p, c_buf_p, u64, c_buf_p]),
    "rrr_probe_gemv_phases": (i32, [c_ctx_p, u32, u32, u32, c_buf_p, c_buf_p, f32, c_buf_p, u32, c_buf_p, u32, u32,
                                    c_buf_p, ctypes.POINTER(u32), ctypes.POINTER(u32)]),
    "rrr_probe_mfma": (i32, [c_ctx_p, u32, u32, u32, c_buf_p]),
    "rrr_probe_cus": (u32, [c_ctx_p]),
    "rrr_rope_kv_store_rows": (i32, [c_ctx_p, c_buf_p, u32, c_buf_p, u32, c_buf_p, c_buf_p, u32, u32, u32, u32, u32,
                                     u32, u32, f32, f32]),
    "rrr_attention_prefill": (i32, [c_ctx_p, c_buf_p, u32, c_buf_p, c_buf_p, c_buf_p, u32, u32, u32, u32, u32]),
    "rrr_gemm_f16": (i32, [c_ctx_p, c_buf_p, c_buf_p, c_buf_p, u32, c_buf_p, u32, u32, u32, u32]),
    "rrr_gemm_f16_rmsnorm": (i32, [c_ctx_p, c_buf_p, c_buf_p, c_buf_p, u32, c_buf_p, u32, u32, u32, u32, c_buf_p, f32,
                                   c_buf_p]),
    "rrr_gemm_f16_silu_gate_f16": (i32, [c_ctx_p, c_buf_p, c_buf_p, u32, c_buf_p, c_buf_p, u32, u32, u32]),
    "rrr_gemm_f16_rope_kv_rows": (i32, [c_ctx_p, c_buf_p, c_buf_p, u32, c_buf_p, u32, u32, u32, c_buf_p, u32, c_buf_p,
                                        c_buf_p, u32, u32, u32, u32, u32, u32, u32, f32, f32]),
    "rrr_rmsnorm_f16": (i32, [c_ctx_p, c_buf_p, c_buf_p, c_buf_p, u32, u32, f32]),
    "rrr_silu_gate_f16": (i32, [c_ctx_p, c_buf_p, c_buf_p, c_buf_p, u32, u32]),
    "rrr_dispatch": (i32, [c_ctx_p, ctypes.c_char_p, ctypes.POINTER(c_buf_p), u32, vp, u32,
                           ctypes.POINTER(u32)]),
    "rrr_dispatch_batch": (i32, [c_ctx_p, ctypes.POINTER(DispatchDesc), u32]),
    "rrr_graph_begin": (i32, [c_ctx_p]),
    "rrr_graph_end": (i32, [c_ctx_p, ctypes.POINTER(vp)]),
    "rrr_graph_launch": (i32, [c_ctx_p, vp]),
    "rrr_graph_destroy": (i32, [c_ctx_p, vp]),
    "rrr_set_async": (i32, [c_ctx_p, i32]),
    "rrr_sync": (i32, [c_ctx_p]),
    "rrr_timer_start": (i32, [c_ctx_p]),
    "rrr_timer_stop": (i32, [c_ctx_p, ctypes.POINTER(f32)]),
    "rrr_matmul_kquant": (i32, [c_ctx_p, c_buf_p, c_buf_p, c_buf_p, u32, vp, vp, u32, u32]),
    # GGUF reader (include/rrr_gguf.h)
    "rrr_gguf_open": (i32, [ctypes.c_char_p, ctypes.POINTER(vp)]),
    "rrr_gguf_open_memory": (i32, [vp, u64, ctypes.POINTER(vp)]),
    "rrr_gguf_close": (i32, [vp]),
    "rrr_gguf_header": (i32, [vp, ctypes.POINTER(u32), ctypes.POINTER(u64), ctypes.POINTER(u64),
                              ctypes.POINTER(u64), ctypes.POINTER(u64)]),
    "rrr_gguf_kv_at": (i32, [vp, u64, ctypes.POINTER(GgufKv)]),
    "rrr_gguf_find_kv": (i32, [vp, ctypes.c_char_p, ctypes.POINTER(u64)]),
    "rrr_gguf_kv_strings": (i32, [vp, u64, u64, u64, ctypes.POINTER(vp), ctypes.POINTER(u64)]),
    "rrr_gguf_get_u64": (i32, [vp, ctypes.c_char_p, ctypes.POINTER(u64)]),
    "rrr_gguf_get_f64": (i32, [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double)]),
    "rrr_gguf_get_str": (i32, [vp, ctypes.c_char_p, ctypes.POINTER(vp), ctypes.POINTER(u64)]),
    "rrr_gguf_tensor_at": (i32, [vp, u64, ctypes.POINTER(GgufTensor)]),
    "rrr_gguf_find_tensor": (i32, [vp, ctypes.c_char_p, ctypes.POINTER(GgufTensor)]),
    "rrr_gguf_type_size": (i32, [u32, ctypes.POINTER(u32), ctypes.POINTER(u32)]),
    "rrr_gguf_upload": (i32, [c_ctx_p, vp, ctypes.c_char_p, ctypes.POINTER(c_buf_p)]),
}

SYNTH_SIGNATURES = {
    "rrr_synth_word": (u64, [u64, u64, u64]),
    "rrr_synth_f32_to_f16": (ctypes.c_uint16, [f32]),
    "rrr_synth_normal_f32": (None, [u64, u64, f32, f32, vp, u64, i32]),
    "rrr_synth_normal_bf16": (None, [u64, u64, f32, f32, vp, u64, i32]),
    "rrr_synth_kquant": (i32, [u64, u64, u32, vp, u64, i32]),
}

_hip = None
_synth = None


def _bind(lib, table):
    for name, (res, args) in table.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def hip():
    """The loaded librrr_hip.so (raises if it has not been built)."""
    global _hip
    if _hip is None:
        if not os.path.exists(HIP_LIB):
            raise RuntimeError(f"{HIP_LIB} is missing: build it with `make -C {PKG_DIR}/csrc` "
                               "(or __graft_entry__.build())")
        _hip = _bind(ctypes.CDLL(HIP_LIB), SIGNATURES)
    return _hip


def synth():
    global _synth
    if _synth is None:
        if not os.path.exists(SYNTH_LIB):
            raise RuntimeError(f"{SYNTH_LIB} is missing: build it with `make -C {PKG_DIR}/csrc`")
        _synth = _bind(ctypes.CDLL(SYNTH_LIB), SYNTH_SIGNATURES)
    return _synth
