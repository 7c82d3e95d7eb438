"""rrr_attention_noalloc: decode attention with the library's own scratch
array (no allocation, no context) against rrr_attention, the entry point
whose kernels it shares, through the C ABI.

Bar: the same bits (same kernels, same launch plan for the same seq_len),
on two calls in a row, the second on a smaller problem (fewer rows and
heads, so stale partials of the first call would show), and within 1e-4
normwise of the fp64 oracle.  The entry point takes plain device pointers
and a stream: the test allocates them with the HIP runtime the library
itself has loaded (found in the process's memory map) and passes the null
stream.
"""
import ctypes
import ctypes.util
import os

import numpy as np
import pytest

import oracle.oracle as orc
import rrr_hip
from rrr_hip import _lib

pytestmark = pytest.mark.gpu

HD = 128
H2D, D2H = 1, 2   # hipMemcpyHostToDevice, hipMemcpyDeviceToHost


def _runtime_path():
    """The libamdhip64 that librrr_hip.so brought into this process."""
    with open("/proc/self/maps") as f:
        for line in f:
            path = line.split()[-1]
            if os.path.basename(path).startswith("libamdhip64.so"):
                return path
    return ctypes.util.find_library("amdhip64") or "libamdhip64.so"


def _hip():
    _lib.hip()   # the library first: it loads the runtime this binds to
    rt = ctypes.CDLL(_runtime_path())
    rt.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    rt.hipFree.argtypes = [ctypes.c_void_p]
    rt.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    for f in (rt.hipMalloc, rt.hipFree, rt.hipMemcpy, rt.hipDeviceSynchronize):
        f.restype = ctypes.c_int
    return rt


class DevArray:
    """Device memory holding a copy of a host array."""

    def __init__(self, rt, host):
        self.rt, self.nbytes = rt, host.nbytes
        self.ptr = ctypes.c_void_p()
        assert rt.hipMalloc(ctypes.byref(self.ptr), self.nbytes) == 0
        assert rt.hipMemcpy(self.ptr, host.ctypes.data, self.nbytes, H2D) == 0

    def get(self, dtype):
        out = np.empty(self.nbytes // np.dtype(dtype).itemsize, dtype)
        assert self.rt.hipMemcpy(out.ctypes.data, self.ptr, self.nbytes, D2H) == 0
        return out

    def free(self):
        self.rt.hipFree(self.ptr)


def _case(rng, seq, nkv, hpk):
    q = rng.standard_normal(nkv * hpk * HD).astype(np.float32)
    k = orc.f32_to_f16_bits(rng.standard_normal(seq * nkv * HD).astype(np.float32))
    v = orc.f32_to_f16_bits(rng.standard_normal(seq * nkv * HD).astype(np.float32))
    return q, k, v


def test_attention_noalloc_matches_rrr_attention(ctx):
    lib = _lib.hip()
    rt = _hip()
    rng = np.random.default_rng(5)
    for seq, nkv, hpk in ((2048, 8, 3), (100, 4, 2)):
        q, k, v = _case(rng, seq, nkv, hpk)
        nq = nkv * hpk * HD
        dq, dk, dv, do = ctx.to_device(q), ctx.to_device(k), ctx.to_device(v), ctx.alloc(nq * 4)
        ctx.attention(dq, dk, dv, do, seq, nkv, hpk, HD)
        ctx.sync()
        ref = ctx.download(do, np.float32, nq)
        for b in (dq, dk, dv, do):
            b.free()
        aq, ak, av = DevArray(rt, q), DevArray(rt, k), DevArray(rt, v)
        ao = DevArray(rt, np.full(nq, np.nan, np.float32))
        rc = lib.rrr_attention_noalloc(aq.ptr, ak.ptr, av.ptr, ao.ptr, seq, nkv, hpk, HD, None)
        assert rc == 0, lib.rrr_last_error()
        assert rt.hipDeviceSynchronize() == 0
        got = ao.get(np.float32)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (seq, nkv, hpk)
        assert orc.normwise_err(got, orc.attention_f64(q, k, v, seq, nkv, hpk, HD)) < 1e-4
        for a in (aq, ak, av, ao):
            a.free()
    # beyond the scratch array's limits: refused before any launch
    z = DevArray(rt, np.zeros(64, np.float32))
    p = z.ptr
    assert lib.rrr_attention_noalloc(p, p, p, p, 2049, 8, 3, HD, None) == rrr_hip.engine.ERR_UNSUPPORTED
    assert lib.rrr_attention_noalloc(p, p, p, p, 16, 16, 8, HD, None) == rrr_hip.engine.ERR_UNSUPPORTED
    assert lib.rrr_attention_noalloc(None, p, p, p, 16, 8, 3, HD, None) == rrr_hip.engine.ERR_NULL
    z.free()
