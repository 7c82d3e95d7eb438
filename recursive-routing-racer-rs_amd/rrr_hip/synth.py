"""Seeded synthetic inputs (csrc/synth.c) as numpy arrays.

Each tensor of a workload draws from its own stream id of the workload's
seed, so every tensor can be regenerated independently and identically on
any machine, with any thread count.
"""
import os

import numpy as np

from . import _lib

BLOCK_BYTES = {12: 144, 13: 176, 14: 210}


def _threads(threads):
    if threads:
        return threads
    return max(1, min(16, os.cpu_count() or 1))


def kquant(seed, stream, qtype, n_blocks, threads=0):
    """n_blocks raw super-blocks of GGUF type 12/13/14 (uint8 array)."""
    out = np.empty(n_blocks * BLOCK_BYTES[qtype], dtype=np.uint8)
    rc = _lib.synth().rrr_synth_kquant(seed, stream, qtype, out.ctypes.data, n_blocks, _threads(threads))
    if rc != 0:
        raise ValueError(f"type {qtype}")
    return out


def weight(seed, stream, qtype, K, N, threads=0):
    """An N x K tensor of K-quant type `qtype` as raw GGUF bytes."""
    return kquant(seed, stream, qtype, N * (K // 256), threads)


def normal_f32(seed, stream, n, mean=0.0, std=1.0, threads=0):
    out = np.empty(n, dtype=np.float32)
    _lib.synth().rrr_synth_normal_f32(seed, stream, mean, std, out.ctypes.data, n, _threads(threads))
    return out


def normal_bf16(seed, stream, n, mean=0.0, std=1.0, threads=0):
    """bf16 bit patterns (uint16) of N(mean, std^2) samples."""
    out = np.empty(n, dtype=np.uint16)
    _lib.synth().rrr_synth_normal_bf16(seed, stream, mean, std, out.ctypes.data, n, _threads(threads))
    return out


def f32_to_f16_bits(x):
    return int(_lib.synth().rrr_synth_f32_to_f16(float(x)))
