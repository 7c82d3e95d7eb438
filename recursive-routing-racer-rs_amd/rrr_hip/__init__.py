"""rrr_hip: MI355X (gfx950) weight-heavy decode path of Recursive Routing Racer.

The compute lives in librrr_hip.so (HIP kernels behind the C ABI of
include/rrr_hip.h); this package is the Python host binding used by the
tests and the benchmark.
"""
from .engine import (ACT_GQA_V, ACT_IDENTITY, ACT_SILU_GATE, BLOCK_BYTES, DEVICE_NONE, F16, F32,
                     LOGITS_CHUNKED, LOGITS_Q6K, LOGITS_ROWS, Q4_K, Q5_K, Q6_K, Buffer, ComputeEngine,
                     Context, DescSetHandle, GpuBuffer, Graph, RrrError, device_count,
                     tensor_bytes)
from . import engine, gguf, synth
from .gguf import GGUFModel, ModelConfig, write_gguf

__all__ = [
    "ACT_GQA_V", "ACT_IDENTITY", "ACT_SILU_GATE", "BLOCK_BYTES", "DEVICE_NONE", "F16", "F32",
    "LOGITS_CHUNKED", "LOGITS_Q6K", "LOGITS_ROWS", "Q4_K", "Q5_K", "Q6_K", "Buffer", "ComputeEngine",
    "Context", "DescSetHandle", "GpuBuffer", "Graph", "RrrError", "device_count",
    "tensor_bytes", "engine", "synth", "gguf", "GGUFModel", "ModelConfig", "write_gguf",
]
