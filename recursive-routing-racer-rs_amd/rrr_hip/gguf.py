"""GGUF models: the bounds-checked reader of librrr_hip (include/rrr_gguf.h),
a writer, and the model configuration read from a file's metadata.

`GGUFModel` mirrors the reference's loader (src/model/gguf.rs:18-195):
`GGUFModel.load(path)` maps and parses the file; `version`, `n_tensors`,
`metadata`, `tensor_infos` and `data_offset` are the reference's fields;
`tensor_bytes(name)` / `tensor_f32(name)` return zero-copy views of the
mapping.  Malformed files raise RrrError (code ERR_FORMAT, ERR_IO, ...)
instead of panicking or reading the wrong bytes.  `upload(ctx, name)` sends a
weight's raw bytes to the device unchanged (rrr_gguf_upload).

`ModelConfig.from_gguf` is the reference's metadata read
(ModelConfig::from_gguf, phi4.rs:31-101), defaults included.

`write_gguf` writes a GGUF v3 file (header, typed metadata, tensor records,
aligned data): it exports a model, e.g. the seeded synthetic one, in the
format the reference and this library load.
"""
import ctypes
import struct
import weakref
from dataclasses import dataclass
from typing import NamedTuple

import numpy as np

from . import _lib
from .engine import Buffer, RrrError, _check, _ptr

(UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64,
 FLOAT64) = range(13)

# value type -> (struct code, numpy dtype) of the fixed-size types
_SCALAR = {UINT8: ("<B", np.uint8), INT8: ("<b", np.int8), UINT16: ("<H", np.uint16), INT16: ("<h", np.int16),
           UINT32: ("<I", np.uint32), INT32: ("<i", np.int32), FLOAT32: ("<f", np.float32), BOOL: ("<?", np.bool_),
           UINT64: ("<Q", np.uint64), INT64: ("<q", np.int64), FLOAT64: ("<d", np.float64)}

GGUF_MAGIC = 0x46554747
DEFAULT_ALIGNMENT = 32


class TensorInfo(NamedTuple):
    """A tensor record (TensorInfo, gguf.rs:10-16) and its byte size."""
    name: str
    shape: tuple      # ne0 (the row length) first
    typ: int          # ggml type
    offset: int       # from data_offset
    n_elements: int
    nbytes: int


def type_size(ggml_type):
    """(elements per block, bytes per block) of a ggml type."""
    e, b = ctypes.c_uint32(), ctypes.c_uint32()
    _check(_lib.hip().rrr_gguf_type_size(ggml_type, ctypes.byref(e), ctypes.byref(b)))
    return e.value, b.value


def _str(raw):
    try:
        return raw.decode("utf-8")
    except UnicodeDecodeError:
        return raw


def _decode_array(buf, pos, et, n):
    """Decode n elements of type et from bytes buf at pos (an already
    validated record); returns (value, new pos).  Numeric arrays become numpy
    arrays, string and nested arrays lists."""
    if et in _SCALAR:
        code, dt = _SCALAR[et]
        size = struct.calcsize(code)
        return np.frombuffer(buf, dt, n, pos).copy(), pos + n * size
    out = []
    for _ in range(n):
        if et == STRING:
            (ln,) = struct.unpack_from("<Q", buf, pos)
            out.append(_str(bytes(buf[pos + 8:pos + 8 + ln])))
            pos += 8 + ln
        else:
            sub_et, sub_n = struct.unpack_from("<IQ", buf, pos)
            val, pos = _decode_array(buf, pos + 12, sub_et, sub_n)
            out.append(val)
    return out, pos


class GGUFModel:
    """A mapped GGUF file (GGUFModel, gguf.rs:18-25)."""

    def __init__(self, path=None, data=None):
        """From a file path, or from an in-memory image `data` (bytes-like,
        kept referenced by the model)."""
        if (path is None) == (data is None):
            raise ValueError("give exactly one of path and data")
        self._lib = _lib.hip()
        h = ctypes.c_void_p()
        self._image = None
        if path is not None:
            _check(self._lib.rrr_gguf_open(str(path).encode(), ctypes.byref(h)))
        else:
            self._image = np.frombuffer(bytes(data), np.uint8)
            _check(self._lib.rrr_gguf_open_memory(_ptr(self._image), self._image.nbytes, ctypes.byref(h)))
        self._handle = h.value
        self._views = []    # weak references to live tensor views
        ver, nt, nkv, al, off = (ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64(),
                                 ctypes.c_uint64())
        _check(self._lib.rrr_gguf_header(self._h, ctypes.byref(ver), ctypes.byref(nt), ctypes.byref(nkv),
                                         ctypes.byref(al), ctypes.byref(off)))
        self.version, self.n_tensors, self.n_kv = ver.value, nt.value, nkv.value
        self.alignment, self.data_offset = al.value, off.value
        self.metadata, self.metadata_types = {}, {}
        for i in range(self.n_kv):
            kv = _lib.GgufKv()
            _check(self._lib.rrr_gguf_kv_at(self._h, i, ctypes.byref(kv)))
            key = kv.key.decode("utf-8")
            self.metadata[key] = self._value(i, kv)
            self.metadata_types[key] = (kv.type, kv.elem_type)
        self.tensor_infos = []
        self._tensors = {}
        for i in range(self.n_tensors):
            t = _lib.GgufTensor()
            _check(self._lib.rrr_gguf_tensor_at(self._h, i, ctypes.byref(t)))
            info = TensorInfo(t.name.decode("utf-8"), tuple(t.dims[:t.n_dims]), t.type, t.offset, t.n_elements,
                              t.bytes)
            self.tensor_infos.append(info)
            self._tensors[info.name] = info

    @classmethod
    def load(cls, path):
        """GGUFModel::load (gguf.rs:125-170)."""
        return cls(path=path)

    @property
    def _h(self):
        if self._handle is None:
            raise RrrError(-10, "GGUF model already closed")
        return self._handle

    def _value(self, index, kv):
        raw = ctypes.string_at(kv.data, kv.bytes) if kv.bytes else b""
        if kv.type in _SCALAR:
            v = struct.unpack(_SCALAR[kv.type][0], raw)[0]
            return bool(v) if kv.type == BOOL else v
        if kv.type == STRING:
            return _str(raw)
        if kv.elem_type == STRING:
            n = kv.count
            ptrs, lens = (ctypes.c_void_p * max(n, 1))(), (ctypes.c_uint64 * max(n, 1))()
            _check(self._lib.rrr_gguf_kv_strings(self._h, index, 0, n, ptrs, lens))
            base = kv.data
            return [_str(raw[ptrs[i] - base:ptrs[i] - base + lens[i]]) for i in range(n)]
        val, _ = _decode_array(memoryview(raw), 0, kv.elem_type, kv.count)
        return val

    # -- metadata (MetaValue::as_u64 / as_f32 / as_str, gguf.rs:41-59) --------
    def get_u64(self, key):
        v = ctypes.c_uint64()
        _check(self._lib.rrr_gguf_get_u64(self._h, key.encode(), ctypes.byref(v)))
        return v.value

    def get_f64(self, key):
        v = ctypes.c_double()
        _check(self._lib.rrr_gguf_get_f64(self._h, key.encode(), ctypes.byref(v)))
        return v.value

    def get_str(self, key):
        p, n = ctypes.c_void_p(), ctypes.c_uint64()
        _check(self._lib.rrr_gguf_get_str(self._h, key.encode(), ctypes.byref(p), ctypes.byref(n)))
        return _str(ctypes.string_at(p.value, n.value)) if n.value else ""

    # -- tensors ---------------------------------------------------------------
    def tensor_info(self, name):
        try:
            return self._tensors[name]
        except KeyError:
            raise RrrError(-12, f"no tensor '{name}'") from None

    def has_tensor(self, name):
        return name in self._tensors

    def tensor_bytes(self, name):
        """The tensor's raw bytes as a read-only uint8 view of the mapping
        (tensor_bytes, gguf.rs:173-195).  Views keep the model from closing."""
        t = _lib.GgufTensor()
        _check(self._lib.rrr_gguf_find_tensor(self._h, name.encode(), ctypes.byref(t)))
        if t.bytes == 0:
            return np.zeros(0, np.uint8)
        arr = (ctypes.c_uint8 * t.bytes).from_address(t.data)
        arr._model = self
        self._views = [r for r in self._views if r() is not None]
        self._views.append(weakref.ref(arr))
        v = np.frombuffer(arr, np.uint8)
        v.flags.writeable = False
        return v

    def tensor_f32(self, name):
        """An F32 tensor as a float32 view (tensor_f32, gguf.rs:198-205)."""
        info = self.tensor_info(name)
        if info.typ != 0:
            raise RrrError(-2, f"tensor '{name}' has ggml type {info.typ}, not F32")
        return self.tensor_bytes(name).view(np.float32)

    def upload(self, ctx, name):
        """The weight's raw bytes in a new device buffer (rrr_gguf_upload)."""
        h = ctypes.c_void_p()
        _check(self._lib.rrr_gguf_upload(ctx._h, self._h, name.encode(), ctypes.byref(h)))
        return Buffer(ctx, h.value, self.tensor_info(name).nbytes)

    def close(self):
        """Unmaps the file; refused while tensor views are alive."""
        if self._handle is None:
            return
        if any(r() is not None for r in self._views):
            raise RrrError(-9, "tensor views of this GGUF model are still alive")
        _check(self._lib.rrr_gguf_close(self._handle))
        self._handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            if getattr(self, "_handle", None) is not None and not any(r() is not None for r in self._views):
                self._lib.rrr_gguf_close(self._handle)
                self._handle = None
        except Exception:
            pass


# ---- writer ------------------------------------------------------------------

def _pack_value(vtype, value):
    if vtype in _SCALAR:
        return struct.pack(_SCALAR[vtype][0], value)
    if vtype == STRING:
        raw = value.encode("utf-8") if isinstance(value, str) else bytes(value)
        return struct.pack("<Q", len(raw)) + raw
    if vtype == ARRAY:
        et, items = value
        if et in _SCALAR and isinstance(items, np.ndarray):
            body = np.ascontiguousarray(items, _SCALAR[et][1]).tobytes()
        else:
            body = b"".join(_pack_value(et, it) for it in items)
        return struct.pack("<IQ", et, len(items)) + body
    raise ValueError(f"unknown GGUF value type {vtype}")


def write_gguf(path, metadata, tensors, alignment=DEFAULT_ALIGNMENT, version=3):
    """Writes a GGUF file.

    metadata: list of (key, value_type, value); an ARRAY value is
    (element_type, items).  tensors: list of (name, ggml_type, shape ne0-first,
    raw bytes); each raw size must match the type's block geometry.  Tensor
    data is placed in order, each at the next multiple of `alignment` (a
    general.alignment key is added when it is not 32 and the caller gave none).
    Returns the data section's file offset."""
    keys = [k for k, _, _ in metadata]
    if len(set(keys)) != len(keys):
        raise ValueError("duplicate metadata keys")
    if alignment != DEFAULT_ALIGNMENT and "general.alignment" not in keys:
        metadata = list(metadata) + [("general.alignment", UINT32, alignment)]
    head = [struct.pack("<IIQQ", GGUF_MAGIC, version, len(tensors), len(metadata))]
    for key, vtype, value in metadata:
        head.append(_pack_value(STRING, key) + struct.pack("<I", vtype) + _pack_value(vtype, value))
    offset, layout = 0, []
    for name, typ, shape, raw in tensors:
        raw = np.frombuffer(raw, np.uint8) if isinstance(raw, (bytes, bytearray)) else raw.reshape(-1).view(np.uint8)
        n = int(np.prod(shape, dtype=np.uint64)) if len(shape) else 1
        be, bb = type_size(typ)
        if shape[0] % be or raw.nbytes != n // be * bb:
            raise ValueError(f"tensor {name}: {raw.nbytes} bytes do not hold a type-{typ} tensor of shape {shape}")
        offset = -(-offset // alignment) * alignment
        head.append(_pack_value(STRING, name) + struct.pack("<I", len(shape)) +
                    struct.pack(f"<{len(shape)}Q", *shape) + struct.pack("<IQ", typ, offset))
        layout.append((offset, raw))
        offset += raw.nbytes
    header = b"".join(head)
    data_offset = -(-len(header) // alignment) * alignment
    with open(path, "wb") as f:
        f.write(header)
        f.write(b"\0" * (data_offset - len(header)))
        pos = 0
        for off, raw in layout:
            f.write(b"\0" * (off - pos))
            f.write(memoryview(raw))
            pos = off + raw.nbytes
    return data_offset


# ---- model configuration -----------------------------------------------------

@dataclass(frozen=True)
class ModelConfig:
    """ModelConfig (phi4.rs:9-28), read from GGUF metadata."""
    arch: str
    d_model: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn_dim: int
    n_layers: int
    vocab_size: int
    rms_eps: float
    rope_dim: int
    rope_theta: float
    rope_attn_factor: float
    has_qkv_bias: bool
    has_rope_factors: bool
    separate_qkv: bool
    separate_gate_up: bool
    has_output_weight: bool

    @classmethod
    def from_gguf(cls, model):
        """ModelConfig::from_gguf (phi4.rs:31-101): architecture prefix,
        integer and float keys with the reference's defaults, and the tensor
        layout flags."""
        md = model.metadata
        arch = md.get("general.architecture")
        arch = arch if isinstance(arch, str) else "llama"

        def get_int(key):
            v = md.get(f"{arch}.{key}")
            return int(v) if isinstance(v, int) and not isinstance(v, bool) and v >= 0 else 0

        def get_float(key):
            v = md.get(f"{arch}.{key}")
            return float(v) if isinstance(v, float) else 0.0

        d = get_int("embedding_length")
        n_heads = get_int("attention.head_count")
        head_dim = d // n_heads if n_heads > 0 else 128
        eps = get_float("attention.layer_norm_rms_epsilon")
        rope_dim = get_int("rope.dimension_count")
        theta = get_float("rope.freq_base")
        attn_factor = get_float("rope.scaling.attn_factor")
        names = {t.name for t in model.tensor_infos}
        emb = model._tensors.get("token_embd.weight")
        has_qkv = "blk.0.attn_qkv.weight" in names
        return cls(
            arch=arch, d_model=d, n_heads=n_heads, n_kv_heads=get_int("attention.head_count_kv"),
            head_dim=head_dim, ffn_dim=get_int("feed_forward_length"), n_layers=get_int("block_count"),
            vocab_size=emb.shape[1] if emb is not None and len(emb.shape) > 1 else 0,
            rms_eps=eps if eps > 0 else 1e-5, rope_dim=rope_dim if rope_dim > 0 else head_dim,
            rope_theta=theta if theta > 0 else 10000.0, rope_attn_factor=attn_factor if attn_factor > 0 else 1.0,
            has_qkv_bias="blk.0.attn_q.bias" in names, has_rope_factors=any("rope_factors" in n for n in names),
            separate_qkv="blk.0.attn_q.weight" in names and not has_qkv,
            separate_gate_up="blk.0.ffn_gate.weight" in names,
            has_output_weight="output.weight" in names)

    @property
    def qkv_dim(self):
        return self.n_heads * self.head_dim + 2 * self.n_kv_heads * self.head_dim

    @property
    def gate_up_dim(self):
        return 2 * self.ffn_dim
