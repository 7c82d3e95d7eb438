"""Restatement of the reference's GGUF reader -- TEST INFRASTRUCTURE ONLY.

A pure-Python statement of src/model/gguf.rs as it behaves, defects
included, so that tests can show (a) that the product reader
(librrr_hip's rrr_gguf_*) returns exactly what the reference returns on
every file the reference reads correctly, and (b) where the two part: the
reference reads UINT8 and INT8 values as 4 bytes (gguf.rs:100-101) and skips
one byte for an unknown value type (gguf.rs:119).  Only tests/ may import it,
and only to check the library's results against.

Panics of the Rust code (slice out of range, failed assert, from_utf8
unwrap, unknown quant type) raise RefPanic here.

Pinned by tests/test_gguf_cpu.py: a hand-assembled byte image whose every
field is written out by hand (the specification's layout), files from the
writer covering every value type the reference decodes as specified, and a
hand-derived value for the UINT8 misread.
"""
import struct

GGUF_MAGIC = 0x46554747


class RefPanic(Exception):
    """A panic of the reference reader."""


class Reader:
    """Reader (gguf.rs:62-122)."""

    def __init__(self, data):
        self.data, self.pos = data, 0

    def _take(self, n):
        # Rust slice indexing: a range past the end panics (gguf.rs:70-96)
        if self.pos + n > len(self.data):
            raise RefPanic(f"range end index {self.pos + n} out of range for slice of length {len(self.data)}")
        b = self.data[self.pos:self.pos + n]
        self.pos += n
        return b

    def u8(self):                        # gguf.rs:70
        return self._take(1)[0]

    def u32(self):                       # gguf.rs:71-74
        return struct.unpack("<I", self._take(4))[0]

    def u64(self):                       # gguf.rs:75-78
        return struct.unpack("<Q", self._take(8))[0]

    def i32(self):                       # gguf.rs:79
        return struct.unpack("<i", struct.pack("<I", self.u32()))[0]

    def i64(self):                       # gguf.rs:80
        return struct.unpack("<q", struct.pack("<Q", self.u64()))[0]

    def f32_raw(self):                   # gguf.rs:83-86
        return struct.unpack("<f", self._take(4))[0]

    def f64_raw(self):                   # gguf.rs:87-90
        return struct.unpack("<d", self._take(8))[0]

    def string(self):                    # gguf.rs:92-96
        n = self.u64()
        raw = self._take(n)
        try:
            return raw.decode("utf-8")
        except UnicodeDecodeError as e:
            raise RefPanic(f"from_utf8: {e}") from None

    def value(self, typ):                # gguf.rs:98-121
        if typ == 0:
            return ("U32", self.u32())   # UINT8 read as 4 bytes (gguf.rs:100)
        if typ == 1:
            return ("I32", self.i32())   # INT8 read as 4 bytes (gguf.rs:101)
        if typ == 2:
            return ("U32", struct.unpack("<H", self._take(2))[0])
        if typ == 3:
            return ("I32", struct.unpack("<h", self._take(2))[0])
        if typ == 4:
            return ("U32", self.u32())
        if typ == 5:
            return ("I32", self.i32())
        if typ == 6:
            return ("F32", self.f32_raw())
        if typ == 7:
            return ("Bool", self.u8() != 0)
        if typ == 8:
            return ("Str", self.string())
        if typ == 9:
            at = self.u32()
            n = self.u64()
            return ("Array", [self.value(at) for _ in range(n)])
        if typ == 10:
            return ("U64", self.u64())
        if typ == 11:
            return ("I64", self.i64())
        if typ == 12:
            return ("F64", self.f64_raw())
        self.pos += 1                    # unknown type: one byte skipped (gguf.rs:119)
        return ("U32", 0)


def as_u64(v):                           # gguf.rs:41-49
    tag, x = v
    if tag in ("U32", "U64"):
        return x
    if tag in ("I32", "I64"):
        return x & 0xFFFFFFFFFFFFFFFF
    return None


class RefModel:
    """GGUFModel::load (gguf.rs:124-170) and tensor_bytes (gguf.rs:173-195)."""

    # gguf.rs:178-191: ggml type -> (elements per block, bytes per block)
    SIZES = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 9: (32, 36),
             12: (256, 144), 13: (256, 176), 14: (256, 210)}

    def __init__(self, data):
        self.data = bytes(data)
        r = Reader(self.data)
        if r.u32() != GGUF_MAGIC:
            raise RefPanic("Not a GGUF file")
        self.version = r.u32()
        self.n_tensors = r.u64()
        n_kv = r.u64()
        self.metadata = {}
        for _ in range(n_kv):
            key = r.string()
            typ = r.u32()
            self.metadata[key] = r.value(typ)     # HashMap::insert: a later duplicate wins
        self.tensor_infos = []
        for _ in range(self.n_tensors):
            name = r.string()
            n_dims = r.u32()
            shape = [r.u64() for _ in range(n_dims)]
            typ = r.u32()
            offset = r.u64()
            self.tensor_infos.append((name, shape, typ, offset))
        a = self.metadata.get("general.alignment")
        a = as_u64(a) if a is not None else None
        alignment = 32 if a is None else a
        if alignment == 0:
            raise RefPanic("attempt to divide by zero")
        self.header_end = r.pos
        self.data_offset = (r.pos + alignment - 1) // alignment * alignment

    def tensor_bytes(self, name):
        info = next((t for t in self.tensor_infos if t[0] == name), None)
        if info is None:
            raise RefPanic(f"Tensor not found: {name}")
        _, shape, typ, offset = info
        n = 1
        for d in shape:
            n *= d
        if typ not in self.SIZES:
            raise RefPanic(f"Unknown quant type {typ} for tensor {name}")
        be, bb = self.SIZES[typ]
        size = n // be * bb
        start = self.data_offset + offset
        if start + size > len(self.data):
            raise RefPanic(f"range end index {start + size} out of range for slice of length {len(self.data)}")
        return self.data[start:start + size]
