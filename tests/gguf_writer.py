"""A small GGUF v2/v3 writer for tests (the layout the reference's
bd::GgufWriter writes, ref/bonsai-decoder/src/gguf.cpp:221-291): "GGUF",
u32 version, u64 n_tensors, u64 n_kv, the key/value pairs, the tensor infos,
zero padding to the alignment, the data section (each tensor's data at an
aligned offset). Knobs for malformed files let the tests exercise the
reader's checks."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
        I64: "<q", F64: "<d"}
# ggml type id -> (elements per block, bytes per block), the formats' sizes
GGML = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 12: (256, 144),
        13: (256, 176), 14: (256, 210), 26: (1, 4), 30: (1, 2), 34: (256, 54), 35: (256, 66), 42: (64, 18),
        142: (128, 34), 143: (128, 28)}


def _str(s):
    b = s if isinstance(s, bytes) else s.encode()
    return struct.pack("<Q", len(b)) + b


def _val(t, v):
    return _str(v) if t == STRING else struct.pack(_FMT[t], v)


class Writer:
    def __init__(self, version=3, alignment=32, write_alignment_key=True):
        self.version, self.alignment, self.write_alignment_key = version, alignment, write_alignment_key
        self.kv, self.tensors = [], []

    def add(self, key, t, value, arr_type=None):
        """value: a scalar, or for t == ARRAY a list of arr_type elements."""
        if t == ARRAY:
            body = struct.pack("<IIQ", ARRAY, arr_type, len(value)) + b"".join(_val(arr_type, x) for x in value)
        else:
            body = struct.pack("<I", t) + _val(t, value)
        self.kv.append(_str(key) + body)
        return self

    def tensor(self, name, ne, ggml_type, data, offset=None):
        self.tensors.append((name, list(ne), ggml_type, bytes(data), offset))
        return self

    def build(self, truncate=None):
        kv = list(self.kv)
        if self.write_alignment_key:
            kv.append(_str("general.alignment") + struct.pack("<II", U32, self.alignment))
        a = self.alignment
        head = b"GGUF" + struct.pack("<IQQ", self.version, len(self.tensors), len(kv)) + b"".join(kv)
        off, offs = 0, []
        for name, ne, ty, data, fixed in self.tensors:
            o = off if fixed is None else fixed
            offs.append(o)
            head += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", x) for x in ne)
            head += struct.pack("<IQ", ty, o)
            off = (max(off, o + len(data)) + a - 1) // a * a
        head += b"\0" * ((-len(head)) % a)
        body = bytearray(off)
        for (_, _, _, data, _), o in zip(self.tensors, offs):
            body[o:o + len(data)] = data
        img = head + bytes(body)
        return img if truncate is None else img[:truncate]

    def write(self, path, **kw):
        img = self.build(**kw)
        with open(path, "wb") as f:
            f.write(img)
        return img


def ptq1_0_bytes(rng, N, K):
    """Random PTQ1_0 rows (any byte values: the codec decodes every byte)."""
    return rng.integers(0, 256, size=N * (K // 128) * 28, dtype=np.uint8)
