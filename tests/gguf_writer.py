"""A small GGUF v3 writer and ggml block packers, for building test files.

Test infrastructure: the files it writes are read back by the product
(cw.Gguf) and by the oracle (oracle.OracleGguf).  The container layout is
GGUF v3 as the reference's reader consumes it (src/loader/gguf.rs:68-106):
magic, version u32, tensor count u64, metadata count u64, metadata
(key string, kind u32, value), tensor infos (name, n_dims u32, dims u64,
dtype u32, offset u64), then the tensor data from the next multiple of the
alignment, each tensor's offset itself aligned.

The block packers write ggml's block layouts from their format definitions
(block_q4_0, block_q4_1, block_q8_0, block_q6_K); they are the inverse of
the decoders under test, written independently of them.
"""
import struct

import numpy as np

KIND = {"u8": 0, "i8": 1, "u16": 2, "i16": 3, "u32": 4, "i32": 5, "f32": 6, "bool": 7,
        "str": 8, "array": 9, "u64": 10, "i64": 11, "f64": 12}
_FMT = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B",
        10: "<Q", 11: "<q", 12: "<d"}

F32, F16, Q4_0, Q4_1, Q8_0, Q6_K = 0, 1, 2, 3, 8, 14


def gstr(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def value_bytes(kind, v):
    """Bytes of one metadata value of `kind` (a name of KIND or its code).
    An array is (element kind, [values])."""
    k = KIND[kind] if isinstance(kind, str) else kind
    if k == 8:
        return gstr(v)
    if k == 9:
        ek, items = v
        ekc = KIND[ek] if isinstance(ek, str) else ek
        return struct.pack("<IQ", ekc, len(items)) + b"".join(
            value_bytes(ekc, x) if ekc == 9 else _scalar(ekc, x) for x in items)
    return _scalar(k, v)


def _scalar(k, v):
    if k == 8:
        return gstr(v)
    return struct.pack(_FMT[k], v)


def _typed(kind, v):
    k = KIND[kind] if isinstance(kind, str) else kind
    return struct.pack("<I", k) + value_bytes(k, v)


class GgufWriter:
    def __init__(self, alignment=32, version=3):
        self.alignment = alignment
        self.version = version
        self.meta = []      # (key, kind, value)
        self.tensors = []   # (name, dims, dtype, raw)

    def add_meta(self, key, kind, value):
        self.meta.append((key, kind, value))
        return self

    def add_tensor(self, name, dims, dtype, raw):
        self.tensors.append((name, list(dims), dtype, bytes(raw)))
        return self

    def tobytes(self):
        out = bytearray(b"GGUF")
        out += struct.pack("<IQQ", self.version, len(self.tensors), len(self.meta))
        for key, kind, value in self.meta:
            out += gstr(key) + _typed(kind, value)
        offsets, off = [], 0
        for _, _, _, raw in self.tensors:
            offsets.append(off)
            off += len(raw)
            off = -(-off // self.alignment) * self.alignment
        for (name, dims, dtype, _), o in zip(self.tensors, offsets):
            out += gstr(name) + struct.pack("<I", len(dims))
            out += b"".join(struct.pack("<Q", d) for d in dims)
            out += struct.pack("<IQ", dtype, o)
        out += b"\0" * ((-len(out)) % self.alignment)
        base = len(out)
        for (_, _, _, raw), o in zip(self.tensors, offsets):
            out += b"\0" * (base + o - len(out))
            out += raw
        return bytes(out)

    def write(self, path):
        with open(path, "wb") as f:
            f.write(self.tobytes())
        return path


# ---------------------------------------------------------------- ggml block packers

def pack_q4_0(scales, quants):
    """block_q4_0 {f16 d; u8 qs[16]} from the split image (scales u16 [nb],
    quants u8 [nb][16])."""
    s = np.ascontiguousarray(scales, np.uint16).reshape(-1)
    q = np.ascontiguousarray(quants, np.uint8).reshape(-1, 16)
    blk = np.empty((s.size, 18), np.uint8)
    blk[:, :2] = s.view(np.uint8).reshape(-1, 2)
    blk[:, 2:] = q
    return blk.tobytes()


def pack_q4_1(d, m, nibbles):
    """block_q4_1 {f16 d; f16 m; u8 qs[16]}: element j < 16 in the low nibble
    of qs[j], element j + 16 in its high nibble.  nibbles [nb][32] in 0..15."""
    n = np.asarray(nibbles, np.uint8).reshape(-1, 32)
    blk = np.empty((n.shape[0], 20), np.uint8)
    blk[:, 0:2] = np.asarray(d, np.uint16).reshape(-1, 1).view(np.uint8)
    blk[:, 2:4] = np.asarray(m, np.uint16).reshape(-1, 1).view(np.uint8)
    blk[:, 4:] = n[:, :16] | (n[:, 16:] << 4)
    return blk.tobytes()


def pack_q8_0(d, q):
    """block_q8_0 {f16 d; i8 qs[32]}."""
    qq = np.asarray(q, np.int8).reshape(-1, 32)
    blk = np.empty((qq.shape[0], 34), np.uint8)
    blk[:, 0:2] = np.asarray(d, np.uint16).reshape(-1, 1).view(np.uint8)
    blk[:, 2:] = qq.view(np.uint8)
    return blk.tobytes()


def pack_q6_k(d, scales, L):
    """block_q6_K {u8 ql[128]; u8 qh[64]; i8 scales[16]; f16 d} of 256 values
    (value e = d * scales[e // 16] * (L[e] - 32), L in 0..63).

    Bit placement (ggml's quantize_row_q6_K packing): within each half of 128
    values, for l < 32 the values l, l+32, l+64, l+96 are a, b, c, e; ql[l]
    holds a's low 4 bits (low nibble) and c's (high nibble), ql[l+32] holds
    b's and e's, and qh[l] holds the top 2 bits of a, b, c, e at bits 0, 2,
    4, 6."""
    L = np.asarray(L, np.uint8).reshape(-1, 2, 4, 32)
    nb = L.shape[0]
    a, b, c, e = L[:, :, 0], L[:, :, 1], L[:, :, 2], L[:, :, 3]
    ql = np.empty((nb, 2, 64), np.uint8)
    ql[:, :, :32] = (a & 15) | ((c & 15) << 4)
    ql[:, :, 32:] = (b & 15) | ((e & 15) << 4)
    qh = (a >> 4) | ((b >> 4) << 2) | ((c >> 4) << 4) | ((e >> 4) << 6)
    blk = np.empty((nb, 210), np.uint8)
    blk[:, :128] = ql.reshape(nb, 128)
    blk[:, 128:192] = qh.reshape(nb, 64)
    blk[:, 192:208] = np.asarray(scales, np.int8).reshape(nb, 16).view(np.uint8)
    blk[:, 208:210] = np.asarray(d, np.uint16).reshape(-1, 1).view(np.uint8)
    return blk.tobytes()
