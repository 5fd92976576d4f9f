"""ctypes wrapper of oracle/liboracle.so -- the CPU restatement of the reference.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as what the device results are checked against.
The product never imports it.
"""
import ctypes as C
import os
import struct
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_P = C.c_void_p
_I = C.c_int
_SZ = C.c_size_t
_F = C.c_float

_SIGS = {
    "or_f16_to_f32": (_F, [C.c_uint16]),
    "or_f32_to_f16": (C.c_uint16, [_F]),
    "or_dequant_q4_0": (None, [_P, _SZ, _P]),
    "or_dequant_q4_0_soa": (None, [_P, _P, _SZ, _P]),
    "or_dequant_f16": (None, [_P, _SZ, _P]),
    "or_dequant_q8_0": (None, [_P, _SZ, _P]),
    "or_dequant_q4_1": (None, [_P, _SZ, _P]),
    "or_dequant_q6_k": (None, [_P, _SZ, _P]),
    "or_quantize_q4_0": (None, [_P, _SZ, _SZ, _P, _P]),
    "or_quantize_q4_0_gguf": (None, [_P, _SZ, _SZ, _P, _P]),
    "or_q4_gemv_refmt": (None, [_P, _P, _P, _I, _I, _P]),
    "or_q4_gemv": (None, [_P, _P, _P, _I, _I, _P]),
    "or_q4_gemv_f64": (None, [_P, _P, _P, _I, _I, _P, _P]),
    "or_naive_matmul": (None, [_P, _P, _I, _I, _I, _P]),
    "or_rmsnorm": (None, [_P, _P, _I, _I, _F, _P]),
    "or_rope_table": (None, [_I, _I, _F, _P, _P]),
    "or_rope": (None, [_P, _I, _I, _I, _P, _P, _P]),
    "or_rope_f32_literal": (None, [_P, _I, _I, _I, _F, _P]),
    "or_swiglu": (None, [_P, _P, _I, _P]),
    "or_add": (None, [_P, _P, _I, _P]),
    "or_argmax": (C.c_uint32, [_P, _I]),
    "or_attention": (None, [_P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "or_attention_f64": (None, [_P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "or_fnv_seed": (C.c_uint64, [C.c_char_p]),
    "or_fill": (None, [C.c_uint64, _SZ, _P]),
    "or_model_new": (_P, [_P, _F, _F]),
    "or_model_free": (None, [_P]),
    "or_model_set": (None, [_P, _I, _I, _P, _P]),
    "or_model_set_globals": (None, [_P, _P, _P, _P, _P]),
    "or_model_prefill_kv": (None, [_P, _P, _P, _I]),
    "or_model_step": (None, [_P, C.c_uint32, _I, _P, _P, _P]),
    "or_model_step_taps": (None, [_P, C.c_uint32, _I, _P, _P, _P, _P, _P]),
    "or_generate": (_I, [_P, _P, _I, _I, _I, _P, _P]),
    "or_model_kv_row": (None, [_P, _I, _I, _P, _P]),
    "or_set_threads": (None, [_I]),
    "or_get_threads": (_I, []),
}

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def set_threads(n):
    lib().or_set_threads(int(n))


def get_threads():
    return int(lib().or_get_threads())


def _p(a):
    return a.ctypes.data_as(_P)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def f16_to_f32(h):
    return lib().or_f16_to_f32(int(h))


def f32_to_f16(f):
    return lib().or_f32_to_f16(float(f))


def dequant_q4_0(blocks, n):
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.empty(n, np.float32)
    lib().or_dequant_q4_0(_p(blocks), n, _p(out))
    return out


def dequant_q4_0_soa(scales, quants):
    s = np.ascontiguousarray(scales, dtype=np.uint16).reshape(-1)
    q = np.ascontiguousarray(quants, dtype=np.uint8).reshape(-1)
    out = np.empty(s.size * 32, np.float32)
    lib().or_dequant_q4_0_soa(_p(s), _p(q), s.size, _p(out))
    return out


def _dequant(fn, raw, n):
    raw = np.ascontiguousarray(np.frombuffer(bytes(raw), np.uint8))
    out = np.empty(n, np.float32)
    getattr(lib(), fn)(_p(raw), n, _p(out))
    return out


def dequant_f16(raw, n):
    return _dequant("or_dequant_f16", raw, n)


def dequant_q8_0(raw, n):
    return _dequant("or_dequant_q8_0", raw, n)


def dequant_q4_1(raw, n):
    return _dequant("or_dequant_q4_1", raw, n)


def dequant_q6_k(raw, n):
    return _dequant("or_dequant_q6_k", raw, n)


# ------------------------------------------------------------------ GGUF container

class OracleGguf:
    """GgufWeights (src/loader/gguf.rs:30-208) restated in Python over bytes.

    parse follows gguf.rs:68-106 (magic, version u32, n_tensors u64, n_meta
    u64, metadata, tensor infos, data at the next general.alignment multiple,
    default 32); metadata values as read_meta_value (gguf.rs:125-151): integer
    kinds widened (signed ones sign-extended to 64 bits), f32/f64 as float,
    strings kept, arrays skipped (the element skip of gguf.rs:153-162).  A
    Python exception (struct.error, IndexError) stands for the reference's
    panic on a truncated file."""

    _SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B",
               10: "<Q", 11: "<q", 12: "<d"}

    def __init__(self, data):
        b = bytes(data)
        self.p = 0
        self.b = b
        if self._take(4) != b"GGUF":
            raise ValueError("not a GGUF file")
        self.version = self._u("<I")
        n_tensors = self._u("<Q")
        n_meta = self._u("<Q")
        self.meta = {}
        for _ in range(n_meta):
            key = self._str()
            self.meta[key] = self._value()
        self.tensors = {}
        for _ in range(n_tensors):
            name = self._str()
            n_dims = self._u("<I")
            dims = [self._u("<Q") for _ in range(n_dims)]
            dtype = self._u("<I")
            offset = self._u("<Q")
            n = 1
            for d in dims:
                n *= d
            self.tensors[name] = (dtype, dims, n, offset)
        align = self.meta.get(b"general.alignment", ("other", None))
        align = align[1] if align[0] == "u" else 32
        self.data_start = -(-self.p // align) * align
        if self.data_start > len(b):   # bytes[data_start..] panics in the reference
            raise IndexError("data section starts past the end")
        self.data = b[self.data_start:]

    def _take(self, n):
        if n > len(self.b) - self.p:
            raise struct.error("truncated")
        out = self.b[self.p:self.p + n]
        self.p += n
        return out

    def _u(self, fmt):
        return struct.unpack(fmt, self._take(struct.calcsize(fmt)))[0]

    def _str(self):
        return self._take(self._u("<Q"))

    def _skip(self, t):
        if t == 8:
            self._str()
        elif t in self._SCALAR:
            self._take(struct.calcsize(self._SCALAR[t]))

    def _value(self):
        t = self._u("<I")
        if t in (6, 12):
            return ("f", float(self._u(self._SCALAR[t])))
        if t in self._SCALAR:
            return ("u", self._u(self._SCALAR[t]) & 0xFFFFFFFFFFFFFFFF)
        if t == 8:
            return ("s", self._str())
        if t == 9:
            et = self._u("<I")
            for _ in range(self._u("<Q")):
                self._skip(et)
        return ("other", None)

    def meta_u32(self, key):
        """gguf.rs:165-179 (f64 -> u32 saturating like Rust `as`)."""
        kind, v = self.meta.get(key.encode() if isinstance(key, str) else key, ("other", None))
        if kind == "u":
            return v & 0xFFFFFFFF
        if kind == "f":
            return 0 if not v > 0 else min(int(v), 0xFFFFFFFF)
        if key.endswith("vocab_size") and b"token_embd.weight" in self.tensors:
            return max(self.tensors[b"token_embd.weight"][1] or [0])
        return 0

    def meta_f32(self, key):
        """gguf.rs:180-186."""
        kind, v = self.meta.get(key.encode(), ("other", None))
        return float(np.float32(v)) if kind in ("u", "f") else 0.0

    def has(self, name):
        return name.encode() in self.tensors

    def tensor_raw(self, name):
        dtype, dims, n, off = self.tensors[name.encode()]
        size = {0: 4 * n, 1: 2 * n, 2: n // 32 * 18, 3: n // 32 * 20, 8: n // 32 * 34,
                14: n // 256 * 210}[dtype]
        if off + size > len(self.data):   # the reference's slice panics
            raise IndexError(f"tensor {name} runs past the data section")
        return dtype, dims, n, self.data[off:off + size]

    def tensor_f32(self, name):
        """tensor_f32 (gguf.rs:109-122)."""
        dtype, dims, n, raw = self.tensor_raw(name)
        if dtype == 0:
            return np.frombuffer(raw, np.float32).copy()
        if dtype == 2:
            return dequant_q4_0(np.frombuffer(raw, np.uint8), n)
        fn = {1: dequant_f16, 3: dequant_q4_1, 8: dequant_q8_0, 14: dequant_q6_k}.get(dtype)
        if fn is None:
            raise ValueError(f"tensor {name}: ggml dtype {dtype} not supported yet")
        return fn(raw, n)


def quantize_q4_0(data):
    """q4.rs:37-61: (f32 scales [out, in/32], u32 quants [out, in/8])."""
    data = _f32(data)
    out_f, in_f = data.shape
    s = np.empty((out_f, in_f // 32), np.float32)
    q = np.empty((out_f, in_f // 8), np.uint32)
    lib().or_quantize_q4_0(_p(data), out_f, in_f, _p(s), _p(q))
    return s, q


def quantize_q4_0_gguf(data):
    data = _f32(data)
    out_f, in_f = data.shape
    s = np.empty((out_f, in_f // 32), np.uint16)
    q = np.empty((out_f, in_f // 32, 16), np.uint8)
    lib().or_quantize_q4_0_gguf(_p(data), out_f, in_f, _p(s), _p(q))
    return s, q


def q4_gemv_refmt(x, scales, quants, in_f, out_f):
    x = _f32(x)
    scales = _f32(scales)
    quants = np.ascontiguousarray(quants, dtype=np.uint32)
    y = np.empty(out_f, np.float32)
    lib().or_q4_gemv_refmt(_p(x), _p(scales), _p(quants), in_f, out_f, _p(y))
    return y


def q4_gemv(x, scales, quants, in_f, out_f):
    x = _f32(x)
    s = np.ascontiguousarray(scales, dtype=np.uint16)
    q = np.ascontiguousarray(quants, dtype=np.uint8)
    y = np.empty(out_f, np.float32)
    lib().or_q4_gemv(_p(x), _p(s), _p(q), in_f, out_f, _p(y))
    return y


def q4_gemv_f64(x, scales, quants, in_f, out_f):
    x = _f32(x)
    s = np.ascontiguousarray(scales, dtype=np.uint16)
    q = np.ascontiguousarray(quants, dtype=np.uint8)
    y = np.empty(out_f, np.float64)
    a = np.empty(out_f, np.float64)
    lib().or_q4_gemv_f64(_p(x), _p(s), _p(q), in_f, out_f, _p(y), _p(a))
    return y, a


def naive_matmul(a, b, m, k, n):
    a, b = _f32(a), _f32(b)
    c = np.empty(m * n, np.float32)
    lib().or_naive_matmul(_p(a), _p(b), m, k, n, _p(c))
    return c


def rmsnorm(x, w, rows, dim, eps):
    x, w = _f32(x), _f32(w)
    y = np.empty(rows * dim, np.float32)
    lib().or_rmsnorm(_p(x), _p(w), rows, dim, eps, _p(y))
    return y


def rope_table(max_pos, head_dim, theta):
    c = np.empty((max_pos, head_dim // 2), np.float32)
    s = np.empty((max_pos, head_dim // 2), np.float32)
    lib().or_rope_table(max_pos, head_dim, theta, _p(c), _p(s))
    return c, s


def rope(x, rows, head_dim, pos, theta):
    c, s = rope_table(pos + 1, head_dim, theta)
    x = _f32(x)
    y = np.empty(rows * head_dim, np.float32)
    lib().or_rope(_p(x), rows, head_dim, pos, _p(c), _p(s), _p(y))
    return y


def rope_f32_literal(x, rows, head_dim, pos, theta):
    x = _f32(x)
    y = np.empty(rows * head_dim, np.float32)
    lib().or_rope_f32_literal(_p(x), rows, head_dim, pos, theta, _p(y))
    return y


def swiglu(g, u):
    g, u = _f32(g), _f32(u)
    o = np.empty(g.size, np.float32)
    lib().or_swiglu(_p(g), _p(u), g.size, _p(o))
    return o


def add(a, b):
    a, b = _f32(a), _f32(b)
    c = np.empty(a.size, np.float32)
    lib().or_add(_p(a), _p(b), a.size, _p(c))
    return c


def argmax(x):
    x = _f32(x)
    return int(lib().or_argmax(_p(x), x.size))


def attention(q, k, v, kv_f16, n_heads, n_kv, seq, hd):
    q = _f32(q)
    dt = np.uint16 if kv_f16 else np.float32
    k = np.ascontiguousarray(k, dtype=dt)
    v = np.ascontiguousarray(v, dtype=dt)
    o = np.empty(n_heads * hd, np.float32)
    lib().or_attention(_p(q), _p(k), _p(v), int(kv_f16), n_heads, n_kv, seq, hd, _p(o))
    return o


def attention_f64(q, k, v, kv_f16, n_heads, n_kv, seq, hd):
    q = _f32(q)
    dt = np.uint16 if kv_f16 else np.float32
    k = np.ascontiguousarray(k, dtype=dt)
    v = np.ascontiguousarray(v, dtype=dt)
    o = np.empty(n_heads * hd, np.float64)
    lib().or_attention_f64(_p(q), _p(k), _p(v), int(kv_f16), n_heads, n_kv, seq, hd, _p(o))
    return o


def fnv_seed(name):
    return int(lib().or_fnv_seed(name.encode()))


def fill(seed, n):
    out = np.empty(n, np.float32)
    lib().or_fill(seed, n, _p(out))
    return out


LAYER_IDS = {"attn_norm": 0, "attn_q_norm": 1, "attn_k_norm": 2, "ffn_norm": 3,
             "attn_q": 4, "attn_k": 5, "attn_v": 6, "attn_output": 7,
             "ffn_gate": 8, "ffn_up": 9, "ffn_down": 10}


class OracleModel:
    """Qwen3 forward + generate on the CPU (qwen3.rs:139-191, mod.rs:57-125).

    `weights` maps GGUF names to f32 vectors or (scales u16, quants u8) tuples,
    as produced for the device model; the arrays are borrowed (kept alive here).
    """

    def __init__(self, cfg, weights, lm_head=None):
        self.cfg = cfg
        spec = np.array([cfg.n_layers, cfg.dim, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim,
                         cfg.hidden, cfg.vocab, cfg.max_seq, int(cfg.kv_dtype == 1)], np.int32)
        self.h = lib().or_model_new(_p(spec), cfg.eps, cfg.rope_theta)
        self._keep = []
        for name, val in weights.items():
            if not name.startswith("blk."):
                continue
            _, li, t, _w = name.split(".")
            tid = LAYER_IDS[t]
            if isinstance(val, tuple):
                s = np.ascontiguousarray(val[0], dtype=np.uint16)
                q = np.ascontiguousarray(val[1], dtype=np.uint8)
                self._keep += [s, q]
                lib().or_model_set(self.h, int(li), tid, _p(s), _p(q))
            else:
                a = _f32(val)
                self._keep.append(a)
                lib().or_model_set(self.h, int(li), tid, _p(a), None)
        emb = _f32(weights["token_embd.weight"])
        fin = _f32(weights["output_norm.weight"])
        if lm_head is None:
            lm_head = weights.get("output.weight")
        if lm_head is None:  # tied head (qwen3.rs:93-98)
            lm_head = quantize_q4_0_gguf(emb.reshape(cfg.vocab, cfg.dim))
        ls = np.ascontiguousarray(lm_head[0], dtype=np.uint16)
        lq = np.ascontiguousarray(lm_head[1], dtype=np.uint8)
        self._keep += [emb, fin, ls, lq]
        self.lm_head = (ls, lq)
        lib().or_model_set_globals(self.h, _p(emb), _p(fin), _p(ls), _p(lq))

    def close(self):
        if self.h:
            lib().or_model_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def prefill_kv(self, k, v, n_pos):
        k = np.ascontiguousarray(k)
        v = np.ascontiguousarray(v)
        lib().or_model_prefill_kv(self.h, _p(k), _p(v), n_pos)

    def kv_row(self, layer, pos):
        """Row `pos` of layer `layer`'s K and V caches as f32 arrays [kv_dim]."""
        kvd = self.cfg.n_kv_heads * self.cfg.head_dim
        k = np.empty(kvd, np.float32)
        v = np.empty(kvd, np.float32)
        lib().or_model_kv_row(self.h, int(layer), int(pos), _p(k), _p(v))
        return k, v

    def step(self, token, pos, want_layers=False):
        logits = np.empty(self.cfg.vocab, np.float32)
        hidden = np.empty(self.cfg.dim, np.float32)
        layers = np.empty((self.cfg.n_layers, self.cfg.dim), np.float32) if want_layers else None
        lib().or_model_step(self.h, int(token), int(pos), _p(logits), _p(hidden),
                            _p(layers) if want_layers else None)
        return (logits, hidden, layers) if want_layers else (logits, hidden)

    def step_taps(self, token, pos):
        """One token with the forward's hook taps (qwen3.rs:165,180,188):
        (logits, {"q": [L][n_heads*hd], "post_attn": [L][dim],
        "layer_out": [L][dim]})."""
        c = self.cfg
        logits = np.empty(c.vocab, np.float32)
        taps = {"q": np.empty((c.n_layers, c.n_heads * c.head_dim), np.float32),
                "post_attn": np.empty((c.n_layers, c.dim), np.float32),
                "layer_out": np.empty((c.n_layers, c.dim), np.float32)}
        lib().or_model_step_taps(self.h, int(token), int(pos), _p(logits), None, _p(taps["q"]),
                                 _p(taps["post_attn"]), _p(taps["layer_out"]))
        return logits, taps

    def generate(self, prompt, max_new, start_pos=0):
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.empty(max_new, np.uint32)
        margins = np.empty(max_new, np.float32)
        n = lib().or_generate(self.h, _p(prompt), len(prompt), max_new, start_pos, _p(out),
                              _p(margins))
        return out[:n], margins[:n]
