"""ctypes binding of libchatwgpu.so (the C ABI in include/chat_wgpu.h).

This is the Python-side host of the MI355X decode path: device buffers,
kernel wrappers named after the reference's (q4::gemv -> q4_gemv,
norm::rmsnorm -> rmsnorm, ...), the Qwen3 model and its greedy loop.  It
loads the in-tree HIP library and raises if it is missing: there is no CPU
fallback.
"""
import ctypes as C
import os

import numpy as np

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libchatwgpu.so")

CW_F32 = 0
CW_F16 = 1

# status codes (include/chat_wgpu.h)
CW_OK = 0
CW_ERR_ARG = -1
CW_ERR_HIP = -2
CW_ERR_OOM = -3
CW_ERR_STATE = -4
CW_ERR_FORMAT = -5
CW_ERR_IO = -6

STEP_EAGER = 0   # one launch per op
STEP_GRAPH = 1   # the op launches of one step replayed as a HIP graph
STEP_FUSED = 2   # one persistent cooperative kernel per step

_P = C.c_void_p
_I = C.c_int
_SZ = C.c_size_t
_U32 = C.c_uint32
_U64 = C.c_uint64
_F = C.c_float


class CwError(RuntimeError):
    def __init__(self, rc, msg):
        super().__init__(f"cw error {rc}: {msg}")
        self.rc = rc


class FamilySpec(C.Structure):
    _fields_ = [("norm_unit_gain", _I), ("act", _I), ("qk_norm", _I), ("qkv_bias", _I)]


class ModelConfig(C.Structure):
    _fields_ = [("family", FamilySpec),
                ("n_layers", _I), ("dim", _I), ("n_heads", _I), ("n_kv_heads", _I),
                ("head_dim", _I), ("hidden", _I), ("vocab", _I),
                ("eps", _F), ("rope_theta", _F),
                ("max_seq", _I), ("kv_dtype", _I)]


# name -> (restype, argtypes); every declaration of include/chat_wgpu.h
_SIGS = {
    "cw_ctx_create": (_I, [_I, C.POINTER(_P)]),
    "cw_ctx_destroy": (_I, [_P]),
    "cw_last_error": (C.c_char_p, []),
    "cw_version": (C.c_char_p, []),
    "cw_device_info": (_I, [_P, C.POINTER(_I), C.POINTER(_SZ), C.c_char_p, _SZ]),
    "cw_alloc": (_I, [_P, _SZ, C.POINTER(_P)]),
    "cw_free": (_I, [_P, _P]),
    "cw_frame_alloc": (_I, [_P, _SZ, C.POINTER(_P)]),
    "cw_frame_reset": (_I, [_P]),
    "cw_upload": (_I, [_P, _P, _P, _SZ]),
    "cw_download": (_I, [_P, _P, _P, _SZ]),
    "cw_copy": (_I, [_P, _P, _P, _SZ]),
    "cw_flush": (_I, [_P]),
    "cw_graph_begin": (_I, [_P]),
    "cw_graph_end": (_I, [_P, C.POINTER(_P)]),
    "cw_graph_launch": (_I, [_P, _P]),
    "cw_graph_destroy": (_I, [_P]),
    "cw_q4_gemv": (_I, [_P, _P, _P, _P, _I, _I, _P]),
    "cw_q4_gemv_add": (_I, [_P, _P, _P, _P, _I, _I, _P, _P]),
    "cw_q4_gemv_swiglu": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _P]),
    "cw_q4_gemm": (_I, [_P, _P, _I, _P, _P, _I, _I, _P]),
    "cw_rmsnorm": (_I, [_P, _P, _P, _I, _I, _F, _P]),
    "cw_rope": (_I, [_P, _P, _I, _I, _I, _F, _P]),
    "cw_attention": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "cw_attention_noalloc": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "cw_add": (_I, [_P, _P, _P, _I, _P]),
    "cw_swiglu": (_I, [_P, _P, _P, _I, _P]),
    "cw_argmax": (_I, [_P, _P, _I, _P]),
    "cw_kv_write": (_I, [_P, _P, _P, _I, _I, _I, _P, _P]),
    "cw_embed": (_I, [_P, _P, _I, _I, _P, _P]),
    "cw_hbm_read_probe": (_I, [_P, _P, _SZ, _I, _P]),
    "cw_q4_quantize": (_I, [_P, _SZ, _SZ, _P, _P]),
    "cw_q4_split_blocks": (_I, [_P, _SZ, _P, _P]),
    "cw_synth_key": (_U64, [_U64, C.c_char_p]),
    "cw_synth_q4": (_I, [_U64, _SZ, _F, _P, _P]),
    "cw_synth_normal_f32": (_I, [_U64, _SZ, _F, _F, _P]),
    "cw_synth_normal_f16": (_I, [_U64, _SZ, _F, _F, _P]),
    "cw_synth_tokens": (_I, [_U64, _SZ, _U32, _P]),
    "cw_model_create": (_I, [_P, C.POINTER(ModelConfig), C.POINTER(_P)]),
    "cw_model_destroy": (_I, [_P]),
    "cw_model_set_q4": (_I, [_P, C.c_char_p, _P, _P]),
    "cw_model_set_f32": (_I, [_P, C.c_char_p, _P]),
    "cw_model_load_synthetic": (_I, [_P, _U64]),
    "cw_model_finalize": (_I, [_P]),
    "cw_model_prefill_kv": (_I, [_P, _P, _P, _I]),
    "cw_model_step": (_I, [_P, _U32, _I, C.POINTER(_U32)]),
    "cw_model_logits": (_I, [_P, _P]),
    "cw_model_hidden": (_I, [_P, _P]),
    "cw_model_set_taps": (_I, [_P, _I]),
    "cw_model_tap": (_I, [_P, C.c_char_p, _I, _P, _I]),
    "cw_generate": (_I, [_P, _P, _I, _I, _I, _I, _P]),
    "cw_model_decode_async": (_I, [_P, _I, _I]),
    "cw_model_decode_next": (_I, [_P, _P]),
    "cw_model_reset_state": (_I, [_P, _U32, _I]),
    "cw_model_prefill": (_I, [_P, _P, _I, _I, C.POINTER(_U32)]),
    "cw_model_tokens": (_I, [_P, _P, _I, C.POINTER(_I)]),
    "cw_model_profile_step": (_I, [_P, _P, _I, C.POINTER(_I), C.POINTER(C.c_double)]),
    "cw_step_layout_check": (_I, [C.POINTER(ModelConfig), _I, _I, C.c_char_p, _SZ]),
    "cw_step_dry_plan": (_I, [C.POINTER(ModelConfig), _I, _I, _P, _SZ, _P, _SZ, _P, _P, _I,
                              C.POINTER(_I)]),
    "cw_gguf_open": (_I, [C.c_char_p, C.POINTER(_P)]),
    "cw_gguf_parse": (_I, [_P, _SZ, C.POINTER(_P)]),
    "cw_gguf_close": (_I, [_P]),
    "cw_gguf_info": (_I, [_P, C.POINTER(_U32), C.POINTER(_U64), C.POINTER(_U64),
                          C.POINTER(_U64)]),
    "cw_gguf_meta_u32": (_I, [_P, C.c_char_p, C.POINTER(_U32)]),
    "cw_gguf_meta_f32": (_I, [_P, C.c_char_p, C.POINTER(_F)]),
    "cw_gguf_meta_str": (_I, [_P, C.c_char_p, C.c_char_p, _SZ, C.POINTER(_SZ)]),
    "cw_gguf_has": (_I, [_P, C.c_char_p]),
    "cw_gguf_tensor_name": (_I, [_P, _U64, C.c_char_p, _SZ]),
    "cw_gguf_tensor_info": (_I, [_P, C.c_char_p, C.POINTER(_U32), C.POINTER(_I),
                                 C.POINTER(_U64), _I, C.POINTER(_U64), C.POINTER(_U64)]),
    "cw_gguf_tensor_f32": (_I, [_P, C.c_char_p, _P, _SZ]),
    "cw_gguf_tensor_q4": (_I, [_P, C.c_char_p, _SZ, _SZ, _P, _P]),
    "cw_gguf_model_config": (_I, [_P, _I, _I, C.POINTER(ModelConfig)]),
    "cw_model_load_gguf": (_I, [_P, _P]),
    "cw_profile_begin": (_I, [_P]),
    "cw_profile_report": (_I, [_P, C.c_char_p, _SZ]),
}

_lib = None


def lib():
    """The loaded library (raises if the HIP build is missing)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with "
                               "`python chat-wgpu_amd/build.py` (no CPU fallback exists)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc):
    if rc != 0:
        raise CwError(rc, lib().cw_last_error().decode())
    return rc


def _ptr(a):
    return a.ctypes.data_as(_P) if isinstance(a, np.ndarray) else a


# ---------------------------------------------------------------- host-side helpers

def step_layout_check(cfg, n_cu, split_gate_up=False):
    """Host-only check of the fused decode step's buffer layout for cfg
    (cw_step_layout_check): (rc, message); rc 0 when every range the step
    touches lies inside an allocation."""
    buf = C.create_string_buffer(256)
    rc = lib().cw_step_layout_check(C.byref(cfg), int(n_cu), int(bool(split_gate_up)), buf, 256)
    return rc, buf.value.decode()


def q4_quantize(data):
    """Re-quantize f32 [out, in] to split GGUF Q4_0 (scales u16 [out, in/32], quants
    u8 [out, in/32, 16]); q4.rs:37-61 with the scale rounded to f16."""
    data = np.ascontiguousarray(data, dtype=np.float32)
    out_f, in_f = data.shape
    s = np.empty((out_f, in_f // 32), np.uint16)
    q = np.empty((out_f, in_f // 32, 16), np.uint8)
    check(lib().cw_q4_quantize(_ptr(data), out_f, in_f, _ptr(s), _ptr(q)))
    return s, q


def q4_split_blocks(blocks):
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    nb = blocks.size // 18
    s = np.empty(nb, np.uint16)
    q = np.empty((nb, 16), np.uint8)
    check(lib().cw_q4_split_blocks(_ptr(blocks), nb, _ptr(s), _ptr(q)))
    return s, q


def synth_key(seed, name):
    return lib().cw_synth_key(seed, name.encode())


def synth_q4(key, out_f, in_f, sigma=0.02):
    nb = out_f * (in_f // 32)
    s = np.empty((out_f, in_f // 32), np.uint16)
    q = np.empty((out_f, in_f // 32, 16), np.uint8)
    check(lib().cw_synth_q4(key, nb, sigma, _ptr(s), _ptr(q)))
    return s, q


def synth_normal_f32(key, n, mean=0.0, std=1.0):
    out = np.empty(n, np.float32)
    check(lib().cw_synth_normal_f32(key, n, mean, std, _ptr(out)))
    return out


def synth_normal_f16(key, n, mean=0.0, std=1.0):
    out = np.empty(n, np.uint16)
    check(lib().cw_synth_normal_f16(key, n, mean, std, _ptr(out)))
    return out


def synth_tokens(key, n, vocab):
    out = np.empty(n, np.uint32)
    check(lib().cw_synth_tokens(key, n, vocab, _ptr(out)))
    return out


# ---------------------------------------------------------------- GGUF container

GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q4_1, GGML_Q8_0, GGML_Q6_K = 0, 1, 2, 3, 8, 14


class Gguf:
    """GgufWeights (src/loader/gguf.rs): a parsed GGUF container, memory-mapped
    (`Gguf(path)`) or copied from bytes (`Gguf(data=b"...")`), with the
    Weights accessors meta_u32 / meta_f32 / has / tensor_f32 (= matrix_raw,
    vector_data) and the split Q4_0 repack tensor_q4."""

    def __init__(self, path=None, data=None):
        h = _P()
        if path is not None:
            check(lib().cw_gguf_open(os.fsencode(path), C.byref(h)))
        else:
            buf = bytes(data)
            check(lib().cw_gguf_parse(buf, len(buf), C.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            lib().cw_gguf_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def info(self):
        v, nt, nm, off = _U32(), _U64(), _U64(), _U64()
        check(lib().cw_gguf_info(self.h, C.byref(v), C.byref(nt), C.byref(nm), C.byref(off)))
        return {"version": v.value, "n_tensors": nt.value, "n_meta": nm.value,
                "data_offset": off.value}

    def meta_u32(self, key):
        r = _U32()
        check(lib().cw_gguf_meta_u32(self.h, key.encode(), C.byref(r)))
        return r.value

    def meta_f32(self, key):
        r = _F()
        check(lib().cw_gguf_meta_f32(self.h, key.encode(), C.byref(r)))
        return r.value

    def meta_str(self, key):
        n = _SZ()
        check(lib().cw_gguf_meta_str(self.h, key.encode(), None, 0, C.byref(n)))
        buf = C.create_string_buffer(n.value + 1)
        check(lib().cw_gguf_meta_str(self.h, key.encode(), buf, len(buf), None))
        return buf.raw[:n.value]

    def has(self, name):
        return bool(lib().cw_gguf_has(self.h, name.encode()))

    def names(self):
        out = []
        buf = C.create_string_buffer(4096)
        for i in range(self.info()["n_tensors"]):
            check(lib().cw_gguf_tensor_name(self.h, i, buf, len(buf)))
            out.append(buf.value.decode())
        return out

    def tensor_info(self, name):
        dt, nd, ne, off = _U32(), _I(), _U64(), _U64()
        dims = (_U64 * 16)()
        check(lib().cw_gguf_tensor_info(self.h, name.encode(), C.byref(dt), C.byref(nd), dims,
                                        16, C.byref(ne), C.byref(off)))
        return {"dtype": dt.value, "dims": list(dims[:nd.value]), "n_elems": ne.value,
                "offset": off.value}

    def tensor_f32(self, name):
        n = self.tensor_info(name)["n_elems"]
        out = np.empty(n, np.float32)
        check(lib().cw_gguf_tensor_f32(self.h, name.encode(), _ptr(out), n))
        return out

    def tensor_q4(self, name, out_f, in_f):
        s = np.empty((out_f, in_f // 32), np.uint16)
        q = np.empty((out_f, in_f // 32, 16), np.uint8)
        check(lib().cw_gguf_tensor_q4(self.h, name.encode(), out_f, in_f, _ptr(s), _ptr(q)))
        return s, q

    def model_config(self, max_seq, kv_dtype=CW_F16):
        cfg = ModelConfig()
        check(lib().cw_gguf_model_config(self.h, max_seq, kv_dtype, C.byref(cfg)))
        return cfg


# ---------------------------------------------------------------- device context

class DeviceArray:
    """A device allocation with a numpy dtype and shape."""

    def __init__(self, ctx, shape, dtype, ptr):
        self.ctx, self.shape, self.dtype, self.ptr = ctx, tuple(shape), np.dtype(dtype), ptr

    @property
    def nbytes(self):
        return int(np.prod(self.shape)) * self.dtype.itemsize

    def upload(self, a):
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes, (a.nbytes, self.nbytes)
        check(lib().cw_upload(self.ctx.h, self.ptr, _ptr(a), a.nbytes))
        return self

    def download(self):
        out = np.empty(self.shape, self.dtype)
        check(lib().cw_download(self.ctx.h, _ptr(out), self.ptr, out.nbytes))
        return out


class Graph:
    """A recorded launch sequence of a Context (cw_graph_*)."""

    def __init__(self, ctx, h):
        self.ctx, self.h = ctx, h

    def launch(self):
        check(lib().cw_graph_launch(self.ctx.h, self.h))

    def close(self):
        if self.h:
            lib().cw_graph_destroy(self.h)
            self.h = None


class Context:
    """GpuContext (src/context.rs): one HIP stream on one device."""

    def __init__(self, device=0):
        h = _P()
        check(lib().cw_ctx_create(device, C.byref(h)))
        self.h = h
        self._arrays = []

    def close(self):
        if self.h:
            lib().cw_ctx_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def info(self):
        n_cu = _I()
        hbm = _SZ()
        arch = C.create_string_buffer(64)
        check(lib().cw_device_info(self.h, C.byref(n_cu), C.byref(hbm), arch, 64))
        return {"n_cu": n_cu.value, "hbm_bytes": hbm.value, "arch": arch.value.decode()}

    def empty(self, shape, dtype=np.float32):
        shape = (shape,) if np.isscalar(shape) else tuple(shape)
        n = max(1, int(np.prod(shape)) * np.dtype(dtype).itemsize)
        p = _P()
        check(lib().cw_alloc(self.h, n, C.byref(p)))
        return DeviceArray(self, shape, dtype, p.value)

    def storage(self, a, dtype=None):
        a = np.asarray(a, dtype=dtype)
        return self.empty(a.shape, a.dtype).upload(a)

    def free(self, d):
        check(lib().cw_free(self.h, d.ptr))

    def flush(self):
        check(lib().cw_flush(self.h))

    def profile_begin(self):
        check(lib().cw_profile_begin(self.h))

    def profile_report(self):
        buf = C.create_string_buffer(1 << 16)
        check(lib().cw_profile_report(self.h, buf, len(buf)))
        rows = []
        for line in buf.value.decode().splitlines():
            name, count, ms = line.split()
            rows.append((name, int(count), float(ms)))
        return rows

    # ---- kernel wrappers (src/kernels/*.rs); outputs are fresh device arrays
    def q4_gemv(self, x, scales, quants, in_f, out_f, y=None):
        y = y or self.empty(out_f)
        check(lib().cw_q4_gemv(self.h, x.ptr, scales.ptr, quants.ptr, in_f, out_f, y.ptr))
        return y

    def q4_gemv_add(self, x, scales, quants, in_f, out_f, residual, y=None):
        y = y or self.empty(out_f)
        check(lib().cw_q4_gemv_add(self.h, x.ptr, scales.ptr, quants.ptr, in_f, out_f,
                                   residual.ptr, y.ptr))
        return y

    def q4_gemv_swiglu(self, x, gs, gq, us, uq, in_f, out_f, y=None):
        y = y or self.empty(out_f)
        check(lib().cw_q4_gemv_swiglu(self.h, x.ptr, gs.ptr, gq.ptr, us.ptr, uq.ptr, in_f,
                                      out_f, y.ptr))
        return y

    def q4_gemm(self, x, m, scales, quants, in_f, out_f, y=None):
        y = y if y is not None else self.empty((m, out_f))
        check(lib().cw_q4_gemm(self.h, x.ptr, m, scales.ptr, quants.ptr, in_f, out_f, y.ptr))
        return y

    def rmsnorm(self, x, w, rows, dim, eps):
        y = self.empty(rows * dim)
        check(lib().cw_rmsnorm(self.h, x.ptr, w.ptr, rows, dim, eps, y.ptr))
        return y

    def rope(self, x, rows, head_dim, pos, theta):
        y = self.empty(rows * head_dim)
        check(lib().cw_rope(self.h, x.ptr, rows, head_dim, pos, theta, y.ptr))
        return y

    def attention(self, q, k, v, kv_dtype, n_heads, n_kv, seq, head_dim):
        o = self.empty(n_heads * head_dim)
        check(lib().cw_attention(self.h, q.ptr, k.ptr, v.ptr, kv_dtype, n_heads, n_kv, seq,
                                 head_dim, o.ptr))
        return o

    def add(self, a, b, n):
        c = self.empty(n)
        check(lib().cw_add(self.h, a.ptr, b.ptr, n, c.ptr))
        return c

    def swiglu(self, g, u, n):
        o = self.empty(n)
        check(lib().cw_swiglu(self.h, g.ptr, u.ptr, n, o.ptr))
        return o

    def argmax(self, logits, n):
        o = self.empty(1, np.uint32)
        check(lib().cw_argmax(self.h, logits.ptr, n, o.ptr))
        return o

    def kv_write(self, kc, vc, kv_dtype, pos, kv_dim, k, v):
        check(lib().cw_kv_write(self.h, kc.ptr, vc.ptr, kv_dtype, pos, kv_dim, k.ptr, v.ptr))

    def embed(self, table, vocab, dim, token_dev):
        o = self.empty(dim)
        check(lib().cw_embed(self.h, table.ptr, vocab, dim, token_dev.ptr, o.ptr))
        return o

    def graph_begin(self):
        """Record the following launches (cw_graph_begin)."""
        check(lib().cw_graph_begin(self.h))

    def graph_end(self):
        """Close the recording; returns a Graph to replay."""
        g = _P()
        check(lib().cw_graph_end(self.h, C.byref(g)))
        return Graph(self, g.value)

    def hbm_read_probe(self, buf, nbytes, blocks, out):
        check(lib().cw_hbm_read_probe(self.h, buf.ptr, nbytes, blocks, out.ptr))


# ---------------------------------------------------------------- model

QWEN3 = FamilySpec(0, 0, 1, 0)

LAYER_VECTORS = ("attn_norm", "attn_q_norm", "attn_k_norm", "ffn_norm")
LAYER_PROJS = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")


def make_config(n_layers, dim, n_heads, n_kv_heads, head_dim, hidden, vocab, max_seq,
                kv_dtype=CW_F32, eps=1e-6, rope_theta=1e6):
    return ModelConfig(QWEN3, n_layers, dim, n_heads, n_kv_heads, head_dim, hidden, vocab,
                       eps, rope_theta, max_seq, kv_dtype)


def proj_shape(cfg, name):
    q_dim = cfg.n_heads * cfg.head_dim
    kv_dim = cfg.n_kv_heads * cfg.head_dim
    return {"attn_q": (q_dim, cfg.dim), "attn_k": (kv_dim, cfg.dim),
            "attn_v": (kv_dim, cfg.dim), "attn_output": (cfg.dim, q_dim),
            "ffn_gate": (cfg.hidden, cfg.dim), "ffn_up": (cfg.hidden, cfg.dim),
            "ffn_down": (cfg.dim, cfg.hidden)}[name]


def synthetic_weights(cfg, seed):
    """Host copies of every tensor cw_model_load_synthetic generates (same keys,
    same generator): {name: array or (scales, quants)}."""
    w = {}
    for i in range(cfg.n_layers):
        for v in LAYER_VECTORS:
            name = f"blk.{i}.{v}.weight"
            n = cfg.head_dim if v in ("attn_q_norm", "attn_k_norm") else cfg.dim
            w[name] = synth_normal_f32(synth_key(seed, name), n, 1.0, 0.02)
        for p in LAYER_PROJS:
            name = f"blk.{i}.{p}.weight"
            out_f, in_f = proj_shape(cfg, p)
            w[name] = synth_q4(synth_key(seed, name), out_f, in_f, 0.02)
    w["output_norm.weight"] = synth_normal_f32(synth_key(seed, "output_norm.weight"), cfg.dim,
                                               1.0, 0.02)
    w["token_embd.weight"] = synth_normal_f32(synth_key(seed, "token_embd.weight"),
                                              cfg.vocab * cfg.dim, 0.0, 0.02)
    return w


class Model:
    """Qwen3 (src/model/qwen3.rs) on the device, with generate (src/model/mod.rs)."""

    def __init__(self, ctx, cfg):
        self.ctx, self.cfg = ctx, cfg
        h = _P()
        check(lib().cw_model_create(ctx.h, C.byref(cfg), C.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            lib().cw_model_destroy(self.h)
            self.h = None

    def set_weights(self, weights):
        for name, val in weights.items():
            if isinstance(val, tuple):
                s, q = (np.ascontiguousarray(a) for a in val)
                check(lib().cw_model_set_q4(self.h, name.encode(), _ptr(s), _ptr(q)))
            else:
                a = np.ascontiguousarray(val, dtype=np.float32)
                check(lib().cw_model_set_f32(self.h, name.encode(), _ptr(a)))

    def load_synthetic(self, seed):
        check(lib().cw_model_load_synthetic(self.h, seed))

    def load_gguf(self, g):
        """Every tensor of a Gguf (Qwen3::load's walk, qwen3.rs:56-100)."""
        check(lib().cw_model_load_gguf(self.h, g.h))

    def finalize(self):
        check(lib().cw_model_finalize(self.h))

    def prefill_kv(self, k, v, n_pos):
        k = np.ascontiguousarray(k)
        v = np.ascontiguousarray(v)
        check(lib().cw_model_prefill_kv(self.h, _ptr(k), _ptr(v), n_pos))

    def step(self, token, pos):
        r = _U32()
        check(lib().cw_model_step(self.h, int(token), int(pos), C.byref(r)))
        return r.value

    def logits(self):
        out = np.empty(self.cfg.vocab, np.float32)
        check(lib().cw_model_logits(self.h, _ptr(out)))
        return out

    def hidden(self):
        out = np.empty(self.cfg.dim, np.float32)
        check(lib().cw_model_hidden(self.h, _ptr(out)))
        return out

    def set_taps(self, enable=True):
        """Keep the forward's hook taps of every decode step (the reference's
        Hook / Capture, mod.rs:158-165, main.rs:193-207)."""
        check(lib().cw_model_set_taps(self.h, 1 if enable else 0))

    TAP_NAMES = ("q", "post_attn", "layer_out")

    def tap(self, name, layer):
        """The tap `name` ("q", "post_attn" or "layer_out") of `layer` from
        the last decode step."""
        n = self.cfg.n_heads * self.cfg.head_dim if name == "q" else self.cfg.dim
        out = np.empty(n, np.float32)
        check(lib().cw_model_tap(self.h, name.encode(), int(layer), _ptr(out), n))
        return out

    def generate(self, prompt, max_new, start_pos=0, mode=STEP_GRAPH):
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.empty(max_new, np.uint32)
        check(lib().cw_generate(self.h, _ptr(prompt), len(prompt), max_new, start_pos,
                                int(mode), _ptr(out)))
        return out

    def prefill(self, tokens, start_pos=0):
        """Batched prompt phase; returns the argmax of the last position."""
        tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
        nxt = _U32(0)
        check(lib().cw_model_prefill(self.h, _ptr(tokens), len(tokens), start_pos, C.byref(nxt)))
        return int(nxt.value)

    def reset_state(self, token, pos):
        check(lib().cw_model_reset_state(self.h, int(token), int(pos)))

    def decode_async(self, n_steps, mode=STEP_GRAPH):
        check(lib().cw_model_decode_async(self.h, n_steps, int(mode)))

    def decode_next(self):
        """One replayed decode step; returns its argmax (one 4-byte read)."""
        nxt = _U32(0)
        check(lib().cw_model_decode_next(self.h, C.byref(nxt)))
        return int(nxt.value)

    def profile_step(self):
        """One fused step with phase stamps, in microseconds from its start:
        (list of (barrier arrive, release) pairs, end of LM head, array
        [layer][phase][after staging, after compute]; 0 where not stamped)."""
        L = self.cfg.n_layers
        n_max = 20 * L + 8
        buf = np.zeros(n_max, np.int64)
        n = _I()
        hz = C.c_double()
        check(lib().cw_model_profile_step(self.h, _ptr(buf), n_max, C.byref(n), C.byref(hz)))
        us = np.where(buf > 0, (buf - buf[0]) / hz.value * 1e6, 0.0)
        nb = 5 * L
        pairs = [(us[2 * e], us[2 * e + 1]) for e in range(1, nb + 1)]
        sub = us[10 * L + 4:10 * L + 4 + 10 * L].reshape(L, 5, 2)
        return pairs, us[10 * L + 2], sub

    def tokens(self, max_n):
        out = np.empty(max_n, np.uint32)
        n = _I()
        check(lib().cw_model_tokens(self.h, _ptr(out), max_n, C.byref(n)))
        return out[:n.value]
