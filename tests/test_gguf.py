"""GGUF container reading and the ggml dtype decoders (src/loader/gguf.rs,
src/loader/dequant.rs), host side, CPU only.

Each check runs the product's reader (cw.Gguf over libchatwgpu's C ABI, no
GPU call) and, where the reference defines the behaviour, the oracle's
restatement (oracle.OracleGguf) on the same bytes:
  * the reference's own known answers: parse_minimal_gguf (gguf.rs:219-251),
    q8_0_block, q4_1_block, q6_k_zero_quants, q4_0_block, f16_roundtrip_known
    (dequant.rs:137-200), from tests/golden/reference_kats.json;
  * bit-exact agreement of every decoded value, f16 over all 65,536 patterns;
  * Q6_K against a packer written from ggml's block layout (a wrong bit
    position, scale index or bias fails it);
  * the error paths: bad magic, every truncation of a file, data past the end,
    unknown dtype, missing tensor, shape mismatch.
Files are built in the test by tests/gguf_writer.py.
"""
import json
import os

import numpy as np
import pytest

import cw
import oracle as orc
from conftest import GOLDEN
import gguf_writer as gw

with open(os.path.join(GOLDEN, "reference_kats.json")) as f:
    KATS = json.load(f)


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def both(data):
    return cw.Gguf(data=data), orc.OracleGguf(data)


# ---------------------------------------------------------------- the reference's KATs

def minimal_gguf():
    k = KATS["parse_minimal_gguf"]
    w = gw.GgufWriter(alignment=k["alignment"], version=k["version"])
    for key, (kind, v) in k["meta"].items():
        w.add_meta(key, kind, v)
    t = k["tensor"]
    w.add_tensor(t["name"], t["dims"], t["dtype"], np.array(t["data"], np.float32).tobytes())
    return w.tobytes()


def test_parse_minimal_gguf_kat():
    """gguf.rs:219-251: block_count 28, output_norm.weight = [1, 2, 3, 4]."""
    data = minimal_gguf()
    g, o = both(data)
    assert g.meta_u32("qwen3.block_count") == 28 == o.meta_u32("qwen3.block_count")
    assert g.tensor_f32("output_norm.weight").tolist() == [1.0, 2.0, 3.0, 4.0]
    assert o.tensor_f32("output_norm.weight").tolist() == [1.0, 2.0, 3.0, 4.0]
    assert g.has("output_norm.weight") and o.has("output_norm.weight")
    assert not g.has("output.weight") and not o.has("output.weight")
    info = g.info()
    assert info["version"] == 3 and info["n_tensors"] == 1 and info["n_meta"] == 1
    assert info["data_offset"] == o.data_start and info["data_offset"] % 32 == 0
    assert g.names() == ["output_norm.weight"]
    assert g.tensor_info("output_norm.weight") == {"dtype": 0, "dims": [4], "n_elems": 4,
                                                   "offset": 0}
    g.close()


def one_tensor(dtype, n, raw, dims=None):
    return gw.GgufWriter().add_tensor("t", dims or [n], dtype, raw).tobytes()


def decode_both(dtype, n, raw):
    g, o = both(one_tensor(dtype, n, raw))
    a, b = g.tensor_f32("t"), o.tensor_f32("t")
    g.close()
    return a, b


def test_dequant_kats():
    k = KATS["q8_0_block"]   # dequant.rs:150-161
    raw = np.array([k["d"]], np.uint16).tobytes() + bytes(range(32))
    for v in decode_both(gw.Q8_0, 32, raw):
        for i, e in k["expect"].items():
            assert v[int(i)] == e
    k = KATS["q4_1_block"]   # dequant.rs:163-173
    raw = np.array([k["d"], k["m"]], np.uint16).tobytes() + bytes([k["byte"]] * 16)
    for v in decode_both(gw.Q4_1, 32, raw):
        for i, e in k["expect"].items():
            assert v[int(i)] == e
    k = KATS["q6_k_zero_quants"]   # dequant.rs:175-188
    raw = bytearray(k["block_bytes"])
    raw[k["scales_at"][0]:k["scales_at"][1]] = bytes([k["scale"]] * 16)
    raw[k["d_at"]:k["d_at"] + 2] = np.array([k["d"]], np.uint16).tobytes()
    for v in decode_both(gw.Q6_K, 256, bytes(raw)):
        for i, e in k["expect"].items():
            assert v[int(i)] == e
        assert np.all(v == -32.0)
    k = KATS["q4_0_block"]   # dequant.rs:190-200
    raw = np.array([k["d"]], np.uint16).tobytes() + bytes([k["byte"]] * 16)
    for v in decode_both(gw.Q4_0, 32, raw):
        for i, e in k["expect"].items():
            assert v[int(i)] == e
    for h, e in KATS["f16_to_f32"]["cases"]:   # dequant.rs:137-142
        for v in decode_both(gw.F16, 1, np.array([h], np.uint16).tobytes()):
            assert v[0] == e


# ---------------------------------------------------------------- whole-dtype agreement

def test_f16_tensor_all_patterns():
    pats = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    a, b = decode_both(gw.F16, pats.size, pats.tobytes())
    assert np.array_equal(bits(a), bits(b))
    ref = pats.view(np.float16).astype(np.float32)
    ok = ~np.isnan(ref)
    assert np.array_equal(bits(a[ok]), bits(ref[ok]))
    # dequant.rs:16-19: NaN -> f32::NAN, sign applied by negation
    assert np.array_equal(bits(a[~ok]), ((pats[~ok] >> 15).astype(np.uint32) << 31) | 0x7FC00000)


def test_q6_k_against_layout_packer(rng):
    nb = 37
    L = rng.integers(0, 64, size=(nb, 256)).astype(np.uint8)
    sc = rng.integers(-128, 128, size=(nb, 16)).astype(np.int8)
    d = np.abs(rng.normal(0, 0.01, size=nb)).astype(np.float16).view(np.uint16)
    raw = gw.pack_q6_k(d, sc, L)
    a, b = decode_both(gw.Q6_K, nb * 256, raw)
    e = np.arange(256)
    df = d.view(np.float16).astype(np.float32)[:, None]
    expect = (df * sc[:, e // 16].astype(np.float32)) * (L.astype(np.float32) - 32.0)
    assert np.array_equal(bits(a), bits(expect.reshape(-1)))
    assert np.array_equal(bits(b), bits(expect.reshape(-1)))


def test_q8_0_and_q4_1_random_and_closed_forms(rng):
    nb = 300
    d = rng.normal(0, 0.05, size=nb).astype(np.float16).view(np.uint16)
    q = rng.integers(-128, 128, size=(nb, 32)).astype(np.int8)
    a, b = decode_both(gw.Q8_0, nb * 32, gw.pack_q8_0(d, q))
    assert np.array_equal(bits(a), bits(b))
    one = np.full(nb, 0x3C00, np.uint16)
    a, _ = decode_both(gw.Q8_0, nb * 32, gw.pack_q8_0(one, q))
    assert np.array_equal(a, q.reshape(-1).astype(np.float32))

    m = rng.normal(0, 0.05, size=nb).astype(np.float16).view(np.uint16)
    nib = rng.integers(0, 16, size=(nb, 32)).astype(np.uint8)
    a, b = decode_both(gw.Q4_1, nb * 32, gw.pack_q4_1(d, m, nib))
    assert np.array_equal(bits(a), bits(b))
    a, _ = decode_both(gw.Q4_1, nb * 32, gw.pack_q4_1(one, np.zeros(nb, np.uint16), nib))
    assert np.array_equal(a, nib.reshape(-1).astype(np.float32))


def test_q4_0_tensor_decode_and_split(rng):
    out_f, in_f = 24, 96
    s, q = cw.synth_q4(cw.synth_key(5, "w"), out_f, in_f, 0.02)
    raw = gw.pack_q4_0(s, q)
    data = gw.GgufWriter().add_tensor("w", [in_f, out_f], gw.Q4_0, raw).tobytes()
    g, o = both(data)
    f = g.tensor_f32("w")
    assert np.array_equal(bits(f), bits(o.tensor_f32("w")))
    # the direct repack keeps the file's bytes, so it decodes to the same values
    s2, q2 = g.tensor_q4("w", out_f, in_f)
    assert np.array_equal(s2, s) and np.array_equal(q2, q)
    assert np.array_equal(bits(orc.dequant_q4_0_soa(s2, q2)), bits(f))
    g.close()


@pytest.mark.parametrize("dtype", [gw.F32, gw.F16, gw.Q8_0, gw.Q6_K])
def test_tensor_q4_requantizes_other_dtypes(rng, dtype):
    """A projection stored as another dtype goes through decode + quantize_q4_0
    (Proj::load, layers.rs:103-116), with the f16 scale of the split image."""
    out_f, in_f = 16, 256
    n = out_f * in_f
    vals = rng.normal(0, 0.05, size=n).astype(np.float32)
    if dtype == gw.F32:
        raw = vals.tobytes()
    elif dtype == gw.F16:
        raw = vals.astype(np.float16).tobytes()
    elif dtype == gw.Q8_0:
        raw = gw.pack_q8_0(np.full(n // 32, 0x2000, np.uint16),
                           rng.integers(-128, 128, size=n).astype(np.int8))
    else:
        raw = gw.pack_q6_k(np.full(n // 256, 0x2000, np.uint16),
                           rng.integers(-128, 128, size=(n // 256, 16)).astype(np.int8),
                           rng.integers(0, 64, size=n).astype(np.uint8))
    data = gw.GgufWriter().add_tensor("w", [in_f, out_f], dtype, raw).tobytes()
    g, o = both(data)
    s, q = g.tensor_q4("w", out_f, in_f)
    f = o.tensor_f32("w").reshape(out_f, in_f)
    s_ref, q_ref = orc.quantize_q4_0_gguf(f)
    assert np.array_equal(s, s_ref) and np.array_equal(q, q_ref)
    g.close()


# ---------------------------------------------------------------- metadata

def meta_file():
    w = gw.GgufWriter()
    w.add_meta("k.u8", "u8", 200).add_meta("k.i8", "i8", -1).add_meta("k.u16", "u16", 60000)
    w.add_meta("k.i16", "i16", -300).add_meta("k.u32", "u32", 4000000000)
    w.add_meta("k.i32", "i32", -5).add_meta("k.f32", "f32", 2.75).add_meta("k.bool", "bool", 1)
    w.add_meta("k.str", "str", "qwen3").add_meta("k.u64", "u64", (1 << 40) + 7)
    w.add_meta("k.i64", "i64", -(1 << 33)).add_meta("k.f64", "f64", 1e-6)
    w.add_meta("k.f64big", "f64", 1e12).add_meta("k.f64neg", "f64", -3.5)
    w.add_meta("k.arr_u8", "array", ("u8", [1, 2, 3]))
    w.add_meta("k.arr_str", "array", ("str", ["a", "bc", ""]))
    w.add_meta("k.arr_f32", "array", ("f32", [0.5] * 1000))
    w.add_meta("k.u32", "u32", 7)   # a repeated key keeps the last value
    w.add_tensor("x", [2], gw.F32, np.array([5.0, -6.0], np.float32).tobytes())
    return w.tobytes()


def test_metadata_kinds_and_conversions():
    g, o = both(meta_file())
    expect_u32 = {"k.u8": 200, "k.i8": 0xFFFFFFFF, "k.u16": 60000, "k.i16": (-300) & 0xFFFFFFFF,
                  "k.u32": 7, "k.i32": (-5) & 0xFFFFFFFF, "k.f32": 2, "k.bool": 1,
                  "k.str": 0, "k.u64": 7, "k.i64": 0, "k.f64": 0, "k.f64big": 0xFFFFFFFF,
                  "k.f64neg": 0, "k.arr_u8": 0, "k.missing": 0}
    for key, v in expect_u32.items():
        assert g.meta_u32(key) == v == o.meta_u32(key), key
    for key in ("k.u8", "k.i8", "k.u16", "k.i16", "k.u32", "k.i32", "k.f32", "k.u64", "k.i64",
                "k.f64", "k.f64big", "k.f64neg", "k.str", "k.arr_str", "k.missing"):
        assert np.float32(g.meta_f32(key)) == np.float32(o.meta_f32(key)), key
    assert g.meta_f32("k.f64") == np.float32(1e-6)
    assert g.meta_f32("k.i8") == np.float32(2.0 ** 64)   # u64 0xFF..FF as f32
    assert g.meta_str("k.str") == b"qwen3"
    with pytest.raises(cw.CwError):
        g.meta_str("k.u32")
    assert g.tensor_f32("x").tolist() == [5.0, -6.0] == o.tensor_f32("x").tolist()
    assert g.info()["n_meta"] == 17
    g.close()


def test_nested_arrays_are_skipped():
    """Arrays of arrays are walked per the GGUF format (the reference's
    skip_scalar leaves their bytes unread, gguf.rs:153-162; real files carry
    none), so the tensor table after them still parses."""
    w = gw.GgufWriter()
    w.add_meta("k.nest", "array", ("array", [("u16", [1, 2]), ("str", ["x", "yz"])]))
    w.add_meta("k.after", "u32", 11)
    w.add_tensor("x", [1], gw.F32, np.array([3.0], np.float32).tobytes())
    g = cw.Gguf(data=w.tobytes())
    assert g.meta_u32("k.after") == 11 and g.tensor_f32("x").tolist() == [3.0]
    g.close()


def test_alignment_and_vocab_fallback():
    for align in (32, 64, 256):
        w = gw.GgufWriter(alignment=align)
        if align != 32:
            w.add_meta("general.alignment", "u32", align)
        emb = np.arange(8 * 50, dtype=np.float32)
        w.add_tensor("a", [3], gw.F32, np.ones(3, np.float32).tobytes())
        w.add_tensor("token_embd.weight", [8, 50], gw.F32, emb.tobytes())
        g, o = both(w.tobytes())
        assert g.info()["data_offset"] % align == 0
        assert g.info()["data_offset"] == o.data_start
        assert np.array_equal(g.tensor_f32("token_embd.weight"), emb)
        assert g.tensor_info("token_embd.weight")["offset"] == align
        # gguf.rs:171-177: no qwen3.vocab_size -> the embedding's largest dim
        assert g.meta_u32("qwen3.vocab_size") == 50 == o.meta_u32("qwen3.vocab_size")
        assert g.meta_u32("qwen3.block_count") == 0
        g.close()


# ---------------------------------------------------------------- errors

def test_not_a_gguf():
    for data in (b"", b"GGU", b"GGML" + bytes(40)):
        with pytest.raises(cw.CwError) as e:
            cw.Gguf(data=data)
        assert e.value.rc == -5 and "not a GGUF file" in str(e.value)
        with pytest.raises(ValueError if data[:4] == b"GGML" else Exception):
            orc.OracleGguf(data)


def test_every_truncation_is_an_error_not_a_crash():
    """Cut a two-tensor file at every length: the header parses exactly when
    the oracle's does, and a tensor whose bytes are cut reads as an error."""
    w = gw.GgufWriter()
    w.add_meta("general.name", "str", "t").add_meta("qwen3.block_count", "u32", 2)
    w.add_meta("k.arr", "array", ("str", ["p", "q"]))
    w.add_tensor("a", [4], gw.F32, np.arange(4, dtype=np.float32).tobytes())
    w.add_tensor("b", [32], gw.Q8_0, gw.pack_q8_0([0x3C00], np.arange(32) - 16))
    full = w.tobytes()
    for n in range(len(full)):
        cut = full[:n]
        try:
            o = orc.OracleGguf(cut)
            o_ok = True
        except Exception:
            o_ok = False
        try:
            g = cw.Gguf(data=cut)
        except cw.CwError as e:
            assert e.rc == -5, (n, e)
            assert not o_ok, n
            continue
        assert o_ok, n
        for name in ("a", "b"):
            try:
                v = g.tensor_f32(name)
            except cw.CwError as e:
                assert "run past the data section" in str(e), (n, name, e)
                v = None
            try:
                ov = o.tensor_f32(name)
            except IndexError:
                ov = None
            assert (v is None) == (ov is None), (n, name)
            if v is not None:
                assert np.array_equal(bits(v), bits(ov)), (n, name)
        g.close()


def test_tensor_errors():
    w = gw.GgufWriter()
    w.add_tensor("bf", [4], 30, bytes(8))   # BF16: not among tensor_f32's dtypes
    w.add_tensor("far", [4], gw.F32, bytes(16))
    w.add_tensor("odd", [40], gw.Q4_0, bytes(36))
    data = bytearray(w.tobytes())
    g = cw.Gguf(data=bytes(data))
    with pytest.raises(cw.CwError, match="tensor bf: ggml dtype 30 not supported yet"):
        g.tensor_f32("bf")
    with pytest.raises(cw.CwError, match="missing tensor nope"):
        g.tensor_f32("nope")
    with pytest.raises(cw.CwError, match="not a whole number"):
        g.tensor_f32("odd")
    with pytest.raises(cw.CwError, match="elements"):
        g.tensor_q4("far", 2, 32)
    assert g.tensor_f32("far").tolist() == [0.0] * 4
    g.close()
    # point "far" past the end of the file
    w2 = gw.GgufWriter()
    w2.add_tensor("far", [4], gw.F32, bytes(16))
    data = bytearray(w2.tobytes())
    off_at = data.index(b"far") + 3 + 4 + 8 + 4
    data[off_at:off_at + 8] = (1 << 40).to_bytes(8, "little")
    g = cw.Gguf(data=bytes(data))
    with pytest.raises(cw.CwError, match="run past the data section"):
        g.tensor_f32("far")
    g.close()
    bad_kind = (b"GGUF" + (3).to_bytes(4, "little") + (0).to_bytes(8, "little")
                + (1).to_bytes(8, "little") + gw.gstr("k") + (13).to_bytes(4, "little"))
    with pytest.raises(cw.CwError, match="bad metadata value"):   # unknown kind 13
        cw.Gguf(data=bad_kind)


@pytest.mark.parametrize("dtype,n", [(gw.F32, 1 << 62), (gw.F16, 1 << 63)])
def test_byte_count_overflow_is_rejected(dtype, n):
    """An element count whose byte size wraps 64 bits (2^62 f32 values are
    2^64 bytes, which would read as 0) is refused before the data-section
    range check, not passed by it."""
    w = gw.GgufWriter()
    w.add_tensor("huge", [n], dtype, bytes(16))
    g = cw.Gguf(data=w.tobytes())
    assert g.tensor_info("huge")["n_elems"] == n
    # straight through the C entry with a small buffer: the byte range is
    # checked before the buffer size, so nothing is written either way
    out = np.zeros(4, np.float32)
    rc = cw.lib().cw_gguf_tensor_f32(g.h, b"huge", out.ctypes.data_as(cw.C.c_void_p), 4)
    assert rc == cw.CW_ERR_FORMAT
    assert "overflow its byte count" in cw.lib().cw_last_error().decode()
    g.close()


def test_open_file_matches_parse(tmp_path):
    data = meta_file()
    p = tmp_path / "m.gguf"
    p.write_bytes(data)
    a, b = cw.Gguf(path=str(p)), cw.Gguf(data=data)
    assert a.info() == b.info()
    assert a.tensor_f32("x").tolist() == b.tensor_f32("x").tolist()
    a.close()
    b.close()
    with pytest.raises(cw.CwError) as e:
        cw.Gguf(path=str(tmp_path / "absent.gguf"))
    assert e.value.rc == -6
    (tmp_path / "empty.gguf").write_bytes(b"")
    with pytest.raises(cw.CwError) as e:
        cw.Gguf(path=str(tmp_path / "empty.gguf"))
    assert e.value.rc == -5


# ---------------------------------------------------------------- model config

def qwen3_meta(w, n_layers=2, dim=64, heads=4, kv=2, hd=16, hidden=128, vocab=None):
    w.add_meta("general.architecture", "str", "qwen3")
    w.add_meta("qwen3.block_count", "u32", n_layers)
    w.add_meta("qwen3.embedding_length", "u32", dim)
    w.add_meta("qwen3.attention.head_count", "u32", heads)
    w.add_meta("qwen3.attention.head_count_kv", "u32", kv)
    w.add_meta("qwen3.attention.key_length", "u32", hd)
    w.add_meta("qwen3.feed_forward_length", "u32", hidden)
    w.add_meta("qwen3.attention.layer_norm_rms_epsilon", "f32", 1e-6)
    w.add_meta("qwen3.rope.freq_base", "f32", 1e6)
    if vocab is not None:
        w.add_meta("qwen3.vocab_size", "u32", vocab)
    return w


def test_model_config_from_metadata():
    w = qwen3_meta(gw.GgufWriter())
    w.add_tensor("token_embd.weight", [64, 300], gw.F16, bytes(64 * 300 * 2))
    g = cw.Gguf(data=w.tobytes())
    c = g.model_config(max_seq=40, kv_dtype=cw.CW_F16)
    assert (c.n_layers, c.dim, c.n_heads, c.n_kv_heads, c.head_dim, c.hidden, c.vocab) == \
        (2, 64, 4, 2, 16, 128, 300)
    assert c.eps == np.float32(1e-6) and c.rope_theta == 1e6
    assert (c.max_seq, c.kv_dtype, c.family.qk_norm) == (40, cw.CW_F16, 1)
    g.close()
    w = gw.GgufWriter().add_meta("general.architecture", "str", "llama")
    with pytest.raises(cw.CwError, match="only qwen3"):
        cw.Gguf(data=w.tobytes()).model_config(10)
    w = qwen3_meta(gw.GgufWriter())   # no vocab_size and no embedding
    with pytest.raises(cw.CwError, match="qwen3.vocab_size"):
        cw.Gguf(data=w.tobytes()).model_config(10)
