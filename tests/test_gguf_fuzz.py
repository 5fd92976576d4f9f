"""Mutation fuzzing of the GGUF reader under AddressSanitizer (CPU only).

tests/gguf_fuzz builds the library with the sanitizer on its host code and a
driver that mutates seed files (bit flips, byte and integer overwrites with
edge values, truncation, duplicated and deleted chunks), parses each result
with cw_gguf_parse and, when it parses, reads every metadata accessor, the
model config and every tensor through cw_gguf_tensor_f32 / cw_gguf_tensor_q4
into buffers of exactly the size cw_gguf_tensor_info reports.  A read or
write outside any buffer, a leak, or a crash fails the test; refusals are
the expected outcome for most inputs."""
import os
import shutil
import subprocess

import numpy as np
import pytest

import gguf_writer as gw
from conftest import ROOT

HERE = os.path.join(ROOT, "tests", "gguf_fuzz")
HIPCC = "/opt/rocm/bin/hipcc"


def seed_files(tmp_path):
    rng = np.random.default_rng(5)
    w = gw.GgufWriter()
    w.add_meta("general.name", "str", "t").add_meta("qwen3.block_count", "u32", 2)
    w.add_meta("k.arr", "array", ("str", ["p", "q"]))
    w.add_tensor("a", [4], gw.F32, np.arange(4, dtype=np.float32).tobytes())
    w.add_tensor("b", [32], gw.Q8_0, gw.pack_q8_0([0x3C00], np.arange(32) - 16))
    s1 = w.tobytes()
    w = gw.GgufWriter()
    for k, kind, v in [("a.u8", "u8", 3), ("a.i8", "i8", -3), ("a.u16", "u16", 7),
                       ("a.i16", "i16", -7), ("a.u32", "u32", 9), ("a.i32", "i32", -9),
                       ("a.f32", "f32", 1.5), ("a.b", "bool", 1), ("a.u64", "u64", 11),
                       ("a.i64", "i64", -11), ("a.f64", "f64", 2.5),
                       ("a.nest", "array", ("array", [("u32", [1, 2]), ("str", ["x"])]))]:
        w.add_meta(k, kind, v)
    for k, v in [("embedding_length", 64), ("attention.head_count", 4),
                 ("attention.head_count_kv", 2), ("feed_forward_length", 128),
                 ("attention.key_length", 16)]:
        w.add_meta("qwen3." + k, "u32", v)
    w.add_meta("qwen3.attention.layer_norm_rms_epsilon", "f32", 1e-6)
    w.add_meta("qwen3.rope.freq_base", "f32", 1e6)
    w.add_tensor("q", [128], gw.Q4_0,
                 gw.pack_q4_0(np.full(4, 0x3C00, np.uint16), rng.integers(0, 256, (4, 16))))
    w.add_tensor("h", [8], gw.F16, np.arange(8, dtype=np.float16).tobytes())
    w.add_tensor("q41", [32], gw.Q4_1,
                 gw.pack_q4_1([0x3C00], [0x0000], rng.integers(0, 16, (1, 32))))
    w.add_tensor("w4", [64, 2], gw.Q4_0,
                 gw.pack_q4_0(np.full(4, 0x2400, np.uint16), rng.integers(0, 256, (4, 16))))
    w.add_tensor("k6", [256], gw.Q6_K,
                 gw.pack_q6_k([0x3C00], rng.integers(-8, 8, 16), rng.integers(0, 64, 256)))
    s2 = w.tobytes()
    paths = []
    for i, b in enumerate((s1, s2)):
        p = tmp_path / f"seed{i}.gguf"
        p.write_bytes(b)
        paths.append(str(p))
    return paths


def test_gguf_reader_survives_mutations(tmp_path):
    if not os.path.exists(HIPCC) or not shutil.which("make"):
        pytest.skip("no hipcc / make for the sanitizer build")
    build = tmp_path / "build"
    r = subprocess.run(["make", "-s", "-j8", "-C", HERE, f"BUILD={build}"], capture_output=True,
                       text=True)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    seeds = seed_files(tmp_path)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0")
    for s in (1, 2, 3):
        env["FUZZ_SEED"] = str(s)
        r = subprocess.run([str(build / "fuzz_gguf"), "100000"] + seeds, capture_output=True,
                           text=True, env=env, timeout=600)
        assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
        assert "iterations 100000" in r.stdout, r.stdout
        parsed = int(r.stdout.split("parsed ")[1].split(",")[0])
        assert parsed > 1000, r.stdout  # the mutations keep many inputs parseable
