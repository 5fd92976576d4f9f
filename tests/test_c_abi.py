"""The C ABI from a C consumer: tests/c_abi/generate_demo.c includes
include/chat_wgpu.h alone, builds as strict C99 and links against the
product library, the way a cgo or Rust FFI binding would.  On the CPU it must
build and fail cleanly without a device; on the GPU its GEMV and its greedy
ids must match the oracle, and misuse must come back as CW_ERR_ARG codes."""
import os
import shutil
import subprocess

import numpy as np
import pytest

import cw
import oracle as orc
from conftest import ROOT

SRC = os.path.join(ROOT, "tests", "c_abi", "generate_demo.c")
LIBDIR = os.path.join(ROOT, "chat-wgpu_amd")
SEED = 11
PROMPT = [3, 141, 59, 265, 358, 979]
N_NEW = 10


def build(tmp_path):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not on PATH")
    exe = str(tmp_path / "generate_demo")
    cmd = [gcc, "-std=c99", "-Wall", "-Wextra", "-Werror", "-pedantic",
           "-I", os.path.join(ROOT, "include"), SRC, "-L", LIBDIR, "-lchatwgpu",
           "-Wl,-rpath," + LIBDIR, "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return exe


def run(exe, mode):
    args = [exe, str(SEED), str(mode), str(N_NEW)] + [str(t) for t in PROMPT]
    return subprocess.run(args, capture_output=True, text=True, timeout=300)


def demo_config():
    # the configuration generate_demo.c builds
    return cw.make_config(2, 256, 4, 2, 64, 512, 1000, 64, cw.CW_F32, 1e-6, 1e6)


def demo_gemv_inputs():
    """generate_demo.c's run_gemv inputs: an LCG (x then the quant bytes),
    every block scale the f16 1/64."""
    s = 12345

    def nxt():
        nonlocal s
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        return s >> 24
    x = np.array([(nxt() - 128) / 128.0 for _ in range(256)], np.float32)
    q = np.array([nxt() for _ in range(64 * 256 // 32 * 16)], np.uint8)
    sc = np.full(64 * 256 // 32, 0x2400, np.uint16)
    return x, sc, q


def test_c_program_builds_and_fails_cleanly_without_a_device(tmp_path):
    exe = build(tmp_path)
    r = run(exe, cw.STEP_GRAPH)
    if r.returncode == 0:  # a device is present: the GPU test checks the output
        return
    assert r.returncode == 2, (r.returncode, r.stderr)
    assert "cw_ctx_create" in r.stderr and "HIP error" in r.stderr, r.stderr


@pytest.mark.gpu
@pytest.mark.parametrize("mode", [cw.STEP_GRAPH, cw.STEP_EAGER])
def test_c_program_matches_the_oracle(tmp_path, mode):
    exe = build(tmp_path)
    print(f"\n[c-abi] generate_demo mode {mode}", flush=True)
    r = run(exe, mode)
    assert r.returncode == 0, r.stderr
    lines = dict(line.split(" ", 1) for line in r.stdout.splitlines() if " " in line)
    # the GEMV, through cw_alloc / cw_upload / cw_q4_gemv / cw_download
    x, sc, q = demo_gemv_inputs()
    y = orc.q4_gemv(x, sc, q, 256, 64)
    w = np.arange(1, 65, dtype=np.float64)
    ref = float(np.dot(y.astype(np.float64), w))
    got = float(lines["gemv"])
    assert abs(got - ref) <= 1e-4 * float(np.dot(np.abs(y).astype(np.float64), w)), (got, ref)
    # greedy ids, through cw_model_* and cw_generate
    cfg = demo_config()
    o = orc.OracleModel(cfg, cw.synthetic_weights(cfg, SEED))
    ids, _ = o.generate(np.array(PROMPT, np.uint32), N_NEW)
    o.close()
    got_ids = [int(t) for t in lines["ids"].split()]
    assert got_ids == [int(t) for t in ids], (got_ids, list(ids))
    # misuse: codes and messages, nothing launched
    refused = [line for line in r.stdout.splitlines() if line.startswith("refused ")]
    assert len(refused) == 2, r.stdout
    assert "positions [0, 69) exceed max_seq 64" in refused[0], refused[0]
    assert "cw_q4_gemv: null argument" in refused[1], refused[1]
