"""CPU execution of the fused decode-step kernel (decode_step.hip) under
AddressSanitizer (tests/step_emu): every thread of the grid runs as a fiber,
the buffers are the library's own plan (cw_step_dry_plan) with one host
allocation of exactly each planned size, and each workgroup's LDS is two
host allocations of exactly the launch's static and dynamic bytes.

The first GPU fault of the fused step (gate|up read as one [2*hidden][dim]
matrix while the model held gate and up apart) is an out-of-range read that
this execution reports; the model's layout runs every step of the shapes the
GPU tests used, with no access outside an allocation, no LDS overrun, no
non-uniform value where the kernel assumes a uniform one, and no deadlock."""
import os
import shutil
import subprocess
import sys

import pytest

import cw

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "step_emu")

CLANG = "/opt/rocm/llvm/bin/clang++"
ENV = {"ASAN_OPTIONS": "detect_leaks=0",
       "ASAN_SYMBOLIZER_PATH": "/opt/rocm/llvm/bin/llvm-symbolizer", "PATH": os.environ["PATH"]}


@pytest.fixture(scope="module")
def emu():
    if not os.path.exists(CLANG) or not shutil.which("make"):
        pytest.skip("no host clang++ for the CPU execution")
    r = subprocess.run(["make", "-s", "-C", HERE], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    return os.path.join(HERE, "step_emu")


def run(emu, cfg, n_cu, steps, tmp_path, split_gate_up=False, prompt=2):
    if HERE not in sys.path:
        sys.path.insert(0, HERE)
    import plan
    path = str(tmp_path / "plan.bin")
    plan.write_plan(cfg, n_cu, path, split_gate_up)
    return subprocess.run([emu, path, str(cfg.kv_dtype), str(n_cu), str(steps), str(prompt)],
                          capture_output=True, text=True, env=ENV, timeout=600)


def small128(max_seq, kv_dtype, n_heads, n_kv):
    return cw.make_config(2, 256, n_heads, n_kv, 128, 512, 1000, max_seq, kv_dtype, 1e-6, 1e6)


CONFIGS = [
    # the configuration whose one GPU run after the gate|up fix faulted
    cw.make_config(2, 256, 4, 2, 128, 512, 1000, 8),
    small128(29, cw.CW_F32, 4, 2),
    small128(29, cw.CW_F16, 8, 2),
    small128(29, cw.CW_F32, 2, 2),
    small128(29, cw.CW_F16, 8, 1),
]


@pytest.mark.parametrize("cfg", CONFIGS, ids=lambda c: f"d{c.dim}h{c.n_heads}kv{c.n_kv_heads}"
                         f"t{c.kv_dtype}s{c.max_seq}")
def test_fused_step_runs_in_bounds(emu, cfg, tmp_path):
    r = run(emu, cfg, 16, 3, tmp_path)
    assert r.returncode == 0, r.stdout + r.stderr[-4000:]
    lines = [ln for ln in r.stdout.splitlines() if ln.startswith("step ")]
    assert len(lines) == 3
    # the state advances one position per step and feeds the prompt, then
    # the argmax (mod.rs:114-122)
    assert "pos 0 -> 1, token 2," in lines[0], lines
    assert "pos 2 -> 3" in lines[2] and "produced 2" in lines[2], lines
    for ln in lines:
        assert ln.endswith("error word 0"), ln


def test_split_gate_up_layout_is_an_out_of_range_read(emu, tmp_path):
    """The first fault's cause: the gate|up phase reads 2*hidden rows from a
    gate matrix of hidden rows, reported at the phase's weight loads."""
    r = run(emu, CONFIGS[0], 8, 1, tmp_path, split_gate_up=True)
    assert r.returncode != 0
    assert "heap-buffer-overflow" in r.stderr, r.stderr[-3000:]
    assert "gemv_load" in r.stderr, r.stderr[-3000:]
