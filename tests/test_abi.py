"""CPU tests of the product library: it loads, exports every declared entry
point, validates arguments on the host, and its host-side helpers (the Q4
re-quantizer, block splitting, synthetic data) are exact."""
import ctypes as C
import os
import re

import numpy as np

import cw
import oracle as orc
from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "chat_wgpu.h")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(cw_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    lib = cw.lib()
    names = declared()
    assert len(names) >= 40
    for n in names:
        assert hasattr(lib, n), n
    # and the binding declares a signature for each
    assert set(names) == set(cw._SIGS), set(names) ^ set(cw._SIGS)


def test_version_and_no_error():
    assert b"gfx950" in cw.lib().cw_version()


def test_host_argument_validation_without_device():
    lib = cw.lib()
    # null context
    rc = lib.cw_q4_gemv(None, None, None, None, 256, 512, None)
    assert rc == -1 and b"null" in lib.cw_last_error()
    # shape errors are reported before the context is touched
    fake = C.c_void_p(16)
    buf = C.c_void_p(4096)
    rc = lib.cw_q4_gemv(fake, buf, buf, buf, 33, 512, buf)
    assert rc == -1 and b"multiple of 32" in lib.cw_last_error()
    rc = lib.cw_q4_gemv(fake, buf, buf, buf, 65536, 512, buf)
    assert rc == -1 and b"32768" in lib.cw_last_error()
    rc = lib.cw_q4_gemv(fake, C.c_void_p(4100), buf, buf, 256, 512, buf)
    assert rc == -1 and b"aligned" in lib.cw_last_error()
    rc = lib.cw_q4_quantize(None, 1, 32, None, None)
    assert rc == -1


def test_quantize_matches_oracle(rng):
    data = (rng.standard_normal((97, 256)) * 0.02).astype(np.float32)
    data[3, :32] = 0.0                      # d == 0 block
    data[5, 7] = np.float32(np.nan)         # NaN ignored by the absmax, q -> 0+8
    data[6, :32] = np.linspace(-1, 1, 32)   # large values
    s, q = cw.q4_quantize(data)
    os_, oq = orc.quantize_q4_0_gguf(data)
    assert np.array_equal(s, os_) and np.array_equal(q, oq)


def test_split_blocks(rng):
    blocks = rng.integers(0, 256, (50, 18)).astype(np.uint8)
    s, q = cw.q4_split_blocks(blocks)
    assert np.array_equal(s, blocks[:, :2].copy().view(np.uint16).reshape(-1))
    assert np.array_equal(q, blocks[:, 2:])
    # the split image dequantizes exactly like the 18-byte blocks
    assert np.array_equal(orc.dequant_q4_0(blocks, 50 * 32), orc.dequant_q4_0_soa(s, q))


def test_synthetic_generators_deterministic():
    k = cw.synth_key(7, "blk.0.attn_q.weight")
    assert k == cw.synth_key(7, "blk.0.attn_q.weight")
    assert k != cw.synth_key(8, "blk.0.attn_q.weight")
    assert k != cw.synth_key(7, "blk.0.attn_k.weight")
    s1, q1 = cw.synth_q4(k, 3072, 1024)
    s2, q2 = cw.synth_q4(k, 3072, 1024)
    assert np.array_equal(s1, s2) and np.array_equal(q1, q2)
    # element i depends only on (key, i): a prefix is a prefix
    s3, q3 = cw.synth_q4(k, 100, 1024)
    assert np.array_equal(s3, s1[:100]) and np.array_equal(q3, q1[:100])
    x1 = cw.synth_normal_f32(k, 1 << 20)
    assert np.array_equal(cw.synth_normal_f32(k, 1000), x1[:1000])


def test_synthetic_distributions():
    k = cw.synth_key(1, "t")
    s, q = cw.synth_q4(k, 4096, 1024, 0.02)
    d = s.view(np.float16).astype(np.float64)
    assert np.all(d >= 0)
    # |N(0, s)| has mean s*sqrt(2/pi)
    assert abs(d.mean() - 0.02 * np.sqrt(2 / np.pi)) < 2e-4
    nib = np.concatenate([q & 15, q >> 4]).astype(np.float64)
    assert abs(nib.mean() - 7.5) < 0.02
    x = cw.synth_normal_f32(k, 1 << 20, 1.0, 0.02).astype(np.float64)
    assert abs(x.mean() - 1.0) < 1e-4 and abs(x.std() - 0.02) < 1e-4
    h = cw.synth_normal_f16(k, 1 << 16)
    assert abs(h.view(np.float16).astype(np.float64).std() - 1.0) < 0.02
    t = cw.synth_tokens(k, 10000, 151936)
    assert t.max() < 151936 and t.min() >= 0 and len(set(t.tolist())) > 9000


def test_synthetic_weights_cover_every_tensor():
    cfg = cw.make_config(2, 64, 4, 2, 16, 128, 256, 16)
    w = cw.synthetic_weights(cfg, 3)
    assert len(w) == 2 * 11 + 2
    s, q = w["blk.1.ffn_down.weight"]
    assert s.shape == (64, 4) and q.shape == (64, 4, 16)


NULL_PROBE = r'''
import sys
sys.path.insert(0, sys.argv[1])
import cw
lib = cw.lib()
for name, (res, args) in sorted(cw._SIGS.items()):
    if res is not cw._I or not args:
        continue
    vals = [0.0 if a is cw._F else 0 if a in (cw._I, cw._U32, cw._SZ, cw._U64) else None
            for a in args]
    rc = getattr(lib, name)(*vals)
    print(name, rc, lib.cw_last_error().decode(), flush=True)
'''


def test_every_entry_point_refuses_null_and_zero_arguments():
    """Every int-returning entry point called with null handles and pointers
    and zero sizes returns a status code, never crashes: CW_ERR_ARG with a
    message naming the call, except the destroy/close calls (a null handle is
    nothing to free) and cw_gguf_has (0: no such tensor).  Run in a child
    process so that a crash would show as its exit status."""
    import subprocess
    import sys as _sys
    r = subprocess.run([_sys.executable, "-c", NULL_PROBE, os.path.join(ROOT, "chat-wgpu_amd")],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    seen = 0
    for line in r.stdout.splitlines():
        name, rc, msg = line.split(" ", 2)
        rc = int(rc)
        seen += 1
        if name in ("cw_ctx_destroy", "cw_model_destroy", "cw_gguf_close", "cw_graph_destroy",
                    "cw_gguf_has"):
            assert rc == 0, line
        else:
            assert rc == -1, line
            assert msg.startswith(name + ":"), line
    assert seen >= 70, r.stdout
