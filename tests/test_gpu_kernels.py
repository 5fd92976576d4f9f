"""Kernel parity on the MI355X: every HIP entry point against the CPU oracle
on the same seeded inputs.

Tolerances (stated per test):
  * Q4 unpack/dequant: bit-exact (one-hot GEMVs return dequantized weights).
  * GEMV / fused GEMV: max|y - y_oracle| / max|y_oracle| <= 1e-4 (f32
    accumulate), and per element |y - y_f64| <= 2e-5 * sum_k |w_k x_k|.
  * RMSNorm / RoPE / SwiGLU / add: 2e-6 relative (f32 rounding only).
  * Attention: 1e-5 * max|V| absolute.
  * argmax, KV write (f32 and f16 rounding), embedding gather: bit-exact.
"""
import json
import os

import numpy as np
import pytest

import cw
import oracle as orc
from conftest import GOLDEN

pytestmark = pytest.mark.gpu

with open(os.path.join(GOLDEN, "reference_kats.json")) as f:
    KATS = json.load(f)


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def rel_err(y, ref):
    return float(np.max(np.abs(y.astype(np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def synth_gemv(out_f, in_f, seed):
    s, q = cw.synth_q4(cw.synth_key(seed, f"w{out_f}x{in_f}"), out_f, in_f, 0.02)
    x = cw.synth_normal_f32(cw.synth_key(seed, f"x{in_f}"), in_f)
    return s, q, x


GEMV_SHAPES = [
    (256, 512),        # reference KAT shape (main.rs:124)
    (1024, 3072),      # single Q4_0 GEMV workload (3072 x 1024)
    (1024, 2048), (1024, 1024), (2048, 1024), (3072, 1024),   # Qwen3-0.6B projections
    (4096, 6144), (4096, 4096), (4096, 12288), (12288, 4096),  # Qwen3-8B projections
    (32, 7), (64, 33), (96, 100), (160, 65), (224, 300), (32768, 40),  # every lane split, tails
    (1024, 151936),    # Qwen3-0.6B LM head
]


@pytest.mark.parametrize("in_f,out_f", GEMV_SHAPES)
def test_q4_gemv_vs_oracle(ctx, in_f, out_f):
    s, q, x = synth_gemv(out_f, in_f, 11)
    y = ctx.q4_gemv(ctx.storage(x), ctx.storage(s), ctx.storage(q), in_f, out_f).download()
    ref = orc.q4_gemv(x, s, q, in_f, out_f)
    assert rel_err(y, ref) <= 1e-4
    y64, absy = orc.q4_gemv_f64(x, s, q, in_f, out_f)
    assert np.all(np.abs(y - y64) <= 2e-5 * absy + 1e-30)


def test_q4_gemv_reference_kat(ctx):
    z = np.load(os.path.join(GOLDEN, "q4_gemv_kat.npz"))
    y = ctx.q4_gemv(ctx.storage(z["x"]), ctx.storage(z["gguf_scales"]),
                    ctx.storage(z["gguf_quants"]), 256, 512).download()
    assert rel_err(y, z["gguf_y"]) <= 1e-4
    assert np.max(np.abs(y - z["gguf_y"])) < KATS["report_tolerance"]["max_abs_err"]


def test_q4_unpack_exhaustive_bit_exact(ctx):
    """Every finite f16 scale x every nibble value at every element position:
    a one-hot x returns d*(q-8) exactly (K=32, one block per row)."""
    d = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    d = d[np.isfinite(d.view(np.float16))]
    n = d.size
    b = np.arange(n)[:, None]
    j = np.arange(16)[None, :]
    qs = (((b + j) % 16) | (((b + 3 * j + 5) % 16) << 4)).astype(np.uint8).reshape(n, 1, 16)
    sd, qd = ctx.storage(d.reshape(n, 1)), ctx.storage(qs)
    for k in range(32):
        e = np.zeros(32, np.float32)
        e[k] = 1.0
        y = ctx.q4_gemv(ctx.storage(e), sd, qd, 32, n).download()
        ref = orc.q4_gemv(e, d.reshape(n, 1), qs, 32, n)
        assert np.array_equal(bits(y), bits(ref)), k


def test_q4_unpack_positions_wide_rows(ctx):
    """One-hot columns across lanes/blocks of wide rows: bit-exact."""
    for in_f, out_f in ((4096, 64), (3072, 96), (1024, 130)):
        s, q, _ = synth_gemv(out_f, in_f, 5)
        sd, qd = ctx.storage(s), ctx.storage(q)
        deq = orc.dequant_q4_0_soa(s, q).reshape(out_f, in_f)
        for k in (0, 1, 15, 16, 17, 31, 32, 33, 1000, in_f - 32, in_f - 17, in_f - 1):
            e = np.zeros(in_f, np.float32)
            e[k] = 1.0
            y = ctx.q4_gemv(ctx.storage(e), sd, qd, in_f, out_f).download()
            assert np.array_equal(bits(y), bits(deq[:, k] + np.float32(0.0))), (in_f, k)


def test_q4_gemv_all_eights_is_zero(ctx):
    """All nibbles 8 (the q4bench input 0x88888888): the weights are exactly
    zero.  Like the reference shader (q4.wgsl:131, s_total = (s_lo + s_hi) -
    8 * x_sum) the kernel factors the -8 out of the block sum, so the result
    is zero up to f32 cancellation: |y| <= 1e-6 * sum_b |d_b| * 8 * sum|x_b|."""
    in_f, out_f = 1024, 3072
    s, _, x = synth_gemv(out_f, in_f, 3)
    q = np.full((out_f, in_f // 32, 16), 0x88, np.uint8)
    y = ctx.q4_gemv(ctx.storage(x), ctx.storage(s), ctx.storage(q), in_f, out_f).download()
    d = s.view(np.float16).astype(np.float64)
    cond = (d * 8 * np.abs(x.astype(np.float64)).reshape(-1, 32).sum(1)).sum(1)
    assert np.all(np.abs(y) <= 1e-6 * cond)


@pytest.mark.parametrize("in_f,out_f", [(2048, 1024), (12288, 4096), (96, 70)])
def test_q4_gemv_add(ctx, in_f, out_f):
    s, q, x = synth_gemv(out_f, in_f, 21)
    r = cw.synth_normal_f32(cw.synth_key(21, "r"), out_f)
    rd = ctx.storage(r)
    y = ctx.q4_gemv_add(ctx.storage(x), ctx.storage(s), ctx.storage(q), in_f, out_f, rd).download()
    ref = orc.add(r, orc.q4_gemv(x, s, q, in_f, out_f))
    assert rel_err(y, ref) <= 1e-4
    # in place: y aliases the residual (hidden += W x)
    ctx.q4_gemv_add(ctx.storage(x), ctx.storage(s), ctx.storage(q), in_f, out_f, rd, rd)
    assert rel_err(rd.download(), ref) <= 1e-4


@pytest.mark.parametrize("in_f,out_f", [(1024, 3072), (4096, 12288), (64, 90)])
def test_q4_gemv_swiglu(ctx, in_f, out_f):
    gs, gq, x = synth_gemv(out_f, in_f, 31)
    us, uq = cw.synth_q4(cw.synth_key(31, "up"), out_f, in_f)
    y = ctx.q4_gemv_swiglu(ctx.storage(x), ctx.storage(gs), ctx.storage(gq), ctx.storage(us),
                           ctx.storage(uq), in_f, out_f).download()
    g = orc.q4_gemv(x, gs, gq, in_f, out_f)
    u = orc.q4_gemv(x, us, uq, in_f, out_f)
    ref = orc.swiglu(g, u)
    assert rel_err(y, ref) <= 1e-4


def test_rmsnorm(ctx, rng):
    k = KATS["rmsnorm_ones"]
    rows, dim, eps = k["rows"], k["dim"], k["eps"]
    y = ctx.rmsnorm(ctx.storage(np.ones(rows * dim, np.float32)),
                    ctx.storage(np.ones(dim, np.float32)), rows, dim, eps).download()
    assert np.max(np.abs(y - 1 / np.sqrt(1 + eps))) < 1e-6
    for rows, dim in ((1, 1024), (16, 128), (8, 128), (1, 4096), (3, 1000)):
        x = rng.standard_normal(rows * dim).astype(np.float32) * 3
        w = (1 + 0.02 * rng.standard_normal(dim)).astype(np.float32)
        y = ctx.rmsnorm(ctx.storage(x), ctx.storage(w), rows, dim, 1e-6).download()
        ref = orc.rmsnorm(x, w, rows, dim, 1e-6)
        assert np.max(np.abs(y - ref)) <= 2e-6 * np.max(np.abs(ref))


def test_rope(ctx, rng):
    k = KATS["rope_pos0"]
    rows, hd = k["rows"], k["head_dim"]
    x = (((np.arange(rows * hd) % 23) - 11) * 0.07).astype(np.float32)
    y = ctx.rope(ctx.storage(x), rows, hd, 0, k["theta"]).download()
    assert np.array_equal(y, x)
    for rows, hd, pos, theta in ((16, 128, 5, 1e6), (8, 128, 4351, 1e6), (4, 16, 77, 1e4),
                                 (32, 128, 4096, 1e6)):
        x = rng.standard_normal(rows * hd).astype(np.float32)
        y = ctx.rope(ctx.storage(x), rows, hd, pos, theta).download()
        ref = orc.rope(x, rows, hd, pos, theta)
        assert np.max(np.abs(y - ref)) <= 2e-6 * np.max(np.abs(ref))


def test_rope_rotation_direction_one_hot(ctx):
    """The device rotation's sign (rope.wgsl:30-31): a one-hot input at i gives
    (cos, sin) in (y_i, y_{i+h}), one at i + h gives (-sin, cos), against
    numpy's f64 cos/sin of pos * theta^(-2i/hd); every other element stays 0."""
    hd, theta, h = 128, 1e6, 64
    probes = [(i, j) for i in (0, 1, 5, 31, h - 1) for j in (i, i + h)]
    x = np.zeros((len(probes), hd), np.float32)
    for r, (_, j) in enumerate(probes):
        x[r, j] = 1.0
    for pos in (1, 7, 100, 4351):
        y = ctx.rope(ctx.storage(x.ravel()), len(probes), hd, pos, theta).download()
        y = y.reshape(len(probes), hd)
        for r, (i, j) in enumerate(probes):
            f = pos * float(np.float32(theta)) ** (-2.0 * i / hd)
            c, s = np.cos(f), np.sin(f)
            want = np.zeros(hd)
            want[i], want[i + h] = (c, s) if j == i else (-s, c)
            assert np.max(np.abs(y[r] - want)) < 2e-7, (pos, i, j)


def test_add_swiglu_kats(ctx):
    k = KATS["swiglu_const"]
    n = k["n"]
    out = ctx.swiglu(ctx.storage(np.full(n, k["g"], np.float32)),
                     ctx.storage(np.full(n, k["u"], np.float32)), n).download()
    ref = orc.swiglu(np.full(n, k["g"]), np.full(n, k["u"]))
    assert np.max(np.abs(out - ref)) <= 2e-6 * np.max(np.abs(ref))
    n = KATS["ewise_add"]["n"]
    a = np.arange(n, dtype=np.float32)
    b = -np.arange(n, dtype=np.float32) * np.float32(0.5)
    c = ctx.add(ctx.storage(a), ctx.storage(b), n).download()
    assert np.array_equal(c, orc.add(a, b))


def test_swiglu_random(ctx, rng):
    g = rng.standard_normal(12288).astype(np.float32) * 4
    u = rng.standard_normal(12288).astype(np.float32)
    out = ctx.swiglu(ctx.storage(g), ctx.storage(u), 12288).download()
    ref = orc.swiglu(g, u)
    assert np.max(np.abs(out - ref)) <= 2e-6 * np.max(np.abs(ref))


def test_argmax(ctx, rng):
    for n in (1, 7, 256, 4097, 151936, 300000):
        x = rng.standard_normal(n).astype(np.float32)
        got = int(ctx.argmax(ctx.storage(x), n).download()[0])
        assert got == orc.argmax(x)
    x = rng.standard_normal(151936).astype(np.float32)
    x[[70000, 10, 150000]] = 50.0
    x[5] = np.nan
    assert int(ctx.argmax(ctx.storage(x), x.size).download()[0]) == 10 == orc.argmax(x)
    x = np.full(1000, -np.inf, np.float32)
    assert int(ctx.argmax(ctx.storage(x), 1000).download()[0]) == 0 == orc.argmax(x)


@pytest.mark.parametrize("kv_dtype", [cw.CW_F32, cw.CW_F16])
def test_kv_write(ctx, rng, kv_dtype):
    kv_dim, max_seq, pos = 1024, 16, 9
    dt = np.float32 if kv_dtype == cw.CW_F32 else np.uint16
    kc = ctx.storage(np.zeros(max_seq * kv_dim, dt))
    vc = ctx.storage(np.zeros(max_seq * kv_dim, dt))
    k = rng.standard_normal(kv_dim).astype(np.float32)
    v = rng.standard_normal(kv_dim).astype(np.float32)
    ctx.kv_write(kc, vc, kv_dtype, pos, kv_dim, ctx.storage(k), ctx.storage(v))
    K = kc.download().reshape(max_seq, kv_dim)
    V = vc.download().reshape(max_seq, kv_dim)
    if kv_dtype == cw.CW_F16:
        ek = np.array([orc.f32_to_f16(t) for t in k], np.uint16)
        ev = np.array([orc.f32_to_f16(t) for t in v], np.uint16)
    else:
        ek, ev = k, v
    assert np.array_equal(K[pos], ek) and np.array_equal(V[pos], ev)
    assert not K[pos - 1].any() and not K[pos + 1].any()


def test_embed(ctx, rng):
    vocab, dim = 1000, 1024
    table = rng.standard_normal(vocab * dim).astype(np.float32)
    tok = ctx.storage(np.array([417], np.uint32))
    out = ctx.embed(ctx.storage(table), vocab, dim, tok).download()
    assert np.array_equal(out, table.reshape(vocab, dim)[417] + np.float32(0))


def _kv(rng, seq, nkv, hd, f16):
    k = rng.standard_normal(seq * nkv * hd).astype(np.float32)
    v = rng.standard_normal(seq * nkv * hd).astype(np.float32)
    if f16:
        return k.astype(np.float16).view(np.uint16), v.astype(np.float16).view(np.uint16)
    return k, v


def test_attention_seq1_kat(ctx):
    k = KATS["attention_seq1"]
    nh, nkv, hd = k["n_heads"], k["n_kv"], k["head_dim"]
    q = (np.arange(nh * hd) * 0.01).astype(np.float32)
    v = (((np.arange(nkv * hd) % 9) - 4) * 0.1).astype(np.float32)
    kc = np.full(nkv * hd, 0.5, np.float32)
    o = ctx.attention(ctx.storage(q), ctx.storage(kc), ctx.storage(v), cw.CW_F32, nh, nkv, 1,
                      hd).download().reshape(nh, hd)
    for h in range(nh):
        assert np.max(np.abs(o[h] - v.reshape(nkv, hd)[h // (nh // nkv)])) < 1e-6


ATTN_CASES = [  # (n_heads, n_kv, hd, seq, f16)
    (32, 8, 128, 4097, True), (32, 8, 128, 4352, True), (16, 8, 128, 160, False),
    (16, 8, 128, 1, False), (16, 8, 128, 33, False), (16, 8, 128, 128, False),
    (16, 8, 128, 129, True), (4, 2, 16, 9, False), (8, 8, 64, 300, True),
    (8, 1, 32, 257, False), (16, 2, 256, 200, True), (64, 8, 128, 1000, True),
    # more than 128 chunks per head: the merge's multi-pass (max, sum) loops
    (32, 8, 128, 9000, False),
    # f16 cache past one merge round (94 chunks of 128 positions)
    (32, 8, 128, 12000, True),
    # the f16 head_dim-128 kernel with one query head per kv head, and with
    # eight per kv head over two kv heads
    (8, 8, 128, 777, True), (16, 2, 128, 513, True),
    # the f32 head_dim-128 kernel at the same groupings
    (8, 8, 128, 300, False), (8, 1, 128, 200, False),
    # the longest sequence an attention call takes (32768 positions), on
    # the 8B shape's heads
    (32, 8, 128, 32768, True), (32, 8, 128, 32768, False),
    # the f16 kernel at 11 and 13 waves per workgroup (the wave count follows
    # the cache length: 9 at 4097, 16 from about 7.7K)
    (32, 8, 128, 5500, True), (32, 8, 128, 6500, True),
]


@pytest.mark.parametrize("nh,nkv,hd,seq,f16", ATTN_CASES)
def test_attention_vs_oracle(ctx, rng, nh, nkv, hd, seq, f16):
    q = rng.standard_normal(nh * hd).astype(np.float32) * 0.3
    k, v = _kv(rng, seq, nkv, hd, f16)
    dt = cw.CW_F16 if f16 else cw.CW_F32
    o = ctx.attention(ctx.storage(q), ctx.storage(k), ctx.storage(v), dt, nh, nkv, seq,
                      hd).download()
    ref = orc.attention(q, k, v, f16, nh, nkv, seq, hd)
    vmax = np.max(np.abs(v.view(np.float16) if f16 else v))
    assert np.max(np.abs(o - ref)) <= 1e-5 * vmax


def test_attention_refuses_sequences_past_its_limit(ctx):
    buf = ctx.empty(16)
    for seq in (0, 32769):
        rc = cw.lib().cw_attention(ctx.h, buf.ptr, buf.ptr, buf.ptr, cw.CW_F16, 32, 8, seq, 128,
                                   buf.ptr)
        assert rc == cw.CW_ERR_ARG, seq
        assert "seq=" in cw.lib().cw_last_error().decode()


def test_attention_repeated_calls(ctx, rng):
    """Calls of other shapes, single-chunk calls and other kernels that reuse
    the context scratch (argmax) in between leave later calls exact."""
    cases = [(32, 8, 128, 700, True), (16, 8, 128, 5, False), (8, 2, 64, 900, False),
             (32, 8, 128, 4100, True), (16, 4, 128, 300, True)]
    logits = rng.standard_normal(151936).astype(np.float32)
    ld = ctx.storage(logits)
    for rep in range(2):
        for nh, nkv, hd, seq, f16 in cases:
            q = rng.standard_normal(nh * hd).astype(np.float32) * 0.3
            k, v = _kv(rng, seq, nkv, hd, f16)
            dt = cw.CW_F16 if f16 else cw.CW_F32
            o = ctx.attention(ctx.storage(q), ctx.storage(k), ctx.storage(v), dt, nh, nkv, seq,
                              hd).download()
            ref = orc.attention(q, k, v, f16, nh, nkv, seq, hd)
            vmax = np.max(np.abs(v.view(np.float16) if f16 else v))
            assert np.max(np.abs(o - ref)) <= 1e-5 * vmax, (rep, nh, nkv, hd, seq, f16)
            # argmax reuses the context scratch that holds attention partials
            assert int(ctx.argmax(ld, logits.size).download()[0]) == int(np.argmax(logits))


def test_attention_constant_keys_mean(ctx, rng):
    nh, nkv, hd, seq = 32, 8, 128, 1000
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = np.tile(rng.standard_normal(nkv * hd).astype(np.float32), seq)
    v = rng.standard_normal(seq * nkv * hd).astype(np.float32)
    o = ctx.attention(ctx.storage(q), ctx.storage(k), ctx.storage(v), cw.CW_F32, nh, nkv, seq,
                      hd).download().reshape(nh, hd)
    mean = v.reshape(seq, nkv, hd).astype(np.float64).mean(0)
    assert np.max(np.abs(o - mean[np.arange(nh) // 4])) < 1e-5


def test_profile_report(ctx):
    s, q, x = synth_gemv(1024, 1024, 1)
    xd, sd, qd = ctx.storage(x), ctx.storage(s), ctx.storage(q)
    ctx.profile_begin()
    for _ in range(3):
        ctx.q4_gemv(xd, sd, qd, 1024, 1024)
    rows = ctx.profile_report()
    assert rows[0][0] == "q4_gemv" and rows[0][1] == 3 and rows[0][2] > 0


def test_attention_rejects_more_kv_heads_than_counters(ctx, rng):
    """The merge counters cover 1024 kv heads; more is an argument error
    raised before any launch."""
    nh = nkv = 1025
    hd = 16
    q = ctx.storage(rng.standard_normal(nh * hd).astype(np.float32))
    k = ctx.storage(rng.standard_normal(2 * nkv * hd).astype(np.float32))
    v = ctx.storage(rng.standard_normal(2 * nkv * hd).astype(np.float32))
    with pytest.raises(cw.CwError, match="exceeds 1024"):
        ctx.attention(q, k, v, cw.CW_F32, nh, nkv, 2, hd)


@pytest.mark.parametrize("n_words,blocks", [(4, 1), (1 << 20, 7), ((1 << 20) + 12, 256)])
def test_hbm_read_probe_folds_every_word(ctx, rng, n_words, blocks):
    """The read-bandwidth probe (examples/q4probe.rs's role) reads every
    16-byte word exactly once: the XOR of its per-workgroup words is the XOR
    of the whole buffer."""
    data = rng.integers(0, 1 << 32, n_words, dtype=np.uint64).astype(np.uint32)
    buf = ctx.storage(data)
    out = ctx.empty(blocks, np.uint32)
    ctx.hbm_read_probe(buf, data.nbytes, blocks, out)
    got = np.bitwise_xor.reduce(out.download())
    assert int(got) == int(np.bitwise_xor.reduce(data))
