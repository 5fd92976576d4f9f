"""Batched prefill on the MI355X: the Q4_0 MFMA GEMM against the oracle's
per-row GEMV, and the batched prompt phase against the oracle's per-token
forward loop (the reference's own prompt phase, src/model/mod.rs:57-125).

Bars:
  * GEMM: max|y - y_oracle| / max|y_oracle| <= 1e-4 (f32 accumulate) and, per
    element, |y - y_f64| <= 2e-5 * sum_k |w_k x_k|.
  * Prefill: logits of the last prompt position within 1e-3 absolute of the
    oracle's, the same next token, and greedy ids identical when decoding
    continues from the prefilled cache.
"""
import numpy as np
import pytest

import cw
import oracle as orc

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3


def rel_err(y, ref):
    return float(np.max(np.abs(y.astype(np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


GEMM_SHAPES = [  # (m, in_f, out_f)
    (1, 256, 512), (7, 1024, 3072), (64, 4096, 256), (65, 2048, 1024), (37, 96, 100),
    (130, 160, 65), (512, 4096, 512), (200, 12288, 128), (3, 32, 7),
    (100, 4160, 200),  # K split in two halves of 65 blocks (odd: a half-empty last stage)
]


@pytest.mark.parametrize("m,in_f,out_f", GEMM_SHAPES)
def test_q4_gemm_vs_oracle(ctx, m, in_f, out_f):
    s, q = cw.synth_q4(cw.synth_key(21, f"g{out_f}x{in_f}"), out_f, in_f, 0.02)
    x = cw.synth_normal_f32(cw.synth_key(21, f"gx{m}x{in_f}"), m * in_f).reshape(m, in_f)
    y = ctx.q4_gemm(ctx.storage(x), m, ctx.storage(s), ctx.storage(q), in_f, out_f).download()
    y = y.reshape(m, out_f)
    orc.set_threads(8)
    worst = 0.0
    for i in range(m):
        ref = orc.q4_gemv(x[i], s, q, in_f, out_f)
        worst = max(worst, rel_err(y[i], ref))
        y64, absy = orc.q4_gemv_f64(x[i], s, q, in_f, out_f)
        assert np.all(np.abs(y[i] - y64) <= 2e-5 * absy + 1e-30), i
    assert worst <= 1e-4, worst


# the four projection shapes of one 8B layer at the 512-token workload:
# QKV (4096 -> 6144), O (4096 -> 4096), gate/up (4096 -> 12288, each) and
# down (12288 -> 4096); (m, in_f, out_f).  These run the split-K and tile
# choices the prefill bench times.
GEMM_8B_512 = [(512, 4096, 6144), (512, 4096, 4096), (512, 4096, 12288), (512, 12288, 4096)]


@pytest.mark.parametrize("m,in_f,out_f", GEMM_8B_512)
def test_q4_gemm_8b_shapes_at_512(ctx, m, in_f, out_f):
    """Every element against an f64 product of the exactly dequantized
    weights (|y - y64| <= 2e-5 * sum_k |w x|, and 1e-4 of max|y| overall);
    sample rows against the oracle's sequential dot (main.rs:133-150)."""
    s, q = cw.synth_q4(cw.synth_key(23, f"g{out_f}x{in_f}"), out_f, in_f, 0.02)
    x = cw.synth_normal_f32(cw.synth_key(23, f"gx{m}x{in_f}"), m * in_f).reshape(m, in_f)
    y = ctx.q4_gemm(ctx.storage(x), m, ctx.storage(s), ctx.storage(q), in_f, out_f).download()
    y = y.reshape(m, out_f).astype(np.float64)
    w = orc.dequant_q4_0_soa(s, q).reshape(out_f, in_f).astype(np.float64)
    x64 = x.astype(np.float64)
    y64 = x64 @ w.T
    bound = np.abs(x64) @ np.abs(w).T
    err = np.abs(y - y64)
    worst = np.unravel_index(np.argmax(err / (bound + 1e-30)), err.shape)
    assert np.all(err <= 2e-5 * bound + 1e-30), (worst, err[worst], bound[worst])
    rel = float(np.max(err) / np.max(np.abs(y64)))
    print(f"\n[q4_gemm {m}x{in_f}->{out_f}] max rel err vs f64 {rel:.2e}", flush=True)
    assert rel <= 1e-4
    orc.set_threads(16)
    for i in (0, 1, 63, 64, 127, 128, 255, 256, 383, 511):
        ref = orc.q4_gemv(x[i], s, q, in_f, out_f)
        assert rel_err(y[i], ref) <= 1e-4, i


def test_q4_gemm_rows_match_gemv(ctx):
    """Every row of the batched GEMM equals the decode GEMV of that row to
    within the same tolerance (two different kernels, one definition)."""
    m, in_f, out_f = 20, 4096, 1024
    s, q = cw.synth_q4(cw.synth_key(22, "w"), out_f, in_f, 0.02)
    x = cw.synth_normal_f32(cw.synth_key(22, "x"), m * in_f).reshape(m, in_f)
    sd, qd = ctx.storage(s), ctx.storage(q)
    y = ctx.q4_gemm(ctx.storage(x), m, sd, qd, in_f, out_f).download().reshape(m, out_f)
    for i in range(m):
        g = ctx.q4_gemv(ctx.storage(x[i]), sd, qd, in_f, out_f).download()
        assert rel_err(y[i], g.astype(np.float64)) <= 1e-4, i


def test_q4_gemm_large_scales(ctx):
    """Block scales up to the f16 maximum (and the smallest subnormal) go
    through the GEMM as they do through the oracle's GEMV: each block's f32
    sum times d."""
    m, in_f, out_f = 37, 512, 96
    s, q = cw.synth_q4(cw.synth_key(24, "w"), out_f, in_f, 0.02)
    big = np.array([8192.0, -30000.0, 65504.0, -65504.0, 2.0 ** -24], np.float16).view(np.uint16)
    rng = np.random.default_rng(24)
    pick = rng.integers(0, s.size, 200)
    s.reshape(-1)[pick] = big[np.arange(200) % big.size]
    x = cw.synth_normal_f32(cw.synth_key(24, "x"), m * in_f).reshape(m, in_f)
    y = ctx.q4_gemm(ctx.storage(x), m, ctx.storage(s), ctx.storage(q), in_f, out_f).download()
    y = y.reshape(m, out_f)
    assert np.all(np.isfinite(y))
    for i in range(m):
        y64, absy = orc.q4_gemv_f64(x[i], s, q, in_f, out_f)
        assert np.all(np.abs(y[i] - y64) <= 2e-5 * absy + 1e-30), i
        assert rel_err(y[i], orc.q4_gemv(x[i], s, q, in_f, out_f)) <= 1e-4, i


def test_q4_gemm_argument_errors(ctx):
    s, q = cw.synth_q4(cw.synth_key(1, "e"), 64, 64, 0.02)
    x = ctx.storage(np.zeros((2, 64), np.float32))
    sd, qd = ctx.storage(s), ctx.storage(q)
    with pytest.raises(cw.CwError):
        ctx.q4_gemm(x, 2, sd, qd, 48, 64)   # in_f not a multiple of 32
    with pytest.raises(cw.CwError):
        ctx.q4_gemm(x, 0, sd, qd, 64, 64)   # no rows


def test_model_rejects_non_finite_scales(ctx):
    """A projection block scale that is not finite is refused at upload;
    large finite ones (8192, the f16 maximum) are accepted."""
    cfg = cw.make_config(1, 64, 2, 1, 32, 64, 100, 8, cw.CW_F16)
    m = cw.Model(ctx, cfg)
    s, q = cw.synth_q4(cw.synth_key(3, "w"), 64, 64, 0.02)
    for bad in (0x7C00, 0xFC00, 0x7E00, 0xFE01):   # +inf, -inf, NaNs
        s2 = s.copy()
        s2[5, 1] = bad
        with pytest.raises(cw.CwError, match="block 11"):
            m.set_weights({"blk.0.attn_q.weight": (s2, q)})
    for big in (0x7000, 0xF000, 0x7BFF):   # 8192, -8192, 65504
        s2 = s.copy()
        s2[5, 1] = big
        m.set_weights({"blk.0.attn_q.weight": (s2, q)})
    m.set_weights({"blk.0.attn_q.weight": (s, q)})
    m.close()


def small_f16(max_seq, n_layers=2, dim=256, n_heads=4, n_kv=2, hidden=512, vocab=1000):
    return cw.make_config(n_layers, dim, n_heads, n_kv, 128, hidden, vocab, max_seq, cw.CW_F16,
                          1e-6, 1e6)


def oracle_prompt_logits(o, prompt, start=0):
    logits = None
    for i, t in enumerate(prompt):
        logits, _ = o.step(int(t), start + i)
    return logits


@pytest.mark.parametrize("P", [1, 5, 64, 100])
def test_prefill_small_model(ctx, P):
    """Batched prompt phase of P tokens (ragged and whole 64-position tiles)
    against the oracle's per-token forward, then 12 greedy decode steps from
    the prefilled cache against the oracle's generate."""
    N = 12
    cfg = small_f16(P + N + 1)
    weights = cw.synthetic_weights(cfg, 77)
    prompt = cw.synth_tokens(cw.synth_key(77, f"p{P}"), P, cfg.vocab)
    m = cw.Model(ctx, cfg)
    m.set_weights(weights)
    m.finalize()
    o = orc.OracleModel(cfg, weights)
    nxt = m.prefill(prompt)
    ref_logits = oracle_prompt_logits(o, prompt)
    diff = float(np.max(np.abs(m.logits() - ref_logits)))
    assert diff <= LOGIT_TOL, diff
    assert nxt == int(np.argmax(ref_logits))
    m.decode_async(N, mode=cw.STEP_GRAPH)
    toks = m.tokens(N)
    ref, margins = o.generate(prompt, N + 1)
    assert int(ref[0]) == nxt
    assert np.array_equal(toks, ref[1:N + 1]), (toks, ref[1:N + 1])
    m.close()
    o.close()


@pytest.mark.parametrize("n_heads,n_kv", [(4, 4), (8, 1), (16, 2)])
def test_prefill_query_groupings(ctx, n_heads, n_kv):
    """The batched prompt phase (130 positions: two whole 64-position tiles
    and a ragged one) with one and with eight query heads per kv head: last
    position's logits within 1e-3 of the oracle's per-token forward, the same
    next token, then 8 greedy decode steps from the prefilled cache."""
    P, N = 130, 8
    cfg = small_f16(P + N + 1, n_heads=n_heads, n_kv=n_kv)
    weights = cw.synthetic_weights(cfg, 78 + n_heads + n_kv)
    prompt = cw.synth_tokens(cw.synth_key(78, f"q{n_heads}x{n_kv}"), P, cfg.vocab)
    m = cw.Model(ctx, cfg)
    m.set_weights(weights)
    m.finalize()
    o = orc.OracleModel(cfg, weights)
    nxt = m.prefill(prompt)
    ref_logits = oracle_prompt_logits(o, prompt)
    diff = float(np.max(np.abs(m.logits() - ref_logits)))
    assert diff <= LOGIT_TOL, diff
    assert nxt == int(np.argmax(ref_logits))
    m.decode_async(N, mode=cw.STEP_GRAPH)
    toks = m.tokens(N)
    ref, _ = o.generate(prompt, N + 1)
    assert int(ref[0]) == nxt
    assert np.array_equal(toks, ref[1:N + 1]), (toks, ref[1:N + 1])
    m.close()
    o.close()


def test_prefill_in_chunks_equals_one_pass(ctx):
    """Two prefill calls (positions 0..39, then 40..99 over the cache the
    first wrote) leave the same logits and next token as one 100-position
    call: attention of a later chunk reads the earlier rows from the cache."""
    cfg = small_f16(128)
    weights = cw.synthetic_weights(cfg, 78)
    prompt = cw.synth_tokens(cw.synth_key(78, "p"), 100, cfg.vocab)
    m = cw.Model(ctx, cfg)
    m.set_weights(weights)
    m.finalize()
    a = m.prefill(prompt)
    la = m.logits()
    m.prefill(prompt[:40])
    b = m.prefill(prompt[40:], start_pos=40)
    lb = m.logits()
    assert a == b
    assert float(np.max(np.abs(la - lb))) <= 1e-4
    m.close()


def test_prefill_qwen3_8b_layers(ctx):
    """Two layers of the Qwen3-8B shape (hidden 4096, 32/8 heads x 128,
    intermediate 12288; vocab cut to 4096 so the oracle finishes quickly):
    a 96-token batched prefill against the oracle's per-token loop, then 8
    greedy steps."""
    P, N = 96, 8
    cfg = cw.make_config(2, 4096, 32, 8, 128, 12288, 4096, P + N + 1, cw.CW_F16, 1e-6, 1e6)
    weights = cw.synthetic_weights(cfg, 80)
    prompt = cw.synth_tokens(cw.synth_key(80, "p"), P, cfg.vocab)
    m = cw.Model(ctx, cfg)
    m.set_weights(weights)
    m.finalize()
    orc.set_threads(16)
    o = orc.OracleModel(cfg, weights)
    nxt = m.prefill(prompt)
    ref_logits = oracle_prompt_logits(o, prompt)
    diff = float(np.max(np.abs(m.logits() - ref_logits)))
    print(f"\n[qwen3-8b x2 layers] prefill {P}: max |logit diff| = {diff:.3e}", flush=True)
    assert diff <= LOGIT_TOL, diff
    assert nxt == int(np.argmax(ref_logits))
    m.decode_async(N, mode=cw.STEP_GRAPH)
    toks = m.tokens(N)
    ref, _ = o.generate(prompt, N + 1)
    assert np.array_equal(toks, ref[1:N + 1]), (toks, ref[1:N + 1])
    m.close()
    o.close()


def test_prefill_qwen3_8b_layers_512(ctx):
    """The benchmarked prompt length: a 512-token batched prefill on two
    layers of the Qwen3-8B shape (vocab cut to 4096 so the oracle's 512
    per-token forwards finish quickly).  Causal MFMA attention over 8 query
    tiles and 512 keys, the M = 512 split-K GEMMs with the in-place residual:
    last-position logits within 1e-3 of the oracle's per-token loop, the same
    next token, then 4 greedy steps from the prefilled cache."""
    P, N = 512, 4
    cfg = cw.make_config(2, 4096, 32, 8, 128, 12288, 4096, P + N + 1, cw.CW_F16, 1e-6, 1e6)
    weights = cw.synthetic_weights(cfg, 81)
    prompt = cw.synth_tokens(cw.synth_key(81, "p512"), P, cfg.vocab)
    m = cw.Model(ctx, cfg)
    m.set_weights(weights)
    m.finalize()
    orc.set_threads(16)
    o = orc.OracleModel(cfg, weights)
    nxt = m.prefill(prompt)
    gl = m.logits()
    ref_logits = oracle_prompt_logits(o, prompt)
    diff = float(np.max(np.abs(gl - ref_logits)))
    top = np.sort(ref_logits)[-2:]
    print(f"\n[qwen3-8b x2 layers] prefill {P}: max |logit diff| = {diff:.3e}, "
          f"oracle top-2 margin {top[1] - top[0]:.3e}", flush=True)
    assert diff <= LOGIT_TOL, diff
    assert nxt == int(np.argmax(ref_logits))
    m.decode_async(N, mode=cw.STEP_GRAPH)
    toks = m.tokens(N)
    # the oracle continues from its own cache (rows 0..P-1 written above)
    ref, t = [], nxt
    for i in range(N):
        lg, _ = o.step(int(t), P + i)
        t = int(np.argmax(lg))
        ref.append(t)
    assert np.array_equal(toks, np.array(ref, np.uint32)), (toks, ref)
    m.close()
    o.close()


def test_prefill_f32_cache_runs_per_token(ctx):
    """An f32 cache takes the per-token step for the prompt: same logits as
    the oracle's loop."""
    cfg = cw.make_config(2, 64, 4, 2, 16, 128, 256, 20, cw.CW_F32, 1e-6, 1e6)
    weights = cw.synthetic_weights(cfg, 79)
    prompt = np.array([3, 1, 4, 1, 5, 9, 2, 6], np.uint32)
    m = cw.Model(ctx, cfg)
    m.set_weights(weights)
    m.finalize()
    o = orc.OracleModel(cfg, weights)
    nxt = m.prefill(prompt)
    ref_logits = oracle_prompt_logits(o, prompt)
    assert float(np.max(np.abs(m.logits() - ref_logits))) <= LOGIT_TOL
    assert nxt == int(np.argmax(ref_logits))
    m.close()
    o.close()
