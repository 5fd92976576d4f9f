"""Token-loop parity on the MI355X: the device-resident Qwen3 decode loop
(HIP graph replay) against the CPU oracle's forward/generate.

Bars: greedy token ids identical over the horizon; teacher-forced logits
within 1e-3 absolute at every step.
"""
import os

import numpy as np
import pytest

import cw
import oracle as orc
from conftest import GOLDEN

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3


def build_pair(ctx, cfg, weights):
    m = cw.Model(ctx, cfg)
    m.set_weights(weights)
    m.finalize()
    o = orc.OracleModel(cfg, weights)
    return m, o


def teacher_forced(m, o, tokens, start_pos=0):
    """Feed the same token sequence to both; return the max |logit diff| and
    the argmax agreement per step."""
    worst = 0.0
    for i, t in enumerate(tokens):
        pos = start_pos + i
        g_arg = m.step(int(t), pos)
        g_logits = m.logits()
        o_logits, _ = o.step(int(t), pos)
        diff = float(np.max(np.abs(g_logits - o_logits)))
        worst = max(worst, diff)
        assert diff <= LOGIT_TOL, (i, diff)
        assert g_arg == int(np.argmax(g_logits))
    return worst


def test_tiny_reference_model(ctx):
    """The reference verify model shape (src/main.rs:165-191) with
    RandomWeights re-quantized to Q4_0: identical greedy ids to the committed
    oracle fixture, graph replay and eager launches alike."""
    import make_golden as mg
    z = np.load(os.path.join(GOLDEN, "tiny_qwen3.npz"))
    cfg = cw.make_config(2, 64, 4, 2, 16, 128, 256, 12, cw.CW_F32, 1e-6, 1e6)
    weights = mg.tiny_weights()
    m, o = build_pair(ctx, cfg, weights)
    prompt = np.array([1, 5, 9, 2], np.uint32)
    for mode in (cw.STEP_GRAPH, cw.STEP_EAGER, cw.STEP_GRAPH):
        toks = m.generate(prompt, 8, mode=mode)
        assert np.array_equal(toks, z["tokens"]), (mode, toks, z["tokens"])
    m2 = cw.Model(ctx, cfg)
    m2.set_weights(weights)
    m2.finalize()
    m2.step(1, 0)
    assert np.max(np.abs(m2.logits() - z["logits_tok1_pos0"])) <= LOGIT_TOL
    teacher_forced(m, o, [1, 5, 9, 2] + list(z["tokens"][:7]))
    m.close()
    m2.close()


@pytest.mark.parametrize("n_heads,n_kv", [(4, 4), (8, 1), (16, 2)])
def test_f16_head128_query_groupings(ctx, n_heads, n_kv):
    """Decode with the f16 head_dim-128 attention fused into the step (QK-norm,
    RoPE and the KV write in its prologue) for one and for eight query heads
    per kv head: greedy ids identical to the oracle's over a 6-token prompt
    and 16 produced tokens, teacher-forced logits within 1e-3."""
    cfg = cw.make_config(2, 256, n_heads, n_kv, 128, 512, 1000, 40, cw.CW_F16, 1e-6, 1e6)
    weights = cw.synthetic_weights(cfg, 90 + n_heads + n_kv)
    prompt = cw.synth_tokens(cw.synth_key(91, f"g{n_heads}x{n_kv}"), 6, cfg.vocab)
    m, o = build_pair(ctx, cfg, weights)
    toks = m.generate(prompt, 16, mode=cw.STEP_GRAPH)
    ref, margins = o.generate(prompt, 16)
    first_diff = np.nonzero(toks != ref)[0]
    msg = "" if not first_diff.size else (
        f"first divergence at step {first_diff[0]}: margin {margins[first_diff[0]]:.3e}")
    assert np.array_equal(toks, ref), msg
    m2, o2 = build_pair(ctx, cfg, weights)
    worst = teacher_forced(m2, o2, list(prompt) + list(ref[:10]))
    print(f"\n[{n_heads}/{n_kv} heads] max |logit diff| = {worst:.3e}", flush=True)
    for x in (m, o, m2, o2):
        x.close()


def test_decode_next_continues_the_prompt_phase(ctx):
    """The chat loop's path: the prompt phase, then one replayed step per
    token read back as its argmax (cw_model_decode_next), gives generate's
    ids; at the last cache position it refuses with CW_ERR_ARG."""
    import make_golden as mg
    z = np.load(os.path.join(GOLDEN, "tiny_qwen3.npz"))
    cfg = cw.make_config(2, 64, 4, 2, 16, 128, 256, 12, cw.CW_F32, 1e-6, 1e6)
    m = cw.Model(ctx, cfg)
    m.set_weights(mg.tiny_weights())
    m.finalize()
    got = [m.prefill(np.array([1, 5, 9, 2], np.uint32))]
    got += [m.decode_next() for _ in range(7)]       # positions 4..10
    assert got == [int(t) for t in z["tokens"][:8]]
    m.decode_next()                                   # position 11, the last row
    with pytest.raises(cw.CwError, match="at max_seq"):
        m.decode_next()
    m.close()


def test_fused_step_refused_while_disabled(ctx):
    """CW_STEP_FUSED is refused with an error, never launched."""
    cfg = cw.make_config(2, 256, 4, 2, 128, 512, 1000, 8)
    m = cw.Model(ctx, cfg)
    m.load_synthetic(3)
    m.finalize()
    with pytest.raises(cw.CwError, match="fused decode step disabled"):
        m.generate(np.array([1, 2], np.uint32), 2, mode=cw.STEP_FUSED)
    m.close()


@pytest.mark.skip(reason="fused decode step disabled: an illegal memory access on the GPU after "
                         "the gate|up layout fix; second cause not found")
def test_fused_step_runs_after_the_layout_check(ctx):
    """CW_STEP_FUSED launches once the host-side range check of its buffer
    layout has passed at cw_model_finalize: the ids equal the graph path's."""
    cfg = cw.make_config(2, 256, 4, 2, 128, 512, 1000, 8)
    m = cw.Model(ctx, cfg)
    m.load_synthetic(3)
    m.finalize()
    g = m.generate(np.array([1, 2], np.uint32), 4, mode=cw.STEP_GRAPH)
    f = m.generate(np.array([1, 2], np.uint32), 4, mode=cw.STEP_FUSED)
    assert np.array_equal(f, g), (f, g)
    m.close()


@pytest.mark.parametrize("kv_dtype", [cw.CW_F16, cw.CW_F32])
def test_cache_rows_past_the_sequence_do_not_reach_the_output(ctx, kv_dtype):
    """Attention reads the cache rows of its chunks before it knows the
    device-resident position (the f16 kernel) or clamps them to the
    sequence (the f32 one); either way rows at or past the sequence must not
    reach the output, whatever they hold.  Two copies of one model: the
    cache rows past the prompt hold NaN and inf in one and zeros in the
    other; 8 replayed greedy steps and the logits of a step give the same
    bits."""
    P, N, max_seq = 40, 8, 96
    cfg = cw.make_config(2, 256, 4, 2, 128, 512, 1000, max_seq, kv_dtype)
    kv_dim = cfg.n_kv_heads * cfg.head_dim
    dt = np.float16 if kv_dtype == cw.CW_F16 else np.float32
    rng = np.random.default_rng(41)
    k = rng.standard_normal((cfg.n_layers, max_seq, kv_dim)).astype(dt)
    v = rng.standard_normal((cfg.n_layers, max_seq, kv_dim)).astype(dt)
    k_bad, v_bad, k_zero, v_zero = k.copy(), v.copy(), k.copy(), v.copy()
    k_bad[:, P:] = np.nan
    v_bad[:, P:] = np.nan
    v_bad[:, P + 1::3] = np.inf
    k_zero[:, P:] = 0
    v_zero[:, P:] = 0
    out = []
    for kk, vv in ((k_bad, v_bad), (k_zero, v_zero)):
        m = cw.Model(ctx, cfg)
        m.load_synthetic(77)
        m.finalize()
        m.prefill_kv(kk, vv, max_seq)
        toks = m.generate(np.array([5], np.uint32), N, start_pos=P, mode=cw.STEP_GRAPH)
        m.step(9, P + N)
        out.append((toks, m.logits()))
        m.close()
    (t_bad, l_bad), (t_zero, l_zero) = out
    assert np.all(np.isfinite(l_bad))
    assert np.array_equal(t_bad, t_zero)
    assert np.array_equal(l_bad.view(np.uint32), l_zero.view(np.uint32))


def test_missing_tensor_is_an_error(ctx):
    cfg = cw.make_config(1, 64, 4, 2, 16, 128, 256, 8)
    m = cw.Model(ctx, cfg)
    with pytest.raises(cw.CwError, match="missing tensor"):
        m.finalize()
    with pytest.raises(cw.CwError, match="not finalized"):
        m.generate(np.array([1], np.uint32), 2)
    m.close()


def qwen3_06b(max_seq, kv_dtype=cw.CW_F32):
    return cw.make_config(28, 1024, 16, 8, 128, 3072, 151936, max_seq, kv_dtype, 1e-6, 1e6)


def qwen3_8b(max_seq, kv_dtype=cw.CW_F16):
    return cw.make_config(36, 4096, 32, 8, 128, 12288, 151936, max_seq, kv_dtype, 1e-6, 1e6)


def test_synthetic_load_matches_host_weights(ctx):
    """cw_model_load_synthetic == set_weights(synthetic_weights) (same keys)."""
    cfg = cw.make_config(2, 256, 4, 2, 64, 512, 1000, 8)
    a = cw.Model(ctx, cfg)
    a.load_synthetic(9)
    a.finalize()
    b = cw.Model(ctx, cfg)
    b.set_weights(cw.synthetic_weights(cfg, 9))
    b.finalize()
    a.step(3, 0)
    b.step(3, 0)
    assert np.array_equal(a.logits(), b.logits())
    a.close()
    b.close()


def test_qwen3_06b_token_loop(ctx):
    """Qwen3-0.6B shape, Q4_0 synthetic weights, 32-token prompt then 128
    greedy steps with an f32 KV cache (the full workload)."""
    P, N = 32, 128
    cfg = qwen3_06b(P + N)
    weights = cw.synthetic_weights(cfg, 2024)
    prompt = cw.synth_tokens(cw.synth_key(2024, "prompt"), P, cfg.vocab)
    m, o = build_pair(ctx, cfg, weights)
    toks = m.generate(prompt, N, mode=cw.STEP_GRAPH)
    ref, margins = o.generate(prompt, N)
    first_diff = np.nonzero(toks != ref)[0]
    msg = "" if not first_diff.size else (
        f"first divergence at step {first_diff[0]}: gpu {toks[first_diff[0]]} oracle "
        f"{ref[first_diff[0]]}, oracle top-2 margin {margins[first_diff[0]]:.3e}")
    assert np.array_equal(toks, ref), msg
    # teacher-forced logits over the whole fed sequence; re-feeding the same
    # tokens rewrites every cache row with the values generate wrote
    seq = list(prompt) + list(ref[:N - 1])
    worst = teacher_forced(m, o, seq)
    print(f"\n[qwen3-0.6b] max |logit diff| over {len(seq)} steps = {worst:.3e}", flush=True)
    m.close()
    o.close()


def test_qwen3_8b_decode_prefilled(ctx):
    """Qwen3-8B shape: KV cache pre-filled with 4096 positions of N(0,1) f16,
    then greedy decode (16 steps here; the bench runs 256)."""
    pre, N = 4096, 16
    cfg = qwen3_8b(pre + N)
    weights = cw.synthetic_weights(cfg, 8008)
    kv_n = cfg.n_layers * pre * cfg.n_kv_heads * cfg.head_dim
    k = cw.synth_normal_f16(cw.synth_key(8008, "kv.k"), kv_n)
    v = cw.synth_normal_f16(cw.synth_key(8008, "kv.v"), kv_n)
    start = cw.synth_tokens(cw.synth_key(8008, "start"), 1, cfg.vocab)
    m, o = build_pair(ctx, cfg, weights)
    m.prefill_kv(k, v, pre)
    o.prefill_kv(k, v, pre)
    toks = m.generate(start, N, start_pos=pre, mode=cw.STEP_GRAPH)
    ref, margins = o.generate(start, N, start_pos=pre)
    first_diff = np.nonzero(toks != ref)[0]
    msg = "" if not first_diff.size else (
        f"first divergence at step {first_diff[0]}: margin {margins[first_diff[0]]:.3e}")
    assert np.array_equal(toks, ref), msg
    # teacher-forced logits at the first 4 decode positions (same tokens as fed)
    worst = teacher_forced(m, o, [int(start[0])] + list(ref[:3]), start_pos=pre)
    print(f"\n[qwen3-8b] max |logit diff| = {worst:.3e}", flush=True)
    m.close()
    o.close()


def test_qwen3_8b_teacher_forced_over_the_decode_range(ctx):
    """Qwen3-8B shape (the decode workload's model) with a cache of 4352
    positions of N(0,1) f16: one forward at each of 16 positions spread over
    4096..4351 (attention over 4097..4352 keys), fed 16 different token ids
    rather than the synthetic model's own greedy output (which repeats one
    id).  Logits within 1e-3 of the oracle at every position and the same
    argmax; the oracle's top-2 margins are printed."""
    n_pre = 4352
    cfg = qwen3_8b(n_pre)
    weights = cw.synthetic_weights(cfg, 8009)
    kv_n = cfg.n_layers * n_pre * cfg.n_kv_heads * cfg.head_dim
    k = cw.synth_normal_f16(cw.synth_key(8009, "kv.k"), kv_n)
    v = cw.synth_normal_f16(cw.synth_key(8009, "kv.v"), kv_n)
    m, o = build_pair(ctx, cfg, weights)
    m.prefill_kv(k, v, n_pre)
    o.prefill_kv(k, v, n_pre)
    del k, v
    orc.set_threads(16)
    positions = np.linspace(4096, 4351, 16).round().astype(int)
    ids = cw.synth_tokens(cw.synth_key(8009, "tf.ids"), 16, cfg.vocab)
    worst = 0.0
    for p, t in zip(positions, ids):
        g_arg = m.step(int(t), int(p))
        gl = m.logits()
        ol, _ = o.step(int(t), int(p))
        diff = float(np.max(np.abs(gl - ol)))
        top = np.sort(ol)[-2:]
        print(f"\n[qwen3-8b tf] pos {p} id {t}: max |logit diff| {diff:.3e}, "
              f"oracle argmax {int(np.argmax(ol))} margin {top[1] - top[0]:.3e}", flush=True)
        worst = max(worst, diff)
        assert diff <= LOGIT_TOL, (p, diff)
        assert g_arg == int(np.argmax(ol)), (p, g_arg, int(np.argmax(ol)))
    print(f"\n[qwen3-8b tf] worst |logit diff| over 16 positions = {worst:.3e}", flush=True)
    m.close()
    o.close()


# ---------------------------------------------------------------- a greedy horizon that moves

HORIZON = 64


@pytest.fixture(scope="module")
def horizon(ctx):
    """Qwen3-8B shape from a cache of 4096 positions of N(0,1) f16, 64 greedy
    steps replayed as a HIP graph, with two changes to the benchmark model so
    that each produced id depends on the fed one: embedding rows drawn with
    std 1e5, and an untied output head (output.weight, which Qwen3::load
    uses when present, qwen3.rs:93-98) drawn like the layer projections.

    With the benchmark model itself every step returns one id: the Q4
    weights' (q - 8) has mean -1/2, so the final hidden state lies along one
    fixed direction whatever the token, and the tied head's argmax is the
    embedding row with the extreme sum there (embedding std 0.02 and 1.0
    both give that id at every step, top-2 margin 0.03 and 1.9).  A loop
    that fed back a stale token would pass such a test; here it cannot."""
    pre, seed = 4096, 8008
    cfg = qwen3_8b(pre + HORIZON)
    w = cw.synthetic_weights(cfg, seed)
    w["token_embd.weight"] = cw.synth_normal_f32(cw.synth_key(seed, "token_embd.weight"),
                                                 cfg.vocab * cfg.dim, 0.0, 1e5)
    w["output.weight"] = cw.synth_q4(cw.synth_key(seed, "output.weight"), cfg.vocab, cfg.dim)
    kv_n = cfg.n_layers * pre * cfg.n_kv_heads * cfg.head_dim
    k = cw.synth_normal_f16(cw.synth_key(seed, "kv.k"), kv_n)
    v = cw.synth_normal_f16(cw.synth_key(seed, "kv.v"), kv_n)
    start = cw.synth_tokens(cw.synth_key(seed, "start"), 1, cfg.vocab)
    m, o = build_pair(ctx, cfg, w)
    m.prefill_kv(k, v, pre)
    o.prefill_kv(k, v, pre)
    del k, v, w
    orc.set_threads(16)
    print(f"\n[qwen3-8b horizon] {HORIZON} greedy steps from {pre} on the GPU", flush=True)
    toks = m.generate(start, HORIZON, start_pos=pre, mode=cw.STEP_GRAPH)
    state = {"m": m, "o": o, "pre": pre, "start": start, "gpu": toks, "ref": []}
    yield state
    m.close()
    o.close()


def horizon_half(h, first):
    """The oracle's greedy ids for one half of the horizon (the second half
    resumes the oracle's own trajectory), compared with the GPU's."""
    n = HORIZON // 2
    if first:
        ref, margins = h["o"].generate(h["start"], n, start_pos=h["pre"])
    else:
        assert len(h["ref"]) == n, "the first half did not pass"
        last = np.array([h["ref"][-1]], np.uint32)
        ref, margins = h["o"].generate(last, n, start_pos=h["pre"] + n)
    lo = 0 if first else n
    gpu = h["gpu"][lo:lo + n]
    print(f"\n[qwen3-8b horizon] steps {lo}..{lo + n - 1}: ids {ref.tolist()}\n"
          f"  top-2 margins min {float(np.min(margins)):.3e} "
          f"{np.round(margins, 3).tolist()}", flush=True)
    first_diff = np.nonzero(gpu != ref)[0]
    msg = "" if not first_diff.size else (
        f"first divergence at step {lo + first_diff[0]}: gpu {gpu[first_diff[0]]} oracle "
        f"{ref[first_diff[0]]}, oracle top-2 margin {margins[first_diff[0]]:.3e}")
    assert np.array_equal(gpu, ref), msg
    h["ref"] += ref.tolist()


def test_qwen3_8b_greedy_horizon_first_half(horizon):
    horizon_half(horizon, True)


def test_qwen3_8b_greedy_horizon_second_half(horizon):
    horizon_half(horizon, False)
    ids = horizon["ref"]
    distinct = len(set(ids))
    print(f"\n[qwen3-8b horizon] {distinct} distinct ids over {len(ids)} steps", flush=True)
    assert len(ids) == HORIZON and distinct >= 4, distinct
    # every produced id is fed back: a loop that kept feeding one token would
    # repeat one id, which the trajectory above does not
    assert any(ids[i] != ids[i + 1] for i in range(len(ids) - 1))


# ---------------------------------------------------------------- fused decode step

# The persistent decode-step kernel raised an illegal memory access here
# (test_fused_step_small_model[f32, 4 heads / 2 kv]): its gate|up phase read
# 2 * hidden rows from the gate matrix alone.  Gate and up now share one
# allocation, and cw_model_finalize checks every range the step touches
# (tests/test_step_layout.py shows the check refusing the old layout), but the
# one run after that fix faulted again, so a second cause remains: the library
# refuses CW_STEP_FUSED and these tests stay skipped.
FUSED_SKIP = pytest.mark.skip(reason="fused decode step disabled: an illegal memory access on "
                                     "the GPU after the gate|up layout fix; second cause not found")


def small128(max_seq, kv_dtype=cw.CW_F32, n_heads=4, n_kv=2):
    """A small model the fused step covers (head_dim 128)."""
    return cw.make_config(2, 256, n_heads, n_kv, 128, 512, 1000, max_seq, kv_dtype, 1e-6, 1e6)


@FUSED_SKIP
@pytest.mark.parametrize("kv_dtype,n_heads,n_kv", [(cw.CW_F32, 4, 2), (cw.CW_F16, 8, 2),
                                                   (cw.CW_F32, 2, 2), (cw.CW_F16, 8, 1)])
def test_fused_step_small_model(ctx, kv_dtype, n_heads, n_kv):
    """One persistent kernel per token: greedy ids equal the oracle's and the
    graph path's; the last step's logits agree with the graph path's to
    1e-4 of their range and with the oracle's to 1e-3 absolute."""
    P, N = 5, 24
    cfg = small128(P + N, kv_dtype, n_heads, n_kv)
    weights = cw.synthetic_weights(cfg, 77)
    prompt = cw.synth_tokens(cw.synth_key(77, "prompt"), P, cfg.vocab)
    m, o = build_pair(ctx, cfg, weights)
    ref, margins = o.generate(prompt, N)
    g = m.generate(prompt, N, mode=cw.STEP_GRAPH)
    lg = m.logits()
    f = m.generate(prompt, N, mode=cw.STEP_FUSED)
    lf = m.logits()
    assert np.array_equal(f, ref), (f, ref, margins)
    assert np.array_equal(g, ref)
    assert np.max(np.abs(lf - lg)) <= 1e-4 * np.max(np.abs(lg))
    # teacher-forced: the oracle's logits at the last fed position
    fed = list(prompt) + list(ref[:N - 1])
    o2 = orc.OracleModel(cfg, weights)
    for i, t in enumerate(fed):
        ol, _ = o2.step(int(t), i)
    assert np.max(np.abs(lf - ol)) <= LOGIT_TOL
    # a second fused run over the same positions gives the same bits
    f2 = m.generate(prompt, N, mode=cw.STEP_FUSED)
    assert np.array_equal(f2, f) and np.array_equal(m.logits(), lf)
    m.close()
    o.close()
    o2.close()


@FUSED_SKIP
def test_fused_step_unsupported_shape_is_an_error(ctx):
    cfg = cw.make_config(2, 64, 4, 2, 16, 128, 256, 12, cw.CW_F32, 1e-6, 1e6)
    import make_golden as mg
    m = cw.Model(ctx, cfg)
    m.set_weights(mg.tiny_weights())
    m.finalize()
    with pytest.raises(cw.CwError, match="head_dim must be 128"):
        m.generate(np.array([1, 5], np.uint32), 2, mode=cw.STEP_FUSED)
    m.close()


@FUSED_SKIP
def test_fused_qwen3_06b_token_loop(ctx):
    """Qwen3-0.6B shape through the fused step: identical greedy ids to the
    oracle over 32 prompt + 128 generated tokens (f32 KV)."""
    P, N = 32, 128
    cfg = qwen3_06b(P + N)
    weights = cw.synthetic_weights(cfg, 2024)
    prompt = cw.synth_tokens(cw.synth_key(2024, "prompt"), P, cfg.vocab)
    m, o = build_pair(ctx, cfg, weights)
    toks = m.generate(prompt, N, mode=cw.STEP_FUSED)
    ref, margins = o.generate(prompt, N)
    first_diff = np.nonzero(toks != ref)[0]
    msg = "" if not first_diff.size else (
        f"first divergence at step {first_diff[0]}: margin {margins[first_diff[0]]:.3e}")
    assert np.array_equal(toks, ref), msg
    m.close()
    o.close()


@FUSED_SKIP
def test_fused_qwen3_8b_decode_prefilled(ctx):
    """Qwen3-8B shape through the fused step from a 4096-position f16 cache:
    identical greedy ids to the oracle, and the last logits within 1e-3."""
    pre, N = 4096, 16
    cfg = qwen3_8b(pre + N)
    weights = cw.synthetic_weights(cfg, 8008)
    kv_n = cfg.n_layers * pre * cfg.n_kv_heads * cfg.head_dim
    k = cw.synth_normal_f16(cw.synth_key(8008, "kv.k"), kv_n)
    v = cw.synth_normal_f16(cw.synth_key(8008, "kv.v"), kv_n)
    start = cw.synth_tokens(cw.synth_key(8008, "start"), 1, cfg.vocab)
    m, o = build_pair(ctx, cfg, weights)
    m.prefill_kv(k, v, pre)
    o.prefill_kv(k, v, pre)
    toks = m.generate(start, N, start_pos=pre, mode=cw.STEP_FUSED)
    lf = m.logits()
    ref, margins = o.generate(start, N, start_pos=pre)
    first_diff = np.nonzero(toks != ref)[0]
    msg = "" if not first_diff.size else (
        f"first divergence at step {first_diff[0]}: margin {margins[first_diff[0]]:.3e}")
    assert np.array_equal(toks, ref), msg
    # the graph path over the same tokens ends with the same logits
    g = m.generate(start, N, start_pos=pre, mode=cw.STEP_GRAPH)
    assert np.array_equal(g, toks)
    lg = m.logits()
    print(f"\n[qwen3-8b fused] max |logit fused - graph| = {np.max(np.abs(lf - lg)):.3e}",
          flush=True)
    assert np.max(np.abs(lf - lg)) <= LOGIT_TOL
    m.close()
    o.close()
