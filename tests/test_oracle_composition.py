"""Pins the oracle's Qwen3 forward / generate composition (oracle/cw_oracle.c
or_model_step_taps, or_generate; the reference's src/model/qwen3.rs:139-191
and src/model/mod.rs:57-125) with weights chosen so that the forward reduces
to a closed form or to a short chain of leaf functions the leaf tests already
pin.  Each case is built so that a plausible composition mistake fails it:

* a projection whose nibbles are all 8 contributes exactly zero, so a
  sublayer can be switched off and the residual stream checked bit for bit;
* at position 0 the softmax over one key is 1, so attention returns v under
  the GQA map (head h reads kv head h // (n_heads / n_kv));
* with q = 0 every score is 0, so attention is the mean of the V rows of
  positions 0..pos (seq = pos + 1), and an identity O projection exposes it;
* non-unit QK-norm gains separate "norm then rope" from "rope then norm" and a
  per-head norm (rows = n_heads) from a whole-vector one;
* the cache rows a step writes are read back: only row pos changes.

CPU only; the oracle is test infrastructure."""
import numpy as np
import pytest

import oracle as orc


class Cfg:
    # q_dim = n_heads * head_dim = dim, so an identity O projection exists
    n_layers, dim, n_heads, n_kv_heads, head_dim, hidden, vocab = 2, 64, 4, 2, 16, 96, 48
    eps, rope_theta, max_seq, kv_dtype = 1e-6, 1e6, 12, 0


C = Cfg
Q_DIM = C.n_heads * C.head_dim
KV_DIM = C.n_kv_heads * C.head_dim
HPK = C.n_heads // C.n_kv_heads
SHAPES = {"attn_q": (Q_DIM, C.dim), "attn_k": (KV_DIM, C.dim), "attn_v": (KV_DIM, C.dim),
          "attn_output": (C.dim, Q_DIM), "ffn_gate": (C.hidden, C.dim),
          "ffn_up": (C.hidden, C.dim), "ffn_down": (C.dim, C.hidden)}


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def rand_q4(rng, out_f, in_f):
    d = (np.abs(rng.standard_normal((out_f, in_f // 32))) * 0.1 + 0.01).astype(np.float16)
    q = rng.integers(0, 256, (out_f, in_f // 32, 16), dtype=np.uint8)
    return d.view(np.uint16), q


def eights_q4(rng, out_f, in_f):
    """Every nibble 8: each weight d * (8 - 8) = 0, so W x = 0 exactly."""
    d, _ = rand_q4(rng, out_f, in_f)
    return d, np.full((out_f, in_f // 32, 16), 0x88, np.uint8)


def identity_q4(n):
    """d = 1 and nibble 9 on the diagonal, 8 elsewhere: W = I exactly."""
    d = np.full((n, n // 32), 0x3C00, np.uint16)
    q = np.full((n, n // 32, 16), 0x88, np.uint8)
    for i in range(n):
        b, j = divmod(i, 32)
        if j < 16:
            q[i, b, j] = (q[i, b, j] & 0xF0) | 9
        else:
            q[i, b, j - 16] = (q[i, b, j - 16] & 0x0F) | (9 << 4)
    return d, q


def make_weights(rng, overrides=None):
    """Random Q4 projections and non-unit gains; overrides[(layer, name)]
    replaces one projection."""
    overrides = overrides or {}
    w = {}
    for i in range(C.n_layers):
        for nm in ("attn_norm", "ffn_norm"):
            w[f"blk.{i}.{nm}.weight"] = (1.0 + 0.3 * rng.standard_normal(C.dim)).astype(np.float32)
        for nm in ("attn_q_norm", "attn_k_norm"):
            w[f"blk.{i}.{nm}.weight"] = (1.0 + 0.5 * rng.standard_normal(C.head_dim)).astype(
                np.float32)
        for nm, (o, k) in SHAPES.items():
            w[f"blk.{i}.{nm}.weight"] = overrides.get((i, nm)) or rand_q4(rng, o, k)
    w["token_embd.weight"] = (0.5 * rng.standard_normal((C.vocab, C.dim))).astype(np.float32)
    w["output_norm.weight"] = (1.0 + 0.3 * rng.standard_normal(C.dim)).astype(np.float32)
    return w


def gemv(w, name, x):
    s, q = w[name]
    o, k = s.shape[0], s.shape[1] * 32
    return orc.q4_gemv(x, s, q, k, o)


def norm(x, g, rows):
    return orc.rmsnorm(x, g, rows, x.size // rows, C.eps)


def gqa_expand(v):
    """[n_kv][hd] -> [n_heads][hd]: head h takes kv head h // HPK."""
    return np.repeat(v.reshape(C.n_kv_heads, C.head_dim), HPK, axis=0).reshape(-1)


def model(w):
    return orc.OracleModel(C, w)


@pytest.fixture
def rng():
    return np.random.default_rng(20261202)


def test_switched_off_sublayers_leave_the_embedding(rng):
    """O and down projections all-8: post_attn and layer_out equal the
    embedding row bit for bit at every layer and position; the logits are the
    tied head (quantize_q4_0 of the embedding) applied to the final RMSNorm of
    that row."""
    ov = {}
    for i in range(C.n_layers):
        ov[(i, "attn_output")] = eights_q4(rng, C.dim, Q_DIM)
        ov[(i, "ffn_down")] = eights_q4(rng, C.dim, C.hidden)
    w = make_weights(rng, ov)
    m = model(w)
    emb = w["token_embd.weight"]
    head = orc.quantize_q4_0_gguf(emb)
    for pos, tok in enumerate([7, 0, 47, 7, 23]):
        logits, taps = m.step_taps(tok, pos)
        for layer in range(C.n_layers):
            assert np.array_equal(bits(taps["post_attn"][layer]), bits(emb[tok])), (pos, layer)
            assert np.array_equal(bits(taps["layer_out"][layer]), bits(emb[tok])), (pos, layer)
        normed = norm(emb[tok], w["output_norm.weight"], 1)
        expect = orc.q4_gemv(normed, head[0], head[1], C.dim, C.vocab)
        assert np.array_equal(bits(logits), bits(expect)), pos
        _, hidden = m.step(tok, pos)
        assert np.array_equal(bits(hidden), bits(normed))
    m.close()


def test_position0_attention_is_v_under_gqa(rng):
    """At position 0 attention over one key returns v, so post_attn = x +
    Wo gqa(Wv rmsnorm(x, attn_norm)) exactly; the down projection is off, so
    the next layer's input is that post_attn."""
    ov = {(i, "ffn_down"): eights_q4(rng, C.dim, C.hidden) for i in range(C.n_layers)}
    w = make_weights(rng, ov)
    m = model(w)
    tok = 11
    _, taps = m.step_taps(tok, 0)
    x = w["token_embd.weight"][tok]
    for layer in range(C.n_layers):
        p = f"blk.{layer}."
        v = gemv(w, p + "attn_v.weight", norm(x, w[p + "attn_norm.weight"], 1))
        expect = orc.add(x, gemv(w, p + "attn_output.weight", gqa_expand(v)))
        assert np.array_equal(bits(taps["post_attn"][layer]), bits(expect)), layer
        assert np.array_equal(bits(taps["layer_out"][layer]), bits(expect)), layer
        # a kv-head map of h % n_kv instead of h // HPK would differ here
        wrong = np.tile(v.reshape(C.n_kv_heads, C.head_dim), (HPK, 1)).reshape(-1)
        assert not np.array_equal(gqa_expand(v), wrong)
        x = expect
    m.close()


def test_qk_norm_then_rope_and_the_row_written(rng):
    """Non-unit gains at position 5: the "q" tap is RoPE(per-head RMSNorm(Wq
    x, q_norm, rows = n_heads)); cache row 5 holds RoPE(per-head RMSNorm(Wk x,
    k_norm, rows = n_kv)) and Wv x; every other row keeps what was there."""
    w = make_weights(rng)
    m = model(w)
    pre = 9
    kpre = rng.standard_normal((C.n_layers, pre, KV_DIM)).astype(np.float32)
    vpre = rng.standard_normal((C.n_layers, pre, KV_DIM)).astype(np.float32)
    m.prefill_kv(kpre, vpre, pre)
    pos, tok = 5, 30
    _, taps = m.step_taps(tok, pos)
    x = w["token_embd.weight"][tok]
    p = "blk.0."
    n = norm(x, w[p + "attn_norm.weight"], 1)
    q = gemv(w, p + "attn_q.weight", n)
    q_expect = orc.rope(norm(q, w[p + "attn_q_norm.weight"], C.n_heads), C.n_heads, C.head_dim,
                        pos, C.rope_theta)
    assert np.array_equal(bits(taps["q"][0]), bits(q_expect))
    # the orders and row counts a composition mistake would use differ
    rope_first = norm(orc.rope(q, C.n_heads, C.head_dim, pos, C.rope_theta),
                      w[p + "attn_q_norm.weight"], C.n_heads)
    one_row = orc.rope(orc.rmsnorm(q, np.tile(w[p + "attn_q_norm.weight"], C.n_heads), 1, Q_DIM,
                                   C.eps), C.n_heads, C.head_dim, pos, C.rope_theta)
    assert np.max(np.abs(rope_first - q_expect)) > 1e-3
    assert np.max(np.abs(one_row - q_expect)) > 1e-3
    k = gemv(w, p + "attn_k.weight", n)
    k_expect = orc.rope(norm(k, w[p + "attn_k_norm.weight"], C.n_kv_heads), C.n_kv_heads,
                        C.head_dim, pos, C.rope_theta)
    v_expect = gemv(w, p + "attn_v.weight", n)
    for layer in range(C.n_layers):
        for r in range(pre):
            kr, vr = m.kv_row(layer, r)
            if r == pos:
                continue
            assert np.array_equal(bits(kr), bits(kpre[layer, r])), (layer, r)
            assert np.array_equal(bits(vr), bits(vpre[layer, r])), (layer, r)
    kr, vr = m.kv_row(0, pos)
    assert np.array_equal(bits(kr), bits(k_expect))
    assert np.array_equal(bits(vr), bits(v_expect))
    m.close()


@pytest.mark.parametrize("pos", [1, 4, 10])
def test_zero_query_attention_is_the_mean_of_v(rng, pos):
    """q = 0 (Wq all-8) makes every score 0, so each head's attention output
    is the mean of its kv head's V rows over positions 0..pos, the new row
    (Wv x at pos) included.  An identity O projection puts that mean into
    post_attn - x.  Wrong sequence lengths (pos, pos + 2), rows or kv-head
    maps give other means."""
    ov = {(0, "attn_q"): eights_q4(rng, Q_DIM, C.dim),
          (0, "attn_output"): identity_q4(C.dim),
          (0, "ffn_down"): eights_q4(rng, C.dim, C.hidden)}
    w = make_weights(rng, ov)
    m = model(w)
    n_pre = C.max_seq
    kpre = rng.standard_normal((C.n_layers, n_pre, KV_DIM)).astype(np.float32)
    vpre = (rng.standard_normal((C.n_layers, n_pre, KV_DIM)) +
            np.repeat(np.arange(C.n_kv_heads) * 3.0, C.head_dim)).astype(np.float32)
    m.prefill_kv(kpre, vpre, n_pre)
    tok = 19
    _, taps = m.step_taps(tok, pos)
    x = w["token_embd.weight"][tok]
    vnew = gemv(w, "blk.0.attn_v.weight", norm(x, w["blk.0.attn_norm.weight"], 1))
    rows = np.concatenate([vpre[0, :pos].astype(np.float64), vnew[None].astype(np.float64)])
    expect = gqa_expand(rows.mean(axis=0))
    got = taps["post_attn"][0].astype(np.float64) - x.astype(np.float64)
    assert np.max(np.abs(got - expect)) < 1e-5, np.max(np.abs(got - expect))
    for wrong in (vpre[0, :pos].mean(axis=0),                      # seq = pos
                  np.concatenate([rows, vpre[0, pos + 1:pos + 2]]).mean(axis=0)):  # pos + 2
        assert np.max(np.abs(got - gqa_expand(wrong))) > 1e-3
    m.close()


def test_ffn_composition(rng):
    """O projection off: layer_out = post_attn + Wdown swiglu(Wgate n, Wup n)
    with n = rmsnorm(post_attn, ffn_norm), bit for bit, chained over the two
    layers (layer 1 reads layer 0's output)."""
    ov = {(i, "attn_output"): eights_q4(rng, C.dim, Q_DIM) for i in range(C.n_layers)}
    w = make_weights(rng, ov)
    m = model(w)
    for pos, tok in enumerate([3, 44]):
        _, taps = m.step_taps(tok, pos)
        x = w["token_embd.weight"][tok]
        for layer in range(C.n_layers):
            p = f"blk.{layer}."
            assert np.array_equal(bits(taps["post_attn"][layer]), bits(x))
            n = norm(x, w[p + "ffn_norm.weight"], 1)
            act = orc.swiglu(gemv(w, p + "ffn_gate.weight", n), gemv(w, p + "ffn_up.weight", n))
            expect = orc.add(x, gemv(w, p + "ffn_down.weight", act))
            assert np.array_equal(bits(taps["layer_out"][layer]), bits(expect)), (pos, layer)
            # silu(up) * gate instead would differ
            swapped = orc.swiglu(gemv(w, p + "ffn_up.weight", n), gemv(w, p + "ffn_gate.weight", n))
            assert not np.array_equal(bits(act), bits(swapped))
            x = expect
    m.close()


def test_generate_runs_prompt_plus_new_minus_one_forwards(rng):
    """generate(prompt of P, N new) from start_pos s runs P + N - 1 forwards:
    cache rows s .. s+P+N-2 are written and row s+P+N-1 is not; the prompt
    is fed in order, then each produced token at the next position; the
    first produced token is the argmax after the last prompt position."""
    w = make_weights(rng)
    P, N, s = 3, 4, 2
    prompt = np.array([5, 17, 40], np.uint32)
    sentinel = np.full((C.n_layers, C.max_seq, KV_DIM), 123.0, np.float32)
    m = model(w)
    m.prefill_kv(sentinel, sentinel, C.max_seq)
    toks, _ = m.generate(prompt, N, start_pos=s)
    assert len(toks) == N
    for layer in range(C.n_layers):
        for r in range(C.max_seq):
            kr, _ = m.kv_row(layer, r)
            written = not np.all(kr == 123.0)
            assert written == (s <= r < s + P + N - 1), (layer, r)
    # explicit steps over the same cache contents give the same rows and ids
    e = model(w)
    e.prefill_kv(sentinel, sentinel, C.max_seq)
    fed = list(prompt) + list(toks[:N - 1])
    for i, t in enumerate(fed):
        logits, _ = e.step(int(t), s + i)
        if i >= P - 1:
            assert orc.argmax(logits) == toks[i - (P - 1)], i
    for layer in range(C.n_layers):
        for r in range(C.max_seq):
            assert np.array_equal(bits(m.kv_row(layer, r)[0]), bits(e.kv_row(layer, r)[0]))
            assert np.array_equal(bits(m.kv_row(layer, r)[1]), bits(e.kv_row(layer, r)[1]))
    m.close()
    e.close()
