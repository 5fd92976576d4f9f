"""Hook taps (src/model/mod.rs:158-165; qwen3.rs:165,180,188; main.rs's
Capture hook, main.rs:193-207) of the device decode step against the
oracle's forward: "q" after QK-norm and RoPE, "post_attn" after the
attention residual, "layer_out" after the FFN residual, per layer."""
import numpy as np
import pytest

import cw
import oracle as orc

pytestmark = pytest.mark.gpu

REL_TOL = 1e-4


def small(max_seq):
    return cw.make_config(2, 256, 4, 2, 128, 512, 1000, max_seq, cw.CW_F16, 1e-6, 1e6)


def build(ctx, cfg, seed):
    weights = cw.synthetic_weights(cfg, seed)
    m = cw.Model(ctx, cfg)
    m.set_weights(weights)
    m.finalize()
    return m, orc.OracleModel(cfg, weights)


def check_taps(m, ref_taps, where):
    for name in cw.Model.TAP_NAMES:
        for layer in range(m.cfg.n_layers):
            got, ref = m.tap(name, layer), ref_taps[name][layer]
            err = float(np.max(np.abs(got - ref)) / np.max(np.abs(ref)))
            assert err <= REL_TOL, (where, name, layer, err)


def test_taps_match_oracle_each_step(ctx):
    P = 10
    m, o = build(ctx, small(P + 2), 61)
    m.set_taps(True)
    prompt = cw.synth_tokens(cw.synth_key(61, "prompt"), P, m.cfg.vocab)
    for pos, t in enumerate(prompt):
        m.step(int(t), pos)
        _, taps = o.step_taps(int(t), pos)
        check_taps(m, taps, pos)
    m.close()
    o.close()


def test_taps_after_graph_decode(ctx):
    """Prompt phase, then N graph-replayed steps: the taps are those of the
    last step's forward (position P + N - 1, input the (N-1)-th produced
    token)."""
    P, N = 12, 6
    m, o = build(ctx, small(P + N + 1), 62)
    m.set_taps(True)
    prompt = cw.synth_tokens(cw.synth_key(62, "prompt"), P, m.cfg.vocab)
    nxt = m.prefill(prompt)
    m.decode_async(N, mode=cw.STEP_GRAPH)
    toks = m.tokens(N)
    for pos, t in enumerate(prompt):
        o.step(int(t), pos)
    inputs = [nxt] + [int(t) for t in toks[:N - 1]]
    for k, t in enumerate(inputs[:-1]):
        o.step(t, P + k)
    _, taps = o.step_taps(inputs[-1], P + N - 1)
    check_taps(m, taps, "graph")
    m.close()
    o.close()


def test_taps_leave_results_unchanged_and_errors(ctx):
    P = 6
    m, o = build(ctx, small(P + 4), 63)
    prompt = cw.synth_tokens(cw.synth_key(63, "prompt"), P, m.cfg.vocab)
    with pytest.raises(cw.CwError, match="taps are off"):
        m.tap("q", 0)
    plain = []
    for pos, t in enumerate(prompt):
        m.step(int(t), pos)
        plain.append(m.logits())
    m.set_taps(True)
    for pos, t in enumerate(prompt):
        m.step(int(t), pos)
        assert np.array_equal(m.logits().view(np.uint32), plain[pos].view(np.uint32)), pos
    with pytest.raises(cw.CwError, match="unknown tap"):
        m.tap("attn", 0)
    with pytest.raises(cw.CwError, match="layer 2"):
        m.tap("q", 2)
    # taps off again: the graph step is captured without them and agrees
    m.set_taps(False)
    toks_off = m.generate(prompt, 4)
    m.set_taps(True)
    toks_on = m.generate(prompt, 4)
    assert np.array_equal(toks_off, toks_on)
    m.close()
    o.close()


def test_taps_of_batched_prompt_phase(ctx):
    """cw_model_prefill with taps on leaves the taps of the last prompt
    position's forward, as the per-token loop's last step would."""
    P = 20
    m, o = build(ctx, small(P + 2), 64)
    m.set_taps(True)
    prompt = cw.synth_tokens(cw.synth_key(64, "prompt"), P, m.cfg.vocab)
    m.prefill(prompt)
    for pos, t in enumerate(prompt[:-1]):
        o.step(int(t), pos)
    _, taps = o.step_taps(int(prompt[-1]), P - 1)
    check_taps(m, taps, "prefill")
    m.close()
    o.close()
