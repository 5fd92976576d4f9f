"""A Qwen3 model loaded from a GGUF file (cw_gguf_model_config +
cw_model_load_gguf, the Qwen3::load walk of src/model/qwen3.rs:44-100) runs
on the MI355X to the same tokens as the oracle model built from the oracle's
own reading of that file (oracle.OracleGguf), and to the same logits, bit for
bit, as the device model given the same arrays through cw_model_set_*.

The file mixes the dtypes a real Q4_0 export carries: Q4_0 projections
(repacked block for block), one projection stored as Q8_0 and an LM head
stored as Q6_K (both decoded and re-quantized to Q4_0), an F16 embedding and
F32 norm gains.
"""
import numpy as np
import pytest

import cw
import oracle as orc
import gguf_writer as gw

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3


def build_file(cfg, seed, head_dtype=None, q8_proj="blk.1.ffn_down.weight"):
    """A GGUF of a synthetic Qwen3: metadata of qwen3.rs:45-53, then every
    tensor under its GGUF name with dims [in, out] (ne0 fastest)."""
    w = gw.GgufWriter()
    w.add_meta("general.architecture", "str", "qwen3")
    for key, v in (("block_count", cfg.n_layers), ("embedding_length", cfg.dim),
                   ("attention.head_count", cfg.n_heads),
                   ("attention.head_count_kv", cfg.n_kv_heads),
                   ("attention.key_length", cfg.head_dim), ("feed_forward_length", cfg.hidden),
                   ("vocab_size", cfg.vocab)):
        w.add_meta(f"qwen3.{key}", "u32", v)
    w.add_meta("qwen3.attention.layer_norm_rms_epsilon", "f32", cfg.eps)
    w.add_meta("qwen3.rope.freq_base", "f32", cfg.rope_theta)
    rng = np.random.default_rng(seed)
    weights = cw.synthetic_weights(cfg, seed)
    for name, val in weights.items():
        if name == "token_embd.weight":
            w.add_tensor(name, [cfg.dim, cfg.vocab], gw.F16,
                         val.astype(np.float16).tobytes())
        elif isinstance(val, tuple):
            out_f, in_f = val[0].shape[0], val[0].shape[1] * 32
            if name == q8_proj:
                n = out_f * in_f
                d = np.abs(rng.normal(0, 0.0005, n // 32)).astype(np.float16).view(np.uint16)
                raw = gw.pack_q8_0(d, rng.integers(-128, 128, n).astype(np.int8))
                w.add_tensor(name, [in_f, out_f], gw.Q8_0, raw)
            else:
                w.add_tensor(name, [in_f, out_f], gw.Q4_0, gw.pack_q4_0(*val))
        else:
            w.add_tensor(name, [val.size], gw.F32, val.astype(np.float32).tobytes())
    if head_dtype == gw.Q6_K:
        n = cfg.vocab * cfg.dim
        d = np.full(n // 256, np.float16(0.0004).view(np.uint16), np.uint16)
        raw = gw.pack_q6_k(d, rng.integers(-64, 64, (n // 256, 16)).astype(np.int8),
                           rng.integers(0, 64, n).astype(np.uint8))
        w.add_tensor("output.weight", [cfg.dim, cfg.vocab], gw.Q6_K, raw)
    return w.tobytes()


def oracle_weights(cfg, data):
    """The oracle's reading of the file: Q4_0 blocks split, every other
    projection decoded and re-quantized (Proj::load, layers.rs:103-116)."""
    o = orc.OracleGguf(data)
    out = {}
    for raw_name in o.tensors:
        name = raw_name.decode()
        dtype, dims, n, raw = o.tensor_raw(name)
        if name.startswith("blk.") and len(dims) == 2 or name == "output.weight":
            in_f, out_f = dims
            if dtype == gw.Q4_0:
                blk = np.frombuffer(raw, np.uint8).reshape(-1, 18)
                out[name] = (blk[:, :2].copy().view(np.uint16).reshape(out_f, in_f // 32),
                             blk[:, 2:].reshape(out_f, in_f // 32, 16).copy())
            else:
                out[name] = orc.quantize_q4_0_gguf(o.tensor_f32(name).reshape(out_f, in_f))
        else:
            out[name] = o.tensor_f32(name)
    return out


def small_cfg(max_seq, kv_dtype=cw.CW_F16):
    return cw.make_config(2, 256, 4, 2, 128, 512, 1000, max_seq, kv_dtype, 1e-6, 1e6)


@pytest.mark.parametrize("head_dtype", [None, gw.Q6_K])
def test_gguf_model_generates_like_oracle(ctx, tmp_path, head_dtype):
    P, N = 9, 12
    cfg0 = small_cfg(P + N + 1)
    data = build_file(cfg0, 41, head_dtype)
    path = tmp_path / "qwen3-small.gguf"
    path.write_bytes(data)
    g = cw.Gguf(path=str(path))
    cfg = g.model_config(P + N + 1, cw.CW_F16)
    assert (cfg.n_layers, cfg.dim, cfg.vocab, cfg.head_dim) == (2, 256, 1000, 128)
    assert g.has("output.weight") == (head_dtype is not None)
    m = cw.Model(ctx, cfg)
    m.load_gguf(g)
    m.finalize()
    g.close()

    weights = oracle_weights(cfg, data)
    o = orc.OracleModel(cfg, weights)
    prompt = cw.synth_tokens(cw.synth_key(41, "prompt"), P, cfg.vocab)
    toks = m.generate(prompt, N, mode=cw.STEP_GRAPH)
    ref, _ = o.generate(prompt, N)
    print(f"\n[gguf head={head_dtype}] tokens {toks.tolist()}", flush=True)
    assert np.array_equal(toks, ref), (toks, ref)

    # the same arrays through cw_model_set_*: the very same device logits
    m2 = cw.Model(ctx, cfg)
    m2.set_weights(weights)
    m2.finalize()
    for pos, t in enumerate(prompt):
        a = m.step(int(t), pos)
        b = m2.step(int(t), pos)
        assert a == b
        la, lb = m.logits(), m2.logits()
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32)), pos
    ref_logits, _ = o.step(int(prompt[-1]), P - 1)
    assert float(np.max(np.abs(la - ref_logits))) <= LOGIT_TOL
    m.close()
    m2.close()
    o.close()


def test_gguf_model_prefill(ctx):
    """The batched prompt phase over a GGUF-loaded model, then graph decode."""
    P, N = 40, 6
    cfg0 = small_cfg(P + N + 1)
    data = build_file(cfg0, 42, gw.Q6_K)
    g = cw.Gguf(data=data)
    cfg = g.model_config(P + N + 1, cw.CW_F16)
    m = cw.Model(ctx, cfg)
    m.load_gguf(g)
    m.finalize()
    g.close()
    o = orc.OracleModel(cfg, oracle_weights(cfg, data))
    prompt = cw.synth_tokens(cw.synth_key(42, "prompt"), P, cfg.vocab)
    nxt = m.prefill(prompt)
    ref, _ = o.generate(prompt, N + 1)
    assert nxt == int(ref[0])
    m.decode_async(N, mode=cw.STEP_GRAPH)
    assert np.array_equal(m.tokens(N), ref[1:N + 1])
    m.close()
    o.close()


def test_gguf_model_shape_errors(ctx):
    cfg0 = small_cfg(8)
    data = build_file(cfg0, 43)
    g = cw.Gguf(data=data)
    other = cw.make_config(2, 256, 4, 2, 128, 1024, 1000, 8, cw.CW_F16)  # hidden differs
    m = cw.Model(ctx, other)
    with pytest.raises(cw.CwError, match="ffn_gate"):
        m.load_gguf(g)
    m.close()
    g.close()
    # a file without one layer tensor
    w = gw.GgufWriter()
    w.add_tensor("output_norm.weight", [256], gw.F32, np.ones(256, np.float32).tobytes())
    g = cw.Gguf(data=w.tobytes())
    m = cw.Model(ctx, cfg0)
    with pytest.raises(cw.CwError, match="missing tensor blk.0.attn_norm.weight"):
        m.load_gguf(g)
    m.close()
    g.close()
