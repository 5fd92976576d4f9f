"""Write the golden fixtures under tests/golden/ from the oracle.

Run from the repository root: `python tests/golden/make_golden.py`.

reference_kats.json  the literal known answers of the reference's own tests
                     (src/loader/dequant.rs:133-201, src/loader/gguf.rs:219-251,
                     src/main.rs:53-161),
                     transcribed as data with their citations.
q4_gemv_kat.npz      the q4_gemv KAT of src/main.rs:120-152 (in=256, out=512,
                     x = fill(0x1234), W = fill(0x5678), quantize_q4_0), with
                     the expected y of the reference's sequential CPU dot
                     (main.rs:133-150) and the same weights re-quantized to
                     GGUF Q4_0 with the GGUF-layout expectation.
tiny_qwen3.npz       the reference verify model shape (src/main.rs:165-191:
                     dim 64, 2 layers, 4/2 heads, hd 16, hidden 128, vocab 256)
                     with RandomWeights tensors (main.rs:209-266) re-quantized
                     to Q4_0, greedy generate of prompt [1,5,9,2] for 8 tokens.
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle as orc  # noqa: E402

KATS = {
    "f16_to_f32": {"source": "src/loader/dequant.rs:137-142",
                   "cases": [[0x3C00, 1.0], [0xC000, -2.0], [0x0000, 0.0]]},
    "bf16_to_f32": {"source": "src/loader/dequant.rs:145-148",
                    "cases": [[0x3F80, 1.0], [0xC000, -2.0]]},
    "q4_0_block": {"source": "src/loader/dequant.rs:190-200",
                   "d": 0x3C00, "byte": 8 | (15 << 4),
                   "expect": {"0": 0.0, "16": 7.0}},
    "q8_0_block": {"source": "src/loader/dequant.rs:150-161",
                   "d": 0x3800, "quants": "0..31", "expect": {"0": 0.0, "1": 0.5, "10": 5.0}},
    "q4_1_block": {"source": "src/loader/dequant.rs:163-173",
                   "d": 0x3C00, "m": 0x3800, "byte": 0 | (15 << 4),
                   "expect": {"0": 0.5, "16": 15.5}},
    "q6_k_zero_quants": {"source": "src/loader/dequant.rs:175-188",
                         "block_bytes": 210, "scales_at": [192, 208], "scale": 1,
                         "d": 0x3C00, "d_at": 208, "expect": {"0": -32.0, "255": -32.0}},
    "parse_minimal_gguf": {"source": "src/loader/gguf.rs:219-251",
                           "version": 3, "meta": {"qwen3.block_count": [4, 28]},
                           "tensor": {"name": "output_norm.weight", "dims": [4], "dtype": 0,
                                      "offset": 0, "data": [1.0, 2.0, 3.0, 4.0]},
                           "alignment": 32},
    "rmsnorm_ones": {"source": "src/main.rs:61-67", "rows": 4, "dim": 1024, "eps": 1e-6},
    "swiglu_const": {"source": "src/main.rs:77-82", "n": 4096, "g": 1.5, "u": -0.7},
    "rope_pos0": {"source": "src/main.rs:93-98", "rows": 16, "head_dim": 128, "theta": 10000.0},
    "attention_seq1": {"source": "src/main.rs:100-118", "n_heads": 4, "n_kv": 2, "head_dim": 16},
    "ewise_add": {"source": "src/main.rs:154-161", "n": 1000},
    "q4_gemv": {"source": "src/main.rs:120-152", "in_f": 256, "out_f": 512,
                "seed_x": 0x1234, "seed_w": 0x5678},
    "report_tolerance": {"source": "src/main.rs:268-273", "max_abs_err": 1e-3},
    "verify_model": {"source": "src/main.rs:165-191", "dim": 64, "n_layers": 2, "n_heads": 4,
                     "n_kv_heads": 2, "head_dim": 16, "hidden": 128, "vocab": 256,
                     "prompt": [1, 5, 9, 2], "max_new": 8, "eps": 1e-6, "rope_theta": 1e6},
}


class TinyCfg:
    n_layers, dim, n_heads, n_kv_heads, head_dim, hidden, vocab = 2, 64, 4, 2, 16, 128, 256
    eps, rope_theta, max_seq, kv_dtype = 1e-6, 1e6, 12, 0


def tiny_weights():
    """RandomWeights (main.rs:209-266): every tensor fill(seed(name)); the
    projections re-quantized to Q4_0 (what Proj::load does with quantize)."""
    c = TinyCfg
    q_dim, kv_dim = c.n_heads * c.head_dim, c.n_kv_heads * c.head_dim
    shapes = {"attn_q": (q_dim, c.dim), "attn_k": (kv_dim, c.dim), "attn_v": (kv_dim, c.dim),
              "attn_output": (c.dim, q_dim), "ffn_gate": (c.hidden, c.dim),
              "ffn_up": (c.hidden, c.dim), "ffn_down": (c.dim, c.hidden)}
    w = {}
    for i in range(c.n_layers):
        for v in ("attn_norm", "attn_q_norm", "attn_k_norm", "ffn_norm"):
            name = f"blk.{i}.{v}.weight"
            n = c.head_dim if v in ("attn_q_norm", "attn_k_norm") else c.dim
            w[name] = orc.fill(orc.fnv_seed(name), n)
        for p, (o, k) in shapes.items():
            name = f"blk.{i}.{p}.weight"
            w[name] = orc.quantize_q4_0_gguf(orc.fill(orc.fnv_seed(name), o * k).reshape(o, k))
    w["output_norm.weight"] = orc.fill(orc.fnv_seed("output_norm.weight"), c.dim)
    w["token_embd.weight"] = orc.fill(orc.fnv_seed("token_embd.weight"), c.vocab * c.dim)
    return w


def main():
    with open(os.path.join(HERE, "reference_kats.json"), "w") as f:
        json.dump(KATS, f, indent=1)

    x = orc.fill(0x1234, 256)
    w = orc.fill(0x5678, 512 * 256).reshape(512, 256)
    s, q = orc.quantize_q4_0(w)
    y = orc.q4_gemv_refmt(x, s, q, 256, 512)
    gs, gq = orc.quantize_q4_0_gguf(w)
    gy = orc.q4_gemv(x, gs, gq, 256, 512)
    np.savez_compressed(os.path.join(HERE, "q4_gemv_kat.npz"), x=x, ref_scales=s,
                        ref_quants=q, ref_y=y, gguf_scales=gs, gguf_quants=gq, gguf_y=gy)

    weights = tiny_weights()
    m = orc.OracleModel(TinyCfg, weights)
    toks, margins = m.generate(np.array([1, 5, 9, 2], np.uint32), 8)
    logits, _ = orc.OracleModel(TinyCfg, weights).step(1, 0)
    m.close()
    np.savez_compressed(os.path.join(HERE, "tiny_qwen3.npz"), tokens=toks, margins=margins,
                        logits_tok1_pos0=logits)
    print("tokens", toks.tolist())


if __name__ == "__main__":
    main()
