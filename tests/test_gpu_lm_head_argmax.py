"""The argmax fused into the LM head's GEMV (argmax.wgsl:18-55, mod.rs:114-122)
on the decode step and on the batched prompt phase, through the C ABI.

The LM head is chosen so that the winning logit is tied across workgroups:
rows with bit-identical bytes give bit-identical logits wherever they sit in
the grid, so the merge over workgroups must keep the lowest index.  Some rows
carry NaN block scales (output.weight is loaded as given, without the finite
check of the layer projections), so their logits are NaN and must never win.
Each id the model returns is compared with cw_argmax over the downloaded
logits and with numpy's lowest-index argmax that ignores NaN.
"""
import numpy as np
import pytest

import cw

pytestmark = pytest.mark.gpu

VOCAB, DIM, NB = 32768, 256, 256 // 32
F16_NAN = np.uint16(0x7E00)


def block_bytes(nib):
    """[..., 32] nibbles -> [..., 16] GGUF Q4_0 bytes (element j low, j + 16 high)."""
    nib = nib.astype(np.uint8)
    return nib[..., :16] | (nib[..., 16:] << 4)


def lm_head(kind, rng):
    """(scales [VOCAB, NB] f16 bits, quants [VOCAB, NB, 16]) and the row sets."""
    pat_a = rng.integers(1, 16, size=(NB, 32))           # nibbles in [1, 15]
    pat_b = 16 - pat_a                                      # (q - 8) negated
    d = np.float16(0.05).view(np.uint16)
    if kind == "all_equal":
        s = np.full((VOCAB, NB), d, np.uint16)
        q = np.broadcast_to(block_bytes(pat_a), (VOCAB, NB, 16)).copy()
        return s, q, {}
    s = np.full((VOCAB, NB), np.float16(0.01).view(np.uint16), np.uint16)
    q = np.full((VOCAB, NB, 16), 0x88, np.uint8)            # q = 8: logits near 0
    sets = {"nan": np.arange(0, 8), "a": np.array([700, 4100, 20000, 32700]),
            "b": np.array([650, 9000, 25000, 32767])}
    for r in sets["a"]:
        s[r], q[r] = d, block_bytes(pat_a)
    for r in sets["b"]:
        s[r], q[r] = d, block_bytes(pat_b)
    s[sets["nan"], :] = F16_NAN
    q[sets["nan"]] = block_bytes(pat_a)
    return s, q, sets


def check_id(ctx, got, logits, sets):
    want = int(np.nanargmax(logits))
    dev = int(ctx.argmax(ctx.storage(logits), VOCAB).download()[0])
    print(f"\n[lm argmax] model {got}, cw_argmax {dev}, numpy {want}, "
          f"max {np.nanmax(logits):.6g}", flush=True)
    assert got == dev == want
    assert not np.isnan(logits[got])
    if sets:
        assert np.isnan(logits[sets["nan"]]).all()
        tied = [k for k in ("a", "b") if got in set(sets[k].tolist())]
        assert tied, got
        vals = logits[sets[tied[0]]]
        assert (vals == vals[0]).all()          # bit-identical across workgroups
        assert got == int(sets[tied[0]].min())  # the lowest index of the tie
    else:
        assert (logits == logits[0]).all() and got == 0


@pytest.mark.parametrize("kind", ["all_equal", "ties_and_nan"])
def test_lm_head_argmax_ties_across_workgroups(ctx, kind):
    rng = np.random.default_rng(515)
    cfg = cw.make_config(2, DIM, 4, 2, 128, 512, VOCAB, 16, cw.CW_F16, 1e-6, 1e6)
    w = cw.synthetic_weights(cfg, 31)
    s, q, sets = lm_head(kind, rng)
    w["output.weight"] = (s, q.reshape(VOCAB, NB * 16))
    m = cw.Model(ctx, cfg)
    m.set_weights(w)
    m.finalize()
    prompt = np.array([11, 4242, 77], np.uint32)
    print(f"\n[lm argmax] {kind}: prefill of {len(prompt)} then 3 decode steps", flush=True)
    got = m.prefill(prompt)
    check_id(ctx, got, m.logits(), sets)
    for _ in range(3):
        got = m.decode_next()
        check_id(ctx, got, m.logits(), sets)
    m.close()
