"""The chat front end on the MI355X: LocalChat over a device model gives the
oracle model's greedy ids for the ChatML-framed prompt, cut at the first
end-of-turn id, and their decoded text (wasm.rs:56-117)."""
import numpy as np
import pytest

import chat
import cw
import oracle as orc
from tiny_tokenizer import tiny_tokenizer

pytestmark = pytest.mark.gpu


def expected_reply(oracle_ids, eos, max_tokens):
    out = []
    for t in oracle_ids[:max_tokens]:
        if int(t) in eos:
            break
        out.append(int(t))
    return out


@pytest.mark.parametrize("batched", [True, False])
def test_local_chat_matches_oracle(ctx, batched):
    tok = tiny_tokenizer()
    vocab = tok.get_vocab_size()
    max_tokens = 12
    lc0 = chat.LocalChat(None, tok)
    ids = lc0.prompt_ids("hello world", system="be brief")
    cfg = cw.make_config(2, 256, 4, 2, 128, 512, vocab, len(ids) + max_tokens, cw.CW_F16, 1e-6,
                         1e6)
    weights = cw.synthetic_weights(cfg, 51)
    m = cw.Model(ctx, cfg)
    m.set_weights(weights)
    m.finalize()
    o = orc.OracleModel(cfg, weights)
    ref, _ = o.generate(np.array(ids, np.uint32), max_tokens)
    lc = chat.LocalChat(m, tok)
    pieces = []
    text = lc.generate("hello world", system="be brief", max_tokens=max_tokens,
                       on_token=pieces.append, batched_prefill=batched)
    want = expected_reply(ref, lc.eos, max_tokens)
    print(f"\n[chat batched={batched}] prompt {len(ids)} ids, reply ids {lc.last_reply_ids}",
          flush=True)
    assert lc.last_prompt_ids == ids
    assert lc.last_reply_ids == want
    assert text == tok.decode(want, skip_special_tokens=True)
    # a second call on the same model starts again from position 0
    assert lc.generate("hello world", system="be brief", max_tokens=max_tokens,
                       batched_prefill=batched) == text
    m.close()
    o.close()


def test_generate_text_matches_oracle(ctx):
    tok = tiny_tokenizer()
    ids = chat.encode(tok, chat.chatml("the kernel"))
    cfg = cw.make_config(2, 256, 4, 2, 128, 512, tok.get_vocab_size(), len(ids) + 8, cw.CW_F16,
                         1e-6, 1e6)
    weights = cw.synthetic_weights(cfg, 52)
    m = cw.Model(ctx, cfg)
    m.set_weights(weights)
    m.finalize()
    o = orc.OracleModel(cfg, weights)
    p_ids, out, reply = chat.generate_text(m, tok, "the kernel", max_new=8)
    ref, _ = o.generate(np.array(ids, np.uint32), 8)
    assert p_ids == ids
    assert out == [int(t) for t in ref]
    assert reply == tok.decode(out, skip_special_tokens=True)
    m.close()
    o.close()
