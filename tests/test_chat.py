"""Chat front end host logic (wasm.rs:56-117, generate.rs:49-60) on the CPU:
the ChatML frame, the end-of-turn ids, the greedy loop's stop / streaming /
position bookkeeping, against a scripted stand-in for the device model."""
import types

import pytest

import chat
from tiny_tokenizer import tiny_tokenizer


class ScriptedModel:
    """prefill / step / generate with a fixed sequence of next ids; records
    what it was fed."""

    def __init__(self, script, max_seq=64):
        self.script = list(script)
        self.cfg = types.SimpleNamespace(max_seq=max_seq)
        self.fed = []       # (token, pos) of every step
        self.prefilled = None
        self.k = 0

    def _next(self):
        v = self.script[self.k]
        self.k += 1
        return v

    def prefill(self, ids):
        self.prefilled = list(ids)
        return self._next()

    def step(self, token, pos):
        self.fed.append((int(token), int(pos)))
        return self._next()

    def generate(self, ids, max_new):
        self.prefilled = list(ids)
        return self.script[:max_new]


@pytest.fixture(scope="module")
def tok():
    return tiny_tokenizer()


def test_chatml_frame():
    assert chat.chatml("hi") == "<|im_start|>user\nhi<|im_end|>\n<|im_start|>assistant\n"
    assert chat.chatml("hi", system="be brief") == (
        "<|im_start|>system\nbe brief<|im_end|>\n"
        "<|im_start|>user\nhi<|im_end|>\n<|im_start|>assistant\n")


def test_eos_ids(tok):
    lc = chat.LocalChat(ScriptedModel([]), tok)
    assert lc.eos == [tok.token_to_id("<|im_end|>"), tok.token_to_id("<|endoftext|>")]
    plain = tiny_tokenizer(specials=["<|im_start|>"])
    assert chat.LocalChat(ScriptedModel([]), plain).eos == []


def test_prompt_encoding_keeps_special_tokens(tok):
    lc = chat.LocalChat(ScriptedModel([]), tok)
    ids = lc.prompt_ids("hello world")
    assert ids[0] == tok.token_to_id("<|im_start|>")
    assert ids.count(tok.token_to_id("<|im_end|>")) == 1
    assert tok.decode(ids, skip_special_tokens=False) == chat.chatml("hello world")


def word_ids(tok, text):
    return tok.encode(text, add_special_tokens=False).ids


def test_generate_stops_at_eos_and_streams(tok):
    body = word_ids(tok, "hello world the model")
    eos = tok.token_to_id("<|im_end|>")
    m = ScriptedModel(body + [eos, 5, 6])
    lc = chat.LocalChat(m, tok)
    pieces = []
    text = lc.generate("hello", max_tokens=20, on_token=pieces.append)
    P = len(lc.last_prompt_ids)
    assert m.prefilled == lc.last_prompt_ids
    assert lc.last_reply_ids == body
    assert text == "hello world the model" == "".join(pieces)
    # each produced id is fed back at the next position; nothing after the stop
    assert m.fed == [(t, P + i) for i, t in enumerate(body)]


def test_endoftext_also_stops(tok):
    body = word_ids(tok, "cache wave")
    m = ScriptedModel(body + [tok.token_to_id("<|endoftext|>")])
    assert chat.LocalChat(m, tok).generate("x", max_tokens=10) == "cache wave"


def test_generate_max_tokens_without_eos(tok):
    body = word_ids(tok, "the model the model the model")
    m = ScriptedModel(body)
    lc = chat.LocalChat(m, tok)
    text = lc.generate("x", max_tokens=4)
    assert lc.last_reply_ids == body[:4]
    assert text == tok.decode(body[:4], skip_special_tokens=True)
    assert len(m.fed) == 3  # no step after the last kept id


def test_eos_first_gives_empty_reply(tok):
    m = ScriptedModel([tok.token_to_id("<|im_end|>")])
    pieces = []
    assert chat.LocalChat(m, tok).generate("x", max_tokens=5, on_token=pieces.append) == ""
    assert pieces == [] and m.fed == []


def test_per_token_prompt_phase(tok):
    eos = tok.token_to_id("<|im_end|>")

    class StepOnly(ScriptedModel):
        def step(self, token, pos):
            self.fed.append((int(token), int(pos)))
            return self.script[len(self.fed) - 1]

    lc0 = chat.LocalChat(ScriptedModel([]), tok)
    P = len(lc0.prompt_ids("hi"))
    body = word_ids(tok, "graph kernel")
    m = StepOnly([0] * (P - 1) + body + [eos])
    text = chat.LocalChat(m, tok).generate("hi", max_tokens=8, batched_prefill=False)
    assert text == "graph kernel"
    assert [p for _, p in m.fed] == list(range(P + len(body)))


def test_cache_limit(tok):
    m = ScriptedModel([1, 2, 3], max_seq=12)
    with pytest.raises(ValueError, match="cache positions"):
        chat.LocalChat(m, tok).generate("hello world", max_tokens=8)


def test_multibyte_reply_is_the_full_decode(tok):
    # byte-level pieces of a multi-byte character: the reply is the decode of
    # all ids, whatever the partial decodes streamed
    body = word_ids(tok, "数据 é ü")
    m = ScriptedModel(body + [tok.token_to_id("<|im_end|>")])
    assert chat.LocalChat(m, tok).generate("x", max_tokens=40) == "数据 é ü"


def test_generate_text_flow(tok):
    body = word_ids(tok, "stream tile")
    m = ScriptedModel(body)
    ids, out, reply = chat.generate_text(m, tok, "hello", max_new=len(body))
    assert ids == chat.encode(tok, chat.chatml("hello")) == m.prefilled
    assert out == body and reply == "stream tile"


def test_load_tokenizer_forms(tok, tmp_path):
    js = tok.to_str()
    p = tmp_path / "tokenizer.json"
    p.write_text(js)
    text = chat.chatml("hello world")
    want = tok.encode(text).ids
    for src in (js, js.encode(), str(p), tok):
        assert chat.load_tokenizer(src).encode(text).ids == want


class ScriptedDeviceLoop(ScriptedModel):
    """A stand-in that also has the device decode loop: after prefill the
    state is (next id, position) on the "device"; decode_next() feeds that
    id at that position and returns the next id."""

    def prefill(self, ids):
        nxt = super().prefill(ids)
        self.state = (nxt, len(ids))
        return nxt

    def decode_next(self):
        token, pos = self.state
        self.fed.append((int(token), int(pos)))
        nxt = self._next()
        self.state = (nxt, pos + 1)
        return nxt

    def step(self, token, pos):  # never used after a batched prompt phase
        raise AssertionError("eager step after the batched prompt phase")


def test_graph_loop_after_batched_prompt(tok):
    """After the batched prompt phase every reply token comes from one
    replay of the device step, fed the previous id at the next position."""
    a, b = tok.token_to_id("a"), tok.token_to_id("b")
    eos = tok.token_to_id("<|im_end|>")
    m = ScriptedDeviceLoop([a, b, a, eos, b])
    lc = chat.LocalChat(m, tok)
    text = lc.generate("x", max_tokens=8)
    n = len(lc.last_prompt_ids)
    assert lc.last_reply_ids == [a, b, a]
    assert text == "aba"
    assert m.fed == [(a, n), (b, n + 1), (a, n + 2)]
    # the per-token prompt path keeps the eager steps
    m2 = ScriptedModel([a] * len(lc.last_prompt_ids) + [b, eos])
    assert chat.LocalChat(m2, tok).generate("x", max_tokens=8, batched_prefill=False) == "ab"
