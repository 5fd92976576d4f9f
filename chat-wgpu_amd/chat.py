"""Chat front end over the device model: the Qwen3 ChatML frame, tokenizer
encode / decode, and greedy generation that stops at an end-of-turn token and
streams the decoded text piece by piece.

Mirrors LocalChat (src/wasm.rs:34-117) and the native example
(examples/generate.rs:49-60).  The tokenizer is the Hugging Face `tokenizers`
library at 0.22.2, the version the reference links (Cargo.lock pins
tokenizers 0.22.2), through its Python binding; it is loaded from a
tokenizer.json the caller supplies, as the reference does.  Sampling is greedy
like the reference's: its `temperature` argument is reserved and unused
(wasm.rs:57,63), and so it is here.

Every forward runs on the device through cw.Model (the batched prompt phase,
then one graph-replayed decode step per token); this module only frames text,
maps it to ids and back, and decides when to stop.
"""
from tokenizers import Tokenizer

# end-of-turn markers looked up in the tokenizer's vocabulary (wasm.rs:48-51)
EOS_TOKENS = ("<|im_end|>", "<|endoftext|>")


def chatml(prompt, system=None):
    """The Qwen3 ChatML frame of one user turn, optionally after a system turn
    (wasm.rs:66-71; generate.rs:50 is the frame without a system turn)."""
    text = ""
    if system is not None:
        text += f"<|im_start|>system\n{system}<|im_end|>\n"
    text += f"<|im_start|>user\n{prompt}<|im_end|>\n<|im_start|>assistant\n"
    return text


def load_tokenizer(src):
    """A Tokenizer from a tokenizer.json path, its bytes or its text
    (Tokenizer::from_file / from_bytes, generate.rs:34, wasm.rs:46); a
    Tokenizer is returned as is."""
    if isinstance(src, Tokenizer):
        return src
    if isinstance(src, (bytes, bytearray)):
        return Tokenizer.from_buffer(bytes(src))
    if isinstance(src, str) and src.lstrip().startswith("{"):
        return Tokenizer.from_str(src)
    return Tokenizer.from_file(str(src))


def encode(tokenizer, text):
    """Token ids of text, special tokens added (tokenizer.encode(text, true))."""
    return list(tokenizer.encode(text, add_special_tokens=True).ids)


class LocalChat:
    """A model and its tokenizer, generating replies to chat turns.

    `model` is a finalized cw.Model (or any object with the same
    prefill / step / cfg.max_seq interface); its KV cache is reused from
    position 0 by every call, as the reference builds a fresh cache per call.
    """

    def __init__(self, model, tokenizer):
        self.model = model
        self.tokenizer = load_tokenizer(tokenizer)
        self.eos = [i for i in (self.tokenizer.token_to_id(t) for t in EOS_TOKENS)
                    if i is not None]

    def prompt_ids(self, prompt, system=None):
        return encode(self.tokenizer, chatml(prompt, system))

    def generate(self, prompt, system=None, max_tokens=256, temperature=0.0, on_token=None,
                 batched_prefill=True):
        """The reply to one user turn (wasm.rs:56-117).

        Greedy: the prompt is run through the model, then each step takes
        the argmax id; an end-of-turn id stops the reply (it is not part of
        it), otherwise the id is appended, all ids so far are decoded with
        special tokens skipped, and the new suffix of that text is passed to
        `on_token`.  Returns the decoded reply.  `temperature` is accepted and
        ignored, like the reference's.  With batched_prefill the prompt goes
        through the batched prompt phase (the same cache and next id as the
        per-token loop the reference runs); otherwise through per-token steps.
        Raises ValueError when prompt + max_tokens exceed the model's cache.
        """
        del temperature  # reserved, as in the reference
        ids = self.prompt_ids(prompt, system)
        self.last_prompt_ids = ids
        max_seq = self.model.cfg.max_seq
        if len(ids) + max_tokens > max_seq:
            raise ValueError(f"prompt of {len(ids)} tokens + max_tokens {max_tokens} exceeds the "
                             f"model's {max_seq} cache positions")
        if batched_prefill:
            nxt = self.model.prefill(ids)
        else:
            for pos, t in enumerate(ids):
                nxt = self.model.step(t, pos)
        # after the batched prompt phase the decode state lives on the device:
        # each further token is one replay of the captured step (the
        # benchmarked path), whose argmax comes back as one 4-byte read
        graph = batched_prefill and hasattr(self.model, "decode_next")
        pos = len(ids)
        produced, shown = [], ""
        for i in range(max_tokens):
            if nxt in self.eos:
                break
            produced.append(nxt)
            full = self.tokenizer.decode(produced, skip_special_tokens=True)
            if len(full) > len(shown):
                piece = full[len(shown):]
                if on_token is not None:
                    on_token(piece)
                shown = full
            if i + 1 < max_tokens:  # the step after the last token would be unused
                if graph:
                    nxt = self.model.decode_next()
                else:
                    nxt = self.model.step(nxt, pos)
                pos += 1
        self.last_reply_ids = produced
        return shown


def generate_text(model, tokenizer, prompt, max_new=32):
    """The native example's flow (generate.rs:49-60): frame the prompt, run
    model.generate for max_new greedy ids (no end-of-turn stop, as
    model::generate has none), decode them with special tokens skipped.
    Returns (prompt ids, reply ids, reply text)."""
    tok = load_tokenizer(tokenizer)
    ids = encode(tok, chatml(prompt))
    out = [int(t) for t in model.generate(ids, max_new)]
    return ids, out, tok.decode(out, skip_special_tokens=True)
