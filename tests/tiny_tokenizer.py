"""A small byte-level BPE tokenizer (the Qwen tokenizer family's model type)
with the ChatML special tokens, trained in-process on a fixed corpus: test
infrastructure for the chat front end (no tokenizer.json ships with the
repository or the reference)."""
import random

from tokenizers import Tokenizer, decoders, models, pre_tokenizers, trainers

SPECIALS = ["<|endoftext|>", "<|im_start|>", "<|im_end|>"]
WORDS = ["the", "model", "token", "decode", "graph", "kernel", "cache", "wave", "tile", "stream",
         "user", "assistant", "system", "hello", "world", "é", "ü", "数据"]


def tiny_tokenizer(vocab_size=400, specials=SPECIALS, seed=7):
    tok = Tokenizer(models.BPE())
    tok.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False)
    tok.decoder = decoders.ByteLevel()
    tr = trainers.BpeTrainer(vocab_size=vocab_size, special_tokens=list(specials),
                             initial_alphabet=pre_tokenizers.ByteLevel.alphabet(),
                             show_progress=False)
    rng = random.Random(seed)
    corpus = [" ".join(rng.choice(WORDS) for _ in range(12)) for _ in range(400)]
    tok.train_from_iterator(corpus, tr)
    return tok
