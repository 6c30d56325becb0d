"""The tokenizer (host only; moert_tokenizer_*, replacing rust/moe-rt/src/tokenizador.rs) against the library that
defines a byte-level BPE tokenizer.json and generated the reference's golden ids: HF `tokenizers` (0.22), on
tokenizers trained here in the Granite configuration (ByteLevel pre-tokenizer without prefix space, BPE without
dropout, byte fallback or unknown token, ByteLevel decoder, special added tokens). The Granite tokenizer.json itself
is not available offline; the reference's own known answers (pre-tokenisation, byte map, date, chat template, odd
inputs) are checked as written in its tests (tokenizador.rs:626-676)."""
import json
import random

import pytest

import moert

tokenizers = pytest.importorskip("tokenizers")
from tokenizers import Tokenizer, decoders, models, pre_tokenizers, trainers  # noqa: E402

SPECIAL = ["<|end_of_text|>", "<|start_of_role|>", "<|end_of_role|>", "<|tool_call|>"]

CORPUS = [
    "Hello world! The quick brown fox jumps over the lazy dog. Don't you think it's great? I'll say we've done it.",
    "def main(x):\n    return x ** 2 + 3 * x - 1  # comment\n\tprint('done')\n",
    "Números: 1234567890, 3.14159, -42, 1e-9; preço R$ 1.234,56 — ação, coração, São Paulo.",
    "日本語のテキストと中文文本，还有한국어 텍스트。",
    "हिन्दी पाठ में मात्राएँ हैं। עברית עם ניקוד: שָׁלוֹם. العربية مع التشكيل: مَرْحَبًا",
    "Roman numerals Ⅰ Ⅱ Ⅻ ⅷ, circled Ⓐ ⓑ, superscripts x² y³, fractions ½ ¾, emoji 😀🚀👍🏽 and ZWJ 👨‍👩‍👧.",
    "Tabs\tand\nnewlines\r\nand   many    spaces nbsp　ideographic em.",
    "<|start_of_role|>user<|end_of_role|>Hi there!<|end_of_text|>\n<|start_of_role|>assistant<|end_of_role|>",
] * 4


def train(vocab=1500, full_alphabet=True):
    tok = Tokenizer(models.BPE())
    tok.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=True)
    tok.decoder = decoders.ByteLevel()
    kw = {"initial_alphabet": pre_tokenizers.ByteLevel.alphabet()} if full_alphabet else {}
    trainer = trainers.BpeTrainer(vocab_size=vocab, special_tokens=SPECIAL, show_progress=False, **kw)
    tok.train_from_iterator(CORPUS, trainer)
    return tok


@pytest.fixture(scope="module")
def pair():
    hf = train()
    return hf, moert.Tokenizer(json_text=hf.to_str())


def random_texts(seed, n):
    rng = random.Random(seed)
    pools = ["abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ", "0123456789", " \t\n\r 　 ",
             "!?.,;:'\"()[]{}<>|-_=+*/\\#@$%^&~`", "áéíóúçãõüñßøåÆŒ", "日本語中文한국어", "हिन्दीमात्राएँ", "שָׁלוֹםمَرْحَبًا",
             "ⅠⅡⅫⅷ²³½¾Ⓐⓑ", "😀🚀👍🏽‍", "́​‍﻿\U0010FFFF�"]
    words = ["'s", "'t", "'re", "'ve", "'m", "'ll", "'d", "'S", "'LL", " don't", "<|end_of_text|>", "<|start_of_role|>",
             "<|end_of_tex", "<|", "<|end_of_role|><|end_of_role|>"]
    out = []
    for _ in range(n):
        parts = []
        for _ in range(rng.randint(1, 12)):
            if rng.random() < 0.2:
                parts.append(rng.choice(words))
            else:
                pool = rng.choice(pools)
                parts.append("".join(rng.choice(pool) for _ in range(rng.randint(1, 6))))
        out.append("".join(parts))
    return out


def test_reference_pretokenization_known_answers():
    """tokenizador.rs:626-634."""
    assert moert.pretokenize("Hello world") == ["Hello", " world"]
    assert moert.pretokenize("don't I'll he's") == ["don", "'t", " I", "'ll", " he", "'s"]
    assert moert.pretokenize("a   b") == ["a", "  ", " b"]
    assert moert.pretokenize("a \n b") == ["a", " \n", " b"]
    assert moert.pretokenize("x  ") == ["x", "  "]
    assert moert.pretokenize(" 12ab!?") == [" 12", "ab", "!?"]
    assert moert.pretokenize("") == []


@pytest.mark.parametrize("seed", range(8))
def test_pretokenization_equals_the_library(seed):
    """Piece boundaries (in characters) equal the library's ByteLevel pre-tokenizer on random mixed-script text."""
    pt = pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=True)
    for text in random_texts(seed, 200):
        want = [e for _, (s, e) in pt.pre_tokenize_str(text)]
        got, pos = [], 0
        for piece in moert.pretokenize(text):
            pos += len(piece)
            got.append(pos)
        assert got == want, repr(text)


def test_encode_and_decode_equal_the_library_on_the_corpus_and_odd_inputs(pair):
    hf, t = pair
    odd = ["", "\u0000", "<", "<|", "<|end_of_tex", "\U0010FFFF", "�", "á", "\r\n\r\n", "​"]
    for text in CORPUS[:8] + odd:
        ids = t.encode(text)
        assert ids == hf.encode(text).ids, repr(text)
        assert t.decode_bytes(ids) == text.encode(), repr(text)  # the round trip of tokenizador.rs:666-671
        assert t.decode(ids) == hf.decode(ids, skip_special_tokens=False), repr(text)


@pytest.mark.parametrize("seed", range(6))
def test_encode_equals_the_library_on_random_text(pair, seed):
    """Random mixed-script text with contractions, special tokens and fragments of them, white-space runs of every
    kind, combining marks, numerals outside the decimal digits: ids equal the library's, bytes round-trip."""
    hf, t = pair
    for text in random_texts(100 + seed, 150):
        ids = t.encode(text)
        assert ids == hf.encode(text).ids, repr(text)
        assert t.decode_bytes(ids) == text.encode(), repr(text)


def test_bytes_outside_the_vocabulary_are_dropped_as_the_library_does():
    """A tokenizer trained without the full byte alphabet has no character for some bytes: the library (no unknown
    token) drops them, and so does this one."""
    hf = train(vocab=400, full_alphabet=False)
    t = moert.Tokenizer(json_text=hf.to_str())
    for text in ["ȸ unseen ☃ snowman", "Zebra QUIZ 🦓 ~`", "plain ascii that was seen"] + random_texts(7, 100):
        assert t.encode(text) == hf.encode(text).ids, repr(text)


def test_lossy_decode_replaces_maximal_invalid_subparts(pair):
    """decode() of an id sequence that splits a character: the whole byte string with each maximal invalid subpart
    replaced by U+FFFD, as Python's (and Rust's from_utf8_lossy) decoding does."""
    hf, t = pair
    ids = t.encode("😀 ação 日本")
    for cut in range(len(ids)):
        part = ids[:cut] + ids[cut + 1:]
        raw = t.decode_bytes(part)
        assert t.decode(part) == raw.decode("utf-8", errors="replace")


def test_loader_refuses_unsupported_configurations_and_sparse_ids(pair):
    """tokenizador.rs:228-282 and the sparse-id regression (tokenizador.rs:679-697)."""
    hf, _ = pair
    base = json.loads(hf.to_str())

    def refused(mutate, match=None):
        j = json.loads(json.dumps(base))
        mutate(j)
        with pytest.raises(moert.MoertError, match=match):
            moert.Tokenizer(json_text=json.dumps(j))

    refused(lambda j: j.__setitem__("normalizer", {"type": "NFC"}), "normalizer")
    refused(lambda j: j["pre_tokenizer"].__setitem__("add_prefix_space", True), "pre_tokenizer")
    refused(lambda j: j["pre_tokenizer"].__setitem__("use_regex", False), "pre_tokenizer")
    refused(lambda j: j.__setitem__("decoder", {"type": "Metaspace"}), "decoder")
    refused(lambda j: j["model"].__setitem__("dropout", 0.1), "dropout")
    refused(lambda j: j["model"].__setitem__("unk_token", "<unk>"), "unk_token")
    refused(lambda j: j["model"].__setitem__("byte_fallback", True), "byte_fallback")
    refused(lambda j: j["added_tokens"][0].__setitem__("lstrip", True), "added token")
    refused(lambda j: j["added_tokens"][0].__setitem__("id", 4294967295), None)
    first = next(iter(base["model"]["vocab"]))
    refused(lambda j: j["model"]["vocab"].__setitem__(first, 4294967295), "sparse")
    refused(lambda j: j["model"]["merges"].append(["Āzz", "q"]), "merge")
    for raw in ("{", "{}", "[]"):
        with pytest.raises(moert.MoertError):
            moert.Tokenizer(json_text=raw)
    with pytest.raises(moert.MoertError):
        moert.Tokenizer(path="/nonexistent/tokenizer.json")


def test_decode_refuses_unknown_ids_and_encode_invalid_utf8(pair):
    _, t = pair
    with pytest.raises(moert.MoertError):
        t.decode_bytes([2 ** 32 - 1])
    with pytest.raises(moert.MoertError):
        t.decode([t.vocab_size()])
    n = moert.ctypes.c_size_t()
    with pytest.raises(moert.MoertError, match="UTF-8"):
        moert.check(moert.lib().moert_tokenizer_encode(t.h, b"\xff\xfe", 2, None, 0, moert.ctypes.byref(n)))


def test_date_and_chat_template_known_answers():
    """tokenizador.rs:645-663."""
    assert moert.format_date(2026, 11, 7) == "November 07, 2026"
    assert moert.format_date(2024, 2, 29) == "February 29, 2024"
    for bad in ((2026, 2, 29), (2026, 13, 1), (2026, 4, 31), (0, 1, 1)):
        with pytest.raises(moert.MoertError):
            moert.format_date(*bad)
    with pytest.raises(moert.MoertError):
        moert.chat_render([], True, "x")
    r = moert.chat_render([(moert.ROLE_USER, "oi")], True, "November 07, 2026")
    assert r == ("<|start_of_role|>system<|end_of_role|>Knowledge Cutoff Date: April 2024.\nToday's Date: November 07, "
                 "2026.\nYou are Granite, developed by IBM. You are a helpful AI assistant.<|end_of_text|>\n"
                 "<|start_of_role|>user<|end_of_role|>oi<|end_of_text|>\n<|start_of_role|>assistant<|end_of_role|>")
    # a first system message replaces the default; the assistant's opening only after the last message
    r = moert.chat_render([(moert.ROLE_SYSTEM, "S"), (moert.ROLE_USER, "u"), (moert.ROLE_ASSISTANT, "a")], False, "")
    assert r == ("<|start_of_role|>system<|end_of_role|>S<|end_of_text|>\n<|start_of_role|>user<|end_of_role|>u"
                 "<|end_of_text|>\n<|start_of_role|>assistant<|end_of_role|>a<|end_of_text|>\n")
    r = moert.chat_render([(moert.ROLE_SYSTEM, "S")], True, "")
    assert r == "<|start_of_role|>system<|end_of_role|>S<|end_of_text|>\n"
