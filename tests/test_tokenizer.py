"""The tokenizer and stream decoder (src/tokenizer.rs) in the library, on the CPU.

Pinned by: the reference's own unit-test vectors (pre-token pieces, the byte table, its tiny
vocabulary with two merges, the stream decoder); the Qwen2 split pattern run by an independent
regex engine (HF `tokenizers`, with the true \\p{L} and \\p{N} classes) on the reference's golden
texts and on extra text; and byte-level BPE against HF `tokenizers` with a vocabulary trained here
on the golden texts (the real Qwen2.5 vocabulary files are not in this image, so the golden ids
themselves are checked only when LS_QWEN_TOKENIZER_DIR names a directory holding them; otherwise
that test says it skipped)."""
import json
import os

import numpy as np
import pytest

import layerstream_amd as LS

HERE = os.path.dirname(os.path.abspath(__file__))
QWEN_PATTERN = r"""(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}| ?[^\s\p{L}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+"""
SPECIALS = {"151643": "<|endoftext|>", "151644": "<|im_start|>", "151645": "<|im_end|>"}


def golden_texts():
    with open(os.path.join(HERE, "golden", "qwen_tokenizer_cases.json")) as f:
        return json.load(f)["cases"]


EXTRA = [
    "Hello, world!", "  spaces  and\ttabs\n", "Café 日本語 😀", "def f(x):\n    return x", "a  b", "x \n y", "trailing   ",
    "!!word", "!word", "end.\n\nNext", "WE'RE HERE, they'LL see", "Ünïcödé: naïve façade", "数字 123 ٣٤٥ Ⅻ ½",
    "\r\n\r\nwindows lines\r\n", "tab\t\tand   nbsp", "emoji 👍🏽 zwj 👨‍👩‍👧", "$100.00 + 50% = ?", "'s 't 're 've 'm 'll 'd 'x",
    "", " ", "\n", "a", "3.14159", "<html><body>text</body></html>", "mixed123abc456",
]


def test_pretoken_pieces_match_the_reference_vectors():
    # src/tokenizer.rs:454-463
    assert LS.pretokens("Hello, world!") == ["Hello", ",", " world", "!"]
    assert LS.pretokens("I'm sure it's 2024") == ["I", "'m", " sure", " it", "'s", " ", "2", "0", "2", "4"]
    assert LS.pretokens("a  b") == ["a", " ", " b"]
    assert LS.pretokens("end.\n\nNext") == ["end", ".\n\n", "Next"]
    assert LS.pretokens("x \n y") == ["x", " \n", " y"]
    assert LS.pretokens("trailing   ") == ["trailing", "   "]
    assert LS.pretokens("!!word") == ["!!", "word"]
    assert LS.pretokens("!word") == ["!word"]


def test_pretoken_split_matches_an_independent_regex_engine():
    from tokenizers import Regex, pre_tokenizers

    split = pre_tokenizers.Split(Regex(QWEN_PATTERN), behavior="isolated", invert=False)
    texts = [c["text"] for c in golden_texts()] + EXTRA
    for text in texts:
        want = [p for p, _ in split.pre_tokenize_str(text)]
        assert LS.pretokens(text) == want, text


def test_stream_decoder_waits_for_complete_characters():
    # src/tokenizer.rs:466-474
    d = LS.StreamDecoder()
    smile = "😀".encode()
    assert d.push(smile[:2]) == ""
    assert d.push(smile[2:]) == "😀"
    assert d.push(b"ab") == "ab"
    assert d.push(bytes([0xFF])) == "�"
    assert d.finish() == ""
    # a cut-short sequence left at the end becomes one replacement
    d = LS.StreamDecoder()
    assert d.push("é".encode()[:1]) == ""
    assert d.finish() == "�"
    # invalid bytes between valid ones: each maximal invalid part is one replacement
    for data in (b"a\xe2\x82b", b"\xf0\x9f\x98\x80\xc3", b"\xed\xa0\x80x", b"\xc0\xaf", b"ok"):
        d = LS.StreamDecoder()
        got = d.push(data) + d.finish()
        assert got == data.decode("utf-8", errors="replace"), data


def byte_table():
    keep = list(range(0x21, 0x7F)) + list(range(0xA1, 0xAD)) + list(range(0xAE, 0x100))
    cps = dict((b, b) for b in keep)
    n = 0
    for b in range(256):
        if b not in cps:
            cps[b] = 256 + n
            n += 1
    return {b: chr(c) for b, c in cps.items()}


def write_files(d, vocab, merges, added):
    with open(os.path.join(d, "vocab.json"), "w", encoding="utf-8") as f:
        json.dump(vocab, f, ensure_ascii=False)
    with open(os.path.join(d, "merges.txt"), "w", encoding="utf-8") as f:
        f.write("#version: 0.2\n" + "".join(f"{a} {b}\n" for a, b in merges))
    with open(os.path.join(d, "tokenizer_config.json"), "w", encoding="utf-8") as f:
        json.dump({"added_tokens_decoder": {str(i): {"content": c, "special": s} for i, (c, s) in added.items()}}, f)


def test_tiny_vocabulary_with_two_merges(tmp_path):
    """src/tokenizer.rs:489-513: the 256 byte tokens, 'hi' and 'hihi', one special token."""
    t = byte_table()
    vocab = {t[b]: b for b in range(256)}
    h, i = t[ord("h")], t[ord("i")]
    vocab[h + i] = 256
    vocab[h + i + h + i] = 257
    write_files(tmp_path, vocab, [(h, i), (h + i, h + i)], {300: ("<|x|>", True)})
    tok = LS.Tokenizer(str(tmp_path))
    assert tok.encode("hihi") == [257]
    assert tok.encode("hihihi") == [257, 256]
    assert tok.encode("hi") == [256]
    assert tok.encode("h") == [ord("h")]
    assert tok.encode("a<|x|>hi") == [ord("a"), 300, 256]
    assert tok.decode(tok.encode("hihihi")) == "hihihi"
    assert tok.token_id("<|x|>") == 300
    assert tok.token_id("nonexistent token") is None
    assert tok.is_special(300) and not tok.is_special(256)
    assert tok.token_bytes(300) == b"" and tok.token_bytes(300, True) == b"<|x|>"
    # the byte table: a bijection onto printable characters, 'A' itself, ' ' -> 'Ġ', '\n' -> 'Ċ'
    assert len(set(t.values())) == 256 and t[ord("A")] == "A" and t[ord(" ")] == "Ġ" and t[ord("\n")] == "Ċ"
    assert tok.encode(" \n") == [ord(" "), ord("\n")]
    assert tok.decode([ord(" "), ord("\n"), 256]) == " \nhi"


def test_files_and_text_errors(tmp_path):
    with pytest.raises(LS.LayerstreamError) as e:
        LS.Tokenizer(str(tmp_path))
    assert e.value.code == -3
    t = byte_table()
    write_files(tmp_path, {t[b]: b for b in range(255)}, [], {})  # a byte token missing
    with pytest.raises(LS.LayerstreamError) as e:
        LS.Tokenizer(str(tmp_path))
    assert e.value.code == -2
    write_files(tmp_path, {t[b]: b for b in range(256)}, [], {})
    tok = LS.Tokenizer(str(tmp_path))
    n = LS.C.c_size_t(0)
    bad = b"ab\xff"
    assert LS.lib().ls_tokenizer_encode(tok.h, bad, len(bad), None, 0, LS.C.byref(n)) == -1


@pytest.fixture(scope="module")
def trained(tmp_path_factory):
    """A byte-level BPE vocabulary trained by HF tokenizers on the golden texts (and some more),
    with the Qwen2 split and three added special tokens, saved as vocab.json + merges.txt."""
    from tokenizers import Regex, Tokenizer, decoders, models, pre_tokenizers, trainers

    d = str(tmp_path_factory.mktemp("bpe"))
    hf = Tokenizer(models.BPE())
    hf.pre_tokenizer = pre_tokenizers.Sequence(
        [pre_tokenizers.Split(Regex(QWEN_PATTERN), behavior="isolated", invert=False), pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)]
    )
    hf.decoder = decoders.ByteLevel()
    corpus = [c["text"] for c in golden_texts()] + EXTRA
    rng = np.random.default_rng(11)
    words = ["the", "speculative", "decoding", "verify", "layer", "stream", "token", "Paris", "model", "über", "naïve", "日本"]
    corpus += [" ".join(rng.choice(words, 12)) + rng.choice([".", "!", "?\n", ",\n\n"]) for _ in range(200)]
    trainer = trainers.BpeTrainer(vocab_size=700, initial_alphabet=pre_tokenizers.ByteLevel.alphabet(), show_progress=False)
    hf.train_from_iterator(corpus, trainer)
    hf.model.save(d)
    # The specials get the next ids, as added tokens after the vocabulary.
    base = hf.get_vocab_size()
    specials = ["<|endoftext|>", "<|im_start|>", "<|im_end|>"]
    hf.add_special_tokens(specials)
    added = {base + k: (s, True) for k, s in enumerate(specials)}
    with open(os.path.join(d, "tokenizer_config.json"), "w") as f:
        json.dump({"added_tokens_decoder": {str(i): {"content": c, "special": True} for i, (c, _) in added.items()}}, f)
    return hf, LS.Tokenizer(d)


def test_bpe_matches_hf_tokenizers_on_a_trained_vocabulary(trained):
    hf, tok = trained
    texts = [c["text"] for c in golden_texts()] + EXTRA
    rng = np.random.default_rng(3)
    alphabet = list("abcdefghij ,.!?\n\t'") + ["é", "日", "😀", "1", "2", "Ä"]
    texts += ["".join(rng.choice(alphabet, int(rng.integers(1, 40)))) for _ in range(300)]
    texts += ["<|im_start|>user\nHi there<|im_end|>\n<|im_start|>assistant\n", "a<|endoftext|><|endoftext|>b"]
    for text in texts:
        want = hf.encode(text, add_special_tokens=False).ids
        assert tok.encode(text) == want, text


def test_decode_inverts_encode_and_hides_special_tokens(trained):
    hf, tok = trained
    for text in ["Hello, world!", "  spaces  and\ttabs\n", "Café 日本語 😀", "def f(x):\n    return x"]:
        assert tok.decode(tok.encode(text)) == text
    ids = tok.encode("<|im_start|>user\nHi<|im_end|>")
    assert ids[0] == tok.token_id("<|im_start|>") and ids[-1] == tok.token_id("<|im_end|>")
    assert tok.decode(ids) == "user\nHi"
    assert tok.decode(ids) == hf.decode(ids, skip_special_tokens=True)


def test_the_golden_ids_of_the_qwen_tokenizer():
    """tests/tokenizer_golden.rs: the reference's golden cases against the real vocabulary, when
    it is available (LS_QWEN_TOKENIZER_DIR)."""
    d = os.environ.get("LS_QWEN_TOKENIZER_DIR")
    if not d or not os.path.exists(os.path.join(d, "vocab.json")):
        pytest.skip("SKIPPED: the Qwen2.5 tokenizer files are not in this image (set LS_QWEN_TOKENIZER_DIR)")
    tok = LS.Tokenizer(d)
    for c in golden_texts():
        assert tok.encode(c["text"]) == c["ids"], c["text"]
