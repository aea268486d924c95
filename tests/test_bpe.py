"""Byte-level BPE tokenizers (gpt2.BPETokenizer, llama.ByteLevelBPE).

There are no checkpoints here, so the reference's own round-trip tests
(tests/test_gpt2.py:60-66, tests/test_llama.py:135-139) run on vocabularies
trained locally with HuggingFace `tokenizers` (an independent byte-level BPE
with the same GPT-2 byte alphabet and merge rule). On ASCII text its
pre-tokenizer splits exactly as the reference's pattern does, so the ids must
agree; on any text, decode(encode(x)) == x. A hand-built merge table pins
the merge order (lowest rank first, every occurrence, left to right), and
the byte alphabet is checked against its definition.
"""

import json

import pytest

from draftkv.bpe import BPETokenizer, ByteLevelBPE, byte_alphabet

CORPUS = [
    "The capital of France is Paris. The capital of Italy is Rome.",
    "Memory bandwidth, not arithmetic, is the binding constraint on modern inference hardware.",
    "def f(x):\n    return x + 1\n\nclass A:\n    pass\n",
    "  leading space and 12345 digits! punctuation, semicolons; and-hyphens.",
    "It's what we'll do, they'd say -- I'm sure you've seen the rest.",
] * 20
ASCII_TEXTS = ["The capital of France is Paris.", "  leading space and 12345 digits!",
               "punctuation, semicolons; and-hyphens.", "def f(x):\n    return x + 1\n",
               "It's raining; they'll stay in, we've heard.", "zzz qqq unseen words 9876543210"]
ANY_TEXTS = ASCII_TEXTS + ["café naïve — ünïcödé ✓ 日本語", "tabs\tand\r\nnewlines  \n"]


@pytest.fixture(scope="module")
def trained(tmp_path_factory):
    tk = pytest.importorskip("tokenizers")
    d = tmp_path_factory.mktemp("bpe")
    t = tk.ByteLevelBPETokenizer(add_prefix_space=False)
    t.train_from_iterator(CORPUS, vocab_size=400, min_frequency=2, show_progress=False)
    t.save_model(str(d))                 # vocab.json + merges.txt (with its version header)
    t.save(str(d / "tokenizer.json"))
    return t, d


def test_byte_alphabet_is_gpt2s():
    m = byte_alphabet()
    assert sorted(m) == list(range(256)) and len(set(m.values())) == 256
    printable = [b for b in range(256) if (0x21 <= b <= 0x7E) or (0xA1 <= b <= 0xAC) or (0xAE <= b <= 0xFF)]
    assert all(m[b] == chr(b) for b in printable) and len(printable) == 188
    others = [b for b in range(256) if b not in printable]
    assert [ord(m[b]) for b in others] == list(range(256, 256 + len(others)))
    assert m[ord(" ")] == "\u0120" and m[ord("\n")] == "\u010a"     # "Ġ", "Ċ" as in GPT-2 vocabularies


@pytest.mark.parametrize("kind", ["gpt2", "tokenizer_json"])
def test_ids_match_an_independent_bpe_on_ascii(trained, kind):
    t, d = trained
    ours = BPETokenizer(d / "vocab.json", d / "merges.txt") if kind == "gpt2" else ByteLevelBPE(d / "tokenizer.json")
    for text in ASCII_TEXTS:
        assert ours.encode(text) == t.encode(text).ids, text


@pytest.mark.parametrize("kind", ["gpt2", "tokenizer_json"])
def test_roundtrip(trained, kind):
    _, d = trained
    ours = BPETokenizer(d / "vocab.json", d / "merges.txt") if kind == "gpt2" else ByteLevelBPE(d / "tokenizer.json")
    for text in ANY_TEXTS:
        assert ours.decode(ours.encode(text)) == text


def test_merge_order_by_hand(tmp_path):
    # symbols a, b, c and merges ranked (b c) < (a b) < (a bc) < (ab c)
    alpha = byte_alphabet()
    vocab = {alpha[b]: b for b in range(256)}
    for i, t in enumerate(["bc", "ab", "abc", "abab"]):
        vocab[t] = 256 + i
    (tmp_path / "vocab.json").write_text(json.dumps(vocab))
    (tmp_path / "merges.txt").write_text("#version: 0.2\nb c\na b\na bc\nab ab\n")
    tok = BPETokenizer(tmp_path / "vocab.json", tmp_path / "merges.txt")
    assert tok.encode("abc") == [vocab["abc"]]               # (b c) first, then (a bc); never (a b)
    assert tok.encode("abab") == [vocab["abab"]]             # (a b) twice, left to right, then (ab ab)
    assert tok.encode("abcab") == [vocab["abc"], vocab["ab"]]
    assert tok.encode("cba") == [vocab["c"], vocab["b"], vocab["a"]]    # no ranked pair
    spec = {"model": {"vocab": vocab, "merges": [["b", "c"], "a b", ["a", "bc"], "ab ab"]}}
    (tmp_path / "tokenizer.json").write_text(json.dumps(spec))
    assert ByteLevelBPE(tmp_path / "tokenizer.json").encode("abcab") == tok.encode("abcab")


def test_unknown_ids_and_invalid_utf8(tmp_path):
    alpha = byte_alphabet()
    vocab = {alpha[b]: b for b in range(256)}
    (tmp_path / "vocab.json").write_text(json.dumps(vocab))
    (tmp_path / "merges.txt").write_text("#version: 0.2\n")
    tok = BPETokenizer(tmp_path / "vocab.json", tmp_path / "merges.txt")
    assert tok.encode("hi") == [ord("h"), ord("i")]
    assert tok.decode([0xC3]) == "\ufffd"                    # a lone lead byte decodes as a replacement
    with pytest.raises(KeyError):
        tok.decode([999])
