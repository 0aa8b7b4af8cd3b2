"""SentencePiece detokenizer (SentencePieceDecoder, Sources/DictatorCore/Decoding/SentencePiece.swift:
5-31): the oracle's restatement pinned against the sentencepiece package's decoder on a model
trained here (byte fallback included), against the Unicode Standard's maximal-subpart example and
hand-built cases of the Swift rules; then the library's C ABI (include/ud_tokenizer.h, host code,
no device) against the oracle on random vocabularies and ids.  CPU only."""
import os
import random

import numpy as np
import pytest

import oracle.oracle as orc


WORDS = ["the", "quick", "brown", "fox", "jumps", "over", "lazy", "dog", "streaming", "encoder", "speech", "audio"]


@pytest.fixture(scope="module")
def sp_model(tmp_path_factory):
    spm = pytest.importorskip("sentencepiece")
    d = tmp_path_factory.mktemp("sp")
    rng = random.Random(1)
    with open(d / "corpus.txt", "w") as f:
        for _ in range(3000):
            f.write(" ".join(rng.choice(WORDS) for _ in range(rng.randint(3, 12))) + "\n")
    spm.SentencePieceTrainer.train(input=str(d / "corpus.txt"), model_prefix=str(d / "m"), vocab_size=300,
                                   byte_fallback=True, character_coverage=1.0, minloglevel=2, hard_vocab_limit=False)
    sp = spm.SentencePieceProcessor(model_file=str(d / "m.model"))
    return sp, str(d / "m.vocab")


def test_oracle_matches_sentencepiece(sp_model):
    """Texts through the trained model's encoder (characters outside the corpus become byte pieces)
    and random runs of its ordinary pieces decode as the sentencepiece package decodes them."""
    sp, vocab = sp_model
    pieces = orc.sp_parse_vocab(open(vocab, "rb").read())
    assert len(pieces) == sp.get_piece_size()
    assert all(pieces[i] == sp.id_to_piece(i) for i in range(len(pieces)))
    texts = ["the quick brown fox", "naïve café über", "日本語の音声 streaming", "  padded   spaces ", "x", "",
             "emoji \U0001F600 and é́ marks", "dog\tover\nlazy"]
    n_bytes = 0
    for t in texts:
        ids = sp.encode(t)
        n_bytes += sum(1 for i in ids if sp.is_byte(i))
        assert orc.sp_decode(pieces, ids) == sp.decode(ids).encode("utf-8"), t
    assert n_bytes > 10                       # the byte-fallback path was exercised
    ordinary = [i for i in range(len(pieces)) if not (sp.is_byte(i) or sp.is_control(i) or sp.is_unknown(i))]
    # (texts that start with two or more spaces differ: the sentencepiece package strips them all,
    # SentencePiece.swift:29 drops one; test_oracle_swift_rules pins that case)
    rng = random.Random(7)
    checked = 0
    for _ in range(300):
        ids = [rng.choice(ordinary) for _ in range(rng.randint(0, 12))]
        if "".join(pieces[i] for i in ids).replace("\u2581", " ").startswith("  "):
            continue
        assert orc.sp_decode(pieces, ids) == sp.decode(ids).encode("utf-8"), ids
        checked += 1
    assert checked > 250
    # control pieces add nothing in both
    ids = [sp.bos_id(), ordinary[5], sp.eos_id(), ordinary[9]]
    assert orc.sp_decode(pieces, ids) == sp.decode(ids).encode("utf-8")


def test_oracle_unicode_maximal_subparts():
    """The Unicode Standard's example of U+FFFD substitution of maximal subparts (Table 3-8):
    61 F1 80 80 E1 80 C2 62 80 63 80 BF 64 -> a FFFD FFFD FFFD b FFFD c FFFD FFFD d."""
    seq = [0x61, 0xF1, 0x80, 0x80, 0xE1, 0x80, 0xC2, 0x62, 0x80, 0x63, 0x80, 0xBF, 0x64]
    pieces = ["<0x%02X>" % b for b in range(256)]
    assert orc.sp_decode(pieces, seq) == "a���b�c��d".encode("utf-8")
    # a truncated 3-byte sequence at the end is one U+FFFD; surrogates and overlongs are ill-formed
    assert orc.sp_decode(pieces, [0x41, 0xE2, 0x96]) == "A�".encode("utf-8")
    assert orc.sp_decode(pieces, [0xED, 0xA0, 0x80]) == "���".encode("utf-8")
    assert orc.sp_decode(pieces, [0xC0, 0xAF]) == "��".encode("utf-8")
    # U+2581 assembled from byte pieces is kept: the replacement applies to ordinary pieces only
    assert orc.sp_decode(pieces, [0xE2, 0x96, 0x81]) == "▁".encode("utf-8")


def test_oracle_swift_rules():
    """Hand-built cases of SentencePiece.swift:8-30."""
    vocab = ("<unk>\t0\n<s>\t0\n</s>\t0\n<pad>\t0\n▁the\t-1.5\n\n\tlead\n\t\t\nab▁cd\t-2\nno_tab\n"
             "<0x41>\t0\n<0x4a>\t0\n<0xZZ>\t0\n<0x4>\t0\na\r\nb\t-1\n▁\t-3\n").encode("utf-8")
    p = orc.sp_parse_vocab(vocab)
    assert p == ["<unk>", "<s>", "</s>", "<pad>", "▁the", "lead", "", "ab▁cd", "no_tab", "<0x41>", "<0x4a>",
                 "<0xZZ>", "<0x4>", "a\r\nb", "▁"]
    d = lambda ids: orc.sp_decode(p, ids).decode("utf-8")
    assert d([4, 7]) == "theab cd"                       # one leading space dropped
    assert d([14, 14, 4]) == "  the"                     # only one of three
    assert d([0, 1, 2, 3, 4]) == "the"                   # specials add nothing
    assert d([-1, 99, 4, 15]) == "the"                   # out of range skipped
    assert d([9, 10, 11, 12]) == "AJ<0xZZ><0x4>"         # byte pieces: two hex digits only
    assert d([5, 6, 8]) == "leadno_tab"
    assert d([13]) == "a\r\nb"
    assert d([]) == ""
    with pytest.raises(UnicodeDecodeError):
        orc.sp_parse_vocab(b"ok\t0\n\xff\xfe\t0\n")      # not UTF-8: the Swift initializer throws


def _random_vocab(rng):
    specials = ["<unk>", "<s>", "</s>", "<pad>"]
    bytes_ = ["<0x%02X>" % b for b in rng.sample(range(256), 40)] + ["<0x%02x>" % b for b in rng.sample(range(256), 10)]
    chars = ["a", "b", "z", "▁", "é", "日", "\U0001F600", "<", ">", "0x", "▁▁"]
    words = ["".join(rng.choice(chars) for _ in range(rng.randint(1, 5))) for _ in range(80)]
    pieces = specials + bytes_ + words + ["<0xZZ>", "<0x4>"]
    rng.shuffle(pieces)
    lines = []
    for pc in pieces:
        form = rng.random()
        if form < 0.7:
            lines.append("%s\t%.4f" % (pc, -rng.random() * 10))
        elif form < 0.85:
            lines.append(pc)
        else:
            lines.append("\t" + pc + "\t-1")
        if rng.random() < 0.05:
            lines.append("")                             # empty lines are dropped
    return ("\n".join(lines) + "\n").encode("utf-8")


def test_library_matches_oracle(ud, tmp_path):
    ud.load_library()
    rng = random.Random(11)
    for trial in range(20):
        data = _random_vocab(rng)
        pieces = orc.sp_parse_vocab(data)
        tok = ud.Tokenizer.from_bytes(data) if trial % 2 else None
        if tok is None:
            path = tmp_path / ("v%d.vocab" % trial)
            path.write_bytes(data)
            tok = ud.Tokenizer(str(path))
        assert len(tok) == len(pieces)
        for i in range(len(pieces)):
            assert tok.piece(i) == pieces[i].encode("utf-8")
        for _ in range(60):
            ids = [rng.randint(-3, len(pieces) + 3) for _ in range(rng.randint(0, 40))]
            assert tok.decode(ids) == orc.sp_decode(pieces, ids), (trial, ids)
        tok.close()


def test_library_edge_cases(ud, tmp_path):
    ud.load_library()
    vocab = "a\r\nb\t0\n▁x\t0\n\n<0xE2>\t0\n<0x96>\t0\n<0x81>\t0\n".encode("utf-8")
    tok = ud.Tokenizer.from_bytes(vocab)
    assert [tok.piece(i) for i in range(len(tok))] == [b"a\r\nb", "▁x".encode(), b"<0xE2>", b"<0x96>", b"<0x81>"]
    assert tok.decode([1, 2, 3, 4]) == "x▁".encode("utf-8")         # " x" (leading space dropped), U+2581 from bytes
    assert tok.decode([2, 3]) == "�".encode("utf-8")             # truncated sequence: one U+FFFD
    assert tok.decode(np.zeros(0, np.int32)) == b""
    # sizing: a call with cap 0 reports the length; a short buffer gets the first cap bytes
    L = ud._lib
    import ctypes
    ids = (ctypes.c_int32 * 2)(0, 1)
    n = ctypes.c_int64(-1)
    assert L.ud_tokenizer_decode(tok.handle, ids, 2, None, 0, ctypes.byref(n)) == 0 and n.value == len(tok.decode([0, 1]))
    buf = ctypes.create_string_buffer(3)
    assert L.ud_tokenizer_decode(tok.handle, ids, 2, buf, 3, ctypes.byref(n)) == 0
    assert buf.raw == tok.decode([0, 1])[:3] and n.value == len(tok.decode([0, 1]))
    # errors
    with pytest.raises(ud.EngineError):
        ud.Tokenizer.from_bytes(b"ok\n\xff\n")                       # not UTF-8
    with pytest.raises(ud.EngineError):
        ud.Tokenizer(str(tmp_path / "missing.vocab"))
    with pytest.raises(ud.EngineError):
        tok.piece(len(tok))
    assert L.ud_tokenizer_decode(tok.handle, None, 3, None, 0, ctypes.byref(n)) == -1
    assert L.ud_tokenizer_decode(None, ids, 2, None, 0, ctypes.byref(n)) == -1
    assert L.ud_tokenizer_decode(tok.handle, ids, 2, None, 5, ctypes.byref(n)) == -1
    tok.close()
