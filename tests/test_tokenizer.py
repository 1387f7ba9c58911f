"""The library's host tokenizer (dn_tokenizer_*, dn_pretokenize, dn_nfc)
against the reference's own test cases, the oracle's line-by-line
restatement of internal/tokenizer/tokenizer.go, HuggingFace `tokenizers`
(the implementation the reference's tokenizer is tested against,
tokenizer_test.go:11-38) and Python's unicodedata. CPU only."""
import json
import os
import random
import unicodedata

import pytest

import oracle.tokenizer as ot
from conftest import GOLDEN

GOLDEN_TEXTS = [c["text"] for c in json.load(open(os.path.join(GOLDEN, "tokenizer_golden.json")))]


def test_pretokenize_reference_cases():
    """TestPreTokenize (internal/tokenizer/tokenizer_test.go:46-65)."""
    from decide_amd.tokenizer import pretokenize

    cases = {"Hello world": ["Hello", " world"], "a  b": ["a", " ", " b"], "it's": ["it", "'s"], "x  ": ["x", "  "],
             "foo\n\nbar": ["foo", "\n", "\n", "bar"], "a1 b2": ["a", "1", " b", "2"], "end.\n": ["end", ".", "\n"],
             " ,": [" ,"]}
    for text, want in cases.items():
        assert pretokenize(text) == want, text
        assert [p.decode() for p in ot.pre_tokenize(text.encode())] == want, text


def test_minimal_tokenizer_is_byte_level():
    """tokenizer.MinimalJSON: ids are the UTF-8 bytes, specials split out,
    [MASK] strips the whitespace before it (the encoding decide.Local's tests
    run on, local_test.go:20-44)."""
    from decide_amd.tokenizer import Tokenizer
    from test_local import byte_encode

    tok = Tokenizer.parse(ot.minimal_json())
    assert (tok.cls_id, tok.sep_id, tok.mask_id, tok.pad_id) == (256, 257, 258, 259)
    o = ot.Tokenizer(ot.minimal_json())
    for text in GOLDEN_TEXTS + ["q st [SEP] [MASK] a [MASK] bc", "x\t [MASK]\n[MASK]", "é"]:
        assert tok.encode(text) == o.encode(text) == byte_encode(text), text
        assert tok.encode(text, add_special=False) == o.encode(text, False)
    assert tok.count("ab c") == 4


def test_parse_errors():
    from decide_amd.native import InvalidArgument
    from decide_amd.tokenizer import Tokenizer

    base = json.loads(ot.minimal_json())
    bad_type = dict(base, model=dict(base["model"], type="WordPiece"))
    with pytest.raises(InvalidArgument, match='unsupported model type "WordPiece"'):
        Tokenizer.parse(json.dumps(bad_type).encode())
    no_mask = dict(base, added_tokens=[a for a in base["added_tokens"] if a["content"] != "[MASK]"])
    with pytest.raises(InvalidArgument, match=r"missing \[CLS\]/\[SEP\]/\[MASK\]"):
        Tokenizer.parse(json.dumps(no_mask).encode())
    bad_merge = dict(base, model=dict(base["model"], merges=["nospace"]))
    with pytest.raises(InvalidArgument, match='bad merge "nospace"'):
        Tokenizer.parse(json.dumps(bad_merge).encode())
    with pytest.raises(InvalidArgument):
        Tokenizer.parse(b"{not json")


def random_texts(seed, count):
    """Words, digits, punctuation, contractions, several kinds of whitespace,
    accents (composed and decomposed), Hangul jamo, CJK, emoji, specials."""
    rng = random.Random(seed)
    words = ["hello", "world", "the", "payment", "failed", "twice", "customer", "ticket", "naïve", "café",
             "café", "日本語", "über", "Straße", "don't", "it's", "we're", "they'll", "I'd", "you've",
             "1,234.56", "3.14", "2026", "😀", "각", "각", "résumé", "(approx.)", "--", "...",
             "!!!", "[MASK]", "[SEP]", "|||EMAIL_ADDRESS|||", "[unused3]", "snake_case", "CamelCase", "x²", "½",
             "٣", "Ⅻ", "Don'T", "'ll", "ậ", "क़"]
    spaces = [" ", "  ", "\t", "\n", "\n\n", "\xa0", " ", " \n ", ""]
    return ["".join(rng.choice(words) + rng.choice(spaces) for _ in range(rng.randint(1, 12)))
            for _ in range(count)]


@pytest.fixture(scope="module")
def trained():
    """A byte-level BPE tokenizer.json trained here with HuggingFace
    `tokenizers` (NFC, ByteLevel pre-tokenizer, ModernBERT's added tokens,
    [CLS] $A [SEP]), and the library instance loaded from it."""
    from tokenizers import AddedToken, Tokenizer as HFTokenizer, models, normalizers, pre_tokenizers, processors, \
        trainers

    from decide_amd.tokenizer import Tokenizer

    hf = HFTokenizer(models.BPE())
    hf.normalizer = normalizers.NFC()
    hf.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=True)
    trainer = trainers.BpeTrainer(vocab_size=600, initial_alphabet=pre_tokenizers.ByteLevel.alphabet(),
                                  show_progress=False)
    hf.train_from_iterator(random_texts(0, 3000) + GOLDEN_TEXTS, trainer)
    hf.add_special_tokens([AddedToken("[CLS]", special=True, normalized=False),
                           AddedToken("[SEP]", special=True, normalized=False),
                           AddedToken("[MASK]", special=True, normalized=False, lstrip=True),
                           AddedToken("[PAD]", special=True, normalized=False),
                           AddedToken("[UNK]", special=True, normalized=False)])
    hf.add_tokens([AddedToken("|||EMAIL_ADDRESS|||", special=False, normalized=True),
                   AddedToken("[unused3]", special=False, normalized=True)])
    hf.post_processor = processors.TemplateProcessing(
        single="[CLS] $A [SEP]", special_tokens=[("[CLS]", hf.token_to_id("[CLS]")), ("[SEP]", hf.token_to_id("[SEP]"))])
    raw = hf.to_str().encode()
    return hf, raw, ot.Tokenizer(raw), Tokenizer.parse(raw)


def test_oracle_matches_huggingface(trained):
    """Pins the oracle: the same ids as HuggingFace's implementation on the
    reference's golden texts and 500 random texts."""
    hf, _, o, _ = trained
    texts = GOLDEN_TEXTS + random_texts(7, 500) + ["", " ", "[MASK]", " [MASK] x", "a[MASK]b", "x  [MASK]  y"]
    for t in texts:
        assert o.encode(t) == hf.encode(t).ids, t


def test_library_matches_oracle(trained):
    """The library tokenizer against the oracle, ids bit for bit, on texts
    that include invalid UTF-8 and random code points from many scripts."""
    _, _, o, tok = trained
    rng = random.Random(3)
    pools = [range(0x20, 0x7F), range(0xA0, 0x250), range(0x300, 0x370), range(0x1100, 0x1200),
             range(0xAC00, 0xAC40), range(0x3040, 0x30FF), range(0x4E00, 0x4E40), range(0x1F600, 0x1F650),
             range(0x2000, 0x2030), range(0x900, 0x980), range(0x660, 0x66A), range(0x2160, 0x2180)]
    texts = [t.encode() for t in GOLDEN_TEXTS + random_texts(11, 300)]
    for i in range(1500):
        b = "".join(chr(rng.choice(rng.choice(pools))) for _ in range(rng.randint(0, 30))).encode()
        if i % 4 == 0:
            bl = bytearray(b)
            for _ in range(rng.randint(1, 3)):
                pos = rng.randint(0, len(bl))
                bl[pos:pos] = rng.choice([b"\xff", b"\xe2\x82", b"\xc3", b"[MASK]", b" [SEP] ", b"\xed\xa0\x80"])
            b = bytes(bl)
        texts.append(b)
    for b in texts:
        assert tok.encode(b) == o.encode(b), b
        assert tok.encode(b, add_special=False) == o.encode(b, False), b


def test_pretokenize_and_nfc_match_oracle():
    from decide_amd.tokenizer import nfc, pretokenize

    rng = random.Random(5)
    for i in range(2000):
        s = "".join(chr(rng.choice([rng.randint(0x20, 0x7E), rng.randint(0xA0, 0x36F), rng.randint(0x1100, 0x11FF),
                                    rng.randint(0xAC00, 0xD7A3), rng.randint(0x2000, 0x206F)]))
                    for _ in range(rng.randint(0, 24)))
        b = s.encode()
        if i % 5 == 0:
            b = b[:len(b) // 2] + b"\xe2\x82" + b[len(b) // 2:]
        assert nfc(b) == ot.nfc(b), b
        assert [p.encode() for p in pretokenize(b)] == ot.pre_tokenize(b), b


def test_nfc_matches_unicodedata():
    """dn_nfc against Python's unicodedata.normalize over every code point
    with a canonical decomposition or a combining class (plus Hangul), alone
    and followed by combining marks in scrambled order."""
    from decide_amd.tokenizer import nfc

    cps = [c for c in range(0x110000) if not (0xD800 <= c <= 0xDFFF) and
           (unicodedata.decomposition(chr(c)) or unicodedata.combining(chr(c)))]
    cps += list(range(0xAC00, 0xAC00 + 400)) + list(range(0x1100, 0x1113)) + list(range(0x1161, 0x1176))
    rng = random.Random(9)
    marks = [0x301, 0x300, 0x323, 0x302, 0x308, 0x327, 0x316, 0x35C, 0x11A8, 0x1161, 0x3099, 0x93C]
    for c in cps:
        s = chr(c) + "".join(chr(rng.choice(marks)) for _ in range(rng.randint(0, 3)))
        want = unicodedata.normalize("NFC", s).encode()
        assert nfc(s) == want, hex(c)
        nfd = unicodedata.normalize("NFD", s)
        assert nfc(nfd) == want, hex(c)


# Hand-derived answers of UAX #15's Stream-Safe Text Process followed by NFC
# (U+0301 acute and U+0316 grave-below are non-starters of class 230 / 220;
# U+00E9's decomposition ends in one non-starter; U+0344 decomposes to two).
A, G, CGJ = "\u0301", "\u0316", "\u034f"
STREAM_SAFE_CASES = [
    ("a" + A * 30, "\u00e1" + A * 29),                       # 30 non-starters: untouched
    ("a" + A * 31, "\u00e1" + A * 29 + CGJ + A),             # the 31st gets a CGJ in front
    ("\u00e9" + A * 30, "\u00e9" + A * 29 + CGJ + A),        # e-acute's own mark counts
    (G * 70, G * 30 + CGJ + G * 30 + CGJ + G * 10),         # no starter at all
    ("a" + A * 29 + "\u0344", "\u00e1" + A * 28 + CGJ + "\u0308\u0301"),  # two at once
    ("a" + A * 30 + G, "\u00e1" + A * 29 + CGJ + G),         # no reordering across the CGJ
    ("a" + G + A * 30, "\u00e1" + G + A * 28 + CGJ + A),     # G + 29 A, then the CGJ
]


def test_stream_safe_known_answers():
    """NFC with x/text's stream-safe step: the oracle and dn_nfc against
    answers worked by hand from UAX #15 D5; an invalid byte restarts the
    count (20 + 20 marks around it stay untouched)."""
    from decide_amd.tokenizer import nfc

    for text, want in STREAM_SAFE_CASES:
        assert ot.nfc(text.encode()) == want.encode(), [hex(ord(c)) for c in text]
        assert nfc(text) == want.encode(), [hex(ord(c)) for c in text]
    b = ("a" + A * 20).encode() + b"\xff" + (A * 20).encode()
    want = ("\u00e1" + A * 19).encode() + b"\xff" + (A * 20).encode()
    assert ot.nfc(b) == want and nfc(b) == want


def test_stream_safe_matches_oracle():
    """Long runs of combining marks (classes 202-240, marks with several
    non-starters in their decompositions, precomposed letters whose
    decompositions end in marks, invalid bytes) through dn_nfc and the
    oracle's stream-safe NFC."""
    from decide_amd.tokenizer import nfc

    rng = random.Random(15)
    marks = [0x301, 0x300, 0x316, 0x323, 0x327, 0x302, 0x308, 0x345, 0x344, 0xF73, 0xF75, 0x93C, 0x3099, 0x5B0]
    starters = ["a", "e", "\u00e9", "\u1e09", "\u00a8", "\uff9e", "\u1100", "\u1161", "\uac00", "x"]
    hits = 0
    for i in range(400):
        parts = []
        for _ in range(rng.randint(1, 4)):
            if rng.random() < 0.7:
                parts.append(rng.choice(starters))
            parts.append("".join(chr(rng.choice(marks)) for _ in range(rng.randint(0, 75))))
        b = "".join(parts).encode()
        if i % 7 == 0:
            cut = rng.randint(0, len(b))
            b = b[:cut] + b"\xc3" + b[cut:]
        want = ot.nfc(b)
        hits += want.count(CGJ.encode())
        assert nfc(b) == want, b
    assert hits > 100  # the cases do exercise the CGJ insertion


def test_merges_outside_the_vocabulary():
    """A merge whose parts or result are not vocabulary entries: the string
    form of bpe (tokenizer.go:320-365) applies it, and a final part that is
    not in the vocabulary falls back to its symbols that are."""
    from decide_amd.tokenizer import Tokenizer

    base = json.loads(ot.minimal_json())
    vocab = dict(base["model"]["vocab"])
    vocab["Ġt"] = 300          # "Ġt"
    vocab["Ġthe"] = 301        # reachable only through "he", which is not in the vocabulary
    merges = ["Ġ t", "h e", "Ġt he", "x y"]
    raw = json.dumps(dict(base, model=dict(base["model"], vocab=vocab, merges=merges))).encode()
    tok, o = Tokenizer.parse(raw), ot.Tokenizer(raw)
    for text in [" the", " them", "the xy", " t", "xyz the the"]:
        assert tok.encode(text) == o.encode(text), text
    assert tok.encode(" the", add_special=False) == [301]
    assert tok.encode(" them", add_special=False) == [301, ord("m")]
