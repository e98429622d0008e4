"""The byte-level BPE tokenizer (dolittle_amd/tokenizer.py) on the CPU.

- The reference's contract cases (tests/core/test_byte_bpe.cpp:31-91) on the
  fixture its tests hold (tests/golden/byte_bpe_tokenizer.json and
  qwen3_tokenizer_config.json, copied from tests/support/text_fixture.h).
- Against the Hugging Face `tokenizers` library 0.22.2 (the version the
  reference's validation bundles record their vectors with), an independent
  implementation of the same pipeline: the fixture on mixed-script text, and
  a tokenizer with 2,000 merges trained here on a synthetic corpus, on
  held-out text, so that rank order, leftmost ties and merges next to earlier
  merges are all exercised.
- Closed forms: the byte alphabet, decode(encode(x)) = NFC(x), contiguous
  byte ranges, and each limit and rejection.
"""
import json
import os
import random
import unicodedata

import pytest

from dolittle_amd import tokenizer as bpe
from dolittle_amd._lib import InvalidArgument, LengthError

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOKENIZER = open(os.path.join(GOLDEN, "byte_bpe_tokenizer.json"), encoding="utf-8").read()
CONFIG = open(os.path.join(GOLDEN, "qwen3_tokenizer_config.json"), encoding="utf-8").read()
LIMITS = bpe.ByteBpeLimits(65536, 4096, 4096, 4096)


def make(tokenizer_json=TOKENIZER, config_json=CONFIG, limits=LIMITS):
    return bpe.make_byte_bpe(tokenizer_json, config_json, "verified-test", limits)


# -- the reference's contract cases (test_byte_bpe.cpp)
def test_reference_contract_cases():
    t = make()
    assert t.encode("abc") == [257]                       # ranked adjacent merges
    assert t.encode("aaaaa") == [259, 259, 97]            # leftmost overlapping merge
    assert t.encode("") == []
    assert t.decode(t.encode(b"e\xcc\x81")).bytes == b"\xc3\xa9"  # NFC
    text = "x<think>abc</think>!"
    ids = t.encode(text)
    decoded = t.decode(ids)
    assert decoded.bytes == text.encode() and len(decoded.tokens) == len(ids)  # added tokens keep their bytes
    raw = t.decode([195, 169, 999999])
    assert raw.bytes == b"\xc3\xa9" and raw.tokens[0].end == 1 and raw.tokens[1].begin == 1
    assert not raw.tokens[2].mapped and raw.tokens[2].begin == raw.tokens[2].end  # unmapped provenance
    reusable = bpe.DecodedBytes()
    reusable.reserve(len(ids), len(ids) * t.max_token_bytes())
    t.decode_into(ids, reusable)
    assert reusable.bytes == decoded.bytes and len(reusable.tokens) == len(ids)
    t.decode_into([], reusable)
    assert reusable.bytes == b"" and reusable.tokens == []  # decode replaces the previous delta
    insufficient = bpe.DecodedBytes()
    with pytest.raises(LengthError):
        t.decode_into(ids, insufficient)
    assert insufficient.bytes == b"" and insufficient.tokens == []  # unchanged on rejection
    zero = b"a\x00b"
    assert t.decode(t.encode(zero)).bytes == zero  # embedded NUL
    with pytest.raises(InvalidArgument):
        t.encode(b"\xff")
    bad = json.loads(TOKENIZER)
    bad["model"]["byte_fallback"] = True
    with pytest.raises(InvalidArgument):
        make(json.dumps(bad))
    small = bpe.ByteBpeLimits(65536, 4096, 2, 4096)
    with pytest.raises(LengthError):
        make(limits=small).encode("abc")


def test_fixture_pattern_is_the_pinned_split():
    data = json.loads(TOKENIZER)
    assert data["pre_tokenizer"]["pretokenizers"][0]["pattern"]["Regex"] == bpe.SPLIT_PATTERN


# -- closed forms
def test_byte_alphabet():
    codes = bpe.byte_alphabet()
    assert len(set(codes)) == 256
    assert all(chr(c).isprintable() and not chr(c).isspace() for c in codes)
    assert codes[ord("a")] == ord("a") and codes[0] == 256 and codes[32] == 256 + 32 and codes[173] == 323
    # Every byte alone encodes to its alphabet symbol's ID in the fixture,
    # whose vocabulary lists the symbols in byte order.
    t = make()
    for b in range(1, 128):
        ids = t.encode(bytes([b]))
        assert ids == [b], (b, ids)


TEXTS = [
    "Hello, world!  It's 2026; we'll test THE tokenizer's splits.\n\n\tTabs\r\nand CRLF",
    "naïve café — résumé 12345 ½ ² Ⅻ",
    "Ελληνικά και русский язык; עברית; العربية",
    "日本語のテキストと中文混合 한국어",
    "emoji 😀🚀👍🏽 and ZWJ 👨‍👩‍👧",
    "combining: é ä ộ and precomposed: é ä",
    "   leading and trailing spaces   ",
    "x<think>reason</think>answer<|im_end|><|endoftext|>",
    "<tool_call>{\"name\": \"f\"}</tool_call>",
    "'S 'T 'RE 'Ve 'm 'LL 'd it's IT'S",
    "a b c　d e",
    "",
]


def random_text(rng: random.Random, n: int) -> str:
    pools = ["abcdefghij ", "ABC xyz", "0123456789", "!?.,;:'\"()[]{}-_", " \t\n\r",
             "éèêëàâäöüß", "αβγδεζ", "абвгде", "日本語中文", "😀🚀", "́̈", "<>|/"]
    return "".join(rng.choice(rng.choice(pools)) for _ in range(n))


def test_round_trip_is_nfc():
    t = make()
    rng = random.Random(7)
    for text in TEXTS + [random_text(rng, rng.randint(1, 60)) for _ in range(200)]:
        ids = t.encode(text)
        decoded = t.decode(ids)
        # Added tokens are matched on the raw text and ordinary spans are
        # normalized on their own, so compare span-wise: here NFC of the
        # whole text equals the concatenation because no span boundary
        # splits a combining sequence in these texts.
        assert decoded.bytes == unicodedata.normalize("NFC", text).encode(), text
        end = 0
        for tb in decoded.tokens:
            assert tb.mapped and tb.begin == end and tb.end >= tb.begin
            end = tb.end
        assert end == len(decoded.bytes)


# -- against the Hugging Face library on the same tokenizer.json.  The
# library numbers added tokens after a model vocabulary smaller than their
# declared IDs (the fixture's 260 entries), where the reference keeps the
# declared IDs (test_reference_contract_cases), so texts holding added tokens
# are compared only without them.
ADDED = ("<think>", "</think>", "<|im_end|>", "<|endoftext|>", "<tool_call>", "</tool_call>")


def plain(texts):
    return [t for t in texts if not any(a in t for a in ADDED)]


def hf(tokenizer_json):
    tokenizers = pytest.importorskip("tokenizers")
    return tokenizers.Tokenizer.from_str(tokenizer_json)


def test_fixture_matches_hf_tokenizers():
    ref = hf(TOKENIZER)
    t = make()
    rng = random.Random(11)
    texts = plain(TEXTS + [random_text(rng, rng.randint(1, 80)) for _ in range(300)])
    assert len(texts) > 250
    for text in texts:
        assert t.encode(text) == ref.encode(text, add_special_tokens=False).ids, repr(text)


def synthetic_lexicon(rng: random.Random, n: int) -> list:
    """Words of 1-4 syllables drawn with skewed frequencies, some accented
    or with digits and punctuation attached."""
    onsets = ["", "b", "c", "d", "f", "g", "h", "k", "l", "m", "n", "p", "r", "s", "t", "v", "w", "st", "tr",
              "ch", "sh", "th", "qu", "gr", "bl", "kn"]
    nuclei = ["a", "e", "i", "o", "u", "ai", "ea", "ou", "ie", "é", "ü", "ö"]
    codas = ["", "", "n", "r", "s", "t", "ng", "ck", "ll", "rd", "st"]
    words = []
    for _ in range(n):
        w = "".join(rng.choice(onsets) + rng.choice(nuclei) + rng.choice(codas)
                    for _ in range(rng.choice([1, 1, 2, 2, 3, 4])))
        words.append(w + rng.choice(["", "", "", "s", "ing", "ed", "'s", "!", "123", ","]))
    return words


def synthetic_sentences(rng: random.Random, n: int, lexicon=None) -> list:
    lexicon = lexicon or synthetic_lexicon(random.Random(1), 3000)
    weights = [1.0 / (i + 1) for i in range(len(lexicon))]
    return [rng.choices(lexicon, weights, k=rng.randint(3, 16)) for _ in range(n)]


def trained_tokenizer_json():
    """The fixture's pipeline with a 2,000-merge model trained here."""
    tokenizers = pytest.importorskip("tokenizers")
    from tokenizers import decoders, models, pre_tokenizers, trainers
    tok = tokenizers.Tokenizer(models.BPE())
    tok.pre_tokenizer = pre_tokenizers.Sequence([
        pre_tokenizers.Split(tokenizers.Regex(bpe.SPLIT_PATTERN), behavior="isolated"),
        pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)])
    tok.decoder = decoders.ByteLevel()
    corpus = [" ".join(sentence) for sentence in synthetic_sentences(random.Random(3), 4000)]
    trainer = trainers.BpeTrainer(vocab_size=256 + 2000, initial_alphabet=pre_tokenizers.ByteLevel.alphabet(),
                                  show_progress=False)
    tok.train_from_iterator(corpus, trainer)
    model = json.loads(tok.to_str())["model"]
    data = json.loads(TOKENIZER)
    data["model"]["vocab"] = model["vocab"]
    data["model"]["merges"] = [m.split(" ") if isinstance(m, str) else m for m in model["merges"]]
    return json.dumps(data), len(data["model"]["merges"])


def test_trained_merges_match_hf_tokenizers():
    text_json, n_merges = trained_tokenizer_json()
    assert n_merges > 1000
    ref = hf(text_json)
    t = make(text_json, limits=bpe.ByteBpeLimits(1 << 22, 4096, 4096, 4096))
    rng = random.Random(5)
    held_out = [" ".join(s) for s in synthetic_sentences(rng, 300, synthetic_lexicon(random.Random(2), 2000))]
    texts = plain(TEXTS + held_out + [" ".join(s) + random_text(rng, 5) for s in synthetic_sentences(rng, 100)]
                  + ["ssss aaaa the the the", "tttttttt", "éééé üüü"])
    assert len(texts) > 350
    for text in texts:
        ids = t.encode(text)
        assert ids == ref.encode(text, add_special_tokens=False).ids, repr(text)
        assert t.decode(ids).bytes == unicodedata.normalize("NFC", text).encode()


# -- limits and rejections
def test_limits():
    t = make(limits=bpe.ByteBpeLimits(65536, 8, 4096, 3))
    with pytest.raises(LengthError):
        t.encode("123456789")          # input bytes
    with pytest.raises(LengthError):
        t.encode("a b c d")            # output tokens
    assert t.encode("a b") == [97, 32, 98]
    with pytest.raises(LengthError):
        t.decode([97] * 4)             # decode token budget
    with pytest.raises(LengthError):
        make(limits=bpe.ByteBpeLimits(100, 4096, 4096, 4096))  # metadata budget
    with pytest.raises(InvalidArgument):
        make(limits=bpe.ByteBpeLimits(65536, 0, 4096, 4096))
    with pytest.raises(InvalidArgument):
        bpe.make_byte_bpe(TOKENIZER, CONFIG, "", LIMITS)


def edited(path, value):
    data = json.loads(TOKENIZER)
    node = data
    for key in path[:-1]:
        node = node[key]
    node[path[-1]] = value
    return json.dumps(data)


@pytest.mark.parametrize("path,value", [
    (("normalizer",), {"type": "NFKC"}),
    (("model", "dropout"), 0.1),
    (("model", "unk_token"), "<unk>"),
    (("model", "continuing_subword_prefix"), "##"),
    (("model", "merges"), [["a", "b"], ["a", "b"]]),       # duplicate pair
    (("model", "merges"), [["a", "q"]]),                   # a + q not in the vocabulary
    (("decoder",), {"type": "Fuse"}),
    (("padding",), {"strategy": "BatchLongest"}),
])
def test_rejected_metadata(path, value):
    with pytest.raises(InvalidArgument):
        make(edited(path, value))


def test_rejected_vocabularies_and_added_tokens():
    data = json.loads(TOKENIZER)
    del data["model"]["vocab"]["Ġ"]                       # a byte symbol missing
    with pytest.raises(InvalidArgument):
        make(json.dumps(data))
    data = json.loads(TOKENIZER)
    data["model"]["vocab"]["zz"] = 97                      # duplicate ID
    with pytest.raises(InvalidArgument):
        make(json.dumps(data))
    data = json.loads(TOKENIZER)
    data["model"]["vocab"]["big"] = 1 << 32                # ID overflow
    with pytest.raises(LengthError):
        make(json.dumps(data))
    data = json.loads(TOKENIZER)
    data["added_tokens"][0]["lstrip"] = True               # stripping added token
    with pytest.raises(InvalidArgument):
        make(json.dumps(data))
    config = json.loads(CONFIG)
    config["added_tokens_decoder"]["151643"]["special"] = False  # config disagrees
    with pytest.raises(InvalidArgument):
        make(config_json=json.dumps(config))
    config = json.loads(CONFIG)
    config["add_bos_token"] = True
    with pytest.raises(InvalidArgument):
        make(config_json=json.dumps(config))


def test_added_token_selection():
    """Earliest match first; at one position the longest content, then the
    lowest ID (byte_bpe.h:22-23)."""
    data = json.loads(TOKENIZER)
    config = json.loads(CONFIG)
    extra = [(151700, "<a>"), (151701, "<a>b"), (151702, "b>")]
    for token_id, content in extra:
        entry = {"id": token_id, "content": content, "single_word": False, "lstrip": False, "rstrip": False,
                 "normalized": False, "special": False}
        data["added_tokens"].append(entry)
        config["added_tokens_decoder"][str(token_id)] = {k: v for k, v in entry.items() if k != "id"}
    t = make(json.dumps(data), json.dumps(config))
    assert t.encode("x<a>b>") == [120, 151701, 62]        # longest at the earliest position
    assert t.encode("xb><a>") == [120, 151702, 151700]
    assert t.contains(151701) and not t.contains(151800)
    assert t.decode([151701]).bytes == b"<a>b"
