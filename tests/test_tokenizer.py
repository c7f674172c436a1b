"""Tokenizer parity: the C++ scanner + BPE (product) against the oracle, which
pre-splits with the `regex` engine and restates tiktoken.rs's merge loop.
CPU only."""
import numpy as np
import pytest

from conftest import MODEL_PATH


@pytest.fixture(scope="module")
def toks(orc):
    import czip_amd
    import tokenizer_oracle as TO
    t, meta = orc.read_czm(MODEL_PATH)
    return czip_amd.Tokenizer(czip_amd.ModelWeights(MODEL_PATH)), TO.Tokenizer.from_model(t, meta)


EDGE = [
    "", " ", "  ", "\n", "\r\n", "a", "Hello world", "Hello  world", "  leading", "trailing  ", "trailing \n",
    "it's I'M we'LL you'Ve they're 'S 'll", "x'y", "'", "''", "don't stop", "ſ 'ſ",
    "12345 1234567 3.14159 1,000,000", "v1.2.3-beta+build", "a\tb\u000bc\u000cd",
    "tabs\t\t\tand\r\r\nmixed \n \n  \n", "!!!\n\n\nabc", "foo!!\r\n\r\nbar", "  !?  ", " nbsp　ideographic em",
    "ünïcödé Ëxàmplé Straße ĳ", "日本語のテキスト、句読点。", "Ελληνικά κείμενο", "кириллица текст", "عربي نص",
    "emoji 😀👍🏽 mixed", "combining é ä", "digits ٣٤٥ ①②③ Ⅻ", "\u0085next-line", "zero​width",
    "<|bos|>", "a<|bos|>b<|eos|>c", "<|bos|><|eos|>", "<|bos", "x <|eos|> y\n<|bos|>\n",
]


@pytest.mark.parametrize("text", EDGE)
def test_edge_cases(toks, text):
    prod, ref = toks
    got = prod.encode(text).tolist()
    exp = ref.encode(text)
    assert got == exp, (text, got, exp)
    assert prod.decode_bytes(got) == text.encode("utf-8")


def test_random_unicode_soup(toks):
    prod, ref = toks
    rng = np.random.default_rng(9)
    pool = list("abcXYZ019 \t\n\r'.,!?-_()\"") + ["é", "ß", "ж", "中", "の", "٣", "😀", " ", "　", "́",
                                                      "ſ", "Ⅻ", " ", "<|bos|>"]
    for _ in range(200):
        n = int(rng.integers(1, 60))
        text = "".join(pool[i] for i in rng.integers(0, len(pool), n))
        assert prod.encode(text).tolist() == ref.encode(text), repr(text)


def test_synthetic_text_and_threads(toks):
    from czip_amd import synth
    prod, ref = toks
    text = synth.synthetic_text(1 << 20, seed=3).decode()
    seq = prod.encode(text)
    assert seq.tolist() == ref.encode(text)
    par = prod.encode(text, threads=8)
    assert np.array_equal(seq, par)
    assert prod.decode_bytes(seq) == text.encode()
    # random-letter words merge little: the corpus tokenizes at ~1.3 bytes per token
    assert 1.0 < len(text) / len(seq) < 4.0


def test_invalid_utf8_and_unknown_token(toks):
    import czip_amd
    prod, _ = toks
    with pytest.raises(czip_amd.CzipError) as e:
        prod.encode(b"abc\xff")
    assert e.value.code == -11
    with pytest.raises(czip_amd.CzipError) as e:
        prod.decode_bytes([5000])
    assert e.value.code == -5
