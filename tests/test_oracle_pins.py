"""Pins of the oracle's attention (attention.rs:197-285), its LUT exp
(lut.rs:213-235 / softmax_cdf.rs:55-77) and the BPE merge (tiktoken.rs:26-107)
against what the mathematics fixes: closed forms of the online softmax on
inputs whose score pattern is known (one key, equal scores, non-increasing
scores, one record, the i32 wrap), the exponent's distance from
2^(16 - t/256) in table steps, and BPE as "merge the lowest-ranked adjacent
pair, leftmost first" run naively.  CPU only."""
import math
from fractions import Fraction

import numpy as np
import pytest

from conftest import GQA_PIN_SHAPES, MODEL_PATH, gqa_pin_logits, write_gqa_pin_model

ACOEF = 378194  # ATTN_COEF_Q24 (attention.rs:17-19)
CCOEF = 37819   # softmax.coef_q24 of the shipped model


def sym_rne(fr: Fraction) -> int:
    """sign(x) * round-half-even(|x|)."""
    a = abs(fr)
    fl = math.floor(a)
    rem = a - fl
    r = fl + 1 if rem > Fraction(1, 2) else fl if rem < Fraction(1, 2) else (fl if fl % 2 == 0 else fl + 1)
    return r if fr >= 0 else -r


def clamp127(x: int) -> int:
    return max(-127, min(127, x))


@pytest.fixture(scope="module")
def lut(orc):
    t, _ = orc.read_czm(MODEL_PATH)
    return np.ascontiguousarray(t["lut.exp2"], np.uint16)


def E(orc, d, lut, coef=ACOEF):
    return int(orc.lib().orc_exp_q16_coef(int(d), lut.ctypes.data, coef))


def score_of(dot: int, mult: int) -> int:
    """sra_rne(sra_rne(dot, 2) * mult, 15) for scores far inside the i32 range."""
    return sym_rne(Fraction(sym_rne(Fraction(dot, 4)) * mult, 1 << 15))


# ---- the exponent ----------------------------------------------------------------

@pytest.mark.parametrize("coef", [ACOEF, CCOEF])
def test_exp_within_half_a_table_step(orc, lut, coef):
    """E(d) = 2^16 * 2^(-t/256) with t the nearest table step to |d|*coef/2^24:
    in table steps, -256*log2(E/2^16) stays within 0.5 (+ the LUT's and the
    final product's rounding, < 0.06 step while E >= 2^12) of |d|*coef/2^24.
    An index off by one step, or truncated instead of rounded, leaves that
    band on most inputs."""
    rng = np.random.default_rng(coef)
    d_max = (4 * 256) * (1 << 24) // coef  # t <= 4 * 256 steps: E >= 2^12
    worst = 0.0
    for d in np.concatenate([rng.integers(1, d_max, 4000), np.arange(1, 600)]):
        e = E(orc, -int(d), lut, coef)
        t_real = int(d) * coef / float(1 << 24)
        err = -256.0 * math.log2(e / 65536.0) - t_real
        worst = max(worst, abs(err))
        assert abs(err) <= 0.56, (int(d), e, err)
    assert worst > 0.45  # the band is reached, so it is not loose by construction


@pytest.mark.parametrize("coef", [ACOEF, CCOEF])
def test_exp_anchors_and_monotone(orc, lut, coef):
    assert E(orc, 0, lut, coef) == 65535
    for d in (1, 17, 1 << 20, (1 << 31) - 1):
        assert E(orc, d, lut, coef) == 65535  # d >= 0 reads "no decay"
    # t >= 17 * 256: the integer part shifts 2^16 to zero; the result is clamped to 1
    d17 = -((17 * 256) * (1 << 24) // coef + 1)
    for d in (d17, d17 - 12345, -(1 << 31)):
        assert E(orc, d, lut, coef) == 1
    prev = 65535
    for d in range(0, d17 - 1000, -max(1, (-d17) // 20000)):
        e = E(orc, d, lut, coef)
        assert 1 <= e <= prev
        prev = e


# ---- attention closed forms ------------------------------------------------------

def test_one_key_gives_its_value(orc, lut):
    """Position 0: one key, w = S = E(0) = 65535, out = RNE(65535 v / 65535) = v
    (clamped to +-127), whatever q, k and the multiplier."""
    rng = np.random.default_rng(1)
    for trial in range(200):
        q = rng.integers(-128, 128, 64)
        k = rng.integers(-128, 128, (1, 64))
        v = rng.integers(-128, 128, (1, 64))
        mult = int(rng.integers(-(1 << 20), 1 << 20))
        out, vacc, S = orc.attend_head(q, k, v, mult, lut)
        assert S == 65535
        assert np.array_equal(vacc, 65535 * v[0])
        assert np.array_equal(out, np.clip(v[0], -127, 127))


def test_equal_scores_give_the_rounded_mean(orc, lut):
    """n keys of one score: no record after the first key, every weight is
    E(0) = 65535, so S = 65535 n and out = clamp(RNE(sum v / n))."""
    rng = np.random.default_rng(2)
    for n in (1, 2, 3, 7, 64, 65, 200, 255):
        q = np.zeros(64, np.int64) if n % 2 else rng.integers(-128, 128, 64)
        k = np.repeat(rng.integers(-128, 128, (1, 64)), n, axis=0)  # one key row repeated: one score
        v = rng.integers(-127, 128, (n, 64))
        out, vacc, S = orc.attend_head(q, k, v, 59000, lut)
        assert S == 65535 * n
        sv = v.sum(axis=0)
        assert np.array_equal(vacc, 65535 * sv)
        assert out.tolist() == [clamp127(sym_rne(Fraction(int(x), n))) for x in sv]


def test_sink_with_an_equal_score(orc, lut):
    """A sink whose score equals every key's (q = 0) adds weight 65535 with a
    zero value: S = 65535 (n + 1), out = RNE(sum v / (n + 1)) (attention.rs:211-224)."""
    rng = np.random.default_rng(3)
    for n in (1, 5, 64, 130):
        k = rng.integers(-128, 128, (n, 64))
        v = rng.integers(-127, 128, (n, 64))
        sink = rng.integers(-128, 128, 64)
        out, vacc, S = orc.attend_head(np.zeros(64), k, v, 40000, lut, sink=sink)
        assert S == 65535 * (n + 1)
        sv = v.sum(axis=0)
        assert out.tolist() == [clamp127(sym_rne(Fraction(int(x), n + 1))) for x in sv]


def test_non_increasing_scores_are_one_weighted_mean(orc, lut):
    """Scores that never rise after the first key: the first key sets the
    max and no rescale follows, so S = sum E(s_t - s_0) and
    out = clamp(RNE(sum E(s_t - s_0) v_t / S)) exactly."""
    rng = np.random.default_rng(4)
    for trial in range(60):
        n = int(rng.integers(2, 160))
        mult = int(rng.integers(1000, 65536))
        q = np.zeros(64, np.int64)
        q[0] = int(rng.integers(1, 128))
        k = rng.integers(-128, 128, (n, 64))
        k[:, 0] = np.sort(rng.integers(-128, 128, n))[::-1]  # dot = q0 * k0 non-increasing
        v = rng.integers(-127, 128, (n, 64))
        s = [score_of(int(q[0]) * int(k[t, 0]), mult) for t in range(n)]
        assert all(s[t + 1] <= s[t] for t in range(n - 1))
        w = [E(orc, s[t] - s[0], lut) for t in range(n)]
        S = sum(w)
        num = [sum(w[t] * int(v[t, i]) for t in range(n)) for i in range(64)]
        assert max(abs(x) for x in num) < 1 << 31
        out, vacc, S_got = orc.attend_head(q, k, v, mult, lut)
        assert S_got == S
        assert vacc.tolist() == num
        assert out.tolist() == [clamp127(sym_rne(Fraction(x, S))) for x in num]


def _rescale(p: int) -> int:
    """attention.rs:246-261: (p + 2^15) >> 16 for p >= 0, (p - 2^15) >> 16 (a
    floor) below 0, i.e. floor((p +- 2^15) / 2^16)."""
    return math.floor(Fraction(p + (1 << 15) if p >= 0 else p - (1 << 15), 1 << 16))


def test_one_record(orc, lut):
    """Keys 0..r-1 at score a, key r at score b > a, keys after at a again:
    one rescale at key r by e = E(a - b) of S and vacc, then key r at full
    weight and the later keys at e:
        S = floor((65535 r e + 2^15) / 2^16) + 65535 + (n - r - 1) e
        vacc = rescale(65535 sum_{t<r} v_t) + 65535 v_r + e sum_{t>r} v_t."""
    rng = np.random.default_rng(5)
    for trial in range(80):
        n = int(rng.integers(2, 150))
        r = int(rng.integers(1, n))
        mult = int(rng.integers(500, 65536))
        q = np.zeros(64, np.int64)
        q[1] = int(rng.integers(1, 128))
        lo, hi = sorted(rng.choice(np.arange(-128, 128), 2, replace=False))
        k = rng.integers(-128, 128, (n, 64))
        k[:, 1] = lo
        k[r, 1] = hi
        v = rng.integers(-127, 128, (n, 64))
        a, b = score_of(int(q[1]) * int(lo), mult), score_of(int(q[1]) * int(hi), mult)
        if b <= a:
            continue
        e = E(orc, a - b, lut)
        S = (65535 * r * e + (1 << 15)) // (1 << 16) + 65535 + (n - r - 1) * e
        pre = v[:r].sum(axis=0)
        post = v[r + 1:].sum(axis=0)
        num = [_rescale(65535 * int(pre[i]) * e) + 65535 * int(v[r, i]) + e * int(post[i]) for i in range(64)]
        out, vacc, S_got = orc.attend_head(q, k, v, mult, lut)
        assert S_got == S
        assert vacc.tolist() == num
        assert out.tolist() == [clamp127(sym_rne(Fraction(x, S))) for x in num]


def test_rescale_rounding_is_not_symmetric():
    """The closed form of attention.rs:246-261 rounds negative products down:
    p = -1 gives -1 where a symmetric rounding would give 0."""
    assert _rescale(-1) == -1 and _rescale(1) == 0
    assert _rescale(-(1 << 15)) == -1 and _rescale((1 << 15) - 1) == 0 and _rescale(1 << 15) == 1


def test_vacc_wraps_like_a_release_build(orc, lut):
    """512 keys of one score with v = +127 (even dims) and -127 (odd dims):
    S = 65535 * 512 and vacc = +-65535 * 127 * 512 mod 2^32 read as i32, the
    wrap of a Rust --release build (attention.rs:207-208, 274); the output is
    the RNE quotient of the wrapped value, +-1 instead of +-127."""
    n = 512
    v = np.tile(np.where(np.arange(64) % 2 == 0, 127, -127), (n, 1))
    k = np.zeros((n, 64), np.int64)
    orc.reset_vacc_wraps()
    out, vacc, S = orc.attend_head(np.zeros(64), k, v, 59000, lut)
    assert orc.vacc_wraps() > 0
    exact = 65535 * 127 * n
    wrapped = (exact + (1 << 31)) % (1 << 32) - (1 << 31)
    assert S == 65535 * n
    assert vacc.tolist() == [wrapped if i % 2 == 0 else -wrapped for i in range(64)]
    q1 = clamp127(sym_rne(Fraction(wrapped, S)))
    assert q1 == -1
    assert out.tolist() == [q1 if i % 2 == 0 else -q1 for i in range(64)]
    # below 2^31 / (65535 * 127) = 258.0 keys nothing wraps
    orc.reset_vacc_wraps()
    out, vacc, S = orc.attend_head(np.zeros(64), k[:258], v[:258], 59000, lut)
    assert orc.vacc_wraps() == 0 and out.tolist() == [127 if i % 2 == 0 else -127 for i in range(64)]


# ---- BPE ---------------------------------------------------------------------------

def naive_bpe(piece: bytes, ranks: dict):
    """BPE by its definition: while some adjacent pair of parts concatenates
    to a ranked token, merge the pair of lowest rank (leftmost among equals)."""
    parts = [piece[i:i + 1] for i in range(len(piece))]
    while len(parts) > 1:
        best = None
        for i in range(len(parts) - 1):
            r = ranks.get(parts[i] + parts[i + 1])
            if r is not None and (best is None or r < best[0]):
                best = (r, i)
        if best is None:
            break
        i = best[1]
        parts[i:i + 2] = [parts[i] + parts[i + 1]]
    return [ranks[p] for p in parts]


@pytest.fixture(scope="module")
def spec(orc):
    import json
    import tokenizer_oracle as TO
    t, _ = orc.read_czm(MODEL_PATH)
    return json.loads(TO.decompress_zstd(bytes(t["tokenizer.data"].reshape(-1))))


def test_bpe_kats(spec):
    """tiktoken.rs:569-588 (byte_pair_encode of b"ab"), plus longer pieces of the same tables."""
    import json
    import czip_amd
    for ranks, text, exp in [({"a": 0, "b": 1, "ab": 2}, "ab", [2]), ({"a": 0, "b": 1}, "ab", [0, 1]),
                             ({"a": 0, "b": 1, "ab": 2}, "abab", [2, 2]), ({"a": 0, "b": 1, "ab": 2}, "aab", [0, 2]),
                             ({"a": 0, "b": 1, "ab": 2, "ba": 3}, "aba", [2, 0]),
                             ({"a": 0, "b": 1, "ba": 2, "ab": 3}, "aba", [0, 2])]:
        s = dict(spec, mergeable_ranks=ranks, special_tokens={}, explicit_n_vocab=None)
        tk = czip_amd.Tokenizer(json_bytes=json.dumps(s).encode())
        assert tk.encode(text).tolist() == exp, (ranks, text)


def test_bpe_against_naive_merge(spec, orc):
    """The product's BPE and the oracle's restated merge loop both equal the
    naive lowest-rank merge (after the whole-piece lookup of tiktoken.rs:249-256)
    on every pre-split piece of a text and on random letter strings (each a
    single piece, 2-39 letters and 100-399 letters), with the shipped model's
    1022 ranks."""
    import czip_amd
    import tokenizer_oracle as TO
    from czip_amd import synth
    ranks = {bytes(ord(ch) for ch in k): v for k, v in spec["mergeable_ranks"].items()}

    def encode_piece(b):
        return [ranks[b]] if b in ranks else naive_bpe(b, ranks)

    prod = czip_amd.Tokenizer(czip_amd.ModelWeights(MODEL_PATH))
    ref = TO.Tokenizer(spec)
    text = synth.synthetic_text(1 << 16, seed=77).decode()
    exp = []
    for p in ref.pieces(text):
        b = p.encode()
        e = encode_piece(b)
        if len(b) > 1:
            assert ref.byte_pair_encode(b) == naive_bpe(b, ranks), p
        exp.extend(e)
    assert prod.encode(text).tolist() == exp
    rng = np.random.default_rng(6)
    for i in range(1560):
        n = int(rng.integers(2, 40)) if i < 1500 else int(rng.integers(100, 400))
        w = "".join(chr(97 + c) for c in rng.integers(0, 26, n))
        assert ref.pieces(w) == [w]
        e = encode_piece(w.encode())
        assert ref.byte_pair_encode(w.encode()) == naive_bpe(w.encode(), ranks)
        assert prod.encode(w).tolist() == e, w


@pytest.mark.parametrize("H,G", GQA_PIN_SHAPES)
def test_gqa_group_mapping_closed_form(orc, tmp_path, H, G):
    """GQA mode (the extension beyond attention.rs:172-194): with zero
    queries and keys and KV group g's values all g + 1, head h's output is
    floor(h G / H) + 1, which the logits of write_gqa_pin_model expose.  A
    mapping h % G, or values taken from the key slice, gives other logits."""
    path = write_gqa_pin_model(str(tmp_path / f"gqa{H}_{G}.czm"), H, G)
    exp = gqa_pin_logits(H, G)
    d = 64 * H
    per_head = exp[:d].reshape(H, 64)
    assert (per_head == per_head[:, :1]).all()
    # distinct groups give distinct logits, so the check sees the grouping
    groups = [h * G // H for h in range(H)]
    vals = {g: int(per_head[h, 0]) for h, g in enumerate(groups)}
    assert len(set(vals.values())) == G
    if G not in (1, H):
        assert [int(per_head[h, 0]) for h in range(H)] != [vals[h % G] for h in range(H)]
    om = orc.Model.from_file(path, orc.KV_GQA)
    inp = np.array([1022] + list(range(0, 700, 7))[:95], np.uint32)
    lg, _ = om.trace(inp)
    assert (lg == exp[None, :]).all()


def test_gqa_one_group_equals_reference_slicing(orc, tmp_path):
    """With one KV group, GQA mode and the reference's slicing
    (attention.rs:174-194) read the same K and V: the same chunk bytes."""
    from czip_amd import synth
    path = synth.write_random_model(str(tmp_path / "g1.czm"), d=384, n_layers=2, n_heads=6, n_kv=1, d_ff=512,
                                    vocab=1024, ctx=128, seed=44)
    toks = synth.zipf_ids(128 * 2 + 40, 1024, seed=45)
    a = orc.Model.from_file(path, orc.KV_GQA).compress_many(toks, 128, threads=4)
    b = orc.Model.from_file(path, orc.KV_RUST_COMPAT).compress_many(toks, 128, threads=4)
    assert a == b
