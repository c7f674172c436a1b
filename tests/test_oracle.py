"""Pins the C oracle against the reference's own known-answer tests and
against what the mathematics fixes (exact rational rounding, integer square
roots, closed forms, round trips).  CPU only."""
import math
from fractions import Fraction

import numpy as np
import pytest

from conftest import MODEL_PATH


def rne(fr: Fraction) -> int:
    """Round a rational to nearest, ties to even (the rounding every RNE
    primitive of rust/src/primitives.rs is specified to perform)."""
    fl = math.floor(fr)
    rem = fr - fl
    if rem > Fraction(1, 2):
        return fl + 1
    if rem < Fraction(1, 2):
        return fl
    return fl if fl % 2 == 0 else fl + 1


def sym_rne(fr: Fraction) -> int:
    """sign(x) * RNE(|x|)"""
    return rne(fr) if fr >= 0 else -rne(-fr)


# ---- reference KATs: rust/src/primitives.rs:305-397 -------------------------

def test_sra_rne_s32_kats(orc):
    L = orc.lib()
    for v, sh, exp in [(100, 1, 50), (64, 2, 16), (-100, 1, -50), (3, 1, 2), (5, 1, 2), (7, 1, 4),
                       (-3, 1, -2), (-5, 1, -2), (-7, 1, -4), (5, 2, 1), (7, 2, 2),
                       # python/tests/test_primitives.py:181-186, test_cross_language.py:217-222
                       (1, 1, 0), (1234567, 10, 1206), (6, 1, 3), (9, 2, 2), (11, 2, 3), (100, 0, 100)]:
        assert L.orc_sra_rne_s32(v, sh) == exp, (v, sh)


def test_isqrt_kats(orc):
    L = orc.lib()
    for x, exp in [(0, 0), (1, 1), (4, 2), (9, 3), (15, 3), (16, 4), (65536, 256), (0xFFFFFFFF, 65535),
                   (1000000, 1000), (2147483647, 46340), (2, 1), (3, 1), (5, 2), (8, 2), (10, 3), (17, 4),
                   (2 ** 30, 2 ** 15)]:
        assert L.orc_isqrt32(x) == exp


def test_udiv_rne_kats(orc):
    L = orc.lib()
    # rust/src/primitives.rs:348-363
    for n, d, exp in [(10, 2, 5), (12, 4, 3), (3, 2, 2), (5, 2, 2), (7, 2, 4), (7, 4, 2),
                      # python/tests/test_primitives.py:99-116 (rows that agree with Rust)
                      (100, 10, 10), (10, 4, 2), (11, 4, 3), (14, 4, 4), (9, 3, 3), (11, 3, 4),
                      (10, 0, 0)]:
        assert L.orc_udiv_rne_u32(n, d) == exp, (n, d)
    # test_cross_language.py:256-257 expects 333334 / 4 (Python's odd-divisor rule);
    # the Rust rule (primitives.rs:88-96) gives the exact round-to-nearest: 333333 / 3.
    assert L.orc_udiv_rne_u32(1000000, 3) == 333333
    assert L.orc_udiv_rne_u32(10, 3) == 3


def test_clamp_argmax_kats(orc):
    L = orc.lib()
    for x, exp in [(0, 0), (127, 127), (128, 127), (-127, -127), (-128, -127), (-129, -127),
                   (1000, 127), (-1000, -127)]:
        assert L.orc_clamp_i8(x) == exp
    for arr, exp in [([1, 3, 2], 1), ([3, 3, 1], 0), ([1, 3, 3], 1), ([5, 5, 5, 5], 0), ([1, 3, 2, 5], 3)]:
        a = np.array(arr, np.int32)
        assert L.orc_argmax(a.ctypes.data, a.size) == exp


def test_inv_rms_kats(orc):
    # rust/src/rmsnorm.rs:136-149
    L = orc.lib()
    for ms, exp in [(1, 32768), (4, 16384), (16, 8192), (16384, 256)]:
        assert L.orc_inv_rms_q15(ms) == exp


def test_reglu_kats(orc):
    # rust/src/reglu.rs:53-99
    L = orc.lib()
    def rg(g, u):
        x = np.array([g, u], np.int8)
        o = np.zeros(1, np.int8)
        L.orc_reglu(x.ctypes.data, 1, o.ctypes.data)
        return int(o[0])
    assert rg(-64, 100) == 0
    assert rg(64, 64) == 32
    assert rg(32, 64) == 16
    assert rg(32, 2) == 0
    assert rg(96, 2) == 2


def test_requant_kat(orc):
    # rust/src/model.rs:502-508
    L = orc.lib()
    x = np.array([8192, 4096, -8192], np.int32)
    o = np.zeros(3, np.int8)
    L.orc_requant(x.ctypes.data, 3, 1, 7, o.ctypes.data)
    assert o.tolist() == [64, 32, -64]


def test_constants(orc):
    L = orc.lib()
    assert L.orc_cdf_coef_q24() == 37819          # test_cross_language.py:37
    assert L.orc_target_total(1024) == 1073739776  # test_cross_language.py:45
    assert L.orc_target_total(256) == (1 << 30) - 256 - 1024
    # attention.rs:19 formula: int(LOG2E/64 * 2^24 + 0.5)
    assert L.orc_attn_coef_q24() == int(1.4426950408889634 / 64.0 * (1 << 24) + 0.5) == 378194


def test_exp_neg_fixed_vectors(orc):
    # python/tests/test_lut.py:155-161
    lut = np.zeros(256, np.uint16)
    orc.lib().orc_gen_exp2_lut(lut.ctypes.data)
    for x, exp in [(0, 65535), (256, 32767), (512, 16383), (768, 8191)]:
        assert orc.lib().orc_exp_q16_from_neg_fixed(x, lut.ctypes.data) == exp


def test_luts_match_shipped_model(orc):
    """The LUT generators (lut.rs:40-52, 97-136) reproduce the tables stored
    in the shipped model, and the tables match the closed forms."""
    t, meta = orc.read_czm(MODEL_PATH)
    lut = np.zeros(256, np.uint16)
    orc.lib().orc_gen_exp2_lut(lut.ctypes.data)
    assert np.array_equal(lut, t["lut.exp2"])
    ref = np.array([min(65535, max(1, round(2 ** (-i / 256) * 65536))) for i in range(256)])
    assert np.array_equal(lut.astype(np.int64), ref)
    ctx = int(meta["context_length"])
    cs = np.zeros(ctx * 32, np.int16)
    sn = np.zeros(ctx * 32, np.int16)
    orc.lib().orc_gen_rope_lut(10000.0, ctx, cs.ctypes.data, sn.ctypes.data)
    assert np.array_equal(cs, t["lut.rope_cos"].reshape(-1))
    assert np.array_equal(sn, t["lut.rope_sin"].reshape(-1))
    assert int(t["softmax.coef_q24"]) == 37819 and int(t["softmax.target_total"]) == 1073739776


# ---- exactness against mathematics -----------------------------------------

def test_sra_rne_exact_rounding(orc):
    L = orc.lib()
    rng = np.random.default_rng(1)
    vals = list(rng.integers(-2 ** 31, 2 ** 31, 3000)) + [-2 ** 31, 2 ** 31 - 1, -1, 0, 1]
    for v in vals:
        v = int(v)
        for sh in (1, 2, 7, 15, 16, 20):
            assert L.orc_sra_rne_s32(v, sh) == max(-2 ** 31, min(2 ** 31 - 1, sym_rne(Fraction(v, 2 ** sh)))) or v == -2 ** 31
    for v in list(rng.integers(-2 ** 50, 2 ** 50, 3000)) + [2 ** 62, -2 ** 62]:
        v = int(v)
        for sh in (1, 15, 20, 31):
            exp = sym_rne(Fraction(v, 2 ** sh))
            assert L.orc_sra_rne_s64_to_s32(v, sh) == max(-2 ** 31, min(2 ** 31 - 1, exp))


def test_isqrt_exact(orc):
    L = orc.lib()
    rng = np.random.default_rng(2)
    for x in list(rng.integers(0, 2 ** 32, 20000)) + list(range(0, 5000)):
        assert L.orc_isqrt32(int(x)) == math.isqrt(int(x))


def test_div_exact(orc):
    L = orc.lib()
    rng = np.random.default_rng(3)
    for _ in range(20000):
        n = int(rng.integers(0, 2 ** 32))
        d = int(rng.integers(1, 2 ** 16))
        assert L.orc_udiv_rne_u32(n, d) == rne(Fraction(n, d)) % 2 ** 32
        s = int(rng.integers(-2 ** 31 + 1, 2 ** 31))
        D = int(rng.integers(1, 2 ** 40))
        assert L.orc_div_rne_s32_by_u64(s, D) == sym_rne(Fraction(s, D))


def test_inv_rms_exhaustive(orc):
    """All mean_sq values a d>=1 row of int8 can produce (<= 127^2 + eps):
    inv = clamp(RNE(2^23 / floor(sqrt(ms*2^16))), 1, 32768)."""
    L = orc.lib()
    for ms in range(1, 127 * 127 + 2):
        s = math.isqrt(ms << 16)
        exp = min(32768, max(1, rne(Fraction(8388608, s))))
        assert L.orc_inv_rms_q15(ms) == exp


def test_inv_rms_f64_form_exhaustive(orc):
    """The device's inv_rms form (f64 sqrt + exact integer correction, f64
    quotient estimate + exact remainder test) against the oracle on every
    mean_sq < 2^16.  The corrections tolerate a +-1 error of either f64
    estimate, so this pins the algorithm whatever the hardware rounding."""
    L = orc.lib()

    def fast(ms, sq_err=0, q_err=0):
        x = max(ms, 1) << 16
        r = int(math.sqrt(float(x))) + sq_err
        if r * r > x:
            r -= 1
        if (r + 1) * (r + 1) <= x:
            r += 1
        q = int(8388608.0 / float(r)) + q_err
        rem = 8388608 - q * r
        if rem < 0:
            q, rem = q - 1, rem + r
        if rem >= r:
            q, rem = q + 1, rem - r
        tr = 2 * rem
        inv = q + 1 if tr > r else (q + (q & 1) if tr == r else q)
        return min(max(inv, 1), 32768)

    for ms in range(0, 1 << 16):
        exp = L.orc_inv_rms_q15(ms)
        assert fast(ms) == exp, ms
        if ms % 97 == 0:
            for e1 in (-1, 1):
                assert fast(ms, sq_err=e1) == exp and fast(ms, q_err=e1) == exp, ms


def test_reglu_exhaustive(orc):
    L = orc.lib()
    g = np.repeat(np.arange(-127, 128), 255).astype(np.int8)
    u = np.tile(np.arange(-127, 128), 255).astype(np.int8)
    n = g.size
    x = np.concatenate([g, u]).astype(np.int8)
    o = np.zeros(n, np.int8)
    L.orc_reglu(x.ctypes.data, n, o.ctypes.data)
    exp = [max(-127, min(127, sym_rne(Fraction(max(int(a), 0) * int(b), 128)))) for a, b in zip(g[::97], u[::97])]
    assert o[::97].tolist() == exp


def test_linear_matches_int64_matmul(orc):
    L = orc.lib()
    rng = np.random.default_rng(4)
    for b, k, n in [(1, 384, 512), (3, 64, 17), (2, 1024, 384)]:
        x = rng.integers(-127, 128, (b, k)).astype(np.int8)
        w = rng.integers(-127, 128, (n, k)).astype(np.int8)
        o = np.zeros((b, n), np.int32)
        L.orc_linear_i8_to_i32(x.ctypes.data, w.ctypes.data, b, k, n, o.ctypes.data)
        assert np.array_equal(o, x.astype(np.int64) @ w.astype(np.int64).T)


def test_rope_closed_form(orc):
    L = orc.lib()
    rng = np.random.default_rng(5)
    for _ in range(200):
        x = rng.integers(-127, 128, 64).astype(np.int8)
        c = rng.integers(-32768, 32768, 32).astype(np.int16)
        s = rng.integers(-32768, 32768, 32).astype(np.int16)
        k = x.copy(); q = x.copy()
        L.orc_rope_k(k.ctypes.data, c.ctypes.data, s.ctypes.data)
        L.orc_rope_q(q.ctypes.data, c.ctypes.data, s.ctypes.data)
        for i in range(32):
            a, b = int(x[i]), int(x[i + 32])
            xr = a * int(c[i]) - b * int(s[i])
            yr = a * int(s[i]) + b * int(c[i])
            cl = lambda v: max(-127, min(127, v))
            assert k[i] == cl(sym_rne(Fraction(xr, 2 ** 15))) and k[i + 32] == cl(sym_rne(Fraction(yr, 2 ** 15)))
            # Q: two successive roundings (attention.rs:68-74)
            assert q[i] == cl(sym_rne(Fraction(sym_rne(Fraction(xr, 2 ** 15)), 2)))
            assert q[i + 32] == cl(sym_rne(Fraction(sym_rne(Fraction(yr, 2 ** 15)), 2)))


def _exp_coef(d, lut, coef):
    """exp2(-|d|*coef/2^24) with the 8-bit LUT fraction, in closed form."""
    if d >= 0:
        return 65535
    t = ((-d) * coef + (1 << 23)) >> 24
    ip, fr = t >> 8, t & 255
    if ip >= 31:
        return 1
    return min(65535, max(1, (((1 << 16) >> ip) * int(lut[fr]) + 0x8000) >> 16))


def test_exp_coef_and_monotone(orc):
    L = orc.lib()
    lut = np.zeros(256, np.uint16)
    L.orc_gen_exp2_lut(lut.ctypes.data)
    prev = 65535
    for d in range(0, -400000, -97):
        e = L.orc_exp_q16_coef(d, lut.ctypes.data, 37819)
        assert e <= prev
        prev = e
        # t256 = |d|*coef/2^24 is the exponent in 1/256 steps: e ~ 2^16 * 2^(-|d|*coef/2^32),
        # accurate to one 8-bit LUT step
        real = 65536 * 2.0 ** (d * 37819 / 2.0 ** 32)
        assert abs(e - min(real, 65535)) <= max(2.0, real * 0.004)
    for d in [-1, -100, -5000, -2 ** 31, 0, 17]:
        assert L.orc_exp_q16_coef(d, lut.ctypes.data, 378194) == _exp_coef(d, lut, 378194)


def test_cumfreqs_properties(orc):
    t, _ = orc.read_czm(MODEL_PATH)
    lut = t["lut.exp2"]
    T = 1073739776
    rng = np.random.default_rng(6)
    # closed form for uniform logits: all e = 65535, f = 1 + floor(R/V), rest to index 0
    for v in (4, 16, 1024):
        cum = orc.build_cumfreqs(np.full(v, 1000, np.int32), lut, 37819, T)
        f = np.diff(np.concatenate([[0], cum.astype(np.int64)]))
        base = 1 + (T - v) // v
        assert (f[1:] == base).all() and f[0] == T - base * (v - 1)
    for v in (2, 16, 1024, 8192):
        lg = rng.integers(-2 ** 21, 2 ** 21, v).astype(np.int32)
        cum = orc.build_cumfreqs(lg, lut, 37819, T)
        f = np.diff(np.concatenate([[0], cum.astype(np.int64)]))
        assert cum[-1] == T and (f >= 1).all()
        e = np.array([_exp_coef(int(x) - int(lg.max()), lut, 37819) for x in lg], np.int64)
        S = int(e.sum())
        exp_f = 1 + (e * (T - v)) // S
        am = int(np.argmax(lg))
        exp_f[am] += T - int(exp_f.sum())
        assert np.array_equal(f, exp_f)
    # rust/src/softmax_cdf.rs:190-248
    lg = np.array([100, 50, 25, 10, 5, 0, -5, -10, -25, -50, -100, -200, -300, -400, -500, -1000], np.int32)
    cum = orc.build_cumfreqs(lg, lut, 37819, orc.lib().orc_target_total(16))
    assert cum[-1] == orc.lib().orc_target_total(16) and (np.diff(cum.astype(np.int64)) > 0).all()


def test_coder_roundtrip_uniform(orc):
    """rust/src/arith_coder.rs:277-331 round trips."""
    cum = np.arange(1, 9, dtype=np.uint32) * 1000
    for syms in ([2], [0, 3, 7, 2, 5, 1], [i % 8 for i in range(16)]):
        enc = orc.encode_symbols(cum, syms)
        assert orc.decode_symbols(enc, cum, len(syms)) == syms


def test_coder_random_distributions(orc):
    L = orc.lib()
    rng = np.random.default_rng(7)
    for trial in range(20):
        v = int(rng.integers(2, 300))
        f = rng.integers(1, 1 << int(rng.integers(1, 20)), v).astype(np.uint64)
        cum = np.cumsum(f).astype(np.uint32)
        syms = rng.integers(0, v, 400).tolist()
        data = orc.encode_symbols(cum, syms)
        assert orc.decode_symbols(data, cum, len(syms)) == syms


def test_chunk_roundtrip_shipped(orc, shipped):
    rng = np.random.default_rng(8)
    toks = rng.integers(0, 1024, 200).astype(np.uint32)
    chunks = shipped.compress_many(toks, 64, threads=2)
    assert len(chunks) == 4
    out = shipped.decompress_many(chunks, [64, 64, 64, 8], threads=2)
    assert np.array_equal(out, toks)
    # a chunk equals its stand-alone compression (fresh state per chunk, main.rs:215)
    assert chunks[1] == shipped.compress_chunk(toks[64:128])


def test_model_check_codes(orc):
    t, meta = orc.read_czm(MODEL_PATH)
    m = orc.Model(t, dict(meta, n_heads="5", d_model="320"))
    assert m.check() == -3    # n_heads not in {4,6,8} panics in attention.rs:172
