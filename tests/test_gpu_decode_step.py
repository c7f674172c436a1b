"""The step-wise decode boundary (czip_decode_begin / czip_decode_step) driven
the way a caller that keeps its own arithmetic decoder drives it: the
per-token loop of main.rs:381-391 for many streams at once, with the
decoder state machine of arith_coder.rs:139-264 on the host.  The chunks are
coded by the oracle; the decoded tokens must be the oracle's input."""
import numpy as np
import pytest

from conftest import MODEL_PATH

pytestmark = pytest.mark.gpu

MASK = (1 << 32) - 1
HALF = 1 << 31
QUARTER = 1 << 30


class HostDecoder:
    """ArithDecoder (arith_coder.rs:139-264) with the symbol search left to the
    device: value() is the target of decode_symbol (:199-203), narrow() its
    interval update (:212-216) and renormalisation (:244-264)."""

    def __init__(self, data: bytes):
        self.data, self.byte_pos, self.bit_pos = data, 0, 7
        self.low, self.high, self.code = 0, MASK, 0
        for _ in range(32):
            self.code = (self.code << 1) | self.bit()

    def bit(self):
        if self.byte_pos >= len(self.data):
            return 0
        b = (self.data[self.byte_pos] >> self.bit_pos) & 1
        self.bit_pos -= 1
        if self.bit_pos < 0:
            self.byte_pos, self.bit_pos = self.byte_pos + 1, 7
        return b

    def value(self, total):
        rng = self.high - self.low + 1
        return ((self.code - self.low + 1) * total - 1) // rng

    def narrow(self, lo, hi, total):
        rng = self.high - self.low + 1
        self.high = self.low + hi * rng // total - 1
        self.low = self.low + lo * rng // total
        while True:
            if (self.low ^ self.high) & HALF == 0:
                self.low = (self.low << 1) & MASK
                self.high = ((self.high << 1) & MASK) | 1
                self.code = ((self.code << 1) & MASK) | self.bit()
            elif self.low & ~self.high & QUARTER:
                self.low = ((self.low << 1) ^ HALF) & MASK
                self.high = (((self.high ^ HALF) << 1) | HALF | 1) & MASK
                self.code = (self.code & HALF) | ((self.code << 1) & (MASK >> 1)) | self.bit()
            else:
                break


@pytest.fixture(scope="module")
def amd():
    import czip_amd
    if czip_amd.device_count() < 1:
        pytest.fail("no HIP device visible")
    return czip_amd


def _decode_streams(gm, chunks, ntoks, T, total, check_tables_every=0):
    S = len(chunks)
    decs = [HostDecoder(c) for c in chunks]
    out = [[] for _ in range(S)]
    gm.decode_begin(S, T)
    try:
        for p in range(max(ntoks)):
            pos = np.array([p if p < n else -1 for n in ntoks], np.int32)
            tok_in = np.array([1022 if p == 0 else (out[s][-1] if p < ntoks[s] else 0) for s in range(S)], np.uint32)
            vals = np.array([decs[s].value(total) if pos[s] >= 0 else 0 for s in range(S)], np.uint32)
            if check_tables_every and p % check_tables_every == 0:
                # the full tables at the same step (the cache write at p is the same again)
                cum = gm.decode_step(tok_in, pos, None)
            res = gm.decode_step(tok_in, pos, vals)
            for s in range(S):
                if pos[s] < 0:
                    assert res[s].tolist() == [0, 0, 0]
                    continue
                sym, lo, hi = (int(x) for x in res[s])
                if check_tables_every and p % check_tables_every == 0:
                    row = cum[s].astype(np.int64)
                    exp = min(int(np.searchsorted(row, int(vals[s]), side="right")), row.size - 1)
                    assert sym == exp and hi == row[sym] and lo == (row[sym - 1] if sym else 0), (s, p)
                    assert row[-1] == total
                decs[s].narrow(lo, hi, total)
                out[s].append(sym)
    finally:
        gm.decode_end()
    return np.concatenate([np.array(o, np.uint32) for o in out])


def test_decode_step_shipped_72_streams(amd, orc):
    """72 streams of 128-token chunks (ragged last one) of the shipped model:
    tokens recovered through the value -> (symbol, interval) boundary, and at
    every 16th step the full tables agree with the symbol search."""
    gm = amd.Model(amd.ModelWeights(MODEL_PATH))
    om = orc.Model.from_file(MODEL_PATH)
    from czip_amd import synth
    n = 71 * 128 + 45
    toks = synth.zipf_ids(n, 1024, seed=101)
    chunks = om.compress_many(toks, 128, threads=8)
    ntoks = [min(128, n - 128 * c) for c in range(len(chunks))]
    print(f"decode_step shipped: {len(chunks)} streams", flush=True)
    got = _decode_streams(gm, chunks, ntoks, 128, gm.target_total, check_tables_every=16)
    assert np.array_equal(got, toks)


def test_decode_step_gqa_model(amd, orc, tmp_path):
    """Two KV heads in GQA mode, two layers, 64 streams of 96 tokens."""
    from czip_amd import synth
    path = synth.write_random_model(str(tmp_path / "g.czm"), d=512, n_layers=2, n_heads=8, n_kv=2, d_ff=1024,
                                    vocab=1024, ctx=256, seed=102)
    gm = amd.Model(amd.ModelWeights(path, amd.KV_GQA))
    om = orc.Model.from_file(path, amd.KV_GQA)
    n = 64 * 96
    toks = synth.zipf_ids(n, 1024, seed=103)
    chunks = om.compress_many(toks, 96, threads=8)
    print("decode_step GQA: 64 streams", flush=True)
    got = _decode_streams(gm, chunks, [96] * 64, 96, gm.target_total, check_tables_every=32)
    assert np.array_equal(got, toks)


def _step_case(i: int) -> dict:
    rng = np.random.default_rng(9100 + i)
    compat = rng.random() < 0.35
    if compat:
        H = int(rng.choice([4, 6, 8]))
        n_kv = int(rng.integers(1, -(-(64 * H + 256) // 128)))  # one MQA row (attention.rs:176)
    else:
        H = int(rng.choice([1, 2, 3, 4, 6, 8, 12, 16]))
        n_kv = int(rng.choice([g for g in range(1, H + 1) if H % g == 0]))
    T = int(rng.integers(16, 161))
    return dict(d=64 * H, n_heads=H, n_kv=n_kv, d_ff=64 * int(rng.integers(1, 33)),
                vocab=int(rng.choice([1024, 1088, 2048, 8192])), n_layers=int(rng.integers(1, 4)),
                sink=bool(rng.random() < 0.3), compat=compat, T=T, ctx=T + int(rng.integers(0, 40)),
                streams=int(rng.integers(3, 25)), tail=int(rng.integers(1, T + 1)), seed=9100 + i)


@pytest.mark.parametrize("i", range(8))
def test_decode_step_random_shapes(amd, orc, tmp_path, i):
    """Seeded random models (1-16 heads, both KV modes, vocabularies to 8192,
    sinks) through the step-wise boundary: 3-24 streams, a ragged last one,
    and the full tables checked against the symbol search every 8 steps."""
    from czip_amd import synth
    c = _step_case(i)
    print(f"decode_step case {i}: {c}", flush=True)
    path = synth.write_random_model(str(tmp_path / f"s{i}.czm"), d=c["d"], n_layers=c["n_layers"], n_heads=c["n_heads"],
                                    n_kv=c["n_kv"], d_ff=c["d_ff"], vocab=c["vocab"], ctx=c["ctx"], seed=c["seed"],
                                    sink=c["sink"])
    kv = amd.KV_RUST_COMPAT if c["compat"] else amd.KV_GQA
    gm = amd.Model(amd.ModelWeights(path, kv))
    om = orc.Model.from_file(path, kv)
    T, S = c["T"], c["streams"]
    n = (S - 1) * T + c["tail"]
    toks = synth.zipf_ids(n, c["vocab"], seed=c["seed"] + 1)
    chunks = om.compress_many(toks, T, threads=8)
    ntoks = [min(T, n - T * k) for k in range(len(chunks))]
    got = _decode_streams(gm, chunks, ntoks, T, gm.target_total, check_tables_every=8)
    assert np.array_equal(got, toks)


def test_decode_step_errors(amd):
    gm = amd.Model(amd.ModelWeights(MODEL_PATH))
    with pytest.raises(amd.CzipError) as e:
        gm.decode_step(np.zeros(2, np.uint32), np.zeros(2, np.int32))
    assert e.value.code == -1  # no session
    with pytest.raises(amd.CzipError) as e:
        gm.decode_begin(4, 2048)  # past the 1024-entry RoPE table
    assert e.value.code == -4
    gm.decode_begin(4, 64)
    try:
        with pytest.raises(amd.CzipError) as e:
            gm.decode_step(np.full(4, 1022, np.uint32), np.array([0, 0, 1, 0], np.int32))
        assert e.value.code == -1  # streams at different positions
        with pytest.raises(amd.CzipError) as e:
            gm.decode_step(np.full(4, 1022, np.uint32), np.full(4, 64, np.int32))
        assert e.value.code == -4  # position past T
        with pytest.raises(amd.CzipError) as e:
            gm.decode_step(np.array([1022, 5000, 1, 2], np.uint32), np.zeros(4, np.int32))
        assert e.value.code == -5
        assert not gm.decode_step(np.zeros(4, np.uint32), np.full(4, -1, np.int32)).any()
        with pytest.raises(amd.CzipError) as e:
            gm.decode_step(np.full(4, 1022, np.uint32), np.full(4, 1, np.int32))
        assert e.value.code == -1  # position 0 never decoded
        bos = np.full(4, 1022, np.uint32)
        gm.decode_step(bos, np.array([0, 0, -1, -1], np.int32))
        gm.decode_step(np.array([5, 6, 0, 0], np.uint32), np.array([1, 1, -1, -1], np.int32))
        with pytest.raises(amd.CzipError) as e:
            # stream 2 joins at position 2 with no cached keys before it
            gm.decode_step(np.array([5, 6, 7, 0], np.uint32), np.array([2, 2, 2, -1], np.int32))
        assert e.value.code == -1
        # streams that begin at 0 (a new chunk) may join at any step, and a
        # stream may repeat a position it has reached
        gm.decode_step(bos, np.array([-1, -1, 0, 0], np.int32))
        gm.decode_step(np.array([5, 6, 0, 0], np.uint32), np.array([1, 1, -1, -1], np.int32))
    finally:
        gm.decode_end()
