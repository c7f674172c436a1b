"""Writes the golden fixtures of tests/golden/ from the reference's Python
mirror (python/compress_zip of the reference tree), as an executor of the
algorithm that is independent of this repository's C oracle and HIP path.

Run where the reference tree is checked out (the GPU tests read only the
fixtures it writes):

    python tests/golden/make_fixtures.py [--ref /root/reference/python] [--jobs 8]

Outputs (committed; the tests read only these files):
  coder_vectors.json  arithmetic-coder bytes of fixed (cumfreqs, symbols)
                      sequences from ArithEncoder (arith_coder.py:23-123,
                      the Python twin of arith_coder.rs:26-130), each decoded
                      back by ArithDecoder.
  v001_chain.npz      the composed chain Model.forward -> get_cumfreqs ->
                      ArithEncoder (model.py:362-501, softmax_cdf.py:88-180)
                      on the shipped model: 32 KiB of seeded synthetic text at
                      level 1 (64-token chunks, the CLI flow of main.rs:206-279)
                      with every chunk's bytes, the CZIPv1 payload and outer
                      header (file_format.py CompressedFile), sample logits and
                      cumulative-frequency rows; five chunks of the same ids at
                      level 4 (512-token chunks).
  sink_chain.npz      the same chain on a seeded random-init 2-layer model with
                      an attention sink (attention.py:308-411 sink branch),
                      at 128-token chunks.

The mirror differs from the Rust crate in a few places (RMSNorm's divide at
mean_sq = 9483, the attention output clip to -128, the running max starting
at -2^30, 64-bit vacc).  The fixtures must hold the Rust semantics, so:
  * the mirror's udiv_rne_tte_u32 (primitives.py:79-111) rounds a remainder
    of (d - 1) / 2 up for odd d, where primitives.rs:80-97 rounds it down.
    The text of the level-1 fixture reaches it (RMSNorm rows with
    mean_sq = 9483): the script runs RMSNorm with the Rust rounding in place
    of the mirror's, and records which (chunk, position) rows it changed, so
    the fixture pins the Rust result at those rows;
  * no attention output is -128;
  * every attention score of the shipped model lies above -2^30
    (|score| <= 8 |score_mult| + 1 < 2^30);
  * no vacc passes the i32 range (the oracle's wrap counter over the same
    chunks stays 0; at 64 keys the bound 64 * 65535 * 127 < 2^31 holds anyway).

model.py cannot be imported as shipped: its LayerWeights dataclass puts
fields without defaults after `sink_key = None` (model.py:90-121), which
`dataclasses` rejects on every Python version.  LayerWeights is only ever
built with keyword arguments (model.py:208-238), so the script imports the
package with that one class made keyword-only and changes nothing else.
"""
from __future__ import annotations

import argparse
import dataclasses
import hashlib
import json
import os
import sys
from concurrent.futures import ProcessPoolExecutor

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for _p in (os.path.join(ROOT, "oracle"), os.path.join(ROOT, "compress-zip_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

MODEL_REL = "models/v001_eng.czm"
MODEL_PATH = os.path.join(ROOT, MODEL_REL)
BOS = 1022
C1_TEXT_BYTES = 32768
C1_TEXT_SEED = 1234
SINK_MODEL = dict(d=256, n_layers=2, n_heads=4, n_kv=1, d_ff=512, vocab=1024, ctx=256, seed=23, sink=True)

_ref = None


def import_reference(ref_path: str):
    """The reference package, with LayerWeights keyword-only (see module doc)."""
    global _ref
    if _ref is not None:
        return _ref
    sys.path.insert(0, ref_path)
    orig = dataclasses.dataclass

    def tolerant(cls=None, **kw):
        def wrap(c):
            try:
                return orig(c, **kw)
            except TypeError:
                if c.__name__ != "LayerWeights":
                    raise
                return orig(c, kw_only=True, **kw)
        return wrap if cls is None else wrap(cls)

    dataclasses.dataclass = tolerant
    try:
        import compress_zip
    finally:
        dataclasses.dataclass = orig
    _ref = compress_zip
    return compress_zip


class Guard:
    """Instruments the mirror's RMSNorm and attention for the Rust-divergence checks."""

    def __init__(self, ref):
        import oracle
        self.L = oracle.lib()
        self.rms_rows = 0
        self.attn_rows = 0
        self.divergent_rows = 0
        model_mod = sys.modules["compress_zip.model"]
        rms_mod = sys.modules["compress_zip.rmsnorm"]
        orig_norm = model_mod.rmsnorm_i8
        orig_attn = model_mod.gqa_attention_mqa_i8_cached
        mirror_udiv = rms_mod.udiv_rne_tte_u32

        def rust_udiv(n, d):
            # primitives.rs:80-97: compare twice the remainder with the divisor
            if d == 0:
                return 0
            q, r = divmod(n, d)
            return q + 1 if 2 * r > d else q + (q & 1) if 2 * r == d else q

        rms_mod.udiv_rne_tte_u32 = rust_udiv

        def norm(x, w, eps_scaled=1):
            ms = max(1, int(np.sum(x.astype(np.int64) ** 2)) // len(x) + eps_scaled)
            inv = rms_mod.compute_inv_rms_q15_from_mean_sq(ms)
            if inv != self.L.orc_inv_rms_q15(ms):
                raise AssertionError(f"RMSNorm row with mean_sq {ms}: inverse RMS differs from the oracle's")
            rms_mod.udiv_rne_tte_u32 = mirror_udiv
            try:
                self.divergent_rows += rms_mod.compute_inv_rms_q15_from_mean_sq(ms) != inv
            finally:
                rms_mod.udiv_rne_tte_u32 = rust_udiv
            self.rms_rows += 1
            return orig_norm(x, w, eps_scaled)

        def attn(*a, **kw):
            out = orig_attn(*a, **kw)
            if (out == -128).any():
                raise AssertionError("attention output -128 (Python clips to [-128, 127], Rust to [-127, 127])")
            self.attn_rows += 1
            return out

        model_mod.rmsnorm_i8 = norm
        model_mod.gqa_attention_mqa_i8_cached = attn


def coder_cases(rng):
    """(cumfreqs, symbols) sequences: uniform, random, skewed, tiny-frequency
    and real-target tables, long enough for E1/E2/E3 runs and pending bits."""
    cases = []
    cases.append((np.arange(1, 9, dtype=np.uint64) * 1000, [2]))
    cases.append((np.arange(1, 9, dtype=np.uint64) * 1000, [0, 3, 7, 2, 5, 1]))
    cases.append((np.arange(1, 9, dtype=np.uint64) * 1000, [i % 8 for i in range(16)]))
    for trial in range(12):
        v = int(rng.integers(2, 300))
        f = rng.integers(1, 1 << int(rng.integers(1, 20)), v).astype(np.uint64)
        cases.append((np.cumsum(f), rng.integers(0, v, int(rng.integers(50, 400))).tolist()))
    for trial in range(4):
        # one dominant symbol: most steps code ~0 bits, E3 straddles build up
        v = int(rng.integers(3, 64))
        f = np.ones(v, np.uint64)
        f[0] = (1 << 30) - (v - 1)
        syms = np.where(rng.random(600) < 0.97, 0, rng.integers(1, v, 600)).tolist()
        cases.append((np.cumsum(f), syms))
    for trial in range(4):
        # frequency 1 out of ~2^30: 30 bits per symbol, long E1/E2 runs
        v = 1024
        f = np.ones(v, np.uint64)
        f[int(rng.integers(0, v))] = (1 << 30) - 1024 - 1024 - (v - 1)
        cases.append((np.cumsum(f), rng.integers(0, v, 120).tolist()))
    return cases


def make_coder_vectors(ref):
    rng = np.random.default_rng(20261202)
    out = []
    for cum, syms in coder_cases(rng):
        cum = cum.astype(np.uint64)
        assert cum[-1] < (1 << 31)
        total = int(cum[-1])
        enc = ref.ArithEncoder()
        for s in syms:
            enc.encode_symbol(cum, int(s), total)
        data = enc.finish()
        dec = ref.ArithDecoder(data)
        back = [dec.decode_symbol(cum, total) for _ in syms]
        assert back == list(map(int, syms)), "ArithDecoder did not recover the symbols"
        out.append({"cum": [int(c) for c in cum], "syms": [int(s) for s in syms], "bytes": data.hex()})
    return out


# ---- the composed chain -------------------------------------------------------

_worker = {}


def _worker_model(ref_path: str, model_path: str):
    key = (ref_path, model_path)
    if key not in _worker:
        ref = import_reference(ref_path)
        guard = Guard(ref)
        w = ref.ModelWeights.load(model_path)
        _worker[key] = (ref, ref.Model(w), guard)
    return _worker[key]


def code_chunk(args):
    """One chunk through the mirror, as the CLI loop does (__main__.py:129-159,
    main.rs:206-238): fresh cache, BOS then the previous token, position from 0."""
    ref_path, model_path, toks, sample_pos = args
    ref, model, guard = _worker_model(ref_path, model_path)
    model.reset()
    enc = ref.ArithEncoder()
    rows_logits, rows_cum, divergent = [], [], []
    for i, tok in enumerate(toks):
        prev = BOS if i == 0 else int(toks[i - 1])
        before = guard.divergent_rows
        logits = model.forward(prev, i)
        if guard.divergent_rows != before:
            divergent.append(i)
        cum, total = model.get_cumfreqs(logits)
        if i in sample_pos:
            rows_logits.append(np.asarray(logits, np.int32).copy())
            rows_cum.append(np.asarray(cum, np.uint32).copy())
        enc.encode_symbol(cum, int(tok), total)
    return enc.finish(), rows_logits, rows_cum, guard.rms_rows, guard.attn_rows, divergent


def run_chunks(pool, ref_path, model_path, ids, chunk, sample_chunks=(), sample_pos=()):
    n = len(ids)
    jobs = []
    for c in range((n + chunk - 1) // chunk):
        toks = [int(t) for t in ids[c * chunk:(c + 1) * chunk]]
        jobs.append((ref_path, model_path, toks, set(sample_pos) if c in sample_chunks else set()))
    return list(pool.map(code_chunk, jobs, chunksize=1))


def model_hash(path_str: str) -> int:
    """main.rs:79-85: the first 8 hex digits of MD5(path as typed), big-endian."""
    return int(hashlib.md5(path_str.encode()).hexdigest()[:8], 16)


def oracle_wraps(model_path, ids, chunk, kv_mode=0):
    import oracle
    om = oracle.Model.from_file(model_path, kv_mode)
    oracle.reset_vacc_wraps()
    om.compress_many(np.asarray(ids, np.uint32), chunk, threads=8)
    return oracle.vacc_wraps()


def pack_chunks(chunks):
    offs = np.zeros(len(chunks) + 1, np.int64)
    offs[1:] = np.cumsum([len(c) for c in chunks])
    return np.frombuffer(b"".join(chunks), np.uint8), offs


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference/python")
    ap.add_argument("--jobs", type=int, default=8)
    args = ap.parse_args()
    ref = import_reference(args.ref)

    import oracle
    import tokenizer_oracle as TO
    from czip_amd import synth

    vec = make_coder_vectors(ref)
    with open(os.path.join(HERE, "coder_vectors.json"), "w") as f:
        json.dump({"source": "python/compress_zip/arith_coder.py ArithEncoder / ArithDecoder", "cases": vec}, f)
    print(f"coder vectors: {len(vec)} cases", flush=True)

    # shipped model: seeded text -> ids (tokenizer oracle: regex pre-split + tiktoken merge loop)
    text = synth.synthetic_text(C1_TEXT_BYTES, seed=C1_TEXT_SEED)
    t, meta = oracle.read_czm(MODEL_PATH)
    ids = np.array(TO.Tokenizer.from_model(t, meta).encode(text.decode()), np.uint32)
    print(f"C1 text: {len(text)} B -> {ids.size} tokens", flush=True)
    assert np.abs(t["layers.0.attn.score_mult"].astype(np.int64)).max() < (1 << 26)

    with ProcessPoolExecutor(args.jobs) as pool:
        # level 1: 64-token chunks, the whole text
        last = (ids.size - 1) // 64
        res = run_chunks(pool, args.ref, MODEL_PATH, ids, 64, sample_chunks=(0, 1, last),
                         sample_pos=(0, 1, 2, 31, 62, 63, (ids.size - 1) % 64))
        l1_chunks = [r[0] for r in res]
        logit_rows = [x for r in res for x in r[1]]
        cum_rows = [x for r in res for x in r[2]]
        sample_index = []
        for c in (0, 1, last):
            n_c = min(64, ids.size - 64 * c)
            for p in sorted({0, 1, 2, 31, 62, 63, (ids.size - 1) % 64}):
                if p < n_c:
                    sample_index.append((c, p))
        assert len(sample_index) == len(logit_rows)
        print(f"level 1: {len(l1_chunks)} chunks, {sum(map(len, l1_chunks))} B", flush=True)
        # level 4: 512-token chunks over the first 4 * 512 + 300 ids
        n4 = 4 * 512 + 300
        res4 = run_chunks(pool, args.ref, MODEL_PATH, ids[:n4], 512)
        l4_chunks = [r[0] for r in res4]
        print(f"level 4: {len(l4_chunks)} chunks, {sum(map(len, l4_chunks))} B", flush=True)
        assert oracle_wraps(MODEL_PATH, ids[:n4], 512) == 0

        # CZIPv1 payload and outer header of the level-1 file (file_format.py)
        ff = sys.modules["compress_zip.file_format"]
        cf = ff.CompressedFile.create(model_id_hash=model_hash(MODEL_REL), tokenizer_id=0, codec=ff.Codec.BROTLI,
                                      context_length_log2=6)
        for i, c in enumerate(l1_chunks):
            is_last = i == len(l1_chunks) - 1
            cf.add_chunk(c, is_last=is_last, last_chunk_tokens=ids.size - 64 * (len(l1_chunks) - 1) if is_last else None)
        cf.finalize(uncompressed_text_len=len(text))
        payload = cf._build_payload()
        outer = cf.outer_header.to_bytes()

        div_l1 = [(c, p) for c, r in enumerate(res) for p in r[5]]
        print(f"level 1: RMSNorm rows where the mirror's divide differs from Rust's: {div_l1}", flush=True)
        l1_data, l1_offs = pack_chunks(l1_chunks)
        l4_data, l4_offs = pack_chunks(l4_chunks)
        np.savez_compressed(
            os.path.join(HERE, "v001_chain.npz"),
            text_sha256=np.frombuffer(hashlib.sha256(text).digest(), np.uint8),
            text_bytes=np.array(C1_TEXT_BYTES), text_seed=np.array(C1_TEXT_SEED),
            ids=ids.astype(np.uint16),
            l1_data=l1_data, l1_offs=l1_offs, l4_data=l4_data, l4_offs=l4_offs, l4_ntokens=np.array(n4),
            sample_index=np.array(sample_index, np.int32), sample_logits=np.stack(logit_rows),
            sample_cum=np.stack(cum_rows), payload=np.frombuffer(payload, np.uint8),
            rust_rounding_rows=np.array(div_l1, np.int32).reshape(-1, 2),
            payload_sha256=np.frombuffer(hashlib.sha256(payload).digest(), np.uint8),
            outer_header=np.frombuffer(outer, np.uint8), model_id_hash=np.array(model_hash(MODEL_REL), np.uint32),
            model_sha256=np.frombuffer(hashlib.sha256(open(MODEL_PATH, "rb").read()).digest(), np.uint8))

        # random-init 2-layer model with an attention sink (written by synth, checked by hash)
        import tempfile
        tmp = tempfile.mkdtemp(prefix="czip_fixture_")
        sink_path = synth.write_random_model(os.path.join(tmp, "sink.czm"), **SINK_MODEL)
        sink_ids = synth.zipf_ids(128 + 77, 1024, seed=24)
        res_s = run_chunks(pool, args.ref, sink_path, sink_ids, 128, sample_chunks=(0, 1),
                           sample_pos=(0, 5, 76, 127))
        assert oracle_wraps(sink_path, sink_ids, 128) == 0
        s_chunks = [r[0] for r in res_s]
        s_data, s_offs = pack_chunks(s_chunks)
        s_index = [(c, p) for c in (0, 1) for p in (0, 5, 76, 127) if p < min(128, sink_ids.size - 128 * c)]
        np.savez_compressed(
            os.path.join(HERE, "sink_chain.npz"),
            model_params=np.frombuffer(json.dumps(SINK_MODEL, sort_keys=True).encode(), np.uint8),
            model_sha256=np.frombuffer(hashlib.sha256(open(sink_path, "rb").read()).digest(), np.uint8),
            ids=sink_ids.astype(np.uint16), chunk=np.array(128), data=s_data, offs=s_offs,
            sample_index=np.array(s_index, np.int32),
            sample_logits=np.stack([x for r in res_s for x in r[1]]),
            sample_cum=np.stack([x for r in res_s for x in r[2]]))
        assert all(r[3] > 0 and r[4] > 0 for r in res + res4 + res_s), "guards were not exercised"
        print(f"sink model: {len(s_chunks)} chunks; guards passed", flush=True)


if __name__ == "__main__":
    main()
