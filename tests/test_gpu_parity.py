"""GPU parity: the HIP path through the C-ABI against the C oracle, bit for
bit, on the shipped model and on random-init models of the benchmark shapes
(reduced depth), in both KV modes, with ragged chunks and an attention sink."""
import os
import sys

import numpy as np
import pytest

from conftest import GQA_PIN_SHAPES, MODEL_PATH, gqa_pin_logits, write_gqa_pin_model

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def amd():
    import czip_amd
    if czip_amd.device_count() < 1:
        pytest.fail("no HIP device visible")
    return czip_amd


@pytest.fixture(scope="module")
def gpu_shipped(amd):
    return amd.Model(amd.ModelWeights(MODEL_PATH))


def _chunk_inputs(toks, lens, T):
    B = len(lens)
    inp = np.zeros((B, T), np.uint32)
    tgt = np.zeros((B, T), np.uint32)
    off = 0
    for b, n in enumerate(lens):
        seg = toks[off:off + n]
        inp[b, 0] = 1022
        inp[b, 1:n] = seg[:n - 1]
        tgt[b, :n] = seg
        off += n
    return inp, tgt


def _model_pair(amd, orc, path, kv_mode):
    return amd.Model(amd.ModelWeights(path, kv_mode)), orc.Model.from_file(path, kv_mode)


def _check_logits(gm, om, T, lens, seed, vocab):
    rng = np.random.default_rng(seed)
    toks = rng.integers(0, vocab, int(sum(lens))).astype(np.uint32)
    inp, tgt = _chunk_inputs(toks, lens, T)
    _say(f"forward_logits B={len(lens)} T={T} lens={lens}")
    got = gm.forward_logits(inp, lens)
    for b, n in enumerate(lens):
        ref, _ = om.trace(inp[b, :n])
        bad = np.argwhere(got[b, :n] != ref)
        assert bad.size == 0, f"chunk {b}: first mismatch at (pos, vocab) {bad[0].tolist()}"
    return inp, tgt


def test_forward_logits_shipped(gpu_shipped, shipped):
    _check_logits(gpu_shipped, shipped, 64, [64, 64, 37, 1], 11, 1024)


def test_cumfreqs_and_cdf_shipped(gpu_shipped, shipped):
    lens = [64, 50]
    rng = np.random.default_rng(12)
    toks = rng.integers(0, 1024, sum(lens)).astype(np.uint32)
    inp, tgt = _chunk_inputs(toks, lens, 64)
    _say("cumfreqs shipped")
    cum = gpu_shipped.cumfreqs(inp, lens)
    lohi = gpu_shipped.prefill_cdf(tgt, lens)
    for b, n in enumerate(lens):
        _, ref = shipped.trace(inp[b, :n])
        assert np.array_equal(cum[b, :n], ref)
        t = tgt[b, :n].astype(np.int64)
        lo = np.where(t > 0, ref[np.arange(n), np.maximum(t - 1, 0)], 0)
        assert np.array_equal(lohi[b, :n, 0], lo)
        assert np.array_equal(lohi[b, :n, 1], ref[np.arange(n), t])


@pytest.mark.parametrize("chunk", [64, 512])
def test_compress_bytes_shipped(amd, gpu_shipped, shipped, chunk):
    rng = np.random.default_rng(13 + chunk)
    n = chunk * 2 + chunk // 3
    toks = rng.integers(0, 1024, n).astype(np.uint32)
    _say(f"compress shipped chunk={chunk} n={n}")
    job = gpu_shipped.compress_plan(toks, chunk)
    try:
        for fetch in (job.fetch, job.fetch_slots):  # nothing to fetch before the job has run
            with pytest.raises(amd.CzipError) as e:
                fetch()
            assert e.value.code == -1
        job.run()
        got = job.fetch()  # packed on the device
        assert job.fetch_slots() == got  # the fixed-slot copy
    finally:
        job.free()
    ref = shipped.compress_many(toks, chunk, threads=8)
    assert len(got) == len(ref)
    for c, (g, r) in enumerate(zip(got, ref)):
        assert g == r, f"chunk {c}: {len(g)} vs {len(r)} bytes"
    out = shipped.decompress_many(got, [chunk, chunk, n - 2 * chunk], threads=4)
    assert np.array_equal(out, toks)


@pytest.fixture(scope="module")
def random_models(tmp_path_factory):
    from czip_amd import synth
    d = tmp_path_factory.mktemp("models")
    paths = {
        "d512": synth.write_random_model(str(d / "d512.czm"), d=512, n_layers=2, n_heads=8, n_kv=2, d_ff=2048,
                                         vocab=1024, ctx=1024, seed=21),
        "d768": synth.write_random_model(str(d / "d768.czm"), d=768, n_layers=2, n_heads=12, n_kv=4, d_ff=3072,
                                         vocab=8192, ctx=4096, seed=22),
        "sink": synth.write_random_model(str(d / "sink.czm"), d=256, n_layers=2, n_heads=4, n_kv=1, d_ff=512,
                                         vocab=1024, ctx=256, seed=23, sink=True),
    }
    return paths


def test_random_d512_compat(amd, orc, random_models):
    gm, om = _model_pair(amd, orc, random_models["d512"], amd.KV_RUST_COMPAT)
    _check_logits(gm, om, 160, [160, 97], 31, 1024)


def test_random_d512_gqa(amd, orc, random_models):
    gm, om = _model_pair(amd, orc, random_models["d512"], amd.KV_GQA)
    _check_logits(gm, om, 128, [128, 70], 32, 1024)


def test_random_d768_gqa(amd, orc, random_models):
    gm, om = _model_pair(amd, orc, random_models["d768"], amd.KV_GQA)
    _check_logits(gm, om, 96, [96], 33, 8192)


def test_random_sink_compat(amd, orc, random_models):
    gm, om = _model_pair(amd, orc, random_models["sink"], amd.KV_RUST_COMPAT)
    _check_logits(gm, om, 128, [128, 5], 34, 1024)


def test_compress_random_d512(amd, orc, random_models):
    gm, om = _model_pair(amd, orc, random_models["d512"], amd.KV_RUST_COMPAT)
    from czip_amd import synth
    toks = synth.zipf_ids(256 + 100, 1024, seed=5)
    _say("compress random d512 chunk=256")
    got = gm.compress_chunks(toks, 256)
    ref = om.compress_many(toks, 256, threads=8)
    assert got == ref


def _write_model(path, t, meta):
    from czip_amd import synth
    synth.write_czm(path, t, meta)
    return path


def test_attention_general_path(amd, orc, tmp_path):
    """Scores that clamp to the i32 range and wrap in their differences, negative
    multipliers and an exp table whose first entry is not 65535: the attention
    kernel's general path against the oracle, with and without a sink."""
    from czip_amd import synth
    for sink in (False, True):
        t, meta = synth.random_model_tensors(d=256, n_layers=1, n_heads=4, n_kv=1, d_ff=256, vocab=1024, ctx=256,
                                             seed=50 + sink, sink=sink)
        t["layers.0.attn.score_mult"] = np.array([1 << 30, -(1 << 30), 1 << 27, -5], np.int32)
        lut = t["lut.exp2"].copy()
        lut[0] = 65000
        t["lut.exp2"] = lut
        path = _write_model(str(tmp_path / f"gen{sink}.czm"), t, meta)
        gm, om = _model_pair(amd, orc, path, amd.KV_RUST_COMPAT)
        _check_logits(gm, om, 192, [192, 77], 60 + sink, 1024)


def test_unfused_norm_path(amd, orc, tmp_path, monkeypatch):
    """The residual + RMSNorm row kernels that back the row GEMM where it has no
    instance (three heads) or is switched off, in both passes; the separate
    LM head + interval kernels behind the fused heads; the tiled GEMMs behind
    the W-stationary ones; and layer 0's QKV GEMM behind its per-token table."""
    from czip_amd import synth
    path = synth.write_random_model(str(tmp_path / "h3.czm"), d=192, n_layers=2, n_heads=3, n_kv=1, d_ff=256,
                                    vocab=1024, ctx=128, seed=90)
    gm, om = _model_pair(amd, orc, path, amd.KV_GQA)
    _check_logits(gm, om, 128, [128, 60], 91, 1024)
    monkeypatch.setenv("CZIP_UNFUSED_NORM", "1")
    monkeypatch.setenv("CZIP_UNFUSED_HEAD", "1")
    monkeypatch.setenv("CZIP_QKV_GEMM", "1")  # layer 0's QKV by the GEMM over gathered rows, not the table
    gm2 = amd.Model(amd.ModelWeights(MODEL_PATH))
    lens = [64, 40]
    toks = synth.zipf_ids(sum(lens), 1024, seed=92)
    ref = orc.Model.from_file(MODEL_PATH).compress_many(toks, 64, threads=2)
    for tiled in (False, True):
        # W-stationary requant / raw-logit GEMMs, then the tiled ones (the
        # switch is read when a context is created)
        if tiled:
            monkeypatch.setenv("CZIP_GEMM_TILED", "1")
            gm2 = amd.Model(amd.ModelWeights(MODEL_PATH))
        _say(f"compress shipped, unfused norms, tiled GEMMs {tiled}")
        assert gm2.compress_chunks(toks, 64) == ref
        out = gm2.decompress_chunks(ref, lens)
        assert np.array_equal(out, toks)


def test_unfused_ffn_path(gpu_shipped, shipped, monkeypatch, amd):
    """The separate FFN up + ReGLU and down + norm kernels behind the fused
    FFN kernel (switched off by environment at context creation)."""
    from czip_amd import synth
    monkeypatch.setenv("CZIP_UNFUSED_FFN", "1")
    gm = amd.Model(amd.ModelWeights(MODEL_PATH))
    lens = [512, 300]
    toks = synth.zipf_ids(sum(lens), 1024, seed=93)
    _say("compress shipped, FFN unfused")
    ref = shipped.compress_many(toks, 512, threads=2)
    assert gm.compress_chunks(toks, 512) == ref
    assert gpu_shipped.compress_chunks(toks, 512) == ref
    assert np.array_equal(gm.decompress_chunks(ref, lens), toks)


@pytest.mark.parametrize("chunk,n_chunks", [(512, 3), (96, 350), (100, 340)])
def test_fused_ffn_small_launches(amd, shipped, monkeypatch, chunk, n_chunks):
    """The fused FFN kernel (used from 2^19 rows) forced onto small launches:
    1,536 rows; 33,600 rows = 262.5 strips of 128 (a partial last strip,
    more strips than the 256 workgroups, so some take a second strip with the
    next strip's input prefetched); 34,000 rows, whose 531.25 row blocks also
    take the persistent LM head through several blocks per workgroup and a
    partial last block; the compressed bytes against the oracle's, and the
    decode, whose steps then run it too."""
    monkeypatch.setenv("CZIP_FFN_MIN_ROWS", "1")
    gm = amd.Model(amd.ModelWeights(MODEL_PATH))
    rng = np.random.default_rng(80 + chunk)
    n = chunk * n_chunks - chunk // 3
    toks = rng.integers(0, 1024, n).astype(np.uint32)
    ref = shipped.compress_many(toks, chunk, threads=8)
    _say(f"fused FFN forced, chunk={chunk} chunks={n_chunks}")
    assert gm.compress_chunks(toks, chunk) == ref
    ntoks = [min(chunk, n - chunk * c) for c in range(len(ref))]
    assert np.array_equal(gm.decompress_chunks(ref, ntoks), toks)


def test_fused_ffn_many_strips(gpu_shipped, shipped):
    """The default FFN choice at the benchmark's scale: 1,100 chunks of 512
    (563,183 rows, above the 2^19 rows from which the fused kernel runs):
    4,400 strips of 128 rows, 17-18 per workgroup, so every workgroup runs
    the next strip's staged input and up weights requested during the
    previous strip.  Ten chunks spread over the batch (the first, the
    ragged last one) against the oracle's bytes, then every chunk decoded
    on the device."""
    chunk, n_chunks = 512, 1100
    rng = np.random.default_rng(1100)
    n = chunk * n_chunks - 17
    toks = rng.integers(0, 1024, n).astype(np.uint32)
    _say(f"compress shipped, fused FFN by default, {n_chunks} x {chunk}")
    got = gpu_shipped.compress_chunks(toks, chunk)
    assert len(got) == n_chunks
    for c in sorted(set(np.linspace(0, n_chunks - 1, 10).astype(int).tolist())):
        ref = shipped.compress_many(toks[c * chunk:(c + 1) * chunk], chunk, threads=1)
        assert got[c] == ref[0], f"chunk {c} differs from the oracle"
    ntoks = [min(chunk, n - chunk * c) for c in range(n_chunks)]
    _say(f"decompress shipped, {n_chunks} streams")
    assert np.array_equal(gpu_shipped.decompress_chunks(got, ntoks), toks)


def test_requant_general_path(amd, orc, tmp_path):
    """Requantization outside the GEMMs' f64 fast path (|mult| >= 2^26, negative
    multipliers, shift <= 0) against the oracle."""
    from czip_amd import synth
    t, meta = synth.random_model_tensors(d=256, n_layers=2, n_heads=4, n_kv=1, d_ff=256, vocab=1024, ctx=128, seed=80)
    t["layers.0.attn.qkv.mult"] = np.array(1 << 27, np.int32)
    t["layers.0.attn.qkv.shift"] = np.array(40, np.int8)
    t["layers.0.attn.out.mult"] = np.array(-(1 << 28), np.int32)
    t["layers.0.attn.out.shift"] = np.array(45, np.int8)
    t["layers.0.ffn.up.mult"] = np.array(3, np.int32)
    t["layers.0.ffn.up.shift"] = np.array(0, np.int8)
    t["layers.1.ffn.down.mult"] = np.array(-819, np.int32)
    path = _write_model(str(tmp_path / "rq.czm"), t, meta)
    gm, om = _model_pair(amd, orc, path, amd.KV_RUST_COMPAT)
    _check_logits(gm, om, 128, [128, 45], 81, 1024)


def record_stress_weights(d, vocab):
    """Token i embeds as 60 cos th_i on the first half of the dims and
    127 sin th_i * s_j on the second (s_j from 0.5 to 1, so the dims round at
    different points), th_i rising with i over [0, pi/4).  Query dims sum the
    cos half (all positive); key dim j sums the first 64 + j dims of the sin
    half, so the keys rise with the token id in fine steps: ~98% of the keys of
    the test sequence are a new running max of every query's row."""
    th = np.arange(vocab) / vocab * (np.pi / 4)
    j = np.arange(d // 2)
    emb = np.zeros((vocab, d), np.int8)
    emb[:, :d // 2] = np.rint(60 * np.cos(th))[:, None].astype(np.int8)
    emb[:, d // 2:] = np.rint(127 * np.sin(th)[:, None] * (0.5 + 0.5 * j / (d // 2 - 1))[None, :]).astype(np.int8)
    qkv = np.zeros((d + 128, d), np.int8)
    qkv[:d, :d // 2] = 1
    for k in range(64):
        qkv[d + k, d // 2:d // 2 + 64 + k] = 1
    qkv[d + 64:, :d // 2] = ((np.arange(64) % 3) - 1)[:, None]
    return emb, np.full(d, 64, np.int8), qkv


def test_attention_every_key_a_record(amd, orc, tmp_path):
    """Scores that rise with almost every key (identity RoPE, keys that grow
    with the token id): nearly every key is a new running max for every query,
    so a 64-key tile carries up to 64 records per row."""
    from czip_amd import synth
    d, vocab, T = 256, 1024, 256
    t, meta = synth.random_model_tensors(d=d, n_layers=1, n_heads=4, n_kv=1, d_ff=256, vocab=vocab, ctx=T, seed=70)
    t["embed.weight"], t["layers.0.attn_norm.weight"], t["layers.0.attn.qkv.weight"] = record_stress_weights(d, vocab)
    t["layers.0.attn.qkv.shift"] = np.array(17, np.int8)
    t["lut.rope_cos"] = np.full_like(t["lut.rope_cos"], 32767)
    t["lut.rope_sin"] = np.zeros_like(t["lut.rope_sin"])
    path = _write_model(str(tmp_path / "records.czm"), t, meta)
    gm, om = _model_pair(amd, orc, path, amd.KV_RUST_COMPAT)
    lens = [T, 131]
    toks = np.concatenate([np.arange(0, vocab, vocab // T)[:T], np.arange(0, 131) * 7]).astype(np.uint32)
    inp, _ = _chunk_inputs(toks, lens, T)
    _say("forward_logits every-key-a-record")
    got = gm.forward_logits(inp, lens)
    for b, n in enumerate(lens):
        ref, _ = om.trace(inp[b, :n])
        bad = np.argwhere(got[b, :n] != ref)
        assert bad.size == 0, f"chunk {b}: first mismatch at (pos, vocab) {bad[0].tolist()}"


@pytest.mark.parametrize("vocab", [2048, 8192])
def test_cdf_large_vocab(amd, orc, tmp_path, vocab):
    """The multi-wave CDF variants (V > 1024) against the oracle's tables and coded bytes."""
    from czip_amd import synth
    path = synth.write_random_model(str(tmp_path / f"v{vocab}.czm"), d=256, n_layers=1, n_heads=4, n_kv=1,
                                    d_ff=256, vocab=vocab, ctx=128, seed=40 + vocab)
    gm, om = _model_pair(amd, orc, path, amd.KV_RUST_COMPAT)
    rng = np.random.default_rng(vocab)
    lens = [96, 33]
    toks = rng.integers(0, vocab, sum(lens)).astype(np.uint32)
    inp, tgt = _chunk_inputs(toks, lens, 96)
    _say(f"cumfreqs V={vocab}")
    cum = gm.cumfreqs(inp, lens)
    for b, n in enumerate(lens):
        _, ref = om.trace(inp[b, :n])
        assert np.array_equal(cum[b, :n], ref)
    assert gm.compress_chunks(toks, 96) == om.compress_many(toks, 96, threads=4)


@pytest.mark.parametrize("chunk", [64, 512])
def test_decompress_shipped(gpu_shipped, shipped, chunk):
    """Batched device decode of oracle-coded chunks recovers the tokens
    (main.rs:377-396), ragged last chunk included."""
    rng = np.random.default_rng(50 + chunk)
    n = chunk * 3 + chunk // 2 + 1
    toks = rng.integers(0, 1024, n).astype(np.uint32)
    chunks = shipped.compress_many(toks, chunk, threads=8)
    ntoks = [min(chunk, n - c * chunk) for c in range(len(chunks))]
    _say(f"decompress shipped chunk={chunk} n={n}")
    out = gpu_shipped.decompress_chunks(chunks, ntoks)
    assert np.array_equal(out, toks)


def test_decompress_random_models(amd, orc, random_models):
    from czip_amd import synth
    for name, kv, vocab, chunk in [("d512", amd.KV_RUST_COMPAT, 1024, 128), ("d768", amd.KV_GQA, 8192, 64),
                                   ("sink", amd.KV_RUST_COMPAT, 1024, 96)]:
        gm, om = _model_pair(amd, orc, random_models[name], kv)
        toks = synth.zipf_ids(chunk * 2 + 17, vocab, seed=60)
        _say(f"decompress {name} chunk={chunk}")
        chunks = gm.compress_chunks(toks, chunk)
        assert chunks == om.compress_many(toks, chunk, threads=8)
        ntoks = [chunk, chunk, 17]
        assert np.array_equal(gm.decompress_chunks(chunks, ntoks), toks)


def _roundtrip(amd, orc, path, kv, toks, chunk):
    gm, om = _model_pair(amd, orc, path, kv)
    ref = om.compress_many(toks, chunk, threads=8)
    assert gm.compress_chunks(toks, chunk) == ref
    ntoks = [min(chunk, toks.size - c * chunk) for c in range(len(ref))]
    assert np.array_equal(gm.decompress_chunks(ref, ntoks), toks)


def test_decompress_attention_edge_cases(amd, orc, tmp_path):
    """Decode attention beyond the plain models: 16 query heads on one KV head
    (all 16 rows of a wavefront live), the general path (clamped, wrapping
    scores; lut[0] != 65535; a sink) and rows where nearly every key is a
    record; each coded by the oracle and decoded on the device."""
    from czip_amd import synth
    path = synth.write_random_model(str(tmp_path / "mqa16.czm"), d=1024, n_layers=1, n_heads=16, n_kv=1, d_ff=256,
                                    vocab=1024, ctx=256, seed=95)
    _say("decompress 16 heads on one KV head")
    _roundtrip(amd, orc, path, amd.KV_GQA, synth.zipf_ids(80 * 2 + 33, 1024, seed=96), 80)

    t, meta = synth.random_model_tensors(d=256, n_layers=1, n_heads=4, n_kv=1, d_ff=256, vocab=1024, ctx=256,
                                         seed=51, sink=True)
    t["layers.0.attn.score_mult"] = np.array([1 << 30, -(1 << 30), 1 << 27, -5], np.int32)
    lut = t["lut.exp2"].copy()
    lut[0] = 65000
    t["lut.exp2"] = lut
    path = _write_model(str(tmp_path / "gen.czm"), t, meta)
    _say("decompress general attention path")
    _roundtrip(amd, orc, path, amd.KV_RUST_COMPAT, synth.zipf_ids(150 + 41, 1024, seed=97), 150)

    d, vocab, T = 256, 1024, 256
    t, meta = synth.random_model_tensors(d=d, n_layers=1, n_heads=4, n_kv=1, d_ff=256, vocab=vocab, ctx=T, seed=70)
    t["embed.weight"], t["layers.0.attn_norm.weight"], t["layers.0.attn.qkv.weight"] = record_stress_weights(d, vocab)
    t["layers.0.attn.qkv.shift"] = np.array(17, np.int8)
    t["lut.rope_cos"] = np.full_like(t["lut.rope_cos"], 32767)
    t["lut.rope_sin"] = np.zeros_like(t["lut.rope_sin"])
    path = _write_model(str(tmp_path / "records.czm"), t, meta)
    toks = np.concatenate([np.arange(0, vocab, vocab // 200)[:200], np.arange(0, 131) * 7]).astype(np.uint32)
    _say("decompress every-key-a-record")
    _roundtrip(amd, orc, path, amd.KV_RUST_COMPAT, toks, 200)


def test_decompress_stream_groups(amd, shipped, monkeypatch):
    """More chunks than streams per group: groups run one after the other
    (the cap is read when a context is created)."""
    monkeypatch.setenv("CZIP_DECODE_STREAMS", "3")
    gm = amd.Model(amd.ModelWeights(MODEL_PATH))
    rng = np.random.default_rng(70)
    toks = rng.integers(0, 1024, 64 * 7 + 5).astype(np.uint32)
    chunks = shipped.compress_many(toks, 64, threads=4)
    ntoks = [64] * 7 + [5]
    out = gm.decompress_chunks(chunks, ntoks)
    assert np.array_equal(out, toks)


@pytest.mark.parametrize("lanes,fused", [(2, True), (2, False), (4, True)])
def test_decompress_lanes(amd, shipped, monkeypatch, lanes, fused):
    """A group's streams decoded as several lanes on their own HIP streams
    (forced on for small groups): odd group sizes, a last group of three (fewer
    streams than lanes), ragged streams; with the fused kernels and with the
    separate norm / FFN / LM head kernels."""
    monkeypatch.setenv("CZIP_DECODE_LANES", str(lanes))
    monkeypatch.setenv("CZIP_DECODE_STREAMS", "5")
    if not fused:
        for k in ("CZIP_UNFUSED_NORM", "CZIP_UNFUSED_HEAD", "CZIP_UNFUSED_FFN"):
            monkeypatch.setenv(k, "1")
    gm = amd.Model(amd.ModelWeights(MODEL_PATH))
    rng = np.random.default_rng(71)
    ntoks = [64] * 12 + [23]
    toks = rng.integers(0, 1024, sum(ntoks)).astype(np.uint32)
    chunks = shipped.compress_many(toks, 64, threads=8)
    _say(f"decompress {lanes} lanes, fused {fused}")
    assert np.array_equal(gm.decompress_chunks(chunks, ntoks), toks)


@pytest.mark.parametrize("kv", ["compat", "gqa"])
def test_config_d512_l8_full_shape(amd, orc, tmp_path, kv):
    """The d512 / 8-layer / 8 heads, 2 KV heads / F 2048 / V 1024 configuration
    at its level-5 chunk size (1024 tokens): chunk bytes against the oracle
    (one full chunk + a ragged one), then decoded on the device as concurrent
    streams (the 4096-stream decode configuration at a test's size)."""
    from czip_amd import synth
    path = synth.write_random_model(str(tmp_path / "d512l8.czm"), seed=31, **synth.MODEL_SHAPES["d512_l8"])
    mode = amd.KV_RUST_COMPAT if kv == "compat" else amd.KV_GQA
    gm, om = _model_pair(amd, orc, path, mode)
    n = 1024 + (333 if kv == "compat" else 96)
    toks = synth.zipf_ids(n, 1024, seed=32)
    _say(f"d512/L8 chunk 1024 {kv}: {n} tokens")
    got = gm.compress_chunks(toks, 1024)
    assert got == om.compress_many(toks, 1024, threads=8)
    assert np.array_equal(gm.decompress_chunks(got, [1024, n - 1024]), toks)


def test_config_d768_l12_full_shape(amd, orc, tmp_path):
    """The d768 / 12-layer / 12 heads, 4 KV heads / F 3072 / V 8192 / 4096-context
    configuration (GQA; the reference rejects 12 heads): a 384-token chunk of a
    4096-token context, coded on the device against the oracle, and decoded."""
    from czip_amd import synth
    path = synth.write_random_model(str(tmp_path / "d768l12.czm"), seed=41, **synth.MODEL_SHAPES["d768_l12"])
    gm, om = _model_pair(amd, orc, path, amd.KV_GQA)
    toks = synth.zipf_ids(384, 8192, seed=42)
    _say("d768/L12/V8192 chunk 4096: 384 tokens")
    got = gm.compress_chunks(toks, 4096)
    assert got == om.compress_many(toks, 4096, threads=8)
    assert np.array_equal(gm.decompress_chunks(got, [384]), toks)


@pytest.mark.parametrize("level", [1, 4])
def test_czip_file_shipped(amd, orc, level):
    """The CLI's whole flow (main.rs:125-399) on the shipped model: text ->
    tokens -> device-coded chunks -> .czip (brotli) -> device decode -> text.
    The container payload equals the one built from the oracle's chunk bytes
    (file_format.rs layout restated in oracle/container.py)."""
    import container as OC
    from czip_amd import synth
    w = amd.ModelWeights(MODEL_PATH)
    gm = amd.Model(w)
    tk = amd.Tokenizer(w)
    text = synth.synthetic_text(24000 + 77 * level, seed=level)
    _say(f"czip file level {level}")
    data = amd.compress_text(gm, tk, text, "models/v001_eng.czm", level=level)
    assert data[:6] == b"CZIPv1" and data[7] == amd.CODEC_BROTLI
    chunk = amd.level_to_context_length(level)
    ids = tk.encode(text)
    ref_chunks = orc.Model.from_file(MODEL_PATH).compress_many(ids, chunk, threads=8)
    last = ids.size - chunk * (len(ref_chunks) - 1)
    exp = OC.payload(OC.model_id_hash("models/v001_eng.czm"), last, 0, chunk.bit_length() - 1, ref_chunks)
    assert OC.decode_outer(amd.CODEC_BROTLI, data[16:]) == exp
    assert data[:16] == OC.outer_header(0, amd.CODEC_BROTLI, len(text), 12 + 2 * len(ref_chunks))
    assert amd.decompress_czip(gm, tk, data) == text


def test_error_codes(gpu_shipped, amd):
    with pytest.raises(amd.CzipError) as e:
        gpu_shipped.compress_plan(np.zeros(10, np.uint32), 2048)   # past the 1024-entry RoPE LUT
    assert e.value.code == -4
    with pytest.raises(amd.CzipError) as e:
        gpu_shipped.compress_plan(np.array([1, 2, 5000], np.uint32), 64)
    assert e.value.code == -5
    assert gpu_shipped.compress_chunks(np.zeros(0, np.uint32), 64) == []


def test_vacc_wrap(amd, orc, tmp_path):
    """Attention sums that wrap the reference's i32 vacc (attention.rs:207-208,
    274: 65535 * 127 * (p + 1) >= 2^31 from position 258 on): prefill logits
    of a 512-token chunk, coded bytes of a full and a ragged chunk, and device
    decode of the oracle's chunks, all against the oracle, whose own sums are
    checked to have wrapped."""
    from conftest import write_vacc_wrap_model
    from czip_amd import synth
    path = write_vacc_wrap_model(str(tmp_path / "wrap.czm"))
    gm, om = _model_pair(amd, orc, path, amd.KV_RUST_COMPAT)
    toks = synth.zipf_ids(512 + 300, 1024, seed=112)
    inp, _ = _chunk_inputs(toks, [512, 300], 512)
    _say("vacc wrap: logits of 512 + 300 rows")
    orc.reset_vacc_wraps()
    got = gm.forward_logits(inp, [512, 300])
    for b, n in enumerate([512, 300]):
        ref, _ = om.trace(inp[b, :n])
        bad = np.argwhere(got[b, :n] != ref)
        assert bad.size == 0, f"chunk {b}: first mismatch at (pos, vocab) {bad[0].tolist()}"
    assert orc.vacc_wraps() > 0
    _say("vacc wrap: compress + decode")
    ref = om.compress_many(toks, 512, threads=2)
    assert gm.compress_chunks(toks, 512) == ref
    assert np.array_equal(gm.decompress_chunks(ref, [512, 300]), toks)


@pytest.mark.parametrize("H,G", GQA_PIN_SHAPES)
def test_gqa_group_mapping_closed_form(amd, tmp_path, H, G):
    """The device's GQA mode against the closed form of write_gqa_pin_model:
    head h's attention output is floor(h G / H) + 1 (query head h on KV
    group floor(h G / H), values from that group's V slice), seen through
    the logits at every position of a full and a ragged chunk."""
    path = write_gqa_pin_model(str(tmp_path / f"gqa{H}_{G}.czm"), H, G)
    gm = amd.Model(amd.ModelWeights(path, amd.KV_GQA))
    lens = [96, 33]
    inp = np.zeros((2, 96), np.uint32)
    inp[:, 0] = 1022
    inp[:, 1:] = np.arange(1, 96) * 5
    _say(f"gqa closed form H={H} G={G}")
    got = gm.forward_logits(inp, lens)
    exp = gqa_pin_logits(H, G)
    for b, n in enumerate(lens):
        assert (got[b, :n] == exp[None, :]).all(), f"chunk {b}"


def test_gqa_one_group_equals_reference_slicing(amd, orc, tmp_path):
    """With one KV group the device's GQA mode and its reference-slicing mode
    give the oracle's reference-slicing chunk bytes."""
    from czip_amd import synth
    path = synth.write_random_model(str(tmp_path / "g1.czm"), d=384, n_layers=2, n_heads=6, n_kv=1, d_ff=512,
                                    vocab=1024, ctx=128, seed=44)
    toks = synth.zipf_ids(128 * 2 + 40, 1024, seed=45)
    ref = orc.Model.from_file(path, orc.KV_RUST_COMPAT).compress_many(toks, 128, threads=4)
    for kv in (amd.KV_GQA, amd.KV_RUST_COMPAT):
        _say(f"one KV group, kv mode {kv}")
        assert amd.Model(amd.ModelWeights(path, kv)).compress_chunks(toks, 128) == ref


@pytest.mark.parametrize("n_chunks,chunk", [(4, 512), (33, 64), (95, 64), (1600, 64), (369, 64), (368, 64)])
def test_small_launch_row_gemm(gpu_shipped, shipped, n_chunks, chunk):
    """Launches of a few thousand rows (fewer than 96 blocks of 64 rows, at
    least 24 of 16) take the 16-row row GEMM for the O and down projections:
    prefill launches of 2,048, 2,112 and 6,075 rows (logits against the
    oracle, then the compressed bytes), and decode steps of 1,600 and 369
    streams (the chunks decoded back); 368 streams (23 blocks) stay on the
    split-K kernels."""
    rng = np.random.default_rng(300 + n_chunks)
    lens = [chunk] * (n_chunks - 1) + [chunk - 5]
    toks = rng.integers(0, 1024, sum(lens)).astype(np.uint32)
    if n_chunks < 100:
        inp, _ = _chunk_inputs(toks, lens, chunk)
        _say(f"row GEMM 16-row blocks, prefill: {n_chunks} x {chunk}")
        got = gpu_shipped.forward_logits(inp, lens)
        for b in (0, n_chunks // 2, n_chunks - 1):
            ref, _ = shipped.trace(inp[b, :lens[b]])
            assert np.array_equal(got[b, :lens[b]], ref), f"chunk {b}"
    ref = shipped.compress_many(toks, chunk, threads=8)
    _say(f"row GEMM 16-row blocks, compress + decode: {n_chunks} x {chunk}")
    assert gpu_shipped.compress_chunks(toks, chunk) == ref
    assert np.array_equal(gpu_shipped.decompress_chunks(ref, lens), toks)
