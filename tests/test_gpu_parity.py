"""GPU parity: the HIP path through the C-ABI against the C oracle, bit for
bit, on the shipped model and on random-init models of the benchmark shapes
(reduced depth), in both KV modes, with ragged chunks and an attention sink."""
import os
import sys

import numpy as np
import pytest

from conftest import MODEL_PATH

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
def test_compress_bytes_shipped(gpu_shipped, shipped, chunk):
    rng = np.random.default_rng(13 + chunk)
    n = chunk * 2 + chunk // 3
    toks = rng.integers(0, 1024, n).astype(np.uint32)
    _say(f"compress shipped chunk={chunk} n={n}")
    got = gpu_shipped.compress_chunks(toks, chunk)
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


def test_decompress_stream_groups(gpu_shipped, shipped, monkeypatch):
    """More chunks than streams per group: groups run one after the other."""
    monkeypatch.setenv("CZIP_DECODE_STREAMS", "3")
    rng = np.random.default_rng(70)
    toks = rng.integers(0, 1024, 64 * 7 + 5).astype(np.uint32)
    chunks = gpu_shipped.compress_chunks(toks, 64)
    ntoks = [64] * 7 + [5]
    out = gpu_shipped.decompress_chunks(chunks, ntoks)
    assert np.array_equal(out, toks)


def test_error_codes(gpu_shipped, amd):
    with pytest.raises(amd.CzipError) as e:
        gpu_shipped.compress_plan(np.zeros(10, np.uint32), 2048)   # past the 1024-entry RoPE LUT
    assert e.value.code == -4
    with pytest.raises(amd.CzipError) as e:
        gpu_shipped.compress_plan(np.array([1, 2, 5000], np.uint32), 64)
    assert e.value.code == -5
    assert gpu_shipped.compress_chunks(np.zeros(0, np.uint32), 64) == []
