"""The HIP path through the C-ABI against the committed golden fixtures:
the reference's Python mirror's chain on the shipped model and on a sink
model (tests/golden/make_fixtures.py), and the oracle-coded chunks of the
d512 / 8-layer and d768 / 12-layer configurations
(tests/golden/make_oracle_fixtures.py), plus the 4096-stream x 512-token
decode configuration as a device round trip."""
import hashlib
import json
import os
import sys

import numpy as np
import pytest

from conftest import MODEL_PATH, ROOT

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(ROOT, "tests", "golden")


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def chunks_of(data, offs):
    return [bytes(data[offs[i]:offs[i + 1]]) for i in range(len(offs) - 1)]


@pytest.fixture(scope="module")
def amd():
    import czip_amd
    if czip_amd.device_count() < 1:
        pytest.fail("no HIP device visible")
    return czip_amd


@pytest.fixture(scope="module")
def v001():
    return np.load(os.path.join(GOLDEN, "v001_chain.npz"))


@pytest.fixture(scope="module")
def gm(amd):
    return amd.Model(amd.ModelWeights(MODEL_PATH))


def test_level1_file_equals_the_mirrors(amd, gm, v001):
    """The 32 KiB text at level 1 through the CLI flow on the device (tokenize,
    code every 64-token chunk, container): chunk bytes, payload and outer
    header equal the mirror's; the file decodes back to the text."""
    import container as OC
    from czip_amd import synth
    text = synth.synthetic_text(int(v001["text_bytes"]), seed=int(v001["text_seed"]))
    tk = amd.Tokenizer(gm.weights)
    _say("level-1 file of the 32 KiB text")
    data = amd.compress_text(gm, tk, text, "models/v001_eng.czm", level=1)
    fields, chunks = amd.unpack_czip(data)
    assert chunks == chunks_of(v001["l1_data"], v001["l1_offs"])
    pay = OC.decode_outer(amd.CODEC_BROTLI, data[16:])
    assert hashlib.sha256(pay).digest() == bytes(v001["payload_sha256"])
    assert data[:16] == bytes(v001["outer_header"])
    assert amd.decompress_czip(gm, tk, data) == text


def test_sample_rows_equal_the_mirrors(gm, v001):
    ids = v001["ids"].astype(np.uint32)
    idx = v001["sample_index"]
    cs = sorted(set(idx[:, 0].tolist()))
    inp = np.zeros((len(cs), 64), np.uint32)
    lens = []
    for b, c in enumerate(cs):
        t = ids[c * 64:(c + 1) * 64]
        inp[b, 0] = 1022
        inp[b, 1:t.size] = t[:-1]
        lens.append(t.size)
    _say("logits / cumfreqs rows of the 32 KiB text")
    lg = gm.forward_logits(inp, lens)
    cum = gm.cumfreqs(inp, lens)
    for r, (c, p) in enumerate(idx):
        b = cs.index(int(c))
        assert np.array_equal(lg[b, p], v001["sample_logits"][r]), (c, p)
        assert np.array_equal(cum[b, p], v001["sample_cum"][r]), (c, p)


def test_level4_chunks_equal_the_mirrors(gm, v001):
    ids = v001["ids"][:int(v001["l4_ntokens"])].astype(np.uint32)
    _say("level-4 chunks")
    exp = chunks_of(v001["l4_data"], v001["l4_offs"])
    assert gm.compress_chunks(ids, 512) == exp
    ntoks = [min(512, ids.size - 512 * c) for c in range(len(exp))]
    assert np.array_equal(gm.decompress_chunks(exp, ntoks), ids)


def test_sink_model_equals_the_mirrors(amd, tmp_path):
    from czip_amd import synth
    fx = np.load(os.path.join(GOLDEN, "sink_chain.npz"))
    params = json.loads(bytes(fx["model_params"]).decode())
    path = synth.write_random_model(str(tmp_path / "sink.czm"), **params)
    assert hashlib.sha256(open(path, "rb").read()).digest() == bytes(fx["model_sha256"])
    g = amd.Model(amd.ModelWeights(path))
    ids = fx["ids"].astype(np.uint32)
    T = int(fx["chunk"])
    exp = chunks_of(fx["data"], fx["offs"])
    _say("sink model chain")
    assert g.compress_chunks(ids, T) == exp
    assert np.array_equal(g.decompress_chunks(exp, [T, ids.size - T]), ids)


def _oracle_fixture(amd, name, tmp_path):
    from czip_amd import synth
    fx = np.load(os.path.join(GOLDEN, name + ".npz"))
    spec = json.loads(bytes(fx["spec"]).decode())
    shape = synth.MODEL_SHAPES[spec["model"]["shape"]]
    path = synth.write_random_model(str(tmp_path / (name + ".czm")), seed=spec["model"]["seed"], **shape)
    assert hashlib.sha256(open(path, "rb").read()).digest() == bytes(fx["model_sha256"])
    ids = synth.zipf_ids(spec["ids"]["n"], shape["vocab"], seed=spec["ids"]["seed"])
    assert hashlib.sha256(ids.tobytes()).digest() == bytes(fx["ids_sha256"])
    g = amd.Model(amd.ModelWeights(path, spec["kv_mode"]))
    return g, ids, spec["chunk"], chunks_of(fx["data"], fx["offs"])


def test_d512l8_ctx512_256_streams(amd, tmp_path):
    """d512 / 8 layers / 8 heads, 2 KV heads at 512-token chunks (reference KV
    semantics): 256 chunks coded on the device equal the oracle's, and the
    oracle's chunks decode on the device as 256 concurrent streams."""
    g, ids, T, exp = _oracle_fixture(amd, "d512l8_ctx512", tmp_path)
    _say(f"d512/L8 ctx {T}: {len(exp)} chunks")
    got = g.compress_chunks(ids, T)
    bad = [i for i, (a, b) in enumerate(zip(got, exp)) if a != b]
    assert len(got) == len(exp) and not bad, bad[:10]
    ntoks = [min(T, ids.size - T * c) for c in range(len(exp))]
    assert np.array_equal(g.decompress_chunks(exp, ntoks), ids)


def test_d768l12_ctx4096_full_chunk(amd, tmp_path):
    """d768 / 12 layers / 12 heads, 4 KV heads / V 8192 (GQA): a full
    4096-token chunk (rows of 4096 keys) and a ragged one of 1000, against
    the oracle, then decoded on the device."""
    g, ids, T, exp = _oracle_fixture(amd, "d768l12_ctx4096", tmp_path)
    _say(f"d768/L12 ctx {T}: {ids.size} tokens")
    assert g.compress_chunks(ids, T) == exp
    assert np.array_equal(g.decompress_chunks(exp, [T, ids.size - T]), ids)


def test_d512l8_4096_streams_x_512_roundtrip(amd, orc, tmp_path):
    """The decode configuration at its full shape: 4096 concurrent streams of
    512 tokens of the d512 / 8-layer model, coded and decoded on the device
    (tokens identical), with a strided sample of the chunks against the oracle."""
    from czip_amd import synth
    path = synth.write_random_model(str(tmp_path / "d512l8.czm"), seed=2024, **synth.MODEL_SHAPES["d512_l8"])
    g = amd.Model(amd.ModelWeights(path))
    ids = synth.zipf_ids(4096 * 512, 1024, seed=7)
    _say("d512/L8 4096 x 512 compress")
    chunks = g.compress_chunks(ids, 512)
    assert len(chunks) == 4096
    _say("d512/L8 4096 x 512 decompress")
    assert np.array_equal(g.decompress_chunks(chunks, [512] * 4096), ids)
    om = orc.Model.from_file(path)
    sample = [0, 1365, 2730, 4095]
    ref = om.compress_many(np.concatenate([ids[c * 512:(c + 1) * 512] for c in sample]), 512, threads=4)
    assert [chunks[c] for c in sample] == ref
