"""The oracle against the golden fixtures of tests/golden/, which the
reference's Python mirror wrote (tests/golden/make_fixtures.py): arithmetic
coder bytes (arith_coder.py:23-123) and the composed chain forward ->
cumulative frequencies -> coder bytes -> CZIPv1 payload on the shipped model
and on a random-init model with an attention sink.  CPU only."""
import hashlib
import json
import os

import numpy as np
import pytest

from conftest import MODEL_PATH, ROOT

GOLDEN = os.path.join(ROOT, "tests", "golden")


def chunks_of(data, offs):
    return [bytes(data[offs[i]:offs[i + 1]]) for i in range(len(offs) - 1)]


def chunk_inputs(ids, c, chunk):
    toks = np.asarray(ids[c * chunk:(c + 1) * chunk], np.uint32)
    return np.concatenate([[1022], toks[:-1]]).astype(np.uint32), toks


@pytest.fixture(scope="module")
def v001():
    return np.load(os.path.join(GOLDEN, "v001_chain.npz"))


@pytest.fixture(scope="module")
def sinkfx():
    return np.load(os.path.join(GOLDEN, "sink_chain.npz"))


def sink_model_path(fx, tmp_dir):
    from czip_amd import synth
    params = json.loads(bytes(fx["model_params"]).decode())
    path = synth.write_random_model(os.path.join(tmp_dir, "sink.czm"), **params)
    assert hashlib.sha256(open(path, "rb").read()).digest() == bytes(fx["model_sha256"]), \
        "the seeded model generator no longer writes the fixture's model"
    return path


def test_coder_bytes(orc):
    """Encoder bytes equal ArithEncoder's for every fixed (table, symbols) case,
    and the oracle's decoder recovers the symbols from them."""
    cases = json.load(open(os.path.join(GOLDEN, "coder_vectors.json")))["cases"]
    assert len(cases) >= 20
    for i, c in enumerate(cases):
        cum = np.array(c["cum"], np.uint32)
        data = bytes.fromhex(c["bytes"])
        assert orc.encode_symbols(cum, c["syms"]) == data, f"case {i}"
        assert orc.decode_symbols(data, cum, len(c["syms"])) == c["syms"], f"case {i}"


def test_fixture_inputs(v001):
    """The fixture's text and model are the ones this tree generates and ships."""
    from czip_amd import synth
    text = synth.synthetic_text(int(v001["text_bytes"]), seed=int(v001["text_seed"]))
    assert hashlib.sha256(text).digest() == bytes(v001["text_sha256"])
    assert hashlib.sha256(open(MODEL_PATH, "rb").read()).digest() == bytes(v001["model_sha256"])
    assert hashlib.sha256(bytes(v001["payload"])).digest() == bytes(v001["payload_sha256"])


def test_tokenizers_give_the_fixture_ids(orc, v001):
    import czip_amd
    import tokenizer_oracle as TO
    from czip_amd import synth
    text = synth.synthetic_text(int(v001["text_bytes"]), seed=int(v001["text_seed"]))
    ids = v001["ids"].astype(np.uint32)
    prod = czip_amd.Tokenizer(czip_amd.ModelWeights(MODEL_PATH))
    assert np.array_equal(prod.encode(text, threads=4), ids)
    t, meta = orc.read_czm(MODEL_PATH)
    assert TO.Tokenizer.from_model(t, meta).encode(text.decode()) == ids.tolist()


def test_sample_rows(shipped, v001):
    """Logits and cumulative-frequency rows of Model.forward / get_cumfreqs."""
    ids = v001["ids"]
    idx = v001["sample_index"]
    for c in sorted(set(idx[:, 0].tolist())):
        inp, _ = chunk_inputs(ids, c, 64)
        lg, cum = shipped.trace(inp)
        for r, (cc, p) in enumerate(idx):
            if cc == c:
                assert np.array_equal(lg[p], v001["sample_logits"][r]), (c, p)
                assert np.array_equal(cum[p], v001["sample_cum"][r]), (c, p)


def test_level1_chunks_and_payload(shipped, v001):
    """All 418 chunks of the 32 KiB text at 64 tokens, byte for byte, and the
    CZIPv1 payload and outer header built from them (file_format.rs layout,
    restated in oracle/container.py)."""
    import container as OC
    ids = v001["ids"].astype(np.uint32)
    exp = chunks_of(v001["l1_data"], v001["l1_offs"])
    got = shipped.compress_many(ids, 64, threads=8)
    assert len(got) == len(exp) == 418
    bad = [i for i, (g, e) in enumerate(zip(got, exp)) if g != e]
    assert not bad, f"chunks differ: {bad[:10]}"
    # the rows where the mirror's RMSNorm divide had to take the Rust rounding
    assert v001["rust_rounding_rows"].shape[0] > 0
    last = ids.size - 64 * (len(exp) - 1)
    pay = OC.payload(int(v001["model_id_hash"]), last, 0, 6, got)
    assert pay == bytes(v001["payload"])
    assert OC.model_id_hash("models/v001_eng.czm") == int(v001["model_id_hash"])
    hdr = OC.outer_header(0, 1, int(v001["text_bytes"]), 12 + 2 * len(got))
    assert hdr == bytes(v001["outer_header"])


def test_level4_chunks(shipped, v001):
    ids = v001["ids"][:int(v001["l4_ntokens"])].astype(np.uint32)
    exp = chunks_of(v001["l4_data"], v001["l4_offs"])
    assert shipped.compress_many(ids, 512, threads=5) == exp


def test_sink_model_chain(orc, sinkfx, tmp_path):
    path = sink_model_path(sinkfx, str(tmp_path))
    om = orc.Model.from_file(path)
    ids = sinkfx["ids"].astype(np.uint32)
    T = int(sinkfx["chunk"])
    assert om.compress_many(ids, T, threads=2) == chunks_of(sinkfx["data"], sinkfx["offs"])
    idx = sinkfx["sample_index"]
    for c in sorted(set(idx[:, 0].tolist())):
        inp, _ = chunk_inputs(ids, c, T)
        lg, cum = om.trace(inp)
        for r, (cc, p) in enumerate(idx):
            if cc == c:
                assert np.array_equal(lg[p], sinkfx["sample_logits"][r]), (c, p)
                assert np.array_equal(cum[p], sinkfx["sample_cum"][r]), (c, p)


def test_vacc_wrap_model_wraps(orc, tmp_path):
    """The wrap model of the GPU test really drives the oracle's vacc past the
    i32 range (and only from position 258 on)."""
    from conftest import write_vacc_wrap_model
    from czip_amd import synth
    om = orc.Model.from_file(write_vacc_wrap_model(str(tmp_path / "wrap.czm")))
    toks = synth.zipf_ids(300, 1024, seed=111)
    inp = np.concatenate([[1022], toks[:-1]]).astype(np.uint32)
    orc.reset_vacc_wraps()
    om.trace(inp[:258], with_cum=False)
    assert orc.vacc_wraps() == 0
    om.trace(inp, with_cum=False)
    assert orc.vacc_wraps() > 0


@pytest.mark.parametrize("name", ["d512l8_ctx512", "d768l12_ctx4096"])
def test_oracle_fixtures_still_match(orc, tmp_path, name):
    """The oracle-coded fixtures of the large configurations: the seeded model
    and ids are the ones the generators write, and (d512 / 8 layers) the
    first and the ragged last chunk re-code to the committed bytes."""
    import sys
    sys.path.insert(0, GOLDEN)
    import make_oracle_fixtures as MOF
    from czip_amd import synth
    fx = np.load(os.path.join(GOLDEN, name + ".npz"))
    spec = json.loads(bytes(fx["spec"]).decode())
    assert spec == json.loads(json.dumps(MOF.FIXTURES[name], sort_keys=True))
    path = MOF.build_model(spec, str(tmp_path))
    assert hashlib.sha256(open(path, "rb").read()).digest() == bytes(fx["model_sha256"])
    ids = MOF.fixture_ids(spec, synth.MODEL_SHAPES[spec["model"]["shape"]]["vocab"])
    assert hashlib.sha256(ids.tobytes()).digest() == bytes(fx["ids_sha256"])
    exp = chunks_of(fx["data"], fx["offs"])
    T = spec["chunk"]
    assert len(exp) == (ids.size + T - 1) // T
    if name == "d512l8_ctx512":
        om = orc.Model.from_file(path, spec["kv_mode"])
        last = len(exp) - 1
        got = om.compress_many(np.concatenate([ids[:T], ids[last * T:]]), T, threads=2)
        assert got == [exp[0], exp[last]]
