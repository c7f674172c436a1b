"""GPU parity over seeded random model shapes: head counts 1-16 in both KV
modes, feed-forward widths, vocabularies up to 8192, 1-4 layers, sinks, odd
chunk lengths with ragged tails, and the library's kernel-path switches.
Each case's chunks are coded by the C oracle and by the HIP path (bytes
equal), then decoded on the device (tokens equal)."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

N_CASES = 96
HEADS_GQA = [1, 2, 3, 4, 5, 6, 7, 8, 10, 12, 14, 16]
VOCABS = [1024, 1024, 1088, 1536, 2048, 4096, 8192]
# switches read when a context is created (each case sets at most one)
SWITCHES = [None, None, None, ("CZIP_UNFUSED_NORM", "1"), ("CZIP_GEMM_TILED", "1"), ("CZIP_UNFUSED_HEAD", "1"),
            ("CZIP_DECODE_STREAMS", "3"), ("CZIP_DECODE_LANES", "2"), ("CZIP_FFN_MIN_ROWS", "1"),
            ("CZIP_QKV_GEMM", "1"), ("CZIP_UNFUSED_FFN", "1")]
ORACLE_MACS = 6e10  # multiply-adds of oracle work per case (a few seconds on the host's cores)


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def case_config(i: int) -> dict:
    rng = np.random.default_rng(7000 + i)
    compat = rng.random() < 0.35
    if compat:
        H = int(rng.choice([4, 6, 8]))
        d = 64 * H
        kv_max = -(-(d + 256) // 128) - 1  # d + 128 n_kv < 2 (d + 128): one MQA row (attention.rs:176)
        n_kv = int(rng.integers(1, kv_max + 1))
    else:
        H = int(rng.choice(HEADS_GQA))
        d = 64 * H
        n_kv = int(rng.choice([g for g in range(1, H + 1) if H % g == 0]))
    cfg = dict(d=d, n_heads=H, n_kv=n_kv, d_ff=64 * int(rng.integers(1, 41)), vocab=int(rng.choice(VOCABS)),
               n_layers=int(rng.integers(1, 5)), sink=bool(rng.random() < 0.3), compat=compat)
    if i % 10 == 9:
        cfg.update(d=384, n_heads=6, n_kv=1, d_ff=1024, compat=True)  # the fused FFN's shape
    T = int(rng.integers(16, 601))
    cfg["T"] = T
    cfg["ctx"] = T + int(rng.integers(0, 100))
    per_tok = cfg["n_layers"] * (cfg["d"] * (cfg["d"] + 128 * cfg["n_kv"]) + cfg["d"] ** 2 + 3 * cfg["d"] * cfg["d_ff"]
                                 + 64 * cfg["n_heads"] * T) + cfg["vocab"] * cfg["d"]
    budget = max(T + 1, int(ORACLE_MACS / per_tok))
    n_chunks = int(rng.integers(1, max(2, min(9, budget // T) + 1)))
    tail = int(rng.integers(0, T)) if rng.random() < 0.7 else 0
    cfg["n_tokens"] = max(1, min(n_chunks * T + tail, max(budget, T + 1)))
    cfg["switch"] = SWITCHES[int(rng.integers(0, len(SWITCHES)))]
    cfg["seed"] = 7000 + i
    return cfg


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_shape_roundtrip(orc, tmp_path, monkeypatch, i):
    import czip_amd
    from czip_amd import synth
    if czip_amd.device_count() < 1:
        pytest.fail("no HIP device visible")
    c = case_config(i)
    _say(f"case {i}: {c}")
    if c["switch"]:
        monkeypatch.setenv(*c["switch"])
    path = synth.write_random_model(str(tmp_path / f"r{i}.czm"), d=c["d"], n_layers=c["n_layers"],
                                    n_heads=c["n_heads"], n_kv=c["n_kv"], d_ff=c["d_ff"], vocab=c["vocab"],
                                    ctx=c["ctx"], seed=c["seed"], sink=c["sink"])
    kv = czip_amd.KV_RUST_COMPAT if c["compat"] else czip_amd.KV_GQA
    gm = czip_amd.Model(czip_amd.ModelWeights(path, kv))
    om = orc.Model.from_file(path, kv)
    toks = synth.zipf_ids(c["n_tokens"], c["vocab"], seed=c["seed"] + 1)
    T = c["T"]
    ref = om.compress_many(toks, T, threads=16)
    got = gm.compress_chunks(toks, T)
    assert len(got) == len(ref)
    for k, (g, r) in enumerate(zip(got, ref)):
        assert g == r, f"case {i}: chunk {k} bytes differ"
    ntoks = [min(T, toks.size - k * T) for k in range(len(ref))]
    out = gm.decompress_chunks(ref, ntoks)
    assert np.array_equal(out, toks), f"case {i}: decoded tokens differ"
