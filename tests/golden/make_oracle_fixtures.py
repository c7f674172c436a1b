"""Writes the oracle-coded fixtures of the two large random-init
configurations, whose oracle runs take minutes (a 4096-token chunk of the
d768 / 12-layer model codes at ~20 tokens/s on one core), so that the GPU
tests compare against them instead of re-running the oracle at test time:

  d512l8_ctx512.npz   d512 / 8 layers / 8 heads, 2 KV heads / F 2048 / V 1024
                      (reference KV semantics): 256 chunks of 512 Zipf(1.1)
                      ids, the last one ragged, coded by the oracle -- the
                      4096-stream decode configuration at 256 streams.
  d768l12_ctx4096.npz d768 / 12 layers / 12 heads, 4 KV heads / F 3072 /
                      V 8192 (GQA): one full 4096-token chunk and a ragged
                      one of 1000 tokens.

Each file holds the model's generator parameters and sha256 (the model is
rebuilt by czip_amd.synth from its seed), the token ids' generator
parameters, and the chunk bytes.  tests/test_golden.py re-codes a few chunks
with the oracle to show the files still match it.

    python tests/golden/make_oracle_fixtures.py [--threads 8]
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys
import tempfile
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for _p in (os.path.join(ROOT, "oracle"), os.path.join(ROOT, "compress-zip_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

FIXTURES = {
    "d512l8_ctx512": dict(model=dict(seed=31, shape="d512_l8"), kv_mode=0, ids=dict(n=255 * 512 + 301, seed=33),
                          chunk=512),
    "d768l12_ctx4096": dict(model=dict(seed=41, shape="d768_l12"), kv_mode=1, ids=dict(n=4096 + 1000, seed=42),
                            chunk=4096),
}


def build_model(spec, tmp_dir):
    from czip_amd import synth
    path = os.path.join(tmp_dir, spec["model"]["shape"] + ".czm")
    synth.write_random_model(path, seed=spec["model"]["seed"], **synth.MODEL_SHAPES[spec["model"]["shape"]])
    return path


def fixture_ids(spec, vocab):
    from czip_amd import synth
    return synth.zipf_ids(spec["ids"]["n"], vocab, seed=spec["ids"]["seed"])


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--threads", type=int, default=8)
    ap.add_argument("--only", default=None)
    args = ap.parse_args()
    import oracle
    from czip_amd import synth
    tmp = tempfile.mkdtemp(prefix="czip_ofix_")
    for name, spec in FIXTURES.items():
        if args.only and name != args.only:
            continue
        path = build_model(spec, tmp)
        om = oracle.Model.from_file(path, spec["kv_mode"])
        ids = fixture_ids(spec, synth.MODEL_SHAPES[spec["model"]["shape"]]["vocab"])
        t = time.time()
        chunks = om.compress_many(ids, spec["chunk"], threads=args.threads)
        offs = np.zeros(len(chunks) + 1, np.int64)
        offs[1:] = np.cumsum([len(c) for c in chunks])
        np.savez_compressed(
            os.path.join(HERE, name + ".npz"),
            spec=np.frombuffer(json.dumps(spec, sort_keys=True).encode(), np.uint8),
            model_sha256=np.frombuffer(hashlib.sha256(open(path, "rb").read()).digest(), np.uint8),
            ids_sha256=np.frombuffer(hashlib.sha256(ids.tobytes()).digest(), np.uint8),
            data=np.frombuffer(b"".join(chunks), np.uint8), offs=offs)
        print(f"{name}: {len(chunks)} chunks, {offs[-1]} B, {time.time() - t:.0f} s", flush=True)


if __name__ == "__main__":
    main()
