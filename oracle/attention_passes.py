"""Record statistics of the prefill attention on real text (analysis, CPU).

Test/analysis infrastructure, like the rest of oracle/: nothing in the
product imports it.  For the shipped model (one layer, six heads) over the
first chunks of the benchmark's seeded synthetic text, it forms every query
row's scores (layer 0's Q/K from the oracle's own RMSNorm / linear / requant
primitives, RoPE as attention.rs:29-83, scores as attention.rs:231-239) and
counts, per 16-row x 64-key tile of the device kernel, the segment passes the
tile needs: 1 + the most splits of any of its rows, a split being a key
whose score exceeds every earlier key of its row (a strict new max,
attention.rs:241-262) other than the row's first key.  Tiles are classed as
the row block's first key tile, its diagonal (last) tile, both, or interior.

    python oracle/attention_passes.py [n_chunks]
"""
from __future__ import annotations

import collections
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
sys.path[:0] = [HERE, os.path.join(ROOT, "compress-zip_amd")]

import oracle as O  # noqa: E402


def _sra(v, sh):
    """sign(v) * RNE(|v| / 2^sh), ties to even (primitives.rs:18-42), on int64 arrays."""
    v = np.asarray(v, np.int64)
    a = np.abs(v)
    q, r, half = a >> sh, a & ((1 << sh) - 1), 1 << (sh - 1)
    q = q + ((r > half) | ((r == half) & ((q & 1) == 1)))
    return np.where(v < 0, -q, q)


def _rope(x, cos, sin, pos, query):
    """RoPE of rows x [T, 64] at positions pos: pairs (i, i + 32); the query
    takes a second RNE shift by one (attention.rs:29-83)."""
    c, s = cos[pos], sin[pos]
    a, b = x[:, :32].astype(np.int64), x[:, 32:].astype(np.int64)
    xa, xb = _sra(a * c - b * s, 15), _sra(a * s + b * c, 15)
    if query:
        xa, xb = _sra(xa, 1), _sra(xb, 1)
    return np.clip(np.concatenate([xa, xb], 1), -127, 127)


def main(n_chunks: int = 64, T: int = 512):
    import czip_amd
    from czip_amd import synth
    path = os.path.join(ROOT, "models", "v001_eng.czm")
    w = czip_amd.ModelWeights(path)
    text = synth.synthetic_text(max(1 << 20, n_chunks * T * 2), seed=1234)
    ids = czip_amd.Tokenizer(w).encode(text, threads=8)
    t, _ = O.read_czm(path)
    L = O.lib()
    E = t["embed.weight"].astype(np.int8)
    d, H = E.shape[1], int(t["layers.0.attn.score_mult"].shape[0])
    an = np.ascontiguousarray(t["layers.0.attn_norm.weight"].astype(np.int8))
    Wq = np.ascontiguousarray(t["layers.0.attn.qkv.weight"].astype(np.int8))
    mult, shift = int(t["layers.0.attn.qkv.mult"]), int(t["layers.0.attn.qkv.shift"])
    smult = t["layers.0.attn.score_mult"].astype(np.int64)
    cos16 = np.ascontiguousarray(t["lut.rope_cos"].astype(np.int16).reshape(-1, 32))
    sin16 = np.ascontiguousarray(t["lut.rope_sin"].astype(np.int16).reshape(-1, 32))
    cos, sin = cos16.astype(np.int64), sin16.astype(np.int64)
    # layer 0's Q/K/V of every token (its input depends on the token only)
    qn = Wq.shape[0]
    tab = np.zeros((E.shape[0], qn), np.int8)
    xn, acc, out = np.zeros(d, np.int8), np.zeros(qn, np.int32), np.zeros(qn, np.int8)
    for v in range(E.shape[0]):
        row = np.ascontiguousarray(E[v])
        L.orc_rmsnorm_i8_to_i8(row.ctypes.data, an.ctypes.data, d, 1, xn.ctypes.data)
        L.orc_linear_i8_to_i32(xn.ctypes.data, Wq.ctypes.data, 1, d, qn, acc.ctypes.data)
        L.orc_requant(acc.ctypes.data, qn, mult, shift, out.ctypes.data)
        tab[v] = out
    # the numpy RoPE equals the oracle's on sample rows
    for pos in (0, 7, 300):
        for query, col, fn in ((True, 0, L.orc_rope_q), (False, d, L.orc_rope_k)):
            x = np.ascontiguousarray(tab[5, col:col + 64].copy())
            ref = x.copy()
            fn(ref.ctypes.data, cos16[pos].ctypes.data, sin16[pos].ctypes.data)
            assert np.array_equal(ref, _rope(x[None], cos, sin, np.array([pos]), query)[0])

    hist = collections.defaultdict(collections.Counter)
    cols = collections.defaultdict(list)
    octets = np.zeros(8)  # splits in the first key tile by key octet, rows 64.. (which see all 64 keys)
    n_rows = 0
    causal = np.tril(np.ones((T, T), bool))
    for c in range(n_chunks):
        toks = ids[c * T:(c + 1) * T]
        inp = np.concatenate([[1022], toks[:-1]]).astype(np.int64)  # main.rs:220-226
        pos = np.arange(T)
        qkv = tab[inp]
        k = _rope(qkv[:, d:d + 64], cos, sin, pos, False)
        for h in range(H):
            q = _rope(qkv[:, 64 * h:64 * h + 64], cos, sin, pos, True)
            sc = np.clip(_sra(_sra(q @ k.T, 2) * smult[h], 15), -2**31, 2**31 - 1)
            sc = np.where(causal, sc, np.iinfo(np.int64).min)
            prev = np.maximum.accumulate(sc, axis=1)
            split = np.zeros_like(sc, bool)
            split[:, 1:] = sc[:, 1:] > prev[:, :-1]
            octets += split[64:, :64].reshape(T - 64, 8, 8).sum(axis=(0, 2))
            n_rows += T - 64
            for b in range(T // 16):
                r0, last = 16 * b, (16 * b + 15) // 64
                for kt in range(last + 1):
                    n = split[r0:r0 + 16, 64 * kt:64 * kt + 64].sum(1)
                    name = ("first+diagonal" if kt == last else "first") if kt == 0 else (
                        "diagonal" if kt == last else "interior")
                    hist[name][int(n.max()) + 1] += 1
                    cols[name].append(int(n.sum()) + 16)
    res = {}
    tot_tiles = tot_passes = 0
    for name in ("first", "first+diagonal", "interior", "diagonal"):
        h = hist[name]
        n = sum(h.values())
        p = sum(k * v for k, v in h.items())
        tot_tiles += n
        tot_passes += p
        res[name] = {"tiles": n, "mean_passes": round(p / n, 2), "mean_useful_columns": round(float(np.mean(cols[name])), 1),
                     "passes_histogram": {int(k): h[k] for k in sorted(h)}}
    res["all"] = {"tiles": tot_tiles, "mean_passes": round(tot_passes / tot_tiles, 2), "chunks": n_chunks, "heads": H,
                  "first_tile_splits_per_row_by_key_octet": [round(float(x) / n_rows, 2) for x in octets]}
    print(json.dumps(res, indent=1))


if __name__ == "__main__":
    main(int(sys.argv[1]) if len(sys.argv) > 1 else 64)
