"""Seeded synthetic workloads: text, Zipf token ids and random-init .czm models.

Everything here is deterministic for a given seed (numpy PCG64), so the GPU
box regenerates byte-identical inputs without shipping them.

* `synthetic_text`: words drawn Zipf(s=1.1) from a 5k-word lexicon of 2-10
  lowercase letters, separated by a space or a punctuation mark + space
  (10 %), with a newline replacing the separator about every 80 characters.
* `zipf_ids`: token ids ~ Zipf(1.1) over [0, vocab) through a seeded
  rank -> id permutation.
* `write_random_model`: an int8 model in the .czm layout read by
  rust/src/model.rs:108-274 (tensor names model.rs:190-256), weights
  clamp(round(N(0, 32^2)), +-127), requant mult 819 with seeded per-layer
  shifts, score_mult ~ 59000 +- jitter, norms 127, LUTs from lut.rs:40-52 /
  97-136, softmax constants coef_q24 = 37819 and target_total = 2^30-V-1024.
"""
from __future__ import annotations

import json
import struct

import numpy as np

PUNCT = np.frombuffer(b".,;:!?", np.uint8)


def _zipf_ranks(rng, n_items: int, count: int, s: float = 1.1) -> np.ndarray:
    w = 1.0 / np.arange(1, n_items + 1, dtype=np.float64) ** s
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    u = rng.random(count)
    return np.minimum(np.searchsorted(cdf, u, side="right"), n_items - 1)


def lexicon(seed: int = 1234, n_words: int = 5000):
    rng = np.random.default_rng(seed)
    words, seen = [], set()
    while len(words) < n_words:
        ln = int(rng.integers(2, 11))
        w = bytes((rng.integers(0, 26, ln) + ord("a")).astype(np.uint8))
        if w not in seen:
            seen.add(w)
            words.append(w)
    return words


def synthetic_text(n_bytes: int, seed: int = 1234) -> bytes:
    """ASCII text of exactly n_bytes bytes."""
    words = lexicon(seed)
    wl = np.array([len(w) for w in words], np.int64)
    flat = np.frombuffer(b"".join(words), np.uint8)
    woff = np.concatenate([[0], np.cumsum(wl)[:-1]])
    rng = np.random.default_rng(seed + 1)
    out = []
    total = 0
    while total < n_bytes:
        n = max(1024, (n_bytes - total) // 5 + 64)
        ranks = _zipf_ranks(rng, len(words), n)
        punct = rng.random(n) < 0.10
        pch = PUNCT[rng.integers(0, len(PUNCT), n)]
        lens = wl[ranks] + np.where(punct, 2, 1)
        ends = np.cumsum(lens) + total
        newline = (ends // 80) != ((ends - lens) // 80)
        buf = np.empty(int(lens.sum()), np.uint8)
        starts = np.concatenate([[0], np.cumsum(lens)[:-1]])
        # word bytes: word i occupies buf[starts[i] : starts[i] + wlr[i]]
        wlr = wl[ranks]
        rep = np.repeat(np.arange(n), wlr)
        within = np.arange(int(wlr.sum())) - np.repeat(np.concatenate([[0], np.cumsum(wlr)[:-1]]), wlr)
        buf[starts[rep] + within] = flat[woff[ranks][rep] + within]
        sep_at = starts + wlr
        buf[sep_at[punct]] = pch[punct]
        last = np.where(punct, sep_at + 1, sep_at)
        buf[last] = np.where(newline, ord("\n"), ord(" ")).astype(np.uint8)
        out.append(buf.tobytes())
        total += buf.size
    return b"".join(out)[:n_bytes]


def zipf_ids(n: int, vocab: int, seed: int = 7, s: float = 1.1) -> np.ndarray:
    rng = np.random.default_rng(seed)
    perm = rng.permutation(vocab).astype(np.uint32)
    return perm[_zipf_ranks(rng, vocab, n, s)]


def exp2_lut() -> np.ndarray:
    return np.clip(np.rint(2.0 ** (-np.arange(256) / 256.0) * 65536.0), 1, 65535).astype(np.uint16)


def rope_luts(ctx: int, theta: float = 10000.0):
    i = np.arange(32, dtype=np.float64)
    freq = 1.0 / theta ** (2 * i / 64.0)
    ang = np.arange(ctx, dtype=np.float64)[:, None] * freq[None, :]
    c = np.clip(np.rint(np.cos(ang) * 32768.0), -32768, 32767).astype(np.int16)
    s = np.clip(np.rint(np.sin(ang) * 32768.0), -32768, 32767).astype(np.int16)
    return c, s


def write_czm(path: str, tensors: dict, metadata: dict):
    """Write tensors (name -> ndarray) + string metadata in the safetensors layout."""
    dt = {np.dtype(np.int8): "I8", np.dtype(np.uint8): "U8", np.dtype(np.int16): "I16",
          np.dtype(np.uint16): "U16", np.dtype(np.int32): "I32", np.dtype(np.uint32): "U32"}
    header = {"__metadata__": {k: str(v) for k, v in metadata.items()}}
    off = 0
    blobs = []
    for name in sorted(tensors):
        a = np.asarray(tensors[name])  # keeps 0-d scalars 0-d (shape [])
        b = a.tobytes()
        header[name] = {"dtype": dt[a.dtype], "shape": list(a.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    hj = json.dumps(header, separators=(",", ":")).encode()
    hj += b" " * ((8 - len(hj) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hj)))
        f.write(hj)
        for b in blobs:
            f.write(b)


def random_model_tensors(d: int, n_layers: int, n_heads: int, n_kv: int, d_ff: int, vocab: int, ctx: int,
                         seed: int = 0, sink: bool = False, max_seq_len: int = 8192):
    rng = np.random.default_rng(seed)

    def w(*shape):
        return np.clip(np.rint(rng.normal(0.0, 32.0, shape)), -127, 127).astype(np.int8)

    t = {"embed.weight": w(vocab, d), "head.weight": w(vocab, d), "norm.weight": np.full(d, 127, np.int8),
         "head.mult": np.array(819, np.int32), "head.shift": np.array(20, np.int8)}
    for l in range(n_layers):
        p = f"layers.{l}"
        t[f"{p}.attn_norm.weight"] = np.full(d, 127, np.int8)
        t[f"{p}.post_attn_norm.weight"] = np.full(d, 127, np.int8)
        t[f"{p}.ffn_norm.weight"] = np.full(d, 127, np.int8)
        t[f"{p}.post_ffn_norm.weight"] = np.full(d, 127, np.int8)
        t[f"{p}.attn.qkv.weight"] = w(d + 2 * n_kv * 64, d)
        t[f"{p}.attn.out.weight"] = w(d, d)
        t[f"{p}.ffn.up.weight"] = w(2 * d_ff, d)
        t[f"{p}.ffn.down.weight"] = w(d, d_ff)
        t[f"{p}.attn.score_mult"] = (59000 + rng.integers(-1500, 1501, n_heads)).astype(np.int32)
        t[f"{p}.attn.score_shift"] = np.array(15, np.int8)
        for nm in ("attn.qkv", "attn.out", "ffn.up", "ffn.down"):
            t[f"{p}.{nm}.mult"] = np.array(819, np.int32)
            t[f"{p}.{nm}.shift"] = np.array(int(rng.integers(18, 22)), np.int8)
        if sink:
            t[f"{p}.attn.sink_key"] = w(64)
    t["lut.exp2"] = exp2_lut()
    c, s = rope_luts(ctx)
    t["lut.rope_cos"], t["lut.rope_sin"] = c, s
    t["softmax.coef_q24"] = np.array(37819, np.uint32)
    t["softmax.target_total"] = np.array((1 << 30) - vocab - 1024, np.uint32)
    meta = {"format": "czip-model-v1", "vocab_size": vocab, "d_model": d, "n_layers": n_layers, "n_heads": n_heads,
            "n_kv_heads": n_kv, "d_ff": d_ff, "head_dim": 64, "context_length": ctx,
            "context_length_log2": int(np.log2(ctx)), "max_seq_len": max_seq_len, "rope_theta_q16": 655360000}
    return t, meta


def write_random_model(path: str, **kw):
    t, meta = random_model_tensors(**kw)
    write_czm(path, t, meta)
    return path


# The random-init workloads (shapes of the configurations the bench names).
MODEL_SHAPES = {
    "d512_l8": dict(d=512, n_layers=8, n_heads=8, n_kv=2, d_ff=2048, vocab=1024, ctx=1024),
    "d768_l12": dict(d=768, n_layers=12, n_heads=12, n_kv=4, d_ff=3072, vocab=8192, ctx=4096),
}
