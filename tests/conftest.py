import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "compress-zip_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

MODEL_PATH = os.path.join(ROOT, "models", "v001_eng.czm")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) to run")
    config.addinivalue_line("markers", "slow: longer CPU test")


def _ensure_oracle():
    import oracle as O
    if not os.path.exists(O.LIB_PATH):
        O.build()
    return O


@pytest.fixture(scope="session")
def orc():
    return _ensure_oracle()


@pytest.fixture(scope="session")
def shipped(orc):
    return orc.Model.from_file(MODEL_PATH)


def gpu_available() -> bool:
    try:
        import czip_amd
        return czip_amd.device_count() > 0
    except Exception:
        return False


def write_vacc_wrap_model(path: str, seed: int = 110) -> str:
    """A 2-layer model whose layer-0 attention sums wrap the i32 `vacc` of
    attention.rs:207-208,274 from position 258 on: Q is zero (every score is
    0, every weight E(0) = 65535), the embeddings are positive so the value
    projection rows of +-127 requantize to V = +127 on even and -127 on odd
    head dims, and 65535 * 127 * (p + 1) passes 2^31 at p + 1 = 259.
    Layer 1 keeps random weights.  Reference KV semantics (V = the 64 QKV
    values after K), context 512."""
    import numpy as np
    from czip_amd import synth
    d = 256
    t, meta = synth.random_model_tensors(d=d, n_layers=2, n_heads=4, n_kv=1, d_ff=256, vocab=1024, ctx=512, seed=seed)
    rng = np.random.default_rng(seed + 1)
    t["embed.weight"] = rng.integers(1, 128, (1024, d)).astype(np.int8)
    qkv = t["layers.0.attn.qkv.weight"].copy()
    qkv[:d] = 0
    qkv[d + 64:d + 128] = np.where(np.arange(64) % 2 == 0, 127, -127)[:, None].astype(np.int8)
    t["layers.0.attn.qkv.weight"] = qkv
    synth.write_czm(path, t, meta)
    return path


# --- GQA pins: a model whose attention output has a closed form -------------
def _sra_rne(v: int, sh: int) -> int:
    """sign(v) * RNE(|v| / 2^sh), ties to even (primitives.rs:18-42)."""
    if sh == 0:
        return v
    a = abs(v)
    q, r = a >> sh, a & ((1 << sh) - 1)
    half = 1 << (sh - 1)
    if r > half or (r == half and q & 1):
        q += 1
    return -q if v < 0 else q


def _udiv_rne(n: int, d: int) -> int:
    q, r = divmod(n, d)
    return q + 1 if 2 * r > d or (2 * r == d and q & 1) else q


def _rmsnorm(v, w: int):
    """rmsnorm_i8_to_i8 of clamp(v) with every weight w (rmsnorm.rs:14-75)."""
    import math
    x8 = [min(127, max(-127, int(t))) for t in v]
    ms = max(sum(t * t for t in x8) // len(x8) + 1, 1)
    inv = min(max(_udiv_rne(1 << 23, math.isqrt(ms << 16)), 1), 32768)
    return [min(127, max(-127, _sra_rne(t * w * inv, 15))) for t in x8]


def write_gqa_pin_model(path: str, H: int, G: int) -> str:
    """One layer whose attention output of head h is exactly
    floor(h G / H) + 1 in every head dim, in the GQA mode's slicing (query
    head h reads KV group floor(h G / H); the QKV rows are [Q | K of groups
    0..G-1 | V of groups 0..G-1], 64 rows per group):
      * every token embeds as all ones, so the pre-attention norm is all ones;
      * Q and K rows are zero: every score is 0, every weight E(0) = 65535,
        so a head's output is the (constant) V of its group;
      * V row r of group g is (g + 1, 0, 0, ...) with requant (mult 1,
        shift 0): V = g + 1 in every dim of group g.
    The rest makes the logits a known function of that output: O projection
    = identity (mult 1, shift 0), FFN up rows zero (the FFN adds rmsnorm(0)
    = 0), LM head row v = unit vector v for v < d, post-attention norm 32,
    final norm 64."""
    import numpy as np
    from czip_amd import synth
    d = 64 * H
    t, meta = synth.random_model_tensors(d=d, n_layers=1, n_heads=H, n_kv=G, d_ff=128, vocab=1024, ctx=128, seed=7)
    t["embed.weight"] = np.ones((1024, d), np.int8)
    t["layers.0.attn_norm.weight"] = np.ones(d, np.int8)
    qkv = np.zeros((d + 2 * G * 64, d), np.int8)
    for g in range(G):
        qkv[d + G * 64 + 64 * g: d + G * 64 + 64 * (g + 1), 0] = g + 1
    t["layers.0.attn.qkv.weight"] = qkv
    t["layers.0.attn.out.weight"] = np.eye(d, dtype=np.int8)
    t["layers.0.ffn_norm.weight"] = np.full(d, 32, np.int8)  # small enough that no group's value clamps
    t["norm.weight"] = np.full(d, 64, np.int8)
    t["layers.0.ffn.up.weight"] = np.zeros_like(t["layers.0.ffn.up.weight"])
    head = np.zeros((1024, d), np.int8)
    head[np.arange(d), np.arange(d)] = 1
    t["head.weight"] = head
    for nm in ("attn.qkv", "attn.out", "ffn.up", "ffn.down"):
        t[f"layers.0.{nm}.mult"] = np.array(1, np.int32)
        t[f"layers.0.{nm}.shift"] = np.array(0, np.int8)
    synth.write_czm(path, t, meta)
    return path


def gqa_pin_logits(H: int, G: int):
    """The logits row of every position of write_gqa_pin_model(H, G): from the
    attention output floor(h G / H) + 1 through the identity O projection,
    the post-attention norm and residual (embedding 1), a zero FFN, the final
    norm and the unit-vector LM head."""
    import numpy as np
    d = 64 * H
    attn = [(i // 64) * G // H + 1 for i in range(d)]
    x = [1 + n for n in _rmsnorm(attn, 32)]
    row = np.zeros(1024, np.int32)
    row[:d] = _rmsnorm(x, 64)
    return row


GQA_PIN_SHAPES = [(8, 2), (12, 4), (6, 3), (16, 4), (4, 4)]
