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
