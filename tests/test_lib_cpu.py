"""CPU-side checks of the C-ABI library: it loads, exports every entry point
the header declares, and its host-only parts (the .czm loader and the
context's configuration checks) behave like the reference."""
import os
import re

import numpy as np
import pytest

from conftest import MODEL_PATH, ROOT


def _header_functions():
    src = open(os.path.join(ROOT, "include", "czip_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(czip_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_header_symbols():
    import czip_amd
    L = czip_amd.lib()
    names = _header_functions()
    assert len(names) >= 20
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(czip_amd.SIGNATURES), set(names) ^ set(czip_amd.SIGNATURES)


def test_loader_matches_oracle_parse(orc):
    import czip_amd
    w = czip_amd.ModelWeights(MODEL_PATH)
    cfg = w.config
    t, meta = orc.read_czm(MODEL_PATH)
    assert cfg["vocab_size"] == 1024 and cfg["d_model"] == 384 and cfg["n_layers"] == 1
    assert cfg["n_heads"] == 6 and cfg["n_kv_heads"] == 1 and cfg["d_ff"] == 1024
    assert cfg["context_length"] == 1024 and cfg["max_seq_len"] == 8192
    assert cfg["coef_q24"] == 37819 and cfg["target_total"] == 1073739776
    d = w.desc
    L0 = d.layers[0]
    assert (L0.qkv_mult, L0.qkv_shift, L0.out_mult, L0.up_shift, L0.down_mult) == (819, 20, 819, 20, 819)
    import ctypes as C
    emb = np.ctypeslib.as_array(C.cast(d.embed, C.POINTER(C.c_int8)), shape=(1024 * 384,))
    assert np.array_equal(emb, t["embed.weight"].reshape(-1))
    assert d.exp2_len == 256 and d.rope_len == 1024 * 32
    data, codec = w.tokenizer_data()
    assert codec == "zstd" and len(data) == 4563


def test_loader_errors(tmp_path):
    import czip_amd
    from czip_amd import synth
    with pytest.raises(czip_amd.CzipError) as e:
        czip_amd.ModelWeights(str(tmp_path / "missing.czm"))
    assert e.value.code == -8
    t, meta = synth.random_model_tensors(d=256, n_layers=1, n_heads=4, n_kv=1, d_ff=256, vocab=256, ctx=64)
    del t["norm.weight"]
    p = str(tmp_path / "nonorm.czm")
    synth.write_czm(p, t, meta)
    with pytest.raises(czip_amd.CzipError) as e:
        czip_amd.ModelWeights(p)
    assert e.value.code == -9          # "Missing tensor" (model.rs:152-154)


def _patch_header(src: str, dst: str, edit):
    """Rewrite the JSON header of a .czm file (same blob after it)."""
    import json
    import struct
    blob = open(src, "rb").read()
    (hlen,) = struct.unpack("<Q", blob[:8])
    hdr = json.loads(blob[8:8 + hlen])
    edit(hdr)
    hj = json.dumps(hdr).encode()
    hj += b" " * ((8 - len(hj) % 8) % 8)
    open(dst, "wb").write(struct.pack("<Q", len(hj)) + hj + blob[8 + hlen:])


@pytest.mark.parametrize("bad", ["neg_offset", "str_offset", "float_offset", "neg_dim", "huge_dim", "past_end",
                                 "swapped"])
def test_loader_rejects_malformed_offsets(tmp_path, bad):
    """data_offsets and shape entries must be non-negative integers inside
    the file (usize in safetensors.rs:287-376): a crafted header gives
    CZIP_E_IO instead of a tensor pointing outside the blob."""
    import czip_amd
    from czip_amd import synth
    good = synth.write_random_model(str(tmp_path / "good.czm"), d=256, n_layers=1, n_heads=4, n_kv=1, d_ff=256,
                                    vocab=256, ctx=64)
    czip_amd.ModelWeights(good)

    def edit(h):
        e = h["embed.weight"]
        a, b = e["data_offsets"]
        if bad == "neg_offset":
            e["data_offsets"] = [a - (1 << 40), b - (1 << 40)]
        elif bad == "str_offset":
            e["data_offsets"] = [str(a), b]
        elif bad == "float_offset":
            e["data_offsets"] = [float(a), float(b)]
        elif bad == "neg_dim":
            e["shape"] = [-e["shape"][0], -e["shape"][1]]
        elif bad == "huge_dim":
            e["shape"] = [1 << 62, 1 << 62]
        elif bad == "past_end":
            e["data_offsets"] = [a + (1 << 30), b + (1 << 30)]
        else:
            e["data_offsets"] = [b, a]
    p = str(tmp_path / f"{bad}.czm")
    _patch_header(good, p, edit)
    with pytest.raises(czip_amd.CzipError) as e:
        czip_amd.ModelWeights(p)
    assert e.value.code == -8


def test_random_model_roundtrip(tmp_path, orc):
    import czip_amd
    from czip_amd import synth
    p = str(tmp_path / "r.czm")
    synth.write_random_model(p, d=512, n_layers=2, n_heads=8, n_kv=2, d_ff=512, vocab=1024, ctx=256, seed=3)
    w = czip_amd.ModelWeights(p)
    t, meta = orc.read_czm(p)
    assert w.config["n_kv_heads"] == 2 and w.config["context_length"] == 256
    assert int(t["softmax.target_total"]) == (1 << 30) - 1024 - 1024
    m = orc.Model(t, meta)
    assert m.check() == 0


def test_context_config_errors(tmp_path):
    """Configuration panics of the reference become status codes before any
    device work (attention.rs:172, lut.rs:148-165)."""
    import czip_amd
    from czip_amd import synth
    t, meta = synth.random_model_tensors(d=320, n_layers=1, n_heads=5, n_kv=1, d_ff=256, vocab=256, ctx=64)
    p = str(tmp_path / "h5.czm")
    synth.write_czm(p, t, meta)
    w = czip_amd.ModelWeights(p)
    with pytest.raises(czip_amd.CzipError) as e:
        czip_amd.Model(w)
    assert e.value.code == -3
    t, meta = synth.random_model_tensors(d=256, n_layers=1, n_heads=4, n_kv=1, d_ff=256, vocab=256, ctx=64)
    t["lut.rope_cos"] = t["lut.rope_cos"][:32]
    p = str(tmp_path / "rope.czm")
    synth.write_czm(p, t, meta)
    with pytest.raises(czip_amd.CzipError) as e:
        czip_amd.Model(czip_amd.ModelWeights(p))
    assert e.value.code == -11


def test_synthetic_text_is_deterministic():
    from czip_amd import synth
    a = synth.synthetic_text(5000, seed=5)
    b = synth.synthetic_text(5000, seed=5)
    assert a == b and len(a) == 5000
    assert set(a) <= set(b"abcdefghijklmnopqrstuvwxyz .,;:!?\n")
    lines = a.split(b"\n")
    assert max(len(x) for x in lines[:-1]) < 100
