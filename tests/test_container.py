"""CZIPv1 container (file_format.rs; main.rs:79-85, 241-279, 339-361) against
the container oracle, the reference's own file_format tests and RFC 1321."""
import hashlib
import os

import numpy as np
import pytest

import container as OC


@pytest.fixture(scope="module")
def amd():
    import czip_amd
    return czip_amd


# RFC 1321, appendix A.5
RFC1321 = [
    ("", "d41d8cd98f00b204e9800998ecf8427e"),
    ("a", "0cc175b9c0f1b6a831c399e269772661"),
    ("abc", "900150983cd24fb0d6963f7d28e17f72"),
    ("message digest", "f96b697d7cb7938d525a2f31aaf161d0"),
    ("abcdefghijklmnopqrstuvwxyz", "c3fcd3d76192e4007dfb496cca67e13b"),
    ("ABCDEFGHIJKLMNOPQRSTUVWXYZabcdefghijklmnopqrstuvwxyz0123456789", "d174ab98d277d9f5a5611c2c9f419d9f"),
    ("1234567890" * 8, "57edf4a22be3c955ac49da2e2107b67a"),
]


def test_model_id_hash_rfc1321(amd):
    for msg, digest in RFC1321:
        assert amd.model_id_hash(msg) == int(digest[:8], 16), msg
        assert OC.model_id_hash(msg) == int(digest[:8], 16), msg


def test_model_id_hash_lengths(amd):
    """Every padding case (0..200 bytes crosses the 55/56 and 64-byte block edges)."""
    rng = np.random.default_rng(1)
    for n in range(0, 201):
        s = "".join(chr(c) for c in rng.integers(33, 127, n))
        assert amd.model_id_hash(s) == OC.model_id_hash(s), n
    assert amd.model_id_hash("models/v001_eng.czm") == OC.model_id_hash("models/v001_eng.czm")


def _pack(amd, chunks, codec, **kw):
    args = dict(model_id_hash=0x12345678, context_length_log2=6, last_chunk_tokens=48, uncompressed_len=2000,
                tokenizer_id=0, flags=0)
    args.update(kw)
    return amd.pack_czip(chunks, codec=codec, **args), args


@pytest.mark.parametrize("codec", [0, 1])
def test_file_layout_against_oracle(amd, codec):
    """Outer header bytes and the decoded payload are the oracle's, byte for byte."""
    rng = np.random.default_rng(codec)
    chunks = [bytes(rng.integers(0, 256, int(n), dtype=np.uint8)) for n in rng.integers(0, 3000, 37)]
    data, a = _pack(amd, chunks, codec, last_chunk_tokens=13, context_length_log2=9, tokenizer_id=3, flags=1)
    exp_payload = OC.payload(a["model_id_hash"], 13, 3, 9, chunks)
    assert data[:16] == OC.outer_header(1, codec, 2000, 12 + 2 * len(chunks))
    assert OC.decode_outer(codec, data[16:]) == exp_payload
    f, back = amd.unpack_czip(data)
    assert back == chunks
    assert (f["flags"], f["codec"], f["uncompressed_len"], f["model_id_hash"], f["chunk_count"],
            f["last_chunk_tokens"], f["tokenizer_id"], f["context_length_log2"]) == \
        (1, codec, 2000, 0x12345678, 37, 13, 3, 9)


def test_reference_file_roundtrip(amd):
    """file_format.rs:475-504 (test_file_roundtrip), through a brotli stream."""
    chunks = [bytes([1, 2, 3, 4, 5]), bytes([6, 7, 8]), bytes([9, 10])]
    data, _ = _pack(amd, chunks, 1, tokenizer_id=1)
    f, back = amd.unpack_czip(data)
    assert f["codec"] == 1 and f["uncompressed_len"] == 2000 and f["model_id_hash"] == 0x12345678
    assert f["tokenizer_id"] == 1 and f["chunk_count"] == 3 and f["last_chunk_tokens"] == 48
    assert back == chunks
    counts = amd.chunk_token_counts(f)
    assert counts == [64, 64, 48] and sum(counts) == 64 + 64 + 48


def test_reference_custom_context_length(amd):
    """file_format.rs:507-527: log2 7 = 128 tokens per chunk."""
    data, _ = _pack(amd, [bytes([1, 2, 3]), bytes([4, 5])], 0, context_length_log2=7, last_chunk_tokens=100,
                    uncompressed_len=4000)
    f, _ = amd.unpack_czip(data)
    assert f["context_length_log2"] == 7 and amd.chunk_token_counts(f) == [128, 100]


def test_inner_header_reference_values(amd):
    """file_format.rs:440-455: hash 0x12345678, lengths [100, 150, 80], last 32."""
    chunks = [bytes(100), bytes(150), bytes(80)]
    data, _ = _pack(amd, chunks, 0, last_chunk_tokens=32)
    pay = OC.decode_outer(0, data[16:])
    assert pay[:18] == bytes.fromhex("78563412" "03000000" "2000" "00" "06" "6400" "9600" "5000")
    assert len(pay) == 18 + 330


def test_log2_zero_reads_as_default(amd):
    """file_format.rs:210-213: a stored log2 of 0 means 64 tokens per chunk."""
    data, _ = _pack(amd, [b"xy"], 0, context_length_log2=0, last_chunk_tokens=5)
    f, _ = amd.unpack_czip(data)
    assert f["context_length_log2"] == 6 and amd.chunk_token_counts(f) == [5]


def test_empty_file(amd):
    data, _ = _pack(amd, [], 1, last_chunk_tokens=64, uncompressed_len=0)
    f, back = amd.unpack_czip(data)
    assert back == [] and f["chunk_count"] == 0 and amd.chunk_token_counts(f) == []


def test_malformed_inputs(amd):
    good, _ = _pack(amd, [bytes(range(50)), bytes(70)], 0)
    with pytest.raises(amd.CzipError) as e:
        amd.unpack_czip(good[:15])                           # outer header too short
    assert e.value.code == -11
    with pytest.raises(amd.CzipError):
        amd.unpack_czip(b"CZIPv2" + good[6:])                # invalid magic
    with pytest.raises(amd.CzipError):
        amd.unpack_czip(good[:7] + bytes([7]) + good[8:])    # unknown codec
    with pytest.raises(amd.CzipError):
        amd.unpack_czip(good[:-5])                           # truncated stream
    # a payload whose chunk table promises more bytes than it holds
    import ctypes as C
    z = C.CDLL("libzstd.so.1")
    z.ZSTD_compress.restype = C.c_size_t
    z.ZSTD_compress.argtypes = [C.c_void_p, C.c_size_t, C.c_char_p, C.c_size_t, C.c_int]
    pay = OC.inner_header(1, 5, 0, 6, [10]) + bytes(4)
    buf = C.create_string_buffer(1024)
    n = z.ZSTD_compress(buf, 1024, pay, len(pay), 3)
    with pytest.raises(amd.CzipError):
        amd.unpack_czip(OC.outer_header(0, 0, 9, 14) + buf.raw[:n])
    with pytest.raises(amd.CzipError) as e:
        amd.pack_czip([bytes(65536)], model_id_hash=0, context_length_log2=6, last_chunk_tokens=1,
                      uncompressed_len=1)                    # "Chunk too large" (file_format.rs:311)
    assert e.value.code == -6


def test_level_mapping(amd):
    """main.rs:113-122."""
    assert [amd.level_to_context_length(l) for l in range(0, 7)] == [64, 64, 128, 256, 512, 1024, 64]
