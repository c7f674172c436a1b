"""CZIPv1 container oracle (test infrastructure only).

Restates the byte layout of rust/src/file_format.rs and the CLI's use of it
(main.rs:79-85, 241-279, 339-361) with `struct` and `hashlib`, and opens the
outer codec streams through the system libzstd / libbrotlidec directly (the
reference's codecs are rust crates that this image does not have, so the
outer stream is only checked to decode to the payload; the payload itself is
the byte-exact contract).  The product library never imports this module.
"""
from __future__ import annotations

import ctypes as C
import hashlib
import struct

MAGIC = b"CZIPv1"                # file_format.rs:22
OUTER_HEADER_SIZE = 16           # file_format.rs:25
DEFAULT_CONTEXT_LENGTH_LOG2 = 6  # file_format.rs:28
CODEC_ZSTD, CODEC_BROTLI = 0, 1  # file_format.rs:45-51


def model_id_hash(path: str) -> int:
    """main.rs:79-85: int(md5(path).hexdigest()[:8], 16)."""
    return int(hashlib.md5(path.encode()).hexdigest()[:8], 16)


def outer_header(flags: int, codec: int, uncompressed_len: int, header_len: int) -> bytes:
    """CZIPv1OuterHeader::to_bytes (file_format.rs:145-153)."""
    return MAGIC + struct.pack("<BBII", flags, codec, uncompressed_len, header_len)


def inner_header(model_id_hash: int, last_chunk_tokens: int, tokenizer_id: int, context_length_log2: int,
                 chunk_lens) -> bytes:
    """CZIPv1InnerHeader::to_bytes (file_format.rs:245-256)."""
    return (struct.pack("<IIHBB", model_id_hash, len(chunk_lens), last_chunk_tokens, tokenizer_id,
                        context_length_log2) + b"".join(struct.pack("<H", n) for n in chunk_lens))


def payload(model_id_hash: int, last_chunk_tokens: int, tokenizer_id: int, context_length_log2: int,
            chunks) -> bytes:
    """CompressedFile::build_payload (file_format.rs:324-331): inner header || chunk bytes."""
    return inner_header(model_id_hash, last_chunk_tokens, tokenizer_id, context_length_log2,
                        [len(c) for c in chunks]) + b"".join(chunks)


def decode_outer(codec: int, stream: bytes) -> bytes:
    """The payload of an outer codec stream, by the system libraries (main.rs:348-359)."""
    if codec == CODEC_ZSTD:
        z = C.CDLL("libzstd.so.1")
        z.ZSTD_getFrameContentSize.restype = C.c_ulonglong
        z.ZSTD_getFrameContentSize.argtypes = [C.c_char_p, C.c_size_t]
        z.ZSTD_decompress.restype = C.c_size_t
        z.ZSTD_decompress.argtypes = [C.c_void_p, C.c_size_t, C.c_char_p, C.c_size_t]
        z.ZSTD_isError.argtypes = [C.c_size_t]
        n = z.ZSTD_getFrameContentSize(stream, len(stream))
        assert n < (1 << 40), "frame without content size"
        buf = C.create_string_buffer(max(int(n), 1))
        r = z.ZSTD_decompress(buf, int(n), stream, len(stream))
        assert not z.ZSTD_isError(r)
        return buf.raw[:r]
    b = C.CDLL("libbrotlidec.so.1")
    b.BrotliDecoderDecompress.argtypes = [C.c_size_t, C.c_char_p, C.POINTER(C.c_size_t), C.c_void_p]
    cap = max(1024, 8 * len(stream))
    while True:
        buf = C.create_string_buffer(cap)
        n = C.c_size_t(cap)
        if b.BrotliDecoderDecompress(len(stream), stream, C.byref(n), buf) == 1:
            return buf.raw[:n.value]
        cap *= 4
        assert cap < (1 << 32)
