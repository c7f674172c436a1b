"""Python mirror of the compress-zip model API over libczip_hip (MI355X).

The reference exposes `ModelWeights::load` (rust/src/model.rs:108),
`Model::new` (model.rs:315), `Model::forward` (model.rs:362) and
`Model::get_cumfreqs` (model.rs:483), called once per token by the chunk
loops of rust/src/main.rs:206-238 / 377-396.  This module binds the batched
C-ABI of include/czip_hip.h that replaces those calls: whole chunks run as
one causal prefill on the GPU, and compression (forward -> CDF -> arithmetic
coding) runs end to end on the device.

There is no CPU fallback: every compute call goes to the HIP library, and
importing this module fails if the library has not been built.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from .build import LIB_PATH

KV_RUST_COMPAT = 0
KV_GQA = 1
CODEC_ZSTD = 0     # outer codecs of the .czip container (file_format.rs:45-51)
CODEC_BROTLI = 1
BOS = 1022  # rust/src/main.rs:222

STATUS = {
    0: "OK", -1: "CZIP_E_ARG", -2: "CZIP_E_CONFIG", -3: "CZIP_E_HEADS", -4: "CZIP_E_RANGE", -5: "CZIP_E_TOKEN",
    -6: "CZIP_E_OVERFLOW", -7: "CZIP_E_HIP", -8: "CZIP_E_IO", -9: "CZIP_E_MISSING", -10: "CZIP_E_NOMEM",
    -11: "CZIP_E_FORMAT",
}


class CzipError(RuntimeError):
    def __init__(self, code: int, msg: str = ""):
        self.code = code
        super().__init__(f"{STATUS.get(code, code)}: {msg}")


class LayerDesc(C.Structure):
    _fields_ = [
        ("attn_norm", C.c_void_p), ("post_attn_norm", C.c_void_p), ("ffn_norm", C.c_void_p),
        ("post_ffn_norm", C.c_void_p), ("qkv_w", C.c_void_p), ("out_w", C.c_void_p), ("up_w", C.c_void_p),
        ("down_w", C.c_void_p), ("score_mult", C.c_void_p), ("sink_key", C.c_void_p),
        ("qkv_mult", C.c_int32), ("out_mult", C.c_int32), ("up_mult", C.c_int32), ("down_mult", C.c_int32),
        ("qkv_shift", C.c_int32), ("out_shift", C.c_int32), ("up_shift", C.c_int32), ("down_shift", C.c_int32),
    ]


class ModelDesc(C.Structure):
    _fields_ = [
        ("vocab", C.c_int32), ("n_layers", C.c_int32), ("n_heads", C.c_int32), ("n_kv_heads", C.c_int32),
        ("d_model", C.c_int32), ("d_ff", C.c_int32), ("head_dim", C.c_int32), ("max_seq_len", C.c_int32),
        ("context_length", C.c_int32), ("kv_mode", C.c_int32),
        ("embed", C.c_void_p), ("final_norm", C.c_void_p), ("head_w", C.c_void_p), ("exp2_lut", C.c_void_p),
        ("rope_cos", C.c_void_p), ("rope_sin", C.c_void_p),
        ("coef_q24", C.c_uint32), ("target_total", C.c_uint32),
        ("layers", C.POINTER(LayerDesc)),
        ("exp2_len", C.c_int64), ("rope_len", C.c_int64),
    ]


class ContainerInfo(C.Structure):
    """czip_container: the header fields of a .czip file (file_format.rs:77-83, 158-165)."""
    _fields_ = [
        ("flags", C.c_uint8), ("codec", C.c_uint8), ("uncompressed_len", C.c_uint32),
        ("model_id_hash", C.c_uint32), ("chunk_count", C.c_uint32), ("last_chunk_tokens", C.c_uint16),
        ("tokenizer_id", C.c_uint8), ("context_length_log2", C.c_uint8),
    ]


# Functions declared in include/czip_hip.h, with their ctypes signatures.
_P = C.c_void_p
SIGNATURES = {
    "czip_model_load": (C.c_int32, [C.c_char_p, C.c_int32, C.POINTER(C.c_void_p)]),
    "czip_model_desc_get": (C.POINTER(ModelDesc), [_P]),
    "czip_model_tokenizer": (C.c_void_p, [_P, C.POINTER(C.c_size_t), C.POINTER(C.c_char_p)]),
    "czip_model_free": (None, [_P]),
    "czip_create": (C.c_int32, [C.POINTER(ModelDesc), C.c_int, C.POINTER(C.c_void_p)]),
    "czip_destroy": (None, [_P]),
    "czip_last_error": (C.c_char_p, [_P]),
    "czip_device_count": (C.c_int, []),
    "czip_forward_logits": (C.c_int32, [_P, _P, _P, C.c_int32, C.c_int32, _P]),
    "czip_prefill_cdf": (C.c_int32, [_P, _P, _P, C.c_int32, C.c_int32, _P]),
    "czip_prefill_cumfreqs": (C.c_int32, [_P, _P, _P, C.c_int32, C.c_int32, _P]),
    "czip_prefill_cdf_noalloc": (C.c_int32, [_P, _P, _P, C.c_int32, C.c_int32, _P]),
    "czip_compress_plan": (C.c_int32, [_P, _P, C.c_int64, C.c_int32, C.POINTER(C.c_void_p)]),
    "czip_job_run": (C.c_int32, [_P]),
    "czip_job_chunks": (C.c_int64, [_P]),
    "czip_compress_fetch": (C.c_int32, [_P, _P, C.c_int64, _P]),
    "czip_compress_fetch_packed": (C.c_int32, [_P, _P, C.c_int64, _P]),
    "czip_job_free": (None, [_P]),
    "czip_chunk_slot_bytes": (C.c_int64, [C.c_int32]),
    "czip_decompress_plan": (C.c_int32, [_P, _P, _P, _P, _P, C.c_int32, C.POINTER(C.c_void_p)]),
    "czip_decompress_fetch": (C.c_int32, [_P, _P, _P]),
    "czip_decode_begin": (C.c_int32, [_P, C.c_int32, C.c_int32]),
    "czip_decode_step": (C.c_int32, [_P, _P, _P, _P, _P]),
    "czip_decode_end": (None, [_P]),
    "czip_tokenizer_load": (C.c_int32, [C.c_char_p, C.c_size_t, C.POINTER(C.c_void_p)]),
    "czip_tokenizer_from_model": (C.c_int32, [_P, C.POINTER(C.c_void_p)]),
    "czip_tokenizer_free": (None, [_P]),
    "czip_tokenize": (C.c_int32, [_P, C.c_char_p, C.c_size_t, C.c_int32, _P, C.c_size_t,
                                  C.POINTER(C.c_size_t)]),
    "czip_detokenize": (C.c_int32, [_P, _P, C.c_size_t, _P, C.c_size_t, C.POINTER(C.c_size_t)]),
    "czip_model_id_hash": (C.c_uint32, [C.c_char_p, C.c_size_t]),
    "czip_container_pack": (C.c_int32, [C.POINTER(ContainerInfo), _P, _P, C.POINTER(C.c_void_p),
                                        C.POINTER(C.c_size_t)]),
    "czip_container_unpack": (C.c_int32, [C.c_char_p, C.c_size_t, C.POINTER(ContainerInfo),
                                          C.POINTER(C.c_void_p), C.POINTER(C.c_void_p)]),
    "czip_buffer_free": (None, [_P]),
    "czip_set_profiling": (None, [_P, C.c_int32]),
    "czip_kernel_stats": (C.c_int32, [_P, C.c_char_p, C.POINTER(C.c_int64), C.POINTER(C.c_double)]),
    "czip_reset_stats": (None, [_P]),
}

_lib = None


def lib():
    """The loaded libczip_hip.so.  Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"libczip_hip.so not built ({LIB_PATH}); run __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def device_count() -> int:
    return int(lib().czip_device_count())


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


class ModelWeights:
    """A loaded .czm file (ModelWeights::load, rust/src/model.rs:108-274)."""

    def __init__(self, path: str, kv_mode: int = KV_RUST_COMPAT):
        self._h = C.c_void_p()
        rc = lib().czip_model_load(os.fsencode(path), kv_mode, C.byref(self._h))
        if rc:
            raise CzipError(rc, f"loading {path}")
        self.path = path
        self.desc = lib().czip_model_desc_get(self._h).contents

    @property
    def config(self) -> dict:
        d = self.desc
        return dict(vocab_size=d.vocab, n_layers=d.n_layers, n_heads=d.n_heads, n_kv_heads=d.n_kv_heads,
                    d_model=d.d_model, d_ff=d.d_ff, head_dim=d.head_dim, max_seq_len=d.max_seq_len,
                    context_length=d.context_length, kv_mode=d.kv_mode, coef_q24=d.coef_q24,
                    target_total=d.target_total)

    def tokenizer_data(self):
        n = C.c_size_t()
        codec = C.c_char_p()
        ptr = lib().czip_model_tokenizer(self._h, C.byref(n), C.byref(codec))
        if not ptr:
            return None, None
        return C.string_at(ptr, n.value), codec.value.decode()

    def __del__(self):
        if getattr(self, "_h", None):
            lib().czip_model_free(self._h)
            self._h = None


class Tokenizer:
    """The model's BPE tokenizer (rust/src/tiktoken.rs), host-side C++."""

    def __init__(self, weights: "ModelWeights" = None, json_bytes: bytes = None):
        self._h = C.c_void_p()
        if json_bytes is not None:
            rc = lib().czip_tokenizer_load(json_bytes, len(json_bytes), C.byref(self._h))
        else:
            rc = lib().czip_tokenizer_from_model(weights._h, C.byref(self._h))
        if rc:
            raise CzipError(rc, "tokenizer load")

    def encode(self, text, threads: int = 1) -> np.ndarray:
        """encode_with_special_tokens (tiktoken.rs:498-501) of UTF-8 text."""
        data = text.encode("utf-8") if isinstance(text, str) else bytes(text)
        out = np.zeros(max(len(data), 1), np.uint32)
        n = C.c_size_t()
        rc = lib().czip_tokenize(self._h, data, len(data), threads, _p(out), out.size, C.byref(n))
        if rc:
            raise CzipError(rc, "tokenize")
        return out[:n.value].copy()

    def decode_bytes(self, ids) -> bytes:
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        n = C.c_size_t()
        rc = lib().czip_detokenize(self._h, _p(ids) if ids.size else None, ids.size, None, 0, C.byref(n))
        if rc not in (0, -6):
            raise CzipError(rc, "detokenize")
        buf = np.zeros(max(n.value, 1), np.uint8)
        rc = lib().czip_detokenize(self._h, _p(ids) if ids.size else None, ids.size, _p(buf), buf.size, C.byref(n))
        if rc:
            raise CzipError(rc, "detokenize")
        return buf[:n.value].tobytes()

    def __del__(self):
        if getattr(self, "_h", None):
            lib().czip_tokenizer_free(self._h)
            self._h = None


class Model:
    """Device context (Model::new, rust/src/model.rs:315-351) with batched
    forward / CDF / compression entry points."""

    def __init__(self, weights: ModelWeights, device: int = 0):
        self._ctx = C.c_void_p()
        self.weights = weights
        rc = lib().czip_create(C.byref(weights.desc), device, C.byref(self._ctx))
        if rc:
            raise CzipError(rc, "czip_create")
        self.vocab = weights.desc.vocab
        self.target_total = weights.desc.target_total

    def _check(self, rc: int):
        if rc:
            raise CzipError(rc, lib().czip_last_error(self._ctx).decode())

    def close(self):
        if getattr(self, "_ctx", None):
            lib().czip_destroy(self._ctx)
            self._ctx = None

    def __del__(self):
        self.close()

    # --- batched forward (debug / parity) ---
    def forward_logits(self, inputs: np.ndarray, lens) -> np.ndarray:
        """inputs [B, T] token ids fed at positions 0..T-1 of each chunk -> logits [B, T, V]."""
        inputs = np.ascontiguousarray(inputs, dtype=np.uint32)
        B, T = inputs.shape
        lens = np.ascontiguousarray(lens, dtype=np.int32)
        out = np.zeros((B, T, self.vocab), np.int32)
        self._check(lib().czip_forward_logits(self._ctx, _p(inputs), _p(lens), B, T, _p(out)))
        return out

    def cumfreqs(self, inputs: np.ndarray, lens) -> np.ndarray:
        inputs = np.ascontiguousarray(inputs, dtype=np.uint32)
        B, T = inputs.shape
        lens = np.ascontiguousarray(lens, dtype=np.int32)
        out = np.zeros((B, T, self.vocab), np.uint32)
        self._check(lib().czip_prefill_cumfreqs(self._ctx, _p(inputs), _p(lens), B, T, _p(out)))
        return out

    def prefill_cdf(self, targets: np.ndarray, lens) -> np.ndarray:
        """(cum_lo, cum_hi) [B, T, 2] of each target under its chunk's CDF."""
        targets = np.ascontiguousarray(targets, dtype=np.uint32)
        B, T = targets.shape
        lens = np.ascontiguousarray(lens, dtype=np.int32)
        out = np.zeros((B, T, 2), np.uint32)
        self._check(lib().czip_prefill_cdf(self._ctx, _p(targets), _p(lens), B, T, _p(out)))
        return out

    # --- compression on the device ---
    def compress_plan(self, tokens: np.ndarray, chunk: int) -> "Job":
        tokens = np.ascontiguousarray(tokens, dtype=np.uint32).reshape(-1)
        h = C.c_void_p()
        self._check(lib().czip_compress_plan(self._ctx, _p(tokens) if tokens.size else None, tokens.size, chunk,
                                             C.byref(h)))
        return Job(self, h, chunk)

    def compress_chunks(self, tokens: np.ndarray, chunk: int):
        """Per-chunk coded bytes, identical to main.rs:206-238's chunk_results."""
        job = self.compress_plan(tokens, chunk)
        try:
            job.run()
            return job.fetch()
        finally:
            job.free()

    # --- decompression on the device ---
    def decompress_plan(self, chunks, ntoks) -> "DecodeJob":
        lens = np.array([len(c) for c in chunks], np.int32)
        offs = np.zeros(len(chunks), np.int64)
        if len(chunks) > 1:
            offs[1:] = np.cumsum(lens[:-1])
        data = np.frombuffer(b"".join(chunks) + b"\0", np.uint8).copy()
        ntoks = np.ascontiguousarray(ntoks, dtype=np.int32)
        h = C.c_void_p()
        self._check(lib().czip_decompress_plan(self._ctx, _p(data), _p(offs), _p(lens), _p(ntoks), len(chunks),
                                               C.byref(h)))
        return DecodeJob(self, h, int(ntoks.sum()))

    def decompress_chunks(self, chunks, ntoks) -> np.ndarray:
        """Decoded tokens of every chunk, concatenated (main.rs:377-399)."""
        job = self.decompress_plan(chunks, ntoks)
        try:
            job.run()
            return job.fetch()
        finally:
            job.free()

    # --- step-wise decode (the caller keeps the arithmetic decoder) ---
    def decode_begin(self, S: int, T: int):
        """Open the decode session of S streams of at most T tokens."""
        self._check(lib().czip_decode_begin(self._ctx, S, T))
        self._dec_S = S

    def decode_step(self, tok_in, pos, values=None) -> np.ndarray:
        """forward + cumfreqs of every stream at its position (-1: inactive);
        with `values` (the decoders' targets) returns [S, 3] (sym, cum_lo,
        cum_hi), else the [S, V] cumulative tables."""
        tok_in = np.ascontiguousarray(tok_in, dtype=np.uint32).reshape(-1)
        S = tok_in.size
        if getattr(self, "_dec_S", None) not in (None, S):
            raise ValueError(f"the decode session has {self._dec_S} streams, got {S}")
        pos = np.ascontiguousarray(pos, dtype=np.int32).reshape(S)
        if values is None:
            out = np.zeros((S, self.vocab), np.uint32)
            vp = None
        else:
            values = np.ascontiguousarray(values, dtype=np.uint32).reshape(S)
            out = np.zeros((S, 3), np.uint32)
            vp = _p(values)
        self._check(lib().czip_decode_step(self._ctx, _p(tok_in), _p(pos), vp, _p(out)))
        return out

    def decode_end(self):
        lib().czip_decode_end(self._ctx)
        self._dec_S = None

    # --- instrumentation ---
    def set_profiling(self, on: bool):
        lib().czip_set_profiling(self._ctx, 1 if on else 0)

    def kernel_stats(self, name: str):
        n = C.c_int64()
        ms = C.c_double()
        self._check(lib().czip_kernel_stats(self._ctx, name.encode(), C.byref(n), C.byref(ms)))
        return int(n.value), float(ms.value)

    def reset_stats(self):
        lib().czip_reset_stats(self._ctx)


class Job:
    def __init__(self, model: Model, handle, chunk: int):
        self.model = model
        self.h = handle
        self.chunk = chunk
        self.nchunks = int(lib().czip_job_chunks(handle))

    def run(self):
        self.model._check(lib().czip_job_run(self.h))

    def fetch_slots(self):
        """Per-chunk coded bytes through the fixed-slot copy (czip_compress_fetch)."""
        slot = int(lib().czip_chunk_slot_bytes(self.chunk))
        buf = np.zeros(max(self.nchunks, 1) * slot, np.uint8)
        lens = np.zeros(max(self.nchunks, 1), np.int32)
        self.model._check(lib().czip_compress_fetch(self.h, _p(buf), slot, _p(lens)))
        return [bytes(buf[c * slot:c * slot + lens[c]]) for c in range(self.nchunks)]

    def fetch_packed(self):
        """(coded bytes of every chunk back to back, offsets [nchunks + 1])."""
        offs = np.zeros(self.nchunks + 1, np.int64)
        self.model._check(lib().czip_compress_fetch_packed(self.h, None, 0, _p(offs)))
        buf = np.zeros(max(int(offs[-1]), 1), np.uint8)
        self.model._check(lib().czip_compress_fetch_packed(self.h, _p(buf), buf.size, _p(offs)))
        return buf[:int(offs[-1])], offs

    def fetch(self):
        """Per-chunk coded bytes (the chunk_results of main.rs:206-238)."""
        buf, offs = self.fetch_packed()
        data = buf.tobytes()
        return [data[offs[c]:offs[c + 1]] for c in range(self.nchunks)]

    def free(self):
        if self.h:
            lib().czip_job_free(self.h)
            self.h = None

    def __del__(self):
        self.free()


class DecodeJob(Job):
    def __init__(self, model: Model, handle, total_tokens: int):
        super().__init__(model, handle, 0)
        self.total_tokens = total_tokens

    def fetch(self):
        out = np.zeros(max(self.total_tokens, 1), np.uint32)
        self.model._check(lib().czip_decompress_fetch(self.h, _p(out), None))
        return out[:self.total_tokens]


# ---------------------------------------------------------------------------
# The .czip container and the whole-file flow of the reference CLI
# (main.rs:125-302 compress, 304-399 decompress).
# ---------------------------------------------------------------------------
def level_to_context_length(level: int) -> int:
    """main.rs:113-122: levels 1-5 are 64..1024 tokens per chunk, others 64."""
    return {1: 64, 2: 128, 3: 256, 4: 512, 5: 1024}.get(level, 64)


def model_id_hash(path: str) -> int:
    """main.rs:79-85: the first 8 hex digits of MD5 of the model path as given."""
    b = os.fsencode(path)
    return int(lib().czip_model_id_hash(b, len(b)))


def pack_czip(chunks, *, model_id_hash: int, context_length_log2: int, last_chunk_tokens: int,
              uncompressed_len: int, codec: int = CODEC_BROTLI, tokenizer_id: int = 0, flags: int = 0) -> bytes:
    """The .czip bytes of coded chunks (file_format.rs:385-392 + main.rs:255-279)."""
    offs = np.zeros(len(chunks) + 1, np.int64)
    offs[1:] = np.cumsum([len(c) for c in chunks]) if chunks else []
    data = np.frombuffer(b"".join(chunks) or b"\0", np.uint8)
    info = ContainerInfo(flags, codec, uncompressed_len, model_id_hash, len(chunks), last_chunk_tokens,
                         tokenizer_id, context_length_log2)
    out, n = C.c_void_p(), C.c_size_t()
    rc = lib().czip_container_pack(C.byref(info), _p(data), _p(offs), C.byref(out), C.byref(n))
    if rc:
        raise CzipError(rc, "czip_container_pack")
    try:
        return C.string_at(out, n.value)
    finally:
        lib().czip_buffer_free(out)


def unpack_czip(data: bytes):
    """(header fields, list of chunk bytes) of a .czip file (main.rs:332-361)."""
    info = ContainerInfo()
    chunks, offs = C.c_void_p(), C.c_void_p()
    rc = lib().czip_container_unpack(data, len(data), C.byref(info), C.byref(chunks), C.byref(offs))
    if rc:
        raise CzipError(rc, "czip_container_unpack")
    try:
        n = info.chunk_count
        o = np.ctypeslib.as_array(C.cast(offs, C.POINTER(C.c_int64)), (n + 1,)).copy()
        body = C.string_at(chunks, int(o[-1])) if o[-1] else b""
    finally:
        lib().czip_buffer_free(chunks)
        lib().czip_buffer_free(offs)
    fields = {f: getattr(info, f) for f, _ in ContainerInfo._fields_}
    return fields, [body[o[i]:o[i + 1]] for i in range(n)]


def chunk_token_counts(fields: dict):
    """Tokens of each chunk (file_format.rs:333-352)."""
    n = fields["chunk_count"]
    per = 1 << fields["context_length_log2"]
    return [per] * (n - 1) + [fields["last_chunk_tokens"]] if n else []


def compress_text(model: "Model", tokenizer: "Tokenizer", text: bytes, model_path: str, level: int = None,
                  codec: int = CODEC_BROTLI, threads: int = 16) -> bytes:
    """main.rs:125-302: tokenize, code every chunk on the device, write the container.
    level=None uses the model's context length, like the CLI without -L."""
    cfg = model.weights.config
    chunk = cfg["context_length"] if level is None else min(level_to_context_length(level), cfg["context_length"])
    log2 = int(np.log2(chunk))
    ids = tokenizer.encode(text, threads=threads)
    chunks = model.compress_chunks(ids, chunk) if ids.size else []
    last = ids.size - chunk * (len(chunks) - 1) if chunks else chunk
    return pack_czip(chunks, model_id_hash=model_id_hash(model_path), context_length_log2=log2,
                     last_chunk_tokens=last, uncompressed_len=len(text), codec=codec)


def decompress_czip(model: "Model", tokenizer: "Tokenizer", data: bytes) -> bytes:
    """main.rs:304-399: read the container, decode every chunk on the device, detokenize."""
    fields, chunks = unpack_czip(data)
    ntoks = chunk_token_counts(fields)
    ids = model.decompress_chunks(chunks, ntoks) if chunks else np.zeros(0, np.uint32)
    return tokenizer.decode_bytes(ids)
