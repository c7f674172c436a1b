"""ctypes binding of the C oracle (test infrastructure only).

The oracle restates the reference Rust crate (rust/src) in C; this module
loads `oracle/_build/liboracle.so`, parses `.czm` files with numpy (the
safetensors layout read by rust/src/safetensors.rs:287-376), and exposes the
model forward, cumulative-frequency builder, arithmetic coder and chunk
driver for the parity tests and for bench.py's CPU baseline.  The product
library never imports this module.
"""
from __future__ import annotations

import ctypes as C
import json
import os
import struct
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
BUILD = os.path.join(HERE, "_build")
LIB_PATH = os.path.join(BUILD, "liboracle.so")

KV_RUST_COMPAT = 0
KV_GQA = 1

# rust/src/safetensors.rs:226-243 ("BOOL" is read as I32 there)
_DTYPES = {
    "I8": np.int8, "I16": np.int16, "I32": np.int32, "BOOL": np.int32, "I64": np.int64,
    "U8": np.uint8, "U16": np.uint16, "U32": np.uint32, "F16": np.float16, "F32": np.float32,
}


def build(native: bool = False, out: str | None = None) -> str:
    """Compile the oracle with gcc (x86-64-v3 portable build, or -march=native)."""
    os.makedirs(BUILD, exist_ok=True)
    out = out or (os.path.join(BUILD, "liboracle_native.so") if native else LIB_PATH)
    arch = "-march=native" if native else "-march=x86-64-v3"
    cmd = ["gcc", "-O3", arch, "-fPIC", "-shared", "-std=c11", "-Wall",
           os.path.join(HERE, "czip_oracle.c"), "-o", out, "-lpthread", "-lm"]
    subprocess.check_call(cmd)
    return out


def read_czm(path: str):
    """Parse a .czm (safetensors) file into ({name: ndarray}, metadata)."""
    with open(path, "rb") as f:
        blob = f.read()
    (hlen,) = struct.unpack("<Q", blob[:8])
    header = json.loads(blob[8:8 + hlen].decode("utf-8"))
    meta = header.pop("__metadata__", {}) or {}
    base = 8 + hlen
    tensors = {}
    for name, info in header.items():
        dt = _DTYPES[info["dtype"]]
        a, b = info["data_offsets"]
        arr = np.frombuffer(blob, dtype=dt, count=(b - a) // np.dtype(dt).itemsize, offset=base + a)
        shape = tuple(info["shape"])
        tensors[name] = arr.reshape(shape) if shape else arr.reshape(())
    return tensors, {k: str(v) for k, v in meta.items()}


class OrcLayer(C.Structure):
    _fields_ = [
        ("attn_norm", C.c_void_p), ("post_attn_norm", C.c_void_p), ("ffn_norm", C.c_void_p),
        ("post_ffn_norm", C.c_void_p), ("qkv_w", C.c_void_p), ("out_w", C.c_void_p),
        ("up_w", C.c_void_p), ("down_w", C.c_void_p), ("score_mult", C.c_void_p),
        ("sink_key", C.c_void_p),
        ("qkv_mult", C.c_int32), ("out_mult", C.c_int32), ("up_mult", C.c_int32), ("down_mult", C.c_int32),
        ("qkv_shift", C.c_int32), ("out_shift", C.c_int32), ("up_shift", C.c_int32), ("down_shift", C.c_int32),
    ]


class OrcModel(C.Structure):
    _fields_ = [
        ("vocab", C.c_int32), ("n_layers", C.c_int32), ("n_heads", C.c_int32), ("n_kv_heads", C.c_int32),
        ("d_model", C.c_int32), ("d_ff", C.c_int32), ("head_dim", C.c_int32), ("max_seq_len", C.c_int32),
        ("context_length", C.c_int32), ("kv_mode", C.c_int32),
        ("embed", C.c_void_p), ("final_norm", C.c_void_p), ("head_w", C.c_void_p),
        ("exp2_lut", C.c_void_p), ("rope_cos", C.c_void_p), ("rope_sin", C.c_void_p),
        ("coef_q24", C.c_uint32), ("target_total", C.c_uint32),
        ("layers", C.POINTER(OrcLayer)),
    ]


class OrcEncoder(C.Structure):
    _fields_ = [("low", C.c_uint64), ("high", C.c_uint64), ("underflow", C.c_uint32),
                ("out", C.c_void_p), ("len", C.c_size_t), ("cap", C.c_size_t),
                ("cur", C.c_uint8), ("bit_pos", C.c_int32)]


class OrcDecoder(C.Structure):
    _fields_ = [("low", C.c_uint64), ("high", C.c_uint64), ("code", C.c_uint64),
                ("inp", C.c_void_p), ("len", C.c_size_t), ("byte_pos", C.c_size_t), ("bit_pos", C.c_int32)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run __graft_entry__.build())")
        _lib = load(LIB_PATH)
    return _lib


def load(path: str):
    L = C.CDLL(path)
    p = C.c_void_p
    L.orc_clamp_i8.restype = C.c_int8; L.orc_clamp_i8.argtypes = [C.c_int32]
    L.orc_sra_rne_s32.restype = C.c_int32; L.orc_sra_rne_s32.argtypes = [C.c_int32, C.c_uint32]
    L.orc_sra_rne_s64_to_s32.restype = C.c_int32; L.orc_sra_rne_s64_to_s32.argtypes = [C.c_int64, C.c_uint32]
    L.orc_udiv_rne_u32.restype = C.c_uint32; L.orc_udiv_rne_u32.argtypes = [C.c_uint32, C.c_uint32]
    L.orc_div_rne_s32.restype = C.c_int32; L.orc_div_rne_s32.argtypes = [C.c_int32, C.c_int32]
    L.orc_div_rne_s32_by_u64.restype = C.c_int32; L.orc_div_rne_s32_by_u64.argtypes = [C.c_int32, C.c_uint64]
    L.orc_isqrt32.restype = C.c_uint32; L.orc_isqrt32.argtypes = [C.c_uint32]
    L.orc_argmax.restype = C.c_size_t; L.orc_argmax.argtypes = [p, C.c_size_t]
    L.orc_exp_q16_from_neg_fixed.restype = C.c_int32; L.orc_exp_q16_from_neg_fixed.argtypes = [C.c_int32, p]
    L.orc_exp_q16_coef.restype = C.c_uint16; L.orc_exp_q16_coef.argtypes = [C.c_int32, p, C.c_uint32]
    L.orc_attn_coef_q24.restype = C.c_uint32; L.orc_attn_coef_q24.argtypes = []
    L.orc_cdf_coef_q24.restype = C.c_uint32; L.orc_cdf_coef_q24.argtypes = []
    L.orc_target_total.restype = C.c_uint32; L.orc_target_total.argtypes = [C.c_uint32]
    L.orc_gen_exp2_lut.restype = None; L.orc_gen_exp2_lut.argtypes = [p]
    L.orc_gen_rope_lut.restype = None; L.orc_gen_rope_lut.argtypes = [C.c_double, C.c_int, p, p]
    L.orc_inv_rms_q15.restype = C.c_int32; L.orc_inv_rms_q15.argtypes = [C.c_int32]
    L.orc_rmsnorm_i8_to_i8.restype = None; L.orc_rmsnorm_i8_to_i8.argtypes = [p, p, C.c_int, C.c_int32, p]
    L.orc_linear_i8_to_i32.restype = None
    L.orc_linear_i8_to_i32.argtypes = [p, p, C.c_int, C.c_int, C.c_int, p]
    L.orc_requant.restype = None; L.orc_requant.argtypes = [p, C.c_int, C.c_int32, C.c_int8, p]
    L.orc_reglu.restype = None; L.orc_reglu.argtypes = [p, C.c_int, p]
    L.orc_rope_k.restype = None; L.orc_rope_k.argtypes = [p, p, p]
    L.orc_rope_q.restype = None; L.orc_rope_q.argtypes = [p, p, p]
    L.orc_attend_head.restype = None
    L.orc_attend_head.argtypes = [p, p, p, C.c_int, C.c_int32, p, p, p, p, p]
    L.orc_vacc_wraps.restype = C.c_int64; L.orc_vacc_wraps.argtypes = []
    L.orc_vacc_wraps_reset.restype = None; L.orc_vacc_wraps_reset.argtypes = []
    L.orc_build_cumfreqs.restype = None
    L.orc_build_cumfreqs.argtypes = [p, C.c_int, p, C.c_uint32, C.c_uint32, p]
    L.orc_model_check.restype = C.c_int; L.orc_model_check.argtypes = [C.POINTER(OrcModel)]
    L.orc_chunk_trace.restype = C.c_int
    L.orc_chunk_trace.argtypes = [C.POINTER(OrcModel), p, C.c_int, p, p]
    L.orc_compress_chunk.restype = C.c_int
    L.orc_compress_chunk.argtypes = [C.POINTER(OrcModel), p, C.c_int, C.POINTER(C.c_void_p), C.POINTER(C.c_size_t)]
    L.orc_compress_many.restype = C.c_int
    L.orc_compress_many.argtypes = [C.POINTER(OrcModel), p, C.c_int64, C.c_int, C.c_int, C.c_int, p,
                                    C.c_int64, p]
    L.orc_decompress_many.restype = C.c_int
    L.orc_decompress_many.argtypes = [C.POINTER(OrcModel), p, p, p, p, C.c_int, C.c_int, p, p]
    E, D = C.POINTER(OrcEncoder), C.POINTER(OrcDecoder)
    L.orc_enc_init.restype = None; L.orc_enc_init.argtypes = [E]
    L.orc_enc_free.restype = None; L.orc_enc_free.argtypes = [E]
    L.orc_enc_encode.restype = None; L.orc_enc_encode.argtypes = [E, p, C.c_int, C.c_int]
    L.orc_enc_encode_range.restype = None
    L.orc_enc_encode_range.argtypes = [E, C.c_uint64, C.c_uint64, C.c_uint64]
    L.orc_enc_finish.restype = None; L.orc_enc_finish.argtypes = [E]
    L.orc_dec_init.restype = None; L.orc_dec_init.argtypes = [D, p, C.c_size_t]
    L.orc_dec_decode.restype = C.c_int; L.orc_dec_decode.argtypes = [D, p, C.c_int]
    return L


def encode_symbols(cum: np.ndarray, syms) -> bytes:
    """Arithmetic-code `syms` under one fixed cumulative table (arith_coder.rs:80-130)."""
    L = lib()
    cum = np.ascontiguousarray(cum, dtype=np.uint32)
    e = OrcEncoder()
    L.orc_enc_init(C.byref(e))
    for s in syms:
        L.orc_enc_encode(C.byref(e), _ptr(cum), cum.size, int(s))
    L.orc_enc_finish(C.byref(e))
    data = C.string_at(e.out, e.len)
    L.orc_enc_free(C.byref(e))
    return data


def decode_symbols(data: bytes, cum: np.ndarray, n: int):
    L = lib()
    cum = np.ascontiguousarray(cum, dtype=np.uint32)
    buf = C.create_string_buffer(data, len(data) + 1)
    d = OrcDecoder()
    L.orc_dec_init(C.byref(d), C.cast(buf, C.c_void_p), len(data))
    return [L.orc_dec_decode(C.byref(d), _ptr(cum), cum.size) for _ in range(n)]


def attend_head(q_rot: np.ndarray, k: np.ndarray, v: np.ndarray, score_mult: int, lut: np.ndarray, sink=None):
    """One query head over keys 0..n-1 (attention.rs:197-285): returns
    (out int8 [64], final i32 vacc [64], final u64 S)."""
    L = lib()
    q_rot = np.ascontiguousarray(q_rot, dtype=np.int8)
    k = np.ascontiguousarray(k, dtype=np.int8)
    v = np.ascontiguousarray(v, dtype=np.int8)
    lut = np.ascontiguousarray(lut, dtype=np.uint16)
    assert q_rot.shape == (64,) and k.ndim == 2 and k.shape[1] == 64 and v.shape == k.shape
    sk = None if sink is None else np.ascontiguousarray(sink, dtype=np.int8)
    out = np.zeros(64, np.int8)
    vacc = np.zeros(64, np.int32)
    S = C.c_uint64(0)
    L.orc_attend_head(_ptr(q_rot), _ptr(k), _ptr(v), k.shape[0], int(score_mult),
                      None if sk is None else _ptr(sk), _ptr(lut), _ptr(out), _ptr(vacc), C.byref(S))
    return out, vacc, S.value


def vacc_wraps() -> int:
    """vacc additions that wrapped the i32 range since the last reset_vacc_wraps()."""
    return int(lib().orc_vacc_wraps())


def reset_vacc_wraps():
    lib().orc_vacc_wraps_reset()


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


class Model:
    """Weights + config of a .czm model, in the oracle's struct layout.

    Config parsing and defaults follow rust/src/model.rs:113-145; scalar
    defaults follow model.rs:157-168 (mult=1, shift=0); softmax constants fall
    back to the computed values (model.rs:336-337).
    """

    def __init__(self, tensors, meta, kv_mode: int = KV_RUST_COMPAT, lib_handle=None):
        self.L = lib_handle or lib()
        self.t = {k: np.ascontiguousarray(v) for k, v in tensors.items()}
        self.meta = meta

        def pu(key, default):
            try:
                return int(meta[key])
            except (KeyError, ValueError):
                return default

        if "context_length" in meta and meta["context_length"].isdigit():
            ctx = int(meta["context_length"])
        elif "context_length_log2" in meta and meta["context_length_log2"].isdigit():
            ctx = 1 << int(meta["context_length_log2"])
        else:
            ctx = pu("max_seq_len", 64)
        self.cfg = dict(vocab=pu("vocab_size", 1024), n_layers=pu("n_layers", 1), n_heads=pu("n_heads", 6),
                        n_kv_heads=pu("n_kv_heads", 1), d_model=pu("d_model", 384), d_ff=pu("d_ff", 1024),
                        head_dim=pu("head_dim", 64), max_seq_len=pu("max_seq_len", 64), context_length=ctx)
        self.kv_mode = kv_mode
        keep = []

        def arr(name, dtype):
            a = np.ascontiguousarray(self.t[name]).astype(dtype, copy=False).reshape(-1)
            keep.append(a)
            return _ptr(a)

        def scalar(name, dtype, default):
            if name in self.t:
                return int(np.asarray(self.t[name]).reshape(-1)[0].astype(dtype))
            return default

        nl = self.cfg["n_layers"]
        self._layers = (OrcLayer * nl)()
        for i in range(nl):
            pre = f"layers.{i}"
            ly = self._layers[i]
            ly.attn_norm = arr(f"{pre}.attn_norm.weight", np.int8)
            ly.post_attn_norm = arr(f"{pre}.post_attn_norm.weight", np.int8)
            ly.ffn_norm = arr(f"{pre}.ffn_norm.weight", np.int8)
            ly.post_ffn_norm = arr(f"{pre}.post_ffn_norm.weight", np.int8)
            ly.qkv_w = arr(f"{pre}.attn.qkv.weight", np.int8)
            ly.out_w = arr(f"{pre}.attn.out.weight", np.int8)
            ly.up_w = arr(f"{pre}.ffn.up.weight", np.int8)
            ly.down_w = arr(f"{pre}.ffn.down.weight", np.int8)
            ly.score_mult = arr(f"{pre}.attn.score_mult", np.int32)
            ly.sink_key = arr(f"{pre}.attn.sink_key", np.int8) if f"{pre}.attn.sink_key" in self.t else None
            ly.qkv_mult = scalar(f"{pre}.attn.qkv.mult", np.int32, 1)
            ly.out_mult = scalar(f"{pre}.attn.out.mult", np.int32, 1)
            ly.up_mult = scalar(f"{pre}.ffn.up.mult", np.int32, 1)
            ly.down_mult = scalar(f"{pre}.ffn.down.mult", np.int32, 1)
            ly.qkv_shift = scalar(f"{pre}.attn.qkv.shift", np.int8, 0)
            ly.out_shift = scalar(f"{pre}.attn.out.shift", np.int8, 0)
            ly.up_shift = scalar(f"{pre}.ffn.up.shift", np.int8, 0)
            ly.down_shift = scalar(f"{pre}.ffn.down.shift", np.int8, 0)
        m = OrcModel()
        for k, v in self.cfg.items():
            setattr(m, k, v)
        m.kv_mode = kv_mode
        m.embed = arr("embed.weight", np.int8)
        m.final_norm = arr("norm.weight", np.int8)
        m.head_w = arr("head.weight", np.int8)
        m.exp2_lut = arr("lut.exp2", np.uint16)
        m.rope_cos = arr("lut.rope_cos", np.int16)
        m.rope_sin = arr("lut.rope_sin", np.int16)
        m.coef_q24 = scalar("softmax.coef_q24", np.uint32, int(self.L.orc_cdf_coef_q24()))
        m.target_total = scalar("softmax.target_total", np.uint32, int(self.L.orc_target_total(self.cfg["vocab"])))
        m.layers = C.cast(self._layers, C.POINTER(OrcLayer))
        self.m = m
        self._keep = keep

    @classmethod
    def from_file(cls, path: str, kv_mode: int = KV_RUST_COMPAT, lib_handle=None):
        t, meta = read_czm(path)
        return cls(t, meta, kv_mode, lib_handle)

    @property
    def vocab(self) -> int:
        return self.cfg["vocab"]

    def check(self) -> int:
        return int(self.L.orc_model_check(C.byref(self.m)))

    def trace(self, inputs: np.ndarray, with_cum: bool = True):
        """Per-token logits [n, V] (and cumfreqs [n, V]) of one chunk whose
        forward inputs are `inputs` at positions 0..n-1."""
        inputs = np.ascontiguousarray(inputs, dtype=np.uint32)
        n = inputs.size
        lg = np.zeros((n, self.vocab), np.int32)
        cum = np.zeros((n, self.vocab), np.uint32) if with_cum else None
        rc = self.L.orc_chunk_trace(C.byref(self.m), _ptr(inputs), n, _ptr(lg), _ptr(cum) if with_cum else None)
        if rc:
            raise RuntimeError(f"oracle forward failed: {rc}")
        return (lg, cum) if with_cum else lg

    def compress_chunk(self, toks: np.ndarray) -> bytes:
        toks = np.ascontiguousarray(toks, dtype=np.uint32)
        out = C.c_void_p()
        n = C.c_size_t()
        rc = self.L.orc_compress_chunk(C.byref(self.m), _ptr(toks), toks.size, C.byref(out), C.byref(n))
        data = C.string_at(out, n.value) if n.value else b""
        C.CDLL(None).free(out)
        if rc:
            raise RuntimeError(f"oracle compress failed: {rc}")
        return data

    def compress_many(self, toks: np.ndarray, chunk: int, threads: int = 1, clone_weights: bool = True):
        """Returns list of per-chunk coded byte strings (main.rs:206-238)."""
        toks = np.ascontiguousarray(toks, dtype=np.uint32)
        nch = (toks.size + chunk - 1) // chunk
        slot = chunk * 4 + 64
        buf = np.zeros(nch * slot, np.uint8)
        lens = np.zeros(nch, np.int32)
        rc = self.L.orc_compress_many(C.byref(self.m), _ptr(toks), toks.size, chunk, threads,
                                      1 if clone_weights else 0, _ptr(buf), slot, _ptr(lens))
        if rc:
            raise RuntimeError(f"oracle compress failed: {rc}")
        return [bytes(buf[c * slot:c * slot + lens[c]]) for c in range(nch)]

    def decompress_many(self, chunks, ntoks, threads: int = 1) -> np.ndarray:
        lens = np.array([len(c) for c in chunks], np.int32)
        offs = np.zeros(len(chunks), np.int64)
        if len(chunks) > 1:
            offs[1:] = np.cumsum(lens[:-1])
        buf = np.frombuffer(b"".join(chunks) + b"\0", np.uint8).copy()
        ntoks = np.ascontiguousarray(ntoks, dtype=np.int32)
        toff = np.zeros(len(chunks), np.int64)
        if len(chunks) > 1:
            toff[1:] = np.cumsum(ntoks[:-1])
        out = np.zeros(int(ntoks.sum()), np.uint32)
        rc = self.L.orc_decompress_many(C.byref(self.m), _ptr(buf), _ptr(offs), _ptr(lens), _ptr(ntoks),
                                        len(chunks), threads, _ptr(out), _ptr(toff))
        if rc:
            raise RuntimeError(f"oracle decompress failed: {rc}")
        return out


def build_cumfreqs(logits: np.ndarray, lut: np.ndarray, coef: int, total: int) -> np.ndarray:
    logits = np.ascontiguousarray(logits, dtype=np.int32)
    lut = np.ascontiguousarray(lut, dtype=np.uint16)
    out = np.zeros(logits.size, np.uint32)
    lib().orc_build_cumfreqs(_ptr(logits), logits.size, _ptr(lut), coef, total, _ptr(out))
    return out


def payload(model_id_hash: int, tokenizer_id: int, ctx_log2: int, chunks, last_chunk_tokens: int) -> bytes:
    """Inner header || chunk bytes (file_format.rs:245-256, 324-330)."""
    hdr = struct.pack("<IIHBB", model_id_hash, len(chunks), last_chunk_tokens, tokenizer_id, ctx_log2)
    hdr += b"".join(struct.pack("<H", len(c)) for c in chunks)
    return hdr + b"".join(chunks)
