"""Tokenizer oracle (test infrastructure only).

Restates the reference tokenizer path of the text configurations:
  * decompress the model's embedded tokenizer JSON (main.rs:88-109);
  * token_str_to_bytes (tiktoken.rs:517-525);
  * encode_with_special_tokens (tiktoken.rs:215-269, 498-501): split on the
    special tokens, pre-split each span with the model's `pat_str` (executed
    here by the `regex` module, an engine independent of the product's
    hand-written scanner), BPE each piece (_byte_pair_merge,
    tiktoken.rs:26-107);
  * decode_bytes (tiktoken.rs:186-198).
"""
from __future__ import annotations

import ctypes as C
import json

import regex


def decompress_zstd(data: bytes) -> bytes:
    z = C.CDLL("libzstd.so.1")
    z.ZSTD_getFrameContentSize.restype = C.c_ulonglong
    z.ZSTD_getFrameContentSize.argtypes = [C.c_char_p, C.c_size_t]
    z.ZSTD_decompress.restype = C.c_size_t
    z.ZSTD_decompress.argtypes = [C.c_void_p, C.c_size_t, C.c_char_p, C.c_size_t]
    n = z.ZSTD_getFrameContentSize(data, len(data))
    out = C.create_string_buffer(n)
    r = z.ZSTD_decompress(out, n, data, len(data))
    return out.raw[:r]


class Tokenizer:
    def __init__(self, spec: dict):
        self.pat = regex.compile(spec["pat_str"])
        self.enc = {}
        for k, v in spec["mergeable_ranks"].items():
            b = bytes(ord(ch) for ch in k)  # each char is one byte (tiktoken.rs:517-525)
            self.enc[b] = v
        self.dec = {v: k for k, v in self.enc.items()}
        self.specials = dict(spec["special_tokens"])
        for k, v in self.specials.items():
            self.dec[v] = k.encode()
        self.special_re = regex.compile("|".join(regex.escape(s) for s in self.specials))

    @classmethod
    def from_model(cls, tensors, meta):
        data = bytes(tensors["tokenizer.data"].reshape(-1))
        assert meta.get("tokenizer_codec", "zstd") == "zstd"
        return cls(json.loads(decompress_zstd(data)))

    def _merge(self, piece: bytes):
        # _byte_pair_merge (tiktoken.rs:26-82)
        MAXR = 2 ** 32 - 1
        parts = []
        min_rank = (MAXR, -1)
        for i in range(len(piece) - 1):
            r = self.enc.get(piece[i:i + 2], MAXR)
            if r < min_rank[0]:
                min_rank = (r, i)
            parts.append([i, r])
        parts.append([len(piece) - 1, MAXR])
        parts.append([len(piece), MAXR])

        def get_rank(i):
            if i + 3 < len(parts):
                return self.enc.get(piece[parts[i][0]:parts[i + 3][0]], MAXR)
            return MAXR

        while min_rank[0] != MAXR:
            i = min_rank[1]
            if i > 0:
                parts[i - 1][1] = get_rank(i - 1)
            parts[i][1] = get_rank(i)
            del parts[i + 1]
            min_rank = (MAXR, -1)
            for k in range(len(parts) - 1):
                if parts[k][1] < min_rank[0]:
                    min_rank = (parts[k][1], k)
        return parts

    def byte_pair_encode(self, piece: bytes):
        if len(piece) == 1:
            return [self.enc[piece]]
        parts = self._merge(piece)
        return [self.enc[piece[a[0]:b[0]]] for a, b in zip(parts, parts[1:])]

    def encode(self, text: str):
        out = []
        cache = {}
        start = 0
        while True:
            m = self.special_re.search(text, start) if self.specials else None
            end = m.start() if m else len(text)
            for mm in self.pat.finditer(text[start:end]):
                piece = mm.group().encode("utf-8")
                if piece in self.enc:
                    out.append(self.enc[piece])
                    continue
                if piece not in cache:
                    cache[piece] = self.byte_pair_encode(piece)
                out.extend(cache[piece])
            if not m:
                break
            out.append(self.specials[m.group()])
            start = m.end()
        return out

    def pieces(self, text: str):
        return [m.group() for m in self.pat.finditer(text)]

    def decode_bytes(self, tokens) -> bytes:
        return b"".join(self.dec[t] for t in tokens)
