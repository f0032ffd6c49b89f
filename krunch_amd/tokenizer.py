"""Tokenizers for the byte-level API.

`load_tokenizer(path)` wraps a `tokenizers` JSON (the reference uses
20B_tokenizer.json, inference.py:171-197, absent here). `ByteTokenizer` maps
each byte to the token id of the same value, which keeps the byte-level API
and the `.krunch` container usable and lossless for any input without the
real tokenizer (ids 0..255 of the 50277-entry vocabulary).
"""
from __future__ import annotations

import numpy as np


class ByteTokenizer:
    tokenizer_id = 0

    def encode_bytes(self, data: bytes) -> np.ndarray:
        return np.frombuffer(bytes(data), dtype=np.uint8).astype(np.int32)

    def decode_bytes(self, ids) -> bytes:
        a = np.asarray(ids, dtype=np.int64)
        if a.size and (a.min() < 0 or a.max() > 255):
            raise ValueError("byte tokenizer: id outside 0..255")
        return a.astype(np.uint8).tobytes()


class JsonTokenizer:
    """A `tokenizers` JSON tokenizer; text is UTF-8 (errors replaced, as the
    reference's compress_chunk does, inference.py:203-230)."""
    tokenizer_id = 1

    def __init__(self, path: str):
        from tokenizers import Tokenizer
        self._tok = Tokenizer.from_file(str(path))

    def encode_bytes(self, data: bytes) -> np.ndarray:
        return np.array(self._tok.encode(bytes(data).decode("utf-8", errors="replace")).ids,
                        dtype=np.int32)

    def decode_bytes(self, ids) -> bytes:
        return self._tok.decode([int(i) for i in ids]).encode("utf-8")


def load_tokenizer(path=None):
    return JsonTokenizer(path) if path else ByteTokenizer()
