"""Input chunking and chunk-entry framing, the reference's
`krunch/chunking.py` (:42-196) with the same names and semantics:

* `compute_chunk_size(total)`: about 4 x target_B chunks per input (at least
  16), never below 64 KiB; `KRUNCH_CHUNK_SIZE` pins it, `KRUNCH_TARGET_B`
  sets target_B (default 128) (chunking.py:42-66).
* `_split_utf8_safe(raw, size)`: chunks of ~size bytes whose boundaries are
  moved back off UTF-8 continuation bytes (0x80-0xBF), so no code point is
  cut (chunking.py:114-137).
* `compress_all(raw, neural_fn, neural_batch_fn=None, chunk_size=None,
  total_size=None) -> (entries, n_chunks)`: one entry per chunk,
  `>II`(orig_len, comp_len) + payload (chunking.py:88-111, :140-147).
* `decompress_all(entries_bytes, n_chunks, neural_fn, neural_batch_fn=None)`:
  parses the entries, decodes (batched when a batch function is given), and
  trims each chunk to its orig_len (chunking.py:150-196).

On this build the batch functions are `InferenceEngine.compress_chunks_batched`
/ `decompress_chunks_batched`, which run all chunks through one batched
packed forward / one lockstep HIP-graph decode.
"""
from __future__ import annotations

import os
import struct
from typing import Callable, List, Optional, Sequence, Tuple

_CHUNK_SIZE_FLOOR = 64 * 1024
_DEFAULT_TARGET_B = 128
CHUNK_SIZE = int(os.environ.get("KRUNCH_CHUNK_SIZE", _CHUNK_SIZE_FLOOR))


def compute_chunk_size(total_size: int) -> int:
    explicit = os.environ.get("KRUNCH_CHUNK_SIZE")
    if explicit is not None:
        return int(explicit)
    if total_size <= 0:
        return _CHUNK_SIZE_FLOOR
    target_b = int(os.environ.get("KRUNCH_TARGET_B", _DEFAULT_TARGET_B))
    target_chunks = max(target_b * 4, 16)
    natural = (total_size + target_chunks - 1) // target_chunks
    return max(_CHUNK_SIZE_FLOOR, natural)


def _split_utf8_safe(raw: bytes, target_size: int) -> List[bytes]:
    if target_size < 1:
        raise ValueError("chunk size must be positive")
    chunks, pos, n = [], 0, len(raw)
    while pos < n:
        end = min(pos + target_size, n)
        if end < n:
            back = end
            while back > pos and 0x80 <= raw[back] < 0xC0:
                back -= 1
            # a run of continuation bytes longer than the chunk: cut at the size
            end = back if back > pos else end
        chunks.append(raw[pos:end])
        pos = end
    return chunks


def _entry(chunk: bytes, compressed: bytes) -> bytes:
    return struct.pack(">II", len(chunk), len(compressed)) + compressed


def compress_all(raw: bytes, neural_fn: Callable[[bytes], bytes],
                 neural_batch_fn: Optional[Callable[[list], list]] = None,
                 chunk_size: Optional[int] = None,
                 total_size: Optional[int] = None) -> Tuple[List[bytes], int]:
    if chunk_size is None:
        chunk_size = compute_chunk_size(total_size if total_size is not None else len(raw))
    chunks = _split_utf8_safe(raw, chunk_size)
    if neural_batch_fn is not None and len(chunks) > 1:
        compressed = neural_batch_fn(chunks)
        entries = [_entry(c, z) for c, z in zip(chunks, compressed)]
    else:
        entries = [_entry(c, neural_fn(c)) for c in chunks]
    return entries, len(entries)


def parse_entries(entries_bytes: bytes, n_chunks: int) -> List[Tuple[int, bytes]]:
    """(orig_len, encoded) per entry; raises ValueError on a truncated blob."""
    out, pos = [], 0
    for i in range(n_chunks):
        if pos + 8 > len(entries_bytes):
            raise ValueError(f"truncated blob: entry {i} header past the end")
        orig_len, comp_len = struct.unpack(">II", entries_bytes[pos:pos + 8])
        pos += 8
        if pos + comp_len > len(entries_bytes):
            raise ValueError(f"truncated blob: entry {i} payload past the end")
        out.append((orig_len, entries_bytes[pos:pos + comp_len]))
        pos += comp_len
    return out


def decompress_all(entries_bytes: bytes, n_chunks: int, neural_fn: Callable[[bytes], bytes],
                   neural_batch_fn: Optional[Callable[[list], list]] = None) -> bytes:
    chunks = parse_entries(entries_bytes, n_chunks)
    if neural_batch_fn is not None and len(chunks) > 1:
        decoded = neural_batch_fn([enc for _, enc in chunks])
        return b"".join(d[:ol] for (ol, _), d in zip(chunks, decoded))
    return b"".join(neural_fn(enc)[:ol] for ol, enc in chunks)
