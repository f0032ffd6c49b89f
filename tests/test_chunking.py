"""Chunking and container framing (krunch/chunking.py semantics), host only."""
import struct

import pytest

from krunch_amd import chunking


def test_chunk_size_policy(monkeypatch):
    monkeypatch.delenv("KRUNCH_CHUNK_SIZE", raising=False)
    monkeypatch.delenv("KRUNCH_TARGET_B", raising=False)
    assert chunking.compute_chunk_size(0) == 64 * 1024
    assert chunking.compute_chunk_size(1000) == 64 * 1024           # floor
    big = 512 * 1024 * 1024
    assert chunking.compute_chunk_size(big) == -(-big // 512)        # 4 x 128 chunks
    monkeypatch.setenv("KRUNCH_TARGET_B", "8")
    assert chunking.compute_chunk_size(big) == -(-big // 32)
    monkeypatch.setenv("KRUNCH_CHUNK_SIZE", "1234")
    assert chunking.compute_chunk_size(big) == 1234


def test_utf8_safe_split():
    text = ("Grüße, 世界! 🙂 " * 300).encode("utf-8")
    for size in (7, 64, 100, 1000):
        parts = chunking._split_utf8_safe(text, size)
        assert b"".join(parts) == text
        for p in parts[:-1]:
            assert size - 3 <= len(p) <= size
            p.decode("utf-8")                                      # never cuts a code point
    # a run of continuation bytes longer than the chunk cannot loop forever
    weird = b"\x80" * 50 + b"abc"
    parts = chunking._split_utf8_safe(weird, 8)
    assert b"".join(parts) == weird and all(parts)


def test_entries_roundtrip_with_mock_codec():
    raw = bytes(range(256)) * 40
    enc = lambda c: c[::-1]
    entries, n = chunking.compress_all(raw, enc, chunk_size=1000)
    assert n == len(entries) == 11
    ol, cl = struct.unpack(">II", entries[0][:8])
    assert ol == 1000 and cl == 1000
    blob = b"".join(entries)
    dec = lambda z: z[::-1] + b"padding"                           # trimmed to orig_len
    assert chunking.decompress_all(blob, n, dec) == raw
    batched = lambda zs: [dec(z) for z in zs]
    assert chunking.decompress_all(blob, n, dec, neural_batch_fn=batched) == raw
    entries2, _ = chunking.compress_all(raw, enc, neural_batch_fn=lambda cs: [enc(c) for c in cs],
                                        chunk_size=1000)
    assert entries2 == entries


def test_truncated_blob():
    entries, n = chunking.compress_all(b"x" * 100, lambda c: c, chunk_size=40)
    blob = b"".join(entries)
    with pytest.raises(ValueError):
        chunking.parse_entries(blob[:-1], n)
    with pytest.raises(ValueError):
        chunking.parse_entries(blob, n + 1)


def test_stream_batch_sizing(monkeypatch):
    from krunch_amd import inference as inf
    monkeypatch.delenv("KRUNCH_DECOMPRESS_BATCH", raising=False)
    monkeypatch.delenv("KRUNCH_COMPRESS_BATCH", raising=False)
    assert inf.compute_decompress_batch() == inf.DEFAULT_STREAM_BATCH == 512
    assert inf.compute_decompress_batch(7) == 7
    assert inf.compute_compress_batch(5000) == 512
    monkeypatch.setenv("KRUNCH_DECOMPRESS_BATCH", "3")
    assert inf.compute_decompress_batch(10) == 3 and inf.compute_decompress_batch(2) == 2
    monkeypatch.setenv("KRUNCH_DECOMPRESS_BATCH", "junk")
    assert inf.compute_decompress_batch(1000) == 512
    monkeypatch.setenv("KRUNCH_COMPRESS_BATCH", "0")
    assert inf.compute_compress_batch(9) == 1


def test_coder_call_split_sizing():
    """Calls are split so the concatenated bitstreams of one call fit the
    int32 stream offsets / uint32 length of the C ABI."""
    from krunch_amd import _lib
    from krunch_amd import inference as inf
    assert inf.MAX_CALL_BYTES == 2 ** 31 - 1
    assert inf.coder_stream_cap(1024) == 4 * 1024 + 64
    parts = inf.split_by_bytes([5, 5, 5, 5, 5], 10)
    assert [list(r) for r in parts] == [[0, 1], [2, 3], [4]]
    assert [list(r) for r in inf.split_by_bytes([3, 9, 1, 1], 10)] == [[0], [1, 2], [3]]
    assert inf.split_by_bytes([], 10) == []
    with pytest.raises(ValueError):
        inf.split_by_bytes([11], 10)
    # 512 streams of 262,144 tokens: 537 MB per call, far under the limit; a
    # 1 GB-per-stream call is split
    per = inf.coder_stream_cap(262144)
    assert 512 * per < inf.MAX_CALL_BYTES
    assert inf.MAX_CALL_BYTES // inf.coder_stream_cap(2 ** 28) == 1
    assert _lib.u32(2 ** 32 - 1) == 2 ** 32 - 1
    for bad in (2 ** 32, 2 ** 32 + 5, -1):
        with pytest.raises(ValueError):
            _lib.u32(bad)
