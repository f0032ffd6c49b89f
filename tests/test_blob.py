"""Blob format (krunch/inference.py:47-83; tests/test_blob.py:24-36 of the reference)."""
import struct

import pytest

from krunch_amd.inference import (BLOB_MAGIC, HEADER_FMT, HEADER_SIZE, decode_header,
                                  encode_header)


def test_header_roundtrip():
    h = encode_header(original_len=123456, n_chunks=7, crc32=0xDEADBEEF)
    assert len(h) == HEADER_SIZE == struct.calcsize(">4sBIIIHHQII") == 37
    d = decode_header(h)
    assert d["original_len"] == 123456 and d["n_chunks"] == 7 and d["crc32"] == 0xDEADBEEF
    assert d["blob_version"] == 1 and d["model_id"] == 1 and d["tokenizer_id"] == 1


def test_header_errors():
    with pytest.raises(ValueError):
        decode_header(b"KRNC")
    bad = b"XXXX" + encode_header(1, 1, 0)[4:]
    with pytest.raises(ValueError):
        decode_header(bad)
    assert HEADER_FMT == ">4sBIIIHHQII" and BLOB_MAGIC == b"KRNC"
