"""The .krunch container end to end on the GPU: bytes -> blob -> bytes with
the byte tokenizer, several chunks decoded in lockstep, codec/CRC/length
checks."""
import struct

import pytest

from krunch_amd import synthetic
from krunch_amd.inference import HEADER_SIZE, InferenceEngine, decode_header, encode_header

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def engines():
    w = synthetic.make_weights()
    return InferenceEngine().load(w), InferenceEngine().load(w, w8a8=True)


def test_container_roundtrip(engines):
    e16, e8 = engines
    raw = ("Grüße aus der Pfalz! 世界 " * 40).encode("utf-8") + bytes(range(256))
    for eng, mid in ((e16, 1), (e8, 2)):
        blob = eng.compress(raw, chunk_size=700)
        hdr = decode_header(blob)
        assert hdr["model_id"] == mid and hdr["tokenizer_id"] == 0
        assert hdr["n_chunks"] == 3 and hdr["original_len"] == len(raw)
        assert eng.decompress(blob) == raw
    assert e16.decompress(e16.compress(b"")) == b""
    assert e16.decompress(e16.compress(b"z")) == b"z"


def test_container_checks(engines):
    e16, e8 = engines
    raw = b"checksummed payload " * 30
    blob = e16.compress(raw, chunk_size=256)
    with pytest.raises(ValueError, match="model_id"):
        e8.decompress(blob)
    bad_crc = blob[:HEADER_SIZE - 4] + struct.pack(">I", (decode_header(blob)["crc32"] ^ 1)) + blob[HEADER_SIZE:]
    with pytest.raises(ValueError, match="CRC32"):
        e16.decompress(bad_crc)
    h = decode_header(blob)
    no_crc = encode_header(h["original_len"], h["n_chunks"], 0, flags=0x01, model_id=1,
                           tokenizer_id=0) + blob[HEADER_SIZE:]      # assembled-from-parts blob
    assert e16.decompress(no_crc) == raw
    short = encode_header(h["original_len"] + 1, h["n_chunks"], h["crc32"], model_id=1,
                          tokenizer_id=0) + blob[HEADER_SIZE:]
    with pytest.raises(ValueError, match="length"):
        e16.decompress(short)
