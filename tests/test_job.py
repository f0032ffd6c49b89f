"""The distributed job contract on the CPU (krunch/job.py semantics): byte
and chunk ranges partition the input, compress parts + finalize give one
blob (flags 0x01, the parts' codec), decompress parts + finalize give the
input back. The engine is a stand-in that frames reversed bytes; the real
engine runs in test_gpu_job.py."""
import struct

import pytest

from krunch_amd import chunking, job
from krunch_amd.inference import HEADER_SIZE, decode_header


class _Fake:
    model_id, tokenizer_id = 1, 0

    def compress_chunk(self, c):
        return self.compress_chunks_batched([c])[0]

    def compress_chunks_batched(self, cs):
        return [struct.pack(">II", len(c), len(c)) + bytes(reversed(c)) for c in cs]

    def decompress_chunk(self, e):
        return self.decompress_chunks_batched([e])[0]

    def decompress_chunks_batched(self, es):
        return [bytes(reversed(e[8:])) for e in es]


def _load(w8a8):
    return _Fake()


@pytest.mark.parametrize("total", [0, 1, 9_999, 10_000, 123_457])
@pytest.mark.parametrize("count", [1, 3, 8])
def test_ranges_partition(monkeypatch, total, count):
    monkeypatch.setenv("KRUNCH_CHUNK_SIZE", "10000")
    pos = 0
    for i in range(count):
        a, b = job.byte_range(i, count, total)
        assert a == pos and a <= b and (a % 10000 == 0 or a == total)
        pos = b
    assert pos == total
    for n in (0, 1, 5, 17):
        got = [job.chunk_range(i, count, n) for i in range(count)]
        assert got[0][0] == 0 and got[-1][1] == n
        assert all(got[i][1] == got[i + 1][0] for i in range(count - 1))


def test_parts_roundtrip(tmp_path, monkeypatch):
    monkeypatch.setenv("KRUNCH_CHUNK_SIZE", "10000")
    raw = bytes((i * 7 + (i >> 5)) & 0xFF for i in range(123_457))
    src, blob, back = tmp_path / "in.bin", tmp_path / "out" / "in.krunch", tmp_path / "back.bin"
    src.write_bytes(raw)
    base = {"KRUNCH_INPUT_URL": f"file://{src}", "KRUNCH_OUTPUT_URL": str(blob),
            "KRUNCH_PART_COUNT": "3", "KRUNCH_INPUT_LEN": str(len(raw))}
    for i in range(3):
        assert job.run({**base, "KRUNCH_MODE": "compress", "KRUNCH_PART_INDEX": str(i)}, _load) == 0
    assert job.run({**base, "KRUNCH_MODE": "finalize"}, _load) == 0
    master = blob.read_bytes()
    hdr = decode_header(master)
    assert hdr["flags"] == job.FLAG_NO_CRC and hdr["original_len"] == len(raw)
    # each part is split on its own (UTF-8-safe cuts can add a chunk per part)
    want = sum(len(chunking._split_utf8_safe(raw[a:b], 10000))
               for a, b in (job.byte_range(i, 3, len(raw)) for i in range(3)))
    assert hdr["n_chunks"] == want and (hdr["model_id"], hdr["tokenizer_id"]) == (1, 0)
    assert not (tmp_path / "out" / "in.krunch.parts").exists()
    # the master is an ordinary container: whole-blob decode gives the input
    ents = chunking.parse_entries(master[HEADER_SIZE:], hdr["n_chunks"])
    assert b"".join(bytes(reversed(e[8:]))[:ol] for ol, e in ents) == raw
    dbase = {"KRUNCH_INPUT_URL": str(blob), "KRUNCH_OUTPUT_URL": str(back), "KRUNCH_PART_COUNT": "4"}
    for i in range(4):
        assert job.run({**dbase, "KRUNCH_MODE": "decompress", "KRUNCH_PART_INDEX": str(i)}, _load) == 0
    assert job.run({**dbase, "KRUNCH_MODE": "finalize", "KRUNCH_FINALIZE_OF": "decompress"}, _load) == 0
    assert back.read_bytes() == raw


def test_contract_errors(tmp_path):
    assert job.run({}, _load) == 1                                   # no mode
    assert job.run({"KRUNCH_MODE": "compress"}, _load) == 1          # missing vars
    assert job.run({"KRUNCH_MODE": "compress", "KRUNCH_INPUT_URL": "s3://b/k",
                    "KRUNCH_OUTPUT_URL": str(tmp_path / "o"), "KRUNCH_PART_COUNT": "1",
                    "KRUNCH_PART_INDEX": "0", "KRUNCH_INPUT_LEN": "5"}, _load) == 1
    with pytest.raises(ValueError):
        job.byte_range(3, 3, 100)
