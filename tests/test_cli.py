"""CLI plumbing on the CPU (krunch/cli.py:1-158 semantics): stdin/stdout or
--in/--out files, the codec chosen from the blob's model_id, errors as exit
status 1. The engine is replaced by a stand-in that frames bytes; the real
engine runs in test_gpu_cli.py."""
import io
import sys

import pytest

from krunch_amd import cli
from krunch_amd.inference import MODEL_ID, MODEL_ID_W8A8, encode_header


class _Fake:
    def __init__(self, w8a8):
        self.mid = MODEL_ID_W8A8 if w8a8 else MODEL_ID

    def compress(self, raw):
        return encode_header(len(raw), 1, 0, model_id=self.mid) + raw

    def decompress(self, blob):
        return blob[37:]


def _loader(calls):
    def load(weights, tokenizer, w8a8):
        calls.append((weights, tokenizer, w8a8))
        return _Fake(w8a8)
    return load


def test_files_and_codec_selection(tmp_path, monkeypatch):
    monkeypatch.delenv("KRUNCH_WEIGHTS", raising=False)
    monkeypatch.setenv("KRUNCH_TOKENIZER", "/tok.json")
    src, mid, dst = tmp_path / "a.txt", tmp_path / "a.krunch", tmp_path / "b.txt"
    src.write_bytes(b"hello krunch")
    calls = []
    assert cli.main(["compress", "--in", str(src), "--out", str(mid), "--w8a8"], _loader(calls)) == 0
    assert cli.main(["decompress", "--in", str(mid), "--out", str(dst),
                     "--weights", "/m.pth"], _loader(calls)) == 0
    assert dst.read_bytes() == b"hello krunch"
    # compress: flag; decompress: model_id 2 read back from the blob
    assert calls == [(None, "/tok.json", True), ("/m.pth", "/tok.json", True)]


def test_stdin_stdout(monkeypatch, capsysbinary):
    monkeypatch.setattr(sys, "stdin", io.TextIOWrapper(io.BytesIO(b"xyz")))
    assert cli.main(["compress"], _loader([])) == 0
    out = capsysbinary.readouterr().out
    assert out[:4] == b"KRNC" and out.endswith(b"xyz")


def test_bad_blob_is_an_error(tmp_path):
    p = tmp_path / "junk"
    p.write_bytes(b"not a blob")
    assert cli.main(["decompress", "--in", str(p), "--out", str(tmp_path / "o")], _loader([])) == 1
    assert not (tmp_path / "o").exists()


def test_parser_requires_command():
    with pytest.raises(SystemExit):
        cli.build_parser().parse_args([])
