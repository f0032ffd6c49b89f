"""The CLI end to end on the GPU: file -> .krunch -> file with the synthetic
model and the byte tokenizer, fp16 and int8 codecs (the int8 one detected
from the blob on decompress)."""
import pytest

from krunch_amd import cli
from krunch_amd.inference import decode_header

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("w8a8", [False, True])
def test_cli_roundtrip(tmp_path, monkeypatch, w8a8):
    monkeypatch.delenv("KRUNCH_WEIGHTS", raising=False)
    monkeypatch.delenv("KRUNCH_TOKENIZER", raising=False)
    raw = ("krunch on MI355X, ünïcödé " * 30).encode("utf-8")
    src, mid, dst = tmp_path / "in", tmp_path / "in.krunch", tmp_path / "out"
    src.write_bytes(raw)
    args = ["compress", "--in", str(src), "--out", str(mid)] + (["--w8a8"] if w8a8 else [])
    print("cli compress, w8a8 =", w8a8, flush=True)
    assert cli.main(args) == 0
    assert decode_header(mid.read_bytes())["model_id"] == (2 if w8a8 else 1)
    print("cli decompress", flush=True)
    assert cli.main(["decompress", "--in", str(mid), "--out", str(dst)]) == 0
    assert dst.read_bytes() == raw
