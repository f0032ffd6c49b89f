"""The job contract end to end on the GPU: two compress workers + finalize
give a master blob that the engine decompresses whole and that three
decompress workers + finalize turn back into the input (synthetic model,
byte tokenizer)."""
import pytest

from krunch_amd import job, synthetic
from krunch_amd.inference import InferenceEngine

pytestmark = pytest.mark.gpu


def test_job_roundtrip(tmp_path, monkeypatch):
    monkeypatch.setenv("KRUNCH_CHUNK_SIZE", "700")
    eng = InferenceEngine().load(synthetic.make_weights())
    load = lambda w8a8: eng       # noqa: E731  (one loaded fp16 engine for every worker)
    raw = ("distributed krunch on MI355X; ünïcödé bytes too. " * 60).encode("utf-8")
    src, blob, back = tmp_path / "in", tmp_path / "in.krunch", tmp_path / "back"
    src.write_bytes(raw)
    base = {"KRUNCH_INPUT_URL": str(src), "KRUNCH_OUTPUT_URL": str(blob),
            "KRUNCH_PART_COUNT": "2", "KRUNCH_INPUT_LEN": str(len(raw))}
    for i in range(2):
        print("compress part", i, flush=True)
        assert job.run({**base, "KRUNCH_MODE": "compress", "KRUNCH_PART_INDEX": str(i)}, load) == 0
    assert job.run({**base, "KRUNCH_MODE": "finalize"}, load) == 0
    master = blob.read_bytes()
    assert eng.decompress(master) == raw
    dbase = {"KRUNCH_INPUT_URL": str(blob), "KRUNCH_OUTPUT_URL": str(back), "KRUNCH_PART_COUNT": "3"}
    for i in range(3):
        print("decompress part", i, flush=True)
        assert job.run({**dbase, "KRUNCH_MODE": "decompress", "KRUNCH_PART_INDEX": str(i)}, load) == 0
    assert job.run({**dbase, "KRUNCH_MODE": "finalize", "KRUNCH_FINALIZE_OF": "decompress"}, load) == 0
    assert back.read_bytes() == raw
