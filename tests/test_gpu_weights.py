"""A real-checkpoint-format file through the engine: a weights_only .pth in
the RWKV-4 layout (the synthetic weights written by to_rwkv4_state_dict)
loads, compresses and decompresses byte-exact, and gives the same stream
as the in-memory weights."""
import pytest
import torch

from krunch_amd import inference, synthetic
from krunch_amd.weights import to_rwkv4_state_dict

pytestmark = pytest.mark.gpu


def test_pth_checkpoint_roundtrip(tmp_path):
    w = synthetic.make_weights(n_layer=2)
    torch.save(to_rwkv4_state_dict(w), tmp_path / "rwkv4.pth")
    data = b"RWKV-4 checkpoint through the MI355X engine. " * 20
    a = inference.InferenceEngine().load(str(tmp_path / "rwkv4.pth"))
    b = inference.InferenceEngine().load(w)
    blob = a.compress(data)
    assert blob == b.compress(data)
    assert a.decompress(blob) == data
