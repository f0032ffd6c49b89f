"""Real-checkpoint loader (krunch_amd/weights.py): RWKV-4 checkpoint layout ->
engine layout. Pinned by construction: transposes and reshapes are exact, the
ln0 fold equals torch's layer_norm in fp32, rescale divides by 2^(i // 6),
and the inverse layout change round-trips bit for bit (also through a
weights_only .pth file and a safetensors file)."""
import numpy as np
import pytest
import torch

from krunch_amd import synthetic
from krunch_amd.weights import convert_rwkv4_state_dict, load_rwkv4, to_rwkv4_state_dict


def _ckpt(n_layer=2, C=256, F=512, V=300, seed=5):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g) * 0.1
    sd = {"emb.weight": r(V, C), "blocks.0.ln0.weight": 1 + r(C), "blocks.0.ln0.bias": r(C),
          "ln_out.weight": 1 + r(C), "ln_out.bias": r(C), "head.weight": r(V, C)}
    for i in range(n_layer):
        b, a, f = f"blocks.{i}.", f"blocks.{i}.att.", f"blocks.{i}.ffn."
        for ln in ("ln1", "ln2"):
            sd[b + ln + ".weight"], sd[b + ln + ".bias"] = 1 + r(C), r(C)
        for n in ("time_mix_k", "time_mix_v", "time_mix_r"):
            sd[a + n] = torch.rand(1, 1, C, generator=g)
        for n in ("time_mix_k", "time_mix_r"):
            sd[f + n] = torch.rand(1, 1, C, generator=g)
        sd[a + "time_decay"] = torch.linspace(-5, 3, C)
        sd[a + "time_first"] = r(C)
        for n in ("key", "value", "receptance", "output"):
            sd[a + n + ".weight"] = r(C, C)
        sd[f + "key.weight"], sd[f + "value.weight"] = r(F, C), r(C, F)
        sd[f + "receptance.weight"] = r(C, C)
    return sd


def test_layout_and_ln0_fold():
    sd = _ckpt()
    w = convert_rwkv4_state_dict(sd)
    emb = torch.nn.functional.layer_norm(sd["emb.weight"], (256,), sd["blocks.0.ln0.weight"],
                                         sd["blocks.0.ln0.bias"], eps=1e-5)
    assert torch.equal(w["emb.weight"], emb.half())
    assert "blocks.0.ln0.weight" not in w
    assert torch.equal(w["blocks.1.att.key.weight"], sd["blocks.1.att.key.weight"].t().half())
    assert w["blocks.0.ffn.key.weight"].shape == (256, 512)     # [in, out]
    assert w["blocks.0.ffn.value.weight"].shape == (512, 256)
    assert w["head.weight"].shape == (256, 300)
    assert w["blocks.0.att.time_mix_k"].shape == (256,)
    assert w["blocks.0.att.time_decay"].dtype == torch.float32
    assert torch.equal(w["blocks.0.att.time_decay"], sd["blocks.0.att.time_decay"])   # raw


def test_rescale():
    sd = _ckpt(n_layer=8)
    w0, w1 = convert_rwkv4_state_dict(sd), convert_rwkv4_state_dict(sd, rescale=True)
    for i in (0, 5, 6, 7):
        s = 2 ** (i // 6)
        for m in ("att.output.weight", "ffn.value.weight"):
            k = f"blocks.{i}.{m}"
            assert torch.equal(w1[k], (sd[k].t() / s).half())
        assert torch.equal(w1[f"blocks.{i}.att.key.weight"], w0[f"blocks.{i}.att.key.weight"])


def test_round_trip_through_files(tmp_path):
    w = synthetic.make_weights(n_layer=2, C=256, F=512, V=400)
    sd = to_rwkv4_state_dict(w)
    torch.save(sd, tmp_path / "m.pth")
    from safetensors.torch import save_file
    save_file(sd, str(tmp_path / "m.safetensors"))
    for name in ("m.pth", "m.safetensors"):
        back = load_rwkv4(str(tmp_path / name))
        assert set(back) == set(w)
        for k in w:
            assert back[k].dtype == w[k].dtype and torch.equal(back[k], w[k]), k


def test_rejects_bad_checkpoints():
    sd = _ckpt()
    del sd["head.weight"]
    with pytest.raises(ValueError):
        convert_rwkv4_state_dict(sd)
    sd = _ckpt()
    sd["blocks.3.ln1.weight"] = sd["blocks.0.ln1.weight"]
    with pytest.raises(ValueError):
        convert_rwkv4_state_dict(sd)
