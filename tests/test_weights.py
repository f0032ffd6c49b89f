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
    w0, w1 = convert_rwkv4_state_dict(sd, rescale=False), convert_rwkv4_state_dict(sd, rescale=True)
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


def test_default_is_the_reference_codecs_weights(tmp_path):
    """The default conversion is the rescaled one (what the reference's codec
    reads from the rwkv package's 'cuda fp16' model.w), also through a file."""
    sd = _ckpt(n_layer=8)
    w = convert_rwkv4_state_dict(sd)
    wr = convert_rwkv4_state_dict(sd, rescale=True)
    assert all(torch.equal(w[k], wr[k]) for k in w)
    assert torch.equal(w["blocks.7.att.output.weight"], (sd["blocks.7.att.output.weight"].t() / 2).half())
    torch.save(sd, tmp_path / "m.pth")
    back = load_rwkv4(str(tmp_path / "m.pth"))
    assert all(torch.equal(back[k], wr[k]) for k in w)


def _forward(w, ids, halve_every=0):
    """oracle.rwkv4's forward, optionally halving x after every
    `halve_every`-th layer (the rwkv package's own fp16 forward)."""
    from oracle import rwkv4
    n_layer = 1 + max(int(k.split(".")[1]) for k in w if k.startswith("blocks."))
    C = w["emb.weight"].shape[1]
    state = rwkv4.new_state(n_layer, ids.shape[0], C)
    f = {k: v.float() for k, v in w.items()}
    x = f["emb.weight"][ids]
    with torch.no_grad():
        for i, st in enumerate(state):
            x = rwkv4.time_mix(x, st, f, i, False)
            x = rwkv4.channel_mix(x, st, f, i, False)
            if halve_every and (i + 1) % halve_every == 0:
                x = x / 2
        x = torch.nn.functional.layer_norm(x, (C,), f["ln_out.weight"], f["ln_out.bias"], 1e-5)
        return (x @ f["head.weight"]).numpy()


def test_rescale_convention_and_what_it_changes():
    """What pins the rescale rule (2^(i // 6) on att.output / ffn.value):
    the rwkv package's own forward, which halves x after every sixth layer,
    computes on rescaled weights what the unscaled weights compute without
    halving (LayerNorm ignores the scale of its input up to eps). A rule off
    by one layer breaks that. The reference codec's function (rescaled
    weights, x never halved; the engine's default) is a different model in
    layers 6 and up."""
    sd = _ckpt(n_layer=12, C=256, F=512, V=300, seed=9)
    plain = convert_rwkv4_state_dict(sd, rescale=False)
    scaled = convert_rwkv4_state_dict(sd, rescale=True)
    ids = torch.as_tensor(np.random.default_rng(3).integers(0, 300, (2, 12)))
    ref = _forward(plain, ids)
    assert np.abs(_forward(scaled, ids, halve_every=6) - ref).max() < 1e-3
    wrong = convert_rwkv4_state_dict(sd, rescale=True, rescale_layer=5)
    assert np.abs(_forward(wrong, ids, halve_every=6) - ref).max() > 1e-2
    assert np.abs(_forward(scaled, ids) - ref).max() > 1e-2
