"""Real-checkpoint loader: an RWKV-4 `.pth` / `.safetensors` state dict ->
the weight dict the engine prepares (`model.prepare`, `cpp_path.init_weights`).

The reference loads the checkpoint through the rwkv package (`rwkv==0.8.26`,
`RWKV(model=..., strategy='cuda fp16')`, krunch/inference.py:171-197) and hands
`model.w` to `cpp_path.init_weights` (cpp_path.py:26-106). That package is not
vendored with the reference and is not installed here. This module restates
the load-time transforms of the RWKV-4 checkpoint format that the engine's
layout needs:

* the 4 attention matrices, the 3 channel-mix matrices and the head are
  stored as torch Linear weights [out, in]; the engine takes them as
  [in, out] (`x @ W`), so they are transposed;
* `blocks.0.ln0` (a LayerNorm applied to the embedding only) is folded into
  `emb.weight` once, in fp32: emb' = LayerNorm(emb; ln0.weight, ln0.bias,
  eps 1e-5), and the ln0 tensors are dropped;
* `time_mix_*` ([1, 1, C]) are flattened to [C];
* `time_decay` stays raw (the engine computes w = -exp(time_decay) itself,
  `kr_prepare_decay`) and `time_first` is used as is (RWKV-4: u = time_first);
* matrices, embedding, LayerNorm and mix vectors become fp16; time_decay and
  time_first stay fp32.

RESCALE: for fp16 strategies ('cuda fp16', the one inference.py:186 picks on
a GPU) the rwkv package divides `att.output.weight` and `ffn.value.weight`
of layer i by 2^(i // 6) at load time, and its own forward halves x after
every sixth layer, so that the package computes the unscaled model. The
reference's codec takes those rescaled weights (`model.w`,
cpp_path.py:26-91) into a layer path that never halves x
(cpp_path.py:131-163, layer_cpp.cpp:456-637): on a real checkpoint the
reference compresses with "rescaled weights, x never halved", which differs
from the unscaled model in layers 6 and up. The default here is therefore
`rescale=True`, so that the engine computes the reference codec's function
on the same checkpoint (its bits/token and bitstreams are the reference's,
up to rounding); `rescale=False` gives the unscaled model, which no
reference stream was coded with.

Checkpoints are read with `torch.load(..., weights_only=True)` or
safetensors, which execute nothing from the file.
"""
from __future__ import annotations

import os
import re
from typing import Dict, Mapping

import torch

_MATRICES = ("att.key.weight", "att.value.weight", "att.receptance.weight",
             "att.output.weight", "ffn.key.weight", "ffn.value.weight",
             "ffn.receptance.weight")


def _n_layer(sd: Mapping[str, torch.Tensor]) -> int:
    ids = {int(m.group(1)) for k in sd for m in [re.match(r"blocks\.(\d+)\.", k)] if m}
    if not ids:
        raise ValueError("checkpoint has no blocks.* tensors")
    n = max(ids) + 1
    if ids != set(range(n)):
        raise ValueError(f"checkpoint layer ids are not contiguous: {sorted(ids)}")
    return n


def convert_rwkv4_state_dict(sd: Mapping[str, torch.Tensor], rescale: bool = True,
                             rescale_layer: int = 6) -> Dict[str, torch.Tensor]:
    """RWKV-4 checkpoint tensors -> the engine's weight dict (CPU tensors)."""
    sd = {k: (v if isinstance(v, torch.Tensor) else torch.as_tensor(v)) for k, v in sd.items()}
    need = ["emb.weight", "ln_out.weight", "ln_out.bias", "head.weight"]
    for k in need:
        if k not in sd:
            raise ValueError(f"checkpoint is missing {k}")
    n_layer = _n_layer(sd)
    V, C = sd["emb.weight"].shape
    out: Dict[str, torch.Tensor] = {}
    emb = sd["emb.weight"].float()
    if "blocks.0.ln0.weight" in sd:
        emb = torch.nn.functional.layer_norm(emb, (C,), sd["blocks.0.ln0.weight"].float(),
                                             sd["blocks.0.ln0.bias"].float(), eps=1e-5)
    out["emb.weight"] = emb.to(torch.float16).contiguous()
    for i in range(n_layer):
        b, a, f = f"blocks.{i}.", f"blocks.{i}.att.", f"blocks.{i}.ffn."
        for ln in ("ln1", "ln2"):
            for p in ("weight", "bias"):
                out[f"{b}{ln}.{p}"] = sd[f"{b}{ln}.{p}"].to(torch.float16).reshape(-1).contiguous()
        for name in ("time_mix_k", "time_mix_v", "time_mix_r"):
            out[a + name] = sd[a + name].to(torch.float16).reshape(-1).contiguous()
        for name in ("time_mix_k", "time_mix_r"):
            out[f + name] = sd[f + name].to(torch.float16).reshape(-1).contiguous()
        out[a + "time_decay"] = sd[a + "time_decay"].float().reshape(-1).contiguous()
        out[a + "time_first"] = sd[a + "time_first"].float().reshape(-1).contiguous()
        for m in _MATRICES:
            t = sd[b + m].float()
            if rescale and rescale_layer > 0 and m in ("att.output.weight", "ffn.value.weight"):
                t = t / (2 ** (i // rescale_layer))
            out[b + m] = t.t().to(torch.float16).contiguous()          # [in, out]
    out["ln_out.weight"] = sd["ln_out.weight"].to(torch.float16).reshape(-1).contiguous()
    out["ln_out.bias"] = sd["ln_out.bias"].to(torch.float16).reshape(-1).contiguous()
    out["head.weight"] = sd["head.weight"].float().t().to(torch.float16).contiguous()   # [C, V]
    F = out["blocks.0.ffn.key.weight"].shape[1]
    if out["blocks.0.ffn.value.weight"].shape != (F, C) or out["head.weight"].shape != (C, V):
        raise ValueError("checkpoint shapes are not RWKV-4 ([C,C] att, [F,C]/[C,F] ffn, [V,C] head)")
    return out


def load_rwkv4(path: str, rescale: bool = True) -> Dict[str, torch.Tensor]:
    """Load an RWKV-4 checkpoint (`.pth` or `.safetensors`) into the engine's
    weight dict. `.pth` files are read with weights_only=True."""
    path = os.fspath(path)
    if path.endswith(".safetensors"):
        from safetensors.torch import load_file
        sd = load_file(path, device="cpu")
    else:
        sd = torch.load(path, map_location="cpu", weights_only=True)
    return convert_rwkv4_state_dict(sd, rescale=rescale)


def to_rwkv4_state_dict(w: Mapping[str, torch.Tensor]) -> Dict[str, torch.Tensor]:
    """The inverse layout change (engine dict -> checkpoint tensors, without
    an ln0, so convert_rwkv4_state_dict gives `w` back exactly), for writing
    test checkpoints."""
    sd: Dict[str, torch.Tensor] = {}
    sd["emb.weight"] = w["emb.weight"].clone()
    for k, v in w.items():
        if k == "emb.weight":
            continue
        if any(k.endswith(m) for m in _MATRICES) or k == "head.weight":
            sd[k] = v.t().contiguous()
        elif "time_mix" in k:
            sd[k] = v.reshape(1, 1, -1).clone()
        else:
            sd[k] = v.clone()
    return sd
