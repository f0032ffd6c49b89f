"""Device-resident RWKV-4 weights in the library's layout, and the
recurrent-state buffer.

`prepare(w)` takes a weight dict in the layout the reference reads
(`krunch/cpp_path.py:59-86`: rwkv-package keys, matrices [in, out], raw
`time_decay`) and builds, on the GPU, the copies the kernels want:
matrices transposed to [out, in] (K contiguous) plus a fragment-packed copy
of each layer matrix (16 x 32 MFMA operand blocks, 1 KB contiguous each) for
the small-M decode GEMMs, fp16 activations/weights, fp32 w = -exp(time_decay) and u = time_first.
Tensor allocation is torch's; every transform is a HIP kernel of the library.

`State` is one contiguous buffer holding all layers' recurrent state for B
streams (per layer: att_xx, ffn_xx fp16 [B,C]; aa, bb, pp fp32 [B,C]) with
views in the reference's layouts: `state[k][i]` as cpp_path.fresh_state
returns (`cpp_path.py:94-106`), and `state.flat()` as
batched_rwkv4.init_state_batched returns (`batched_rwkv4.py:60-82`).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import torch

from krunch_amd import _lib

MAT_KEYS_ATT = ("key", "value", "receptance", "output")


def _dev(device):
    return torch.device(device if device is not None else "cuda")


def _fragments(Wt: torch.Tensor) -> torch.Tensor:
    """Fragment-packed copy of Wt [N, K] (kr_pack_fragments) for the small-M GEMM."""
    N, K = Wt.shape
    nbytes = _lib.lib().kr_fragment_bytes(N, K)
    out = torch.empty(nbytes // 2, dtype=torch.float16, device=Wt.device)
    _lib.call("kr_pack_fragments", Wt.data_ptr(), K, N, K, out.data_ptr(), _lib.stream_ptr())
    return out


def _quantized(Wt: torch.Tensor):
    """w8a8 copy of Wt [N, K]: int8 rows (one fp32 scale per output channel,
    kr_quantize_rows) and their fragment-packed copy for the small-M GEMM."""
    N, K = Wt.shape
    q = torch.empty((N, K), dtype=torch.int8, device=Wt.device)
    scale = torch.empty(N, dtype=torch.float32, device=Wt.device)
    _lib.call("kr_quantize_rows", Wt.data_ptr(), K, N, K, q.data_ptr(), scale.data_ptr(), 0,
              _lib.stream_ptr())
    qf = torch.empty(_lib.lib().kr_fragment_bytes(N, K // 2), dtype=torch.int8, device=Wt.device)
    _lib.call("kr_pack_fragments", q.data_ptr(), K // 2, N, K // 2, qf.data_ptr(),
              _lib.stream_ptr())
    return q, qf, scale


def _transposed(W: torch.Tensor, device) -> torch.Tensor:
    """[K, N] -> [N, K] fp16 on the device via kr_transpose_f16."""
    src = W.to(device=device, dtype=torch.float16).contiguous()
    K, N = src.shape
    out = torch.empty((N, K), dtype=torch.float16, device=device)
    _lib.call("kr_transpose_f16", src.data_ptr(), N, K, N, out.data_ptr(), K, _lib.stream_ptr())
    return out


@dataclass
class Prepared:
    n_layer: int
    C: int
    F: int
    V: int
    device: torch.device
    tensors: dict = field(default_factory=dict)
    layers_c: object = None
    model_c: object = None
    w8a8: bool = False
    q8_c: object = None

    @property
    def ptr(self):
        return ctypes.byref(self.model_c)

    def layer_ptr(self, i: int):
        return ctypes.byref(self.layers_c[i])


def prepare(w: dict, device=None, w8a8: bool = False) -> Prepared:
    """w8a8=True also builds the int8 codec's weights: the
    seven layer matrices quantised per output channel; the head stays fp16."""
    device = _dev(device)
    n_layer = 1 + max(int(k.split(".")[1]) for k in w if k.startswith("blocks."))
    V, C = w["emb.weight"].shape
    F = w["blocks.0.ffn.key.weight"].shape[1]
    P = Prepared(n_layer, C, F, V, device, w8a8=w8a8)
    t = P.tensors
    h = lambda x: x.to(device=device, dtype=torch.float16).reshape(-1).contiguous()
    t["emb"] = w["emb.weight"].to(device=device, dtype=torch.float16).contiguous()
    t["ln_out_w"], t["ln_out_b"] = h(w["ln_out.weight"]), h(w["ln_out.bias"])
    t["headT"] = _transposed(w["head.weight"], device)
    t["headF"] = _fragments(t["headT"])
    layers = (_lib.KrLayerWeights * n_layer)()
    for i in range(n_layer):
        a, f, b = f"blocks.{i}.att.", f"blocks.{i}.ffn.", f"blocks.{i}."
        L = {}
        L["ln1_w"], L["ln1_b"] = h(w[b + "ln1.weight"]), h(w[b + "ln1.bias"])
        L["ln2_w"], L["ln2_b"] = h(w[b + "ln2.weight"]), h(w[b + "ln2.bias"])
        L["tm_k"], L["tm_v"], L["tm_r"] = (h(w[a + n]) for n in ("time_mix_k", "time_mix_v", "time_mix_r"))
        L["ftm_k"], L["ftm_r"] = h(w[f + "time_mix_k"]), h(w[f + "time_mix_r"])
        raw = w[a + "time_decay"].to(device=device, dtype=torch.float32).reshape(-1).contiguous()
        L["decay"] = torch.empty_like(raw)
        _lib.call("kr_prepare_decay", raw.data_ptr(), L["decay"].data_ptr(), raw.numel(),
                  _lib.stream_ptr())
        L["first"] = w[a + "time_first"].to(device=device, dtype=torch.float32).reshape(-1).contiguous()
        for src, dst in zip(MAT_KEYS_ATT, ("Kt", "Vt", "Rt", "Ot")):
            L[dst] = _transposed(w[a + src + ".weight"], device)
        L["fKt"] = _transposed(w[f + "key.weight"], device)
        L["fVt"] = _transposed(w[f + "value.weight"], device)
        L["fRt"] = _transposed(w[f + "receptance.weight"], device)
        for src in ("K", "V", "R", "O", "fK", "fV", "fR"):
            L[src + "f"] = _fragments(L[src + "t"])
        if w8a8:
            for src in ("K", "V", "R", "O", "fK", "fV", "fR"):
                L[src + "_q"], L[src + "_qf"], L[src + "_qs"] = _quantized(L[src + "t"])
        for name, tensor in L.items():
            t[f"{i}.{name}"] = tensor
            if "_q" not in name:
                setattr(layers[i], name, tensor.data_ptr())
    if w8a8:
        q8 = (_lib.KrLayerQ8 * n_layer)()
        for i in range(n_layer):
            for src in ("K", "V", "R", "O", "fK", "fV", "fR"):
                m = getattr(q8[i], src)
                m.q = t[f"{i}.{src}_q"].data_ptr()
                m.qf = t[f"{i}.{src}_qf"].data_ptr()
                m.scale = t[f"{i}.{src}_qs"].data_ptr()
            layers[i].q8 = ctypes.pointer(q8[i])
        P.q8_c = q8
    P.layers_c = layers
    P.model_c = _lib.KrModelWeights(n_layer, C, F, V, t["emb"].data_ptr(), t["ln_out_w"].data_ptr(),
                                    t["ln_out_b"].data_ptr(), t["headT"].data_ptr(),
                                    ctypes.cast(layers, ctypes.POINTER(_lib.KrLayerWeights)),
                                    t["headF"].data_ptr())
    return P


class State:
    """All layers' recurrent state for B streams in one device buffer."""

    def __init__(self, n_layer: int, B: int, C: int, device=None):
        self.n_layer, self.B, self.C = n_layer, B, C
        self.device = _dev(device)
        nbytes = _lib.lib().kr_state_bytes(n_layer, B, C)
        self.buf = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        self.reset()

    def reset(self):
        _lib.call("kr_state_init", self.buf.data_ptr(), self.n_layer, self.B, self.C,
                  _lib.stream_ptr())

    def _layer(self, i):
        B, C = self.B, self.C
        per = B * C * 16
        raw = self.buf[i * per:(i + 1) * per]
        att_xx = raw[:B * C * 2].view(torch.float16).view(B, C)
        ffn_xx = raw[B * C * 2:B * C * 4].view(torch.float16).view(B, C)
        f = raw[B * C * 4:].view(torch.float32).view(3, B, C)
        return att_xx, f[0], f[1], f[2], ffn_xx

    def __getitem__(self, k: int):
        """state[k][i] with k = 0 att_xx, 1 aa, 2 bb, 3 pp, 4 ffn_xx (cpp_path layout)."""
        return [self._layer(i)[k] for i in range(self.n_layer)]

    def __len__(self):
        return 5

    def flat(self):
        """[att_xx, aa, bb, pp, ffn_xx] * n_layer (batched_rwkv4 layout)."""
        out = []
        for i in range(self.n_layer):
            out.extend(self._layer(i))
        return out

    @property
    def ptr(self):
        return self.buf.data_ptr()

    def clone(self):
        s = State.__new__(State)
        s.n_layer, s.B, s.C, s.device = self.n_layer, self.B, self.C, self.device
        s.buf = self.buf.clone()
        return s
