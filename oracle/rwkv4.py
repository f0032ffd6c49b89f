"""Oracle: RWKV-4 forward in fp32 torch on the CPU (test infrastructure only).

Layer math restated from the reference's torch path
`krunch/batched_rwkv4.py:85-172` (channel mix :85-101, time mix :104-172),
the model loop `:219-262`, and the production op order of
`krunch_ac/cuda/layer_cpp.cpp:456-637`. The WKV recurrence follows the
production kernel `krunch_ac/cuda/wkv_kernel.cu:52-73` (bonus u applied to the
current token, w = -exp(time_decay_raw)), not the pure-torch branch at
batched_rwkv4.py:138-154, which applies u to the carried state instead.
Initial state as in `krunch/cpp_path.py:94-106` (pp = -1e30).

Weights use the rwkv-package layout the reference reads (`cpp_path.py:59-86`):
matrices are [in, out] so that y = x @ W; `time_decay` is the raw value.

`fp16=True` rounds every activation to fp16 where the production layer
stores one (`layer_cpp.cpp:456-637`: fp16 activations, fp32 k/v/WKV): the
residual stream, LayerNorm outputs, token-shift mixes, the sigmoid / ReLU^2
products, fp16(y) and r * y, and every fp16 GEMM output before the residual
add or gate. The int8 codec (`w8a8=True`) quantises those fp16 values, as the
GPU kernels do; with fp16=False it quantises fp32 activations (the scheme in
exact arithmetic).

`rowwise=True` computes every matrix product with one fixed summation order
per output (oracle/rowgemm.c: k ascending), so a token's result does not
depend on how many rows share the call (packed T=1024 and stepped T=1 give
identical bits); that makes the CPU round trip byte-exact.

Pinned by: golden logits from the reference's own `forward_batched`
(tests/golden/make_golden.py), the WKV closed form (direct weighted sums in
float64) and T=1 from the initial state (y = v), and the packed == stepped /
windowed == single-shot invariants (tests/test_oracle_rwkv.py).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

LN_EPS = 1e-5


def new_state(n_layer: int, B: int, C: int):
    z = lambda: torch.zeros(B, C, dtype=torch.float32)
    return [dict(att_xx=z(), aa=z(), bb=z(), pp=torch.full((B, C), -1e30), ffn_xx=z())
            for _ in range(n_layer)]


def _mm_q8(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """w8a8 product (oracle/quant.py): x quantised per row, w [in, out] per
    output channel, exact integer sums, two float32 scale multiplies."""
    from oracle import quant
    qw, sw = quant.quantize_rows(w.t().contiguous().numpy())
    flat = x.reshape(-1, x.shape[-1]).numpy()
    qa, sa = quant.quantize_rows(flat)
    y = torch.from_numpy(quant.matmul_i8(qa, sa, qw, sw))
    return y.reshape(*x.shape[:-1], w.shape[-1])


def _mm(x: torch.Tensor, w: torch.Tensor, rowwise: bool, q8: bool = False) -> torch.Tensor:
    if q8:
        return _mm_q8(x, w)
    if not rowwise:
        return x @ w
    from oracle import crc
    flat = x.reshape(-1, x.shape[-1]).contiguous().numpy()
    out = torch.from_numpy(crc.gemm_rows(flat, w.contiguous().numpy()))
    return out.reshape(*x.shape[:-1], w.shape[-1])


def _shift(xx: torch.Tensor, prev: torch.Tensor) -> torch.Tensor:
    """Token shift: row t sees row t-1, row 0 sees the carried state."""
    return torch.cat((prev.unsqueeze(1), xx[:, :-1, :]), dim=1)


def wkv(k, v, w, u, st):
    """WKV recurrence over T (k, v: [B,T,C] fp32); updates st['aa','bb','pp']."""
    aa, bb, pp = st["aa"], st["bb"], st["pp"]
    ys = []
    for t in range(k.shape[1]):
        kt, vt = k[:, t], v[:, t]
        ww = u + kt
        p = torch.maximum(pp, ww)
        e1, e2 = torch.exp(pp - p), torch.exp(ww - p)
        ys.append((e1 * aa + e2 * vt) / (e1 * bb + e2))
        ww = w + pp
        p = torch.maximum(ww, kt)
        e1, e2 = torch.exp(ww - p), torch.exp(kt - p)
        aa, bb, pp = e1 * aa + e2 * vt, e1 * bb + e2, p
    st["aa"], st["bb"], st["pp"] = aa, bb, pp
    return torch.stack(ys, dim=1)


def _f32(t):
    return t.to(torch.float32)


def _round(fp16: bool):
    return (lambda t: t.half().float()) if fp16 else (lambda t: t)


def time_mix(x, st, w, i, rowwise, q8=False, fp16=False):
    a, b = f"blocks.{i}.att.", f"blocks.{i}."
    C = x.shape[-1]
    h = _round(fp16)
    xx = h(F.layer_norm(x, (C,), _f32(w[b + "ln1.weight"]), _f32(w[b + "ln1.bias"]), LN_EPS))
    sx = _shift(xx, st["att_xx"])
    mk, mv, mr = (_f32(w[a + n]).reshape(C) for n in ("time_mix_k", "time_mix_v", "time_mix_r"))
    kx = h(xx * mk + sx * (1 - mk))
    vx = h(xx * mv + sx * (1 - mv))
    rx = h(xx * mr + sx * (1 - mr))
    r = h(torch.sigmoid(h(_mm(rx, _f32(w[a + "receptance.weight"]), rowwise, q8))))
    k = _mm(kx, _f32(w[a + "key.weight"]), rowwise, q8)
    v = _mm(vx, _f32(w[a + "value.weight"]), rowwise, q8)
    decay = -torch.exp(_f32(w[a + "time_decay"]).reshape(C))
    y = wkv(k, v, decay, _f32(w[a + "time_first"]).reshape(C), st)
    st["att_xx"] = xx[:, -1, :].clone()
    return h(x + h(_mm(h(r * h(y)), _f32(w[a + "output.weight"]), rowwise, q8)))


def channel_mix(x, st, w, i, rowwise, q8=False, fp16=False):
    f, b = f"blocks.{i}.ffn.", f"blocks.{i}."
    C = x.shape[-1]
    h = _round(fp16)
    xx = h(F.layer_norm(x, (C,), _f32(w[b + "ln2.weight"]), _f32(w[b + "ln2.bias"]), LN_EPS))
    sx = _shift(xx, st["ffn_xx"])
    mk, mr = (_f32(w[f + n]).reshape(C) for n in ("time_mix_k", "time_mix_r"))
    kx = h(xx * mk + sx * (1 - mk))
    rx = h(xx * mr + sx * (1 - mr))
    r = h(torch.sigmoid(h(_mm(rx, _f32(w[f + "receptance.weight"]), rowwise, q8))))
    kk = h(torch.relu(h(_mm(kx, _f32(w[f + "key.weight"]), rowwise, q8))) ** 2)
    st["ffn_xx"] = xx[:, -1, :].clone()
    return h(x + h(r * h(_mm(kk, _f32(w[f + "value.weight"]), rowwise, q8))))


def forward(w: dict, ids: torch.Tensor, state, rowwise: bool = False,
            w8a8: bool = False, fp16: bool = False) -> torch.Tensor:
    """ids [B, T] int -> logits [B, T, V] fp32; mutates `state` (list per layer).
    w8a8=True runs the seven layer products as the int8 codec defines them
    (oracle/quant.py); the head stays floating point. fp16=True rounds
    activations to fp16 where the production kernels store them."""
    ids = torch.as_tensor(ids, dtype=torch.long)
    if ids.dim() == 1:
        ids = ids.unsqueeze(0)
    h = _round(fp16)
    x = h(_f32(w["emb.weight"])[ids])
    with torch.no_grad():
        for i, st in enumerate(state):
            x = time_mix(x, st, w, i, rowwise, w8a8, fp16)
            x = channel_mix(x, st, w, i, rowwise, w8a8, fp16)
        C = x.shape[-1]
        x = h(F.layer_norm(x, (C,), _f32(w["ln_out.weight"]), _f32(w["ln_out.bias"]), LN_EPS))
        return h(_mm(x, _f32(w["head.weight"]), rowwise))
