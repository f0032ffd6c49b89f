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
add or gate. In that mode LayerNorm sums in the order the GPU's one-wave row
kernel does (`layer_norm`: per lane over its 4-column groups, then a 64-lane
butterfly), so its fp16 outputs are the GPU's. The int8 codec (`w8a8=True`)
quantises those fp16 values, as the GPU kernels do; with fp16=True it also
takes its exps from the deterministic kexp (oracle/softmax.py, the GPU's
kr_kexp), in the sigmoid and the WKV update, as the GPU's int8 codec does:
the int8 activations are then the GPU's bit for bit
(tests/test_gpu_w8a8.py). With fp16=False it quantises fp32 activations (the
scheme in exact arithmetic).

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

import numpy as np
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


def _kexp(t: torch.Tensor) -> torch.Tensor:
    from oracle import softmax as osm
    return torch.from_numpy(osm.kexp(t.numpy()))


def wkv(k, v, w, u, st, det: bool = False):
    """WKV recurrence over T (k, v: [B,T,C] fp32); updates st['aa','bb','pp'].
    det: exps by kexp (every argument is <= 0), as the GPU's int8 codec."""
    ex = _kexp if det else torch.exp
    aa, bb, pp = st["aa"], st["bb"], st["pp"]
    ys = []
    for t in range(k.shape[1]):
        kt, vt = k[:, t], v[:, t]
        ww = u + kt
        p = torch.maximum(pp, ww)
        e1, e2 = ex(pp - p), ex(ww - p)
        ys.append((e1 * aa + e2 * vt) / (e1 * bb + e2))
        ww = w + pp
        p = torch.maximum(ww, kt)
        e1, e2 = ex(ww - p), ex(kt - p)
        aa, bb, pp = e1 * aa + e2 * vt, e1 * bb + e2, p
    st["aa"], st["bb"], st["pp"] = aa, bb, pp
    return torch.stack(ys, dim=1)


def _f32(t):
    return t.to(torch.float32)


def _round(fp16: bool):
    return (lambda t: t.half().float()) if fp16 else (lambda t: t)


def _butterfly_sum(v: np.ndarray) -> np.ndarray:
    """[R, 64] float32 lane values -> [R] sums, added as a 64-lane xor
    butterfly (strides 32, 16, ..., 1; each lane adds its partner's value)."""
    lanes = np.arange(64)
    for o in (32, 16, 8, 4, 2, 1):
        v = (v + v[:, lanes ^ o]).astype(np.float32)
    return v[:, 0]


def layer_norm(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """LayerNorm of float32 rows [..., C] (C = 256 G), in float32 with the
    summation order of the GPU's one-wave row kernel (kr_layer.hip
    layer_norm_row): lane l holds columns 256 i + 4 l + q and sums them over
    (i, q) in order from 0; the 64 lane sums meet in a butterfly; mean =
    sum * RN(1/C); the squared deviations likewise; rstd = 1 / sqrt(var +
    1e-5); y = ((x - mean) * rstd) * w + b, every operation rounded on its own.
    Pinned against torch.nn.functional.layer_norm in tests/test_oracle_rwkv.py."""
    C = x.shape[-1]
    G = C // 256
    f = np.float32
    v = x.reshape(-1, C).numpy().astype(f).reshape(-1, G, 64, 4)
    inv_c = f(1.0) / f(C)
    s = np.zeros(v.shape[:1] + (64,), f)
    for i in range(G):
        for q in range(4):
            s = (s + v[:, i, :, q]).astype(f)
    mean = (_butterfly_sum(s) * inv_c).astype(f)[:, None, None, None]
    d = (v - mean).astype(f)
    ss = np.zeros_like(s)
    for i in range(G):
        for q in range(4):
            ss = (ss + (d[:, i, :, q] * d[:, i, :, q]).astype(f)).astype(f)
    var = (_butterfly_sum(ss) * inv_c).astype(f)
    rstd = (f(1.0) / np.sqrt((var + f(LN_EPS)).astype(f))).astype(f)[:, None, None, None]
    wv = w.numpy().astype(f).reshape(G, 64, 4)
    bv = b.numpy().astype(f).reshape(G, 64, 4)
    y = ((d * rstd).astype(f) * wv).astype(f)
    y = (y + bv).astype(f)
    return torch.from_numpy(y.reshape(x.shape))


def _ln(x, w, b, fp16: bool):
    C = x.shape[-1]
    if fp16 and C % 256 == 0:
        return layer_norm(x, w, b)
    return F.layer_norm(x, (C,), w, b, LN_EPS)


def _sigmoid(t: torch.Tensor, det: bool) -> torch.Tensor:
    """det: 1 / (1 + e) for x >= 0, e / (1 + e) for x < 0, e = kexp(-|x|),
    as the GPU's int8 codec computes it."""
    if not det:
        return torch.sigmoid(t)
    e = _kexp(-t.abs())
    d = 1.0 + e
    return torch.where(t >= 0, 1.0 / d, e / d)


def time_mix(x, st, w, i, rowwise, q8=False, fp16=False, decay=None):
    """decay: the layer's w = -exp(time_decay) as given (e.g. the GPU's
    prepared vector), instead of computing it here."""
    a, b = f"blocks.{i}.att.", f"blocks.{i}."
    C = x.shape[-1]
    h = _round(fp16)
    det = q8 and fp16
    xx = h(_ln(x, _f32(w[b + "ln1.weight"]), _f32(w[b + "ln1.bias"]), fp16))
    sx = _shift(xx, st["att_xx"])
    mk, mv, mr = (_f32(w[a + n]).reshape(C) for n in ("time_mix_k", "time_mix_v", "time_mix_r"))
    kx = h(xx * mk + sx * (1 - mk))
    vx = h(xx * mv + sx * (1 - mv))
    rx = h(xx * mr + sx * (1 - mr))
    r = h(_sigmoid(h(_mm(rx, _f32(w[a + "receptance.weight"]), rowwise, q8)), det))
    k = _mm(kx, _f32(w[a + "key.weight"]), rowwise, q8)
    v = _mm(vx, _f32(w[a + "value.weight"]), rowwise, q8)
    if decay is None:
        decay = -torch.exp(_f32(w[a + "time_decay"]).reshape(C))
    y = wkv(k, v, _f32(decay).reshape(C), _f32(w[a + "time_first"]).reshape(C), st, det)
    st["att_xx"] = xx[:, -1, :].clone()
    return h(x + h(_mm(h(r * h(y)), _f32(w[a + "output.weight"]), rowwise, q8)))


def channel_mix(x, st, w, i, rowwise, q8=False, fp16=False):
    f, b = f"blocks.{i}.ffn.", f"blocks.{i}."
    C = x.shape[-1]
    h = _round(fp16)
    det = q8 and fp16
    xx = h(_ln(x, _f32(w[b + "ln2.weight"]), _f32(w[b + "ln2.bias"]), fp16))
    sx = _shift(xx, st["ffn_xx"])
    mk, mr = (_f32(w[f + n]).reshape(C) for n in ("time_mix_k", "time_mix_r"))
    kx = h(xx * mk + sx * (1 - mk))
    rx = h(xx * mr + sx * (1 - mr))
    r = h(_sigmoid(h(_mm(rx, _f32(w[f + "receptance.weight"]), rowwise, q8)), det))
    kr = torch.relu(h(_mm(kx, _f32(w[f + "key.weight"]), rowwise, q8)))
    kk = h(kr * kr)
    st["ffn_xx"] = xx[:, -1, :].clone()
    return h(x + h(r * h(_mm(kk, _f32(w[f + "value.weight"]), rowwise, q8))))


def forward(w: dict, ids: torch.Tensor, state, rowwise: bool = False,
            w8a8: bool = False, fp16: bool = False, decays=None) -> torch.Tensor:
    """ids [B, T] int -> logits [B, T, V] fp32; mutates `state` (list per layer).
    w8a8=True runs the seven layer products as the int8 codec defines them
    (oracle/quant.py); the head stays floating point. fp16=True rounds
    activations to fp16 where the production kernels store them. decays:
    optional per-layer w = -exp(time_decay) vectors (time_mix's decay)."""
    ids = torch.as_tensor(ids, dtype=torch.long)
    if ids.dim() == 1:
        ids = ids.unsqueeze(0)
    h = _round(fp16)
    x = h(_f32(w["emb.weight"])[ids])
    with torch.no_grad():
        for i, st in enumerate(state):
            x = time_mix(x, st, w, i, rowwise, w8a8, fp16, None if decays is None else decays[i])
            x = channel_mix(x, st, w, i, rowwise, w8a8, fp16)
        x = h(_ln(x, _f32(w["ln_out.weight"]), _f32(w["ln_out.bias"]), fp16))
        return h(_mm(x, _f32(w["head.weight"]), rowwise))
