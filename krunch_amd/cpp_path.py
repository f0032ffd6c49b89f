"""Drop-in for the reference's `krunch.cpp_path` forward orchestration
(`krunch/cpp_path.py:26-585`), running on the HIP library.

Same function names and argument meaning: `init_weights`, `fresh_state`,
`fresh_state_batched`, `forward_packed`, `forward_packed_window`,
`forward_stepped`, `forward_stepped_batched`, `softmax_cdfs_per_row`,
`softmax_cdf_one_row`, `compute_decompress_batch`. Packed and stepped calls
are bit-identical per row (one GEMM reduction order, shared elementwise
code), which is what makes compress/decompress round trips byte-exact.

Additions: `forward_packed_batched` runs B chunks x T tokens in one call
(the reference op already accepts [B,T,C], layer_cpp.cpp:469-474).
"""
from __future__ import annotations

import os

import torch

from krunch_amd import _lib
from krunch_amd.model import Prepared, State, prepare

N_LAYER = 12
CDF_PRECISION = 24
_WEIGHTS_CACHE: dict = {}


class Workspace:
    """Grow-only device scratch for the layer kernels, per device."""

    def __init__(self, device):
        self.device = device
        self.buf = None

    def get(self, nbytes: int) -> torch.Tensor:
        if self.buf is None or self.buf.numel() < nbytes:
            self.buf = None
            self.buf = torch.zeros(nbytes, dtype=torch.uint8, device=self.device)
        return self.buf


_WS: dict = {}



def logits_ld(V: int) -> int:
    """Row stride (elements) for engine-internal logits buffers: V rounded up
    to a multiple of 8, so the head GEMM stores 8-byte vectors."""
    return (int(V) + 7) // 8 * 8

def workspace(weights, M: int):
    P: Prepared = weights["prepared"]
    nbytes = _lib.lib().kr_forward_workspace_bytes(M, P.C, P.F)
    ws = _WS.setdefault(str(P.device), Workspace(P.device)).get(nbytes)
    return ws, nbytes


def init_weights(model, device: str = "cuda", w8a8: bool = False) -> dict:
    """Prepare weights once per (model, device, codec); `model` has `.w`
    (rwkv-package keys, [in,out] matrices, raw time_decay) or is such a dict.
    w8a8=True selects the int8 codec (head stays fp16)."""
    key = (id(model), str(device), bool(w8a8))
    if key in _WEIGHTS_CACHE:
        return _WEIGHTS_CACHE[key]
    w = model.w if hasattr(model, "w") else model
    P = prepare(w, device, w8a8=w8a8)
    bundle = {"prepared": P, "n_embd": P.C, "n_att": P.C, "n_ffn": P.F, "n_vocab": P.V,
              "n_layer": P.n_layer, "device": P.device, "model": model}
    _WEIGHTS_CACHE[key] = bundle
    return bundle


def fresh_state(weights: dict) -> State:
    return fresh_state_batched(weights, 1)


def fresh_state_batched(weights: dict, B: int) -> State:
    P: Prepared = weights["prepared"]
    return State(P.n_layer, B, P.C, P.device)


def _ids(t, device):
    t = torch.as_tensor(t, device=device)
    return t.to(torch.int32).contiguous()


def _check_ids(ids: torch.Tensor, V: int):
    if ids.numel() and (int(ids.min()) < 0 or int(ids.max()) >= V):
        raise ValueError(f"token id out of range [0, {V})")


def forward_packed_batched(weights: dict, input_ids, state: State) -> torch.Tensor:
    """input_ids [B, T] -> fp16 logits [B*T, V]; state (B streams) carried."""
    P: Prepared = weights["prepared"]
    ids = _ids(input_ids, P.device)
    if ids.dim() == 1:
        ids = ids.unsqueeze(0)
    B, T = ids.shape
    assert state.B == B, f"state holds {state.B} streams, input has {B}"
    _check_ids(ids, P.V)
    M = B * T
    x = torch.empty((M, P.C), dtype=torch.float16, device=P.device)
    s = _lib.stream_ptr()
    _lib.call("kr_embed", P.ptr, ids.data_ptr(), M, x.data_ptr(), s)
    ws, nbytes = workspace(weights, M)
    _lib.call("kr_forward_layers", P.ptr, x.data_ptr(), B, T, state.ptr, ws.data_ptr(), nbytes, s)
    xn = torch.empty_like(x)
    logits = torch.empty((M, P.V), dtype=torch.float16, device=P.device)
    _lib.call("kr_head_logits", P.ptr, x.data_ptr(), M, xn.data_ptr(), logits.data_ptr(), P.V, s)
    return logits


def forward_packed(weights: dict, input_ids, state: State) -> torch.Tensor:
    ids = torch.as_tensor(input_ids)
    return forward_packed_window(weights, ids, state, 0, int(ids.shape[-1]))


def forward_packed_window(weights: dict, input_ids, state: State, off: int, n: int):
    """Layer stack on the window [off, off+n) of one stream; returns fp16
    logits [n, V]. Consecutive windows give the same result as one call."""
    ids = torch.as_tensor(input_ids).reshape(-1)[off:off + n]
    return forward_packed_batched(weights, ids.reshape(1, -1), state)


def forward_stepped_batched(weights: dict, last_tokens, state: State) -> torch.Tensor:
    """One token for each of B streams; returns fp16 logits [B, V]."""
    ids = torch.as_tensor(last_tokens).reshape(-1, 1)
    return forward_packed_batched(weights, ids, state)


def forward_stepped(weights: dict, last_token: int, state: State) -> torch.Tensor:
    return forward_stepped_batched(weights, [int(last_token)], state).reshape(-1)


def softmax_cdfs_per_row(logits_TxV: torch.Tensor) -> torch.Tensor:
    """fp16 logits [T, V] -> int32 CDF [T, V+1] (softmax + cdf.py + scan, one kernel)."""
    from krunch_amd import krunch_ac_hip
    return krunch_ac_hip.softmax_cdf(logits_TxV.contiguous(), 1 << CDF_PRECISION)


def softmax_cdf_one_row(logits_V: torch.Tensor) -> torch.Tensor:
    return softmax_cdfs_per_row(logits_V.reshape(1, -1))[0].contiguous()


def cpp_path_enabled() -> bool:
    return True


def compute_decompress_batch(n_chunks: int = -1, default: int = 256) -> int:
    """Streams decoded in lockstep. The fused decode step runs one 1024-thread
    workgroup per stream, so 256 streams fill the 256 CUs of one MI355X once;
    memory per stream is ~0.5 MB (state, logits, workspace), so HBM never
    binds. Override with KRUNCH_DECOMPRESS_BATCH (cpp_path.py:531-580)."""
    env = os.environ.get("KRUNCH_DECOMPRESS_BATCH")
    upper = default
    if env:
        try:
            upper = max(1, int(env))
        except ValueError:
            pass
    return max(1, min(n_chunks, upper)) if n_chunks > 0 else upper


def pick_decompress_batch(default: int = 256) -> int:
    return compute_decompress_batch(n_chunks=-1, default=default)
