"""Drop-in for the reference's `krunch.cpp_path` forward orchestration
(`krunch/cpp_path.py:26-585`), running on the HIP library.

Same function names and argument meaning: `init_weights`, `fresh_state`,
`fresh_state_batched`, `forward_packed`, `forward_packed_window`,
`forward_stepped`, `forward_stepped_graphed`, `forward_stepped_batched`,
`softmax_cdfs_per_row`, `softmax_cdf_one_row`, `compute_decompress_batch`,
`pick_decompress_batch`. Packed and stepped calls
are bit-identical per row (one GEMM reduction order, shared elementwise
code), which is what makes compress/decompress round trips byte-exact.

Additions: `forward_packed_batched` runs B chunks x T tokens in one call
(the reference op already accepts [B,T,C], layer_cpp.cpp:469-474).
"""
from __future__ import annotations

import os
from collections import OrderedDict

import torch

from krunch_amd import _lib
from krunch_amd.model import Prepared, State, prepare

N_LAYER = 12
CDF_PRECISION = 24
# Prepared bundles by (id(model), device, codec), least recently used first.
# Each entry holds the model itself, so its id cannot be reused while the
# entry lives; at most WEIGHTS_CACHE_SIZE entries are kept (one prepared
# 169M-shape fp16 model is ~350 MB of device memory).
WEIGHTS_CACHE_SIZE = 4
_WEIGHTS_CACHE: "OrderedDict" = OrderedDict()


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
    hit = _WEIGHTS_CACHE.get(key)
    if hit is not None and hit["model"] is model:
        _WEIGHTS_CACHE.move_to_end(key)
        return hit
    w = model.w if hasattr(model, "w") else model
    P = prepare(w, device, w8a8=w8a8)
    bundle = {"prepared": P, "n_embd": P.C, "n_att": P.C, "n_ffn": P.F, "n_vocab": P.V,
              "n_layer": P.n_layer, "device": P.device, "model": model}
    _WEIGHTS_CACHE[key] = bundle
    while len(_WEIGHTS_CACHE) > WEIGHTS_CACHE_SIZE:
        _WEIGHTS_CACHE.popitem(last=False)
    return bundle


def release_weights(model=None):
    """Drop the prepared copies of `model` (every device and codec), or of
    every model when None. Bundles a caller still holds stay valid."""
    for key in [k for k, v in _WEIGHTS_CACHE.items() if model is None or v["model"] is model]:
        del _WEIGHTS_CACHE[key]
        for gk in [g for g, hit in _STEP_GRAPHS.items() if hit[-1]["model"] is model or model is None]:
            del _STEP_GRAPHS[gk]


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


_STEP_GRAPHS: dict = {}


def forward_stepped_graphed(weights: dict, last_token: int, state: State) -> torch.Tensor:
    """forward_stepped replayed from one captured HIP graph (the role of
    cpp_path.py:369-410): embedding lookup, all layers and the head of one
    token. The graph is captured on the first call for (weights, state) and
    replayed after; capturing executes nothing, so every call advances the
    state exactly once (the reference's per-layer capture advances it three
    times on the first call, which its docstring records as broken). Same
    bits as forward_stepped. Returns fp16 logits [V]."""
    P: Prepared = weights["prepared"]
    assert state.B == 1, "forward_stepped_graphed decodes one stream"
    key = (id(weights), state.ptr)
    hit = _STEP_GRAPHS.get(key)
    if hit is None:
        dev = P.device
        ids = torch.zeros(1, dtype=torch.int32, device=dev)
        x = torch.empty((16, P.C), dtype=torch.float16, device=dev)
        xn = torch.empty((16, P.C), dtype=torch.float16, device=dev)
        logits = torch.empty((1, P.V), dtype=torch.float16, device=dev)
        ws, nbytes = workspace(weights, 16)
        ws = ws.clone()        # private to the graph: the shared workspace may grow
        torch.cuda.synchronize(dev)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            s = _lib.stream_ptr()
            _lib.call("kr_embed", P.ptr, ids.data_ptr(), 1, x.data_ptr(), s)
            _lib.call("kr_forward_layers", P.ptr, x.data_ptr(), 1, 1, state.ptr, ws.data_ptr(),
                      nbytes, s)
            _lib.call("kr_head_logits", P.ptr, x.data_ptr(), 1, xn.data_ptr(), logits.data_ptr(),
                      P.V, s)
        # the entry holds the weights bundle, so its id cannot be reused for
        # another bundle while the graph (which points into it) is cached
        hit = (graph, ids, x, xn, logits, ws, weights)
        _STEP_GRAPHS[key] = hit
    graph, ids, _, _, logits, _, _ = hit
    tok = int(last_token)
    if not 0 <= tok < P.V:
        raise ValueError(f"token id out of range [0, {P.V})")
    ids.fill_(tok)
    graph.replay()
    return logits.reshape(-1).clone()


def clear_graph_cache():
    """Drop the graphs forward_stepped_graphed captured (call when weights or
    state buffers are freed)."""
    _STEP_GRAPHS.clear()


def softmax_cdfs_per_row(logits_TxV: torch.Tensor) -> torch.Tensor:
    """fp16 logits [T, V] -> int32 CDF [T, V+1] (softmax + cdf.py + scan, one kernel)."""
    from krunch_amd import krunch_ac_hip
    return krunch_ac_hip.softmax_cdf(logits_TxV.contiguous(), 1 << CDF_PRECISION)


def softmax_cdf_one_row(logits_V: torch.Tensor) -> torch.Tensor:
    return softmax_cdfs_per_row(logits_V.reshape(1, -1))[0].contiguous()


def cpp_path_enabled() -> bool:
    return True


# Streams per lockstep call, for compress and decompress alike (the role of
# cpp_path.py:531-580, sized for MI355X by measurement rather than by CU
# count). Decompress at the config-5 window on one MI355X: B = 128, 256, 384,
# 512 give 1,074, 1,799, 1,857, 2,283 KB/s. 512 rows is the largest batch the
# fused stepped kernels take (small-M GEMMs, fragment-packed operands), and
# B x 1024-token windows stay under the forward's 2^31 / F row limit.
DEFAULT_STREAM_BATCH = 512


def env_batch(name: str, n_chunks: int, default: int) -> int:
    B = default
    env = os.environ.get(name)
    if env:
        try:
            B = max(1, int(env))
        except ValueError:
            pass
    return max(1, min(n_chunks, B)) if n_chunks > 0 else B


def compute_decompress_batch(n_chunks: int = -1, default: int = DEFAULT_STREAM_BATCH) -> int:
    """Streams decoded in one lockstep call, clamped to n_chunks when given;
    $KRUNCH_DECOMPRESS_BATCH overrides (cpp_path.py:531-580). Memory is never
    the limit: ~0.5 MB per stream (state, logits, workspace) against 288 GB."""
    return env_batch("KRUNCH_DECOMPRESS_BATCH", n_chunks, default)


def pick_decompress_batch(default: int = DEFAULT_STREAM_BATCH) -> int:
    return compute_decompress_batch(n_chunks=-1, default=default)
