"""Drop-in for the reference's `krunch_ac_cuda` extension ops, on the HIP library.

Same op names, argument order and in-place semantics as the pybind module
(`krunch_ac/cuda/main.cpp:114-303,354-466`, `layer_cpp.cpp:824-1052`): the
range-coder ops, det_softmax_cdf, det_matmul, rwkv4_layer_step_cpp,
rwkv4_layer_step_cpp_t1, rwkv4_layer_step_cpp_graphed,
clear_layer_graph_cache, read_phase_times and reset_phase_times;
the caller owns coder state and buffers (mutated in place, launches are
asynchronous on the current stream); ops that produce tensors allocate them.
Argument errors raise RuntimeError, as TORCH_CHECK does. Differences: every
call is bounds-checked against the buffers it is given; the CDF precision is
taken from the CDF itself (cdf[:, -1] = 2^precision) or passed explicitly;
the graphed layer op advances the state once per call (the reference's first
call advances it three times); the phase profiler reports this build's seven
kernel phases rather than the reference's eleven.
"""
from __future__ import annotations

import weakref

import torch

from krunch_amd import _lib

CDF_PRECISION = 24


def _check(cond, msg):
    if not cond:
        raise RuntimeError(msg)


def _cuda(t, dtype, name):
    _check(t.is_cuda, f"{name} must be a device tensor")
    _check(t.dtype == dtype, f"{name} must be {dtype}, got {t.dtype}")
    _check(t.is_contiguous(), f"{name} must be contiguous")


def _nbytes(t):
    return t.numel() * t.element_size()


def _cap(buf):
    """A coder buffer's byte length as the uint32 the C ABI takes (raises
    rather than truncating past 2^32 - 1)."""
    return _lib.u32(_nbytes(buf), "coder buffer bytes")


# ---------------------------------------------------------------------------
# range coder (encode_kernel.cu / decode_kernel.cu ops)
# ---------------------------------------------------------------------------

def encode_step(cdf, symbols, output_buf, state, precision: int = CDF_PRECISION):
    """Encode N rows of one stream: cdf int32 [N, V+1], symbols int32 [N]."""
    _cuda(cdf, torch.int32, "cdf"); _cuda(symbols, torch.int32, "symbols")
    _cuda(output_buf, torch.uint8, "output_buf"); _cuda(state, torch.uint32, "state")
    _check(cdf.dim() == 2 and symbols.numel() == cdf.shape[0], "cdf/symbols shape mismatch")
    _check(state.numel() >= 4, "state must hold 4 uint32")
    _lib.call("kr_encode_step", cdf.data_ptr(), cdf.shape[1], symbols.data_ptr(), cdf.shape[0],
              output_buf.data_ptr(), _cap(output_buf), state.data_ptr(), precision, None,
              _lib.stream_ptr())


def encode_finalize(output_buf, state):
    _cuda(output_buf, torch.uint8, "output_buf"); _cuda(state, torch.uint32, "state")
    _lib.call("kr_encode_finalize", output_buf.data_ptr(), _cap(output_buf), state.data_ptr(),
              None, _lib.stream_ptr())


def decode_init(input_buf, state):
    _cuda(input_buf, torch.uint8, "input_buf"); _cuda(state, torch.uint32, "state")
    _lib.call("kr_decode_init_batched", input_buf.data_ptr(), _cap(input_buf), None, None,
              state.data_ptr(), 1, _lib.stream_ptr())


def decode_step(cdf, input_buf, state, out_sym, precision: int = CDF_PRECISION):
    """Decode one symbol: cdf int32 [V+1]; out_sym int32 [1]."""
    _cuda(cdf, torch.int32, "cdf"); _cuda(input_buf, torch.uint8, "input_buf")
    _cuda(state, torch.uint32, "state"); _cuda(out_sym, torch.int32, "out_sym")
    V = cdf.numel() - 1
    _lib.call("kr_decode_step_batched", cdf.data_ptr(), V, input_buf.data_ptr(),
              _cap(input_buf), None, None, state.data_ptr(), out_sym.data_ptr(), 1, precision,
              _lib.stream_ptr())


def encode_step_batched(cdfs, symbols, output_buf, base_byte_offsets, states,
                        precision: int = CDF_PRECISION):
    _cuda(cdfs, torch.int32, "cdfs"); _cuda(symbols, torch.int32, "symbols")
    _cuda(output_buf, torch.uint8, "output_buf"); _cuda(base_byte_offsets, torch.int32, "offsets")
    _cuda(states, torch.uint32, "states")
    B = symbols.numel()
    _check(cdfs.dim() == 2 and cdfs.shape[0] == B and base_byte_offsets.numel() == B
           and states.numel() == 4 * B, "batched shapes mismatch")
    _lib.call("kr_encode_step_batched", cdfs.data_ptr(), cdfs.shape[1] - 1, symbols.data_ptr(),
              output_buf.data_ptr(), _cap(output_buf), base_byte_offsets.data_ptr(),
              states.data_ptr(), B, precision, None, _lib.stream_ptr())


def encode_finalize_batched(output_buf, base_byte_offsets, states):
    _cuda(output_buf, torch.uint8, "output_buf"); _cuda(base_byte_offsets, torch.int32, "offsets")
    _cuda(states, torch.uint32, "states")
    B = base_byte_offsets.numel()
    _check(states.numel() == 4 * B, "states must be [4*B]")
    _lib.call("kr_encode_finalize_batched", output_buf.data_ptr(), _cap(output_buf),
              base_byte_offsets.data_ptr(), states.data_ptr(), B, None, _lib.stream_ptr())


def decode_init_batched(input_buf, base_byte_offsets, states, byte_limits=None):
    _cuda(input_buf, torch.uint8, "input_buf"); _cuda(base_byte_offsets, torch.int32, "offsets")
    _cuda(states, torch.uint32, "states")
    B = base_byte_offsets.numel()
    _check(states.numel() == 4 * B, "states must be [4*B]")
    _lib.call("kr_decode_init_batched", input_buf.data_ptr(), _cap(input_buf),
              base_byte_offsets.data_ptr(), _lib.ptr(byte_limits), states.data_ptr(), B,
              _lib.stream_ptr())


def decode_step_batched(cdfs, input_buf, base_byte_offsets, states, out_syms, byte_limits=None,
                        precision: int = CDF_PRECISION):
    _cuda(cdfs, torch.int32, "cdfs"); _cuda(input_buf, torch.uint8, "input_buf")
    _cuda(base_byte_offsets, torch.int32, "offsets"); _cuda(states, torch.uint32, "states")
    _cuda(out_syms, torch.int32, "out_syms")
    B = out_syms.numel()
    _check(cdfs.dim() == 2 and cdfs.shape[0] == B and states.numel() == 4 * B,
           "batched shapes mismatch")
    _lib.call("kr_decode_step_batched", cdfs.data_ptr(), cdfs.shape[1] - 1, input_buf.data_ptr(),
              _cap(input_buf), base_byte_offsets.data_ptr(), _lib.ptr(byte_limits),
              states.data_ptr(), out_syms.data_ptr(), B, precision, _lib.stream_ptr())


# ---------------------------------------------------------------------------
# softmax -> CDF (det_softmax_cdf.cu op)
# ---------------------------------------------------------------------------

def _precision_of(cdf_T_value: int) -> int:
    p = int(cdf_T_value).bit_length() - 1
    _check(p >= 1 and (1 << p) == int(cdf_T_value), "cdf_T_value must be a power of two")
    return p


def det_softmax_cdf(logits, cdf_T_value: int):
    """fp16 logits [T, V] -> int32 [T, V+1]: column 0 = 0, columns 1..V the
    per-symbol counts (deficit applied); the caller scans (cpp_path.py:490-501)."""
    _cuda(logits, torch.float16, "logits")
    _check(logits.dim() == 2, "logits must be [T, V]")
    T, V = logits.shape
    out = torch.empty((T, V + 1), dtype=torch.int32, device=logits.device)
    _lib.call("kr_softmax_cdf", logits.data_ptr(), T, V, V, out.data_ptr(), 0,
              _precision_of(cdf_T_value), _lib.stream_ptr())
    return out


def softmax_cdf(logits, cdf_T_value: int = 1 << CDF_PRECISION):
    """fp16 logits [T, V] -> cumulative int32 CDF [T, V+1] in one kernel."""
    _cuda(logits, torch.float16, "logits")
    T, V = logits.shape
    out = torch.empty((T, V + 1), dtype=torch.int32, device=logits.device)
    _lib.call("kr_softmax_cdf", logits.data_ptr(), T, V, V, out.data_ptr(), 1,
              _precision_of(cdf_T_value), _lib.stream_ptr())
    return out


def softmax_probs(logits):
    """fp16 logits [T, V] -> float32 softmax probabilities (the CDF's input)."""
    _cuda(logits, torch.float16, "logits")
    T, V = logits.shape
    out = torch.empty((T, V), dtype=torch.float32, device=logits.device)
    _lib.call("kr_softmax_probs", logits.data_ptr(), T, V, V, out.data_ptr(), _lib.stream_ptr())
    return out


# ---------------------------------------------------------------------------
# matmul / layer ops (layer_cpp.cpp)
# ---------------------------------------------------------------------------

_WT_CACHE: dict = {}


def _wt(W):
    """Transposed copy of a [K, N] weight, cached per live tensor object and version."""
    key = id(W)
    hit = _WT_CACHE.get(key)
    if hit is None or hit[0]() is not W or hit[1] != W._version:
        K, N = W.shape
        wt = torch.empty((N, K), dtype=torch.float16, device=W.device)
        _lib.call("kr_transpose_f16", W.data_ptr(), N, K, N, wt.data_ptr(), K, _lib.stream_ptr())
        hit = (weakref.ref(W, lambda _r, k=key: _WT_CACHE.pop(k, None)), W._version, wt)
        _WT_CACHE[key] = hit
    return hit[2]


def det_matmul(x, W, out_dtype=None):
    """y = x @ W, x fp16 [M, K], W fp16 [K, N]; fp32 accumulation in a fixed
    K order, so each row's result does not depend on M."""
    _cuda(x, torch.float16, "x"); _cuda(W, torch.float16, "W")
    M, K = x.shape
    _check(W.shape[0] == K, "inner dimensions differ")
    N = W.shape[1]
    dtype = out_dtype or torch.float16
    out = torch.empty((M, N), dtype=dtype, device=x.device)
    ep = 0 if dtype == torch.float32 else 1
    _lib.call("kr_det_matmul", x.data_ptr(), M, K, _wt(W).data_ptr(), K, N, out.data_ptr(), N,
              ep, None, None, _lib.stream_ptr())
    return out


def _layer_struct(x, att_xx, aa, bb, pp, ffn_xx, ln1_w, ln1_b, tm_k, tm_v, tm_r, time_decay,
                  time_first, Kw, Vw, Rw, Ow, ln2_w, ln2_b, ffn_tm_k, ffn_tm_r, ffn_Kw, ffn_Vw,
                  ffn_Rw):
    """Validate one layer call and build its kr_layer_weights; returns the
    struct, (C, F) and the device copies it points at (keep them alive)."""
    _cuda(x, torch.float16, "x")
    _check(x.dim() == 3, "x must be [B, T, C]")
    B, T, C = x.shape
    F = ffn_Kw.shape[1]
    dev = x.device
    keep = []

    def h(t):
        t = t.to(device=dev, dtype=torch.float16).reshape(-1).contiguous()
        _check(t.numel() == C, "layer vectors must hold C values")
        keep.append(t)
        return t.data_ptr()

    def f32(t):
        t = t.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
        _check(t.numel() == C, "time_decay / time_first must hold C values")
        keep.append(t)
        return t.data_ptr()

    def wt(m, k, n):
        _cuda(m, torch.float16, "weight")
        _check(tuple(m.shape) == (k, n), f"weight must be [{k}, {n}], got {tuple(m.shape)}")
        t = _wt(m)
        keep.append(t)
        return t.data_ptr()

    L = _lib.KrLayerWeights()
    L.ln1_w, L.ln1_b, L.tm_k, L.tm_v, L.tm_r = map(h, (ln1_w, ln1_b, tm_k, tm_v, tm_r))
    L.decay, L.first = f32(time_decay), f32(time_first)
    L.Kt, L.Vt, L.Rt, L.Ot = (wt(m, C, C) for m in (Kw, Vw, Rw, Ow))
    L.ln2_w, L.ln2_b, L.ftm_k, L.ftm_r = map(h, (ln2_w, ln2_b, ffn_tm_k, ffn_tm_r))
    L.fKt, L.fVt, L.fRt = wt(ffn_Kw, C, F), wt(ffn_Vw, F, C), wt(ffn_Rw, C, C)
    for t, dt, n in ((att_xx, torch.float16, "att_xx"), (aa, torch.float32, "aa"),
                     (bb, torch.float32, "bb"), (pp, torch.float32, "pp"),
                     (ffn_xx, torch.float16, "ffn_xx")):
        _cuda(t, dt, n)
        _check(t.numel() == B * C, f"{n} must be [B, C] = [{B}, {C}]")
    return L, C, F, keep


def _layer_call(L, C, F, x_inout, att_xx, aa, bb, pp, ffn_xx, ws, ws_bytes):
    B, T, _ = x_inout.shape
    _lib.call("kr_layer_step", L, C, F, x_inout.data_ptr(), B, T, att_xx.data_ptr(),
              aa.data_ptr(), bb.data_ptr(), pp.data_ptr(), ffn_xx.data_ptr(), ws.data_ptr(),
              ws_bytes, _lib.stream_ptr())


def rwkv4_layer_step_cpp(x, att_xx, aa, bb, pp, ffn_xx, ln1_w, ln1_b, tm_k, tm_v, tm_r,
                         time_decay, time_first, Kw, Vw, Rw, Ow, ln2_w, ln2_b, ffn_tm_k,
                         ffn_tm_r, ffn_Kw, ffn_Vw, ffn_Rw):
    """One RWKV-4 layer over x [B, T, C] fp16 (any B, T); state mutated in
    place; returns the new x (layer_cpp.cpp:456-637). `time_decay` is
    w = -exp(raw) as the reference's rwkv loader passes it (wkv_kernel.cu:41-45).
    Matrices are [in, out] (y = x @ W)."""
    args = (x, att_xx, aa, bb, pp, ffn_xx, ln1_w, ln1_b, tm_k, tm_v, tm_r, time_decay,
            time_first, Kw, Vw, Rw, Ow, ln2_w, ln2_b, ffn_tm_k, ffn_tm_r, ffn_Kw, ffn_Vw, ffn_Rw)
    L, C, F, _keep = _layer_struct(*args)
    B, T, _ = x.shape
    out = x.contiguous().clone()
    ws_bytes = _lib.lib().kr_forward_workspace_bytes(B * T, C, F)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    _layer_call(L, C, F, out, att_xx, aa, bb, pp, ffn_xx, ws, ws_bytes)
    return out


def rwkv4_layer_step_cpp_t1(x, att_xx, aa, bb, pp, ffn_xx, *weights):
    """The B = 1, T = 1 form of rwkv4_layer_step_cpp (layer_cpp.cpp:294-443):
    x [1, 1, C], state tensors [1, C]. Same kernels and bits as the general
    op at that shape (the decode step's)."""
    _check(x.dim() == 3 and x.shape[0] == 1 and x.shape[1] == 1, "x must be [1, 1, C]")
    return rwkv4_layer_step_cpp(x, att_xx, aa, bb, pp, ffn_xx, *weights)


_LAYER_GRAPHS: dict = {}


def rwkv4_layer_step_cpp_graphed(layer_id, x_buf, x_out_buf, att_xx, aa, bb, pp, ffn_xx,
                                 *weights):
    """Graph-replayed rwkv4_layer_step_cpp (layer_cpp.cpp:654-717):
    x_out_buf = layer(x_buf) with the state mutated in place; returns
    x_out_buf. The first call for a (layer_id, T, buffers) key captures the
    layer step into a HIP graph, later calls replay it, so the buffers must
    stay allocated and keep their addresses (as in the reference). Capturing
    executes nothing here, so every call - the first included - advances the
    state exactly once; the reference's warm-up runs and capture advance it
    three times on the first call (cpp_path.py:369-384 records that as a bug).
    The graph also keys on the buffer addresses and shapes, so new buffers get
    a new graph instead of a stale replay. The graph runs on the transposed
    weight copies made at capture time: after an in-place change of a
    weight tensor (same address), call clear_layer_graph_cache()."""
    _cuda(x_buf, torch.float16, "x_buf")
    _cuda(x_out_buf, torch.float16, "x_out_buf")
    _check(x_buf.shape == x_out_buf.shape, "x_buf and x_out_buf must have the same shape")
    bufs = (x_buf, x_out_buf, att_xx, aa, bb, pp, ffn_xx)
    key = (int(layer_id), tuple((t.data_ptr(), tuple(t.shape)) for t in bufs),
           tuple((w.data_ptr(), tuple(w.shape)) for w in weights))
    hit = _LAYER_GRAPHS.get(key)
    if hit is None:
        L, C, F, keep = _layer_struct(x_buf, att_xx, aa, bb, pp, ffn_xx, *weights)
        B, T, _ = x_buf.shape
        ws_bytes = _lib.lib().kr_forward_workspace_bytes(B * T, C, F)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x_buf.device)
        torch.cuda.synchronize(x_buf.device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            x_out_buf.copy_(x_buf)
            _layer_call(L, C, F, x_out_buf, att_xx, aa, bb, pp, ffn_xx, ws, ws_bytes)
        hit = (graph, L, keep, ws)
        _LAYER_GRAPHS[key] = hit
    hit[0].replay()
    return x_out_buf


def clear_layer_graph_cache():
    """Drop every cached layer graph (layer_cpp.cpp:719-722); call when
    weights change or before freeing the buffers a graph was captured on."""
    _LAYER_GRAPHS.clear()


# ---------------------------------------------------------------------------
# phase profiler (layer_cpp.cpp:111-157, read/reset at :825-836)
# ---------------------------------------------------------------------------

def set_phase_profile(on: bool) -> bool:
    """Turn the per-call layer profiler on or off (KRUNCH_PHASE_PROFILE=1 does
    it at first use); returns the previous setting."""
    return bool(_lib.lib().kr_phase_profile(1 if on else 0))


def read_phase_times() -> dict:
    """Accumulated milliseconds per layer phase over the profiled
    rwkv4_layer_step_cpp calls, plus "call_count". This build's phases:
    ln1_mix, kvr_matmul, wkv, ow_matmul_residual, ln2_mix, ffn_rk_matmul,
    ffn_v_matmul_residual (the reference's eleven, grouped as its fused
    kernels run them; a phase absorbed by a fused launch reads 0)."""
    import ctypes
    L = _lib.lib()
    n = L.kr_phase_count()
    ms = (ctypes.c_double * n)()
    calls = ctypes.c_longlong(0)
    _lib.call("kr_read_phase_times", ms, n, ctypes.byref(calls))
    out = {L.kr_phase_name(i).decode(): float(ms[i]) for i in range(n)}
    out["call_count"] = int(calls.value)
    return out


def reset_phase_times():
    _lib.call("kr_reset_phase_times")
