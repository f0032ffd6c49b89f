#!/usr/bin/env python3
"""Benchmark: krunch compress & decompress throughput on one MI355X.

Workload (one window per step): B = 256 chunks of
Zipf(1.1) tokens with 5% repeated 64-token spans, RWKV-4-169M-shaped
random-init weights in fp16. One step = one 1024-token window of every
chunk: packed compress (12 layers over B*T = 262,144 rows, head, softmax ->
CDF interval, range encode), then stepped decompress of the same window
(1024 lockstep steps of B tokens, fused CDF search + range decode, replayed
from a HIP graph). RNN and coder state carry across windows on both sides.
Inputs are resident in HBM before the timed region; after it, every decoded
token is checked against the input (byte-exact round trip).

value = input KB/s of the round trip, KB = 1024 B at 4 B/token:
  K*B*T*4/1024 / (t_compress + t_decompress).
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

BYTES_PER_TOKEN = 4
FLOP_PER_TOKEN = 261_250_560        # 12 x 2 x (5*768^2 + 2*768*3072) + 2*768*50277
MI355X_FP16_PEAK = 2.5e15
MI355X_HBM_PEAK = 8.0e12


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--batch", type=int, default=256)
    ap.add_argument("--window", type=int, default=1024)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-decode-steps", type=int, default=1024,
                    help="CPU baseline: tokens decoded (all of the window by default)")
    ap.add_argument("--head-rows", type=int, default=8192,
                    help="compress: rows per head GEMM + CDF block (the logits buffer holds this many rows)")
    ap.add_argument("--groups", type=int, default=1,
                    help="decode the B streams as this many concurrent groups (graph branches)")
    ap.add_argument("--no-w8a8", action="store_true",
                    help="skip the w8a8 codec (BASELINE config 4) run on the same windows")
    ap.add_argument("--hbm-table", metavar="CSV",
                    help="print the per-kernel HBM fraction of a decode step from a rocprofv3 "
                         "kernel-trace CSV of this bench (no GPU work)")
    ap.add_argument("--roofline-json", metavar="OUT",
                    help="with --hbm-table: also write the in-step durations of the two "
                         "roofline launches to OUT (bench.py reads profiles/"
                         "decode_step_B256_roofline.json for its roofline lines)")
    ap.add_argument("--bench-line", metavar="JSON",
                    help="with --roofline-json: the bench line printed by the profiled run, "
                         "whose live in-step wave spans are recorded beside the trace figures")
    ap.add_argument("--kernel-probe", action="store_true",
                    help="only run a 256 MiB device copy (counter calibration), 8 launches of "
                         "the dominant kernel and 2 eager launches of each other hot kernel at "
                         "the bench shapes (the packed products and head included), for "
                         "rocprofv3 --pmc runs")
    return ap.parse_args()


def kernel_probe(weights16, B, head_rows):
    """A plain copy of known size, then the dominant kernel, eagerly (one
    dispatch each), so hardware counters can be read per dispatch."""
    import ctypes
    import torch
    from krunch_amd import _lib, cpp_path

    dev = torch.device("cuda")
    src = torch.ones(64 << 20, dtype=torch.float32, device=dev)       # 256 MiB
    dst = torch.empty_like(src)
    dst.copy_(src)
    W = cpp_path.init_weights(weights16, "cuda")
    P = W["prepared"]
    K, N, M = P.F, P.C, B
    A = torch.rand((M, K), device=dev).half()
    res = torch.randn((M, N), device=dev).half()
    gate = torch.rand((M, N), device=dev).half()
    out = torch.empty((M, N), dtype=torch.float16, device=dev)
    Wf = P.tensors["0.fVf"]
    Af = torch.empty(_lib.lib().kr_fragment_bytes(M, K) // 2, dtype=torch.float16, device=dev)
    _lib.call("kr_pack_fragments", A.data_ptr(), K, M, K, Af.data_ptr(), _lib.stream_ptr())
    for _ in range(8):
        _lib.call("kr_det_matmul_packed", Af.data_ptr(), M, K, Wf.data_ptr(), N, out.data_ptr(), N,
                  5, res.data_ptr(), gate.data_ptr(), 0, _lib.stream_ptr())
    torch.cuda.synchronize()
    # 8 launches of the channel-mix R + K products (one launch, as the step runs them)
    xr = _pack(torch.rand((M, N), device=dev).half())
    xk = _pack(torch.rand((M, N), device=dev).half())
    rf = torch.empty((M, N), dtype=torch.float16, device=dev)
    kf = torch.empty(_lib.lib().kr_fragment_bytes(M, K) // 2, dtype=torch.float16, device=dev)
    jobs = (_lib.KrPackedJob * 2)()
    jobs[0] = _lib.KrPackedJob(xr.data_ptr(), P.tensors["0.fRf"].data_ptr(), N, rf.data_ptr(), N,
                               2, None, None, 0)
    jobs[1] = _lib.KrPackedJob(xk.data_ptr(), P.tensors["0.fKf"].data_ptr(), K, kf.data_ptr(), K,
                               3, None, None, 1)
    for _ in range(8):
        _lib.call("kr_det_matmul_packed_multi", jobs, 2, M, N, _lib.stream_ptr())
    torch.cuda.synchronize()
    del xr, xk, rf, kf
    del A, Af, res, gate, out
    s = _lib.stream_ptr()
    # one stepped layer (LN-mix, K/V/R+WKV, output projection, LN-mix, ffn R/K, ffn V) at B rows
    from krunch_amd.model import State
    st = State(P.n_layer, B, P.C, dev)
    ws, nbytes = cpp_path.workspace(W, B)
    x = torch.randn((B, P.C), device=dev).half()
    L0 = P.layers_c[0]
    att_xx, aa0, bb0, pp0, ffn_xx = st._layer(0)
    for _ in range(2):
        _lib.call("kr_layer_step", ctypes.byref(L0), P.C, P.F, x.data_ptr(), B, 1,
                  att_xx.data_ptr(), aa0.data_ptr(), bb0.data_ptr(), pp0.data_ptr(),
                  ffn_xx.data_ptr(), ws.data_ptr(), nbytes, s)
    torch.cuda.synchronize()
    # the decode head at B rows (LN_out, then the small-M head kernel)
    xn = torch.empty((B, P.C), dtype=torch.float16, device=dev)   # B % 16 == 0 at the bench shapes
    ld = cpp_path.logits_ld(P.V)
    hl = torch.empty((B, ld), dtype=torch.float16, device=dev)
    for _ in range(2):
        _lib.call("kr_head_logits", P.ptr, x.data_ptr(), B, xn.data_ptr(), hl.data_ptr(), ld, s)
    torch.cuda.synchronize()
    del ws, xn, hl
    # packed channel-mix value product at the window shape (B * 1024 rows) on the large-M kernel
    Mp = B * 1024
    A = torch.rand((Mp, K), device=dev).half()
    res = torch.randn((Mp, N), device=dev).half()
    gate = torch.rand((Mp, N), device=dev).half()
    out = torch.empty((Mp, N), dtype=torch.float16, device=dev)
    Wt = P.tensors["0.fVt"]
    for _ in range(2):
        _lib.call("kr_det_matmul", A.data_ptr(), Mp, K, Wt.data_ptr(), K, N, out.data_ptr(), N, 5,
                  res.data_ptr(), gate.data_ptr(), s)
    torch.cuda.synchronize()
    del A, res, gate, out
    # packed channel-mix key product (K = 768, N = 3072, relu^2) at the window shape
    A = torch.rand((Mp, N), device=dev).half()
    out = torch.empty((Mp, K), dtype=torch.float16, device=dev)
    for _ in range(2):
        _lib.call("kr_det_matmul", A.data_ptr(), Mp, N, P.tensors["0.fKt"].data_ptr(), N, K,
                  out.data_ptr(), K, 3, None, None, s)
    torch.cuda.synchronize()
    del A, out
    # the compress head: LN_out + the 768 x 50277 product on one block of head_rows rows
    xh = torch.randn((head_rows, P.C), device=dev).half()
    xnh = torch.empty((head_rows, P.C), dtype=torch.float16, device=dev)
    lh = torch.empty((head_rows, cpp_path.logits_ld(P.V)), dtype=torch.float16, device=dev)
    for _ in range(2):
        _lib.call("kr_head_logits", P.ptr, xh.data_ptr(), head_rows, xnh.data_ptr(), lh.data_ptr(),
                  cpp_path.logits_ld(P.V), s)
    torch.cuda.synchronize()
    del xh, xnh, lh
    # packed WKV over a 1024-token window of B streams
    k = torch.randn((B, 1024, P.C), device=dev)
    v = torch.randn((B, 1024, P.C), device=dev)
    r = torch.rand((B, 1024, P.C), device=dev).half()
    ry = torch.empty_like(r)
    aa = torch.zeros((B, P.C), device=dev)
    bb = torch.zeros((B, P.C), device=dev)
    pp = torch.full((B, P.C), -1e30, device=dev)
    dec = P.tensors["0.decay"]
    fst = P.tensors["0.first"]
    for _ in range(2):
        _lib.call("kr_wkv", B, 1024, P.C, dec.data_ptr(), fst.data_ptr(), k.data_ptr(), v.data_ptr(),
                  r.data_ptr(), aa.data_ptr(), bb.data_ptr(), pp.data_ptr(), ry.data_ptr(), s)
    torch.cuda.synchronize()
    del k, v, r, ry
    # softmax -> CDF -> symbol interval for head_rows rows of logits (the compress CDF stage)
    rows = head_rows
    ld = cpp_path.logits_ld(P.V)
    logits = (torch.randn((rows, ld), device=dev) * 3).half()
    syms = torch.randint(0, P.V, (rows,), device=dev, dtype=torch.int32)
    pairs = torch.empty((rows, 2), dtype=torch.int32, device=dev)
    for _ in range(2):
        _lib.call("kr_softmax_cdf_pairs", logits.data_ptr(), rows, P.V, ld, syms.data_ptr(),
                  pairs.data_ptr(), 24, s)
    torch.cuda.synchronize()
    # the fused CDF search + range decode of one decode step (B rows; zeroed
    # decoder states over a zeroed stream are valid inputs)
    buf = torch.zeros(1 << 16, dtype=torch.uint8, device=dev)
    states = torch.zeros(4 * B, dtype=torch.int32, device=dev)
    out_syms = torch.empty(B, dtype=torch.int32, device=dev)
    for _ in range(2):
        _lib.call("kr_softmax_cdf_decode", logits.data_ptr(), B, P.V, ld, buf.data_ptr(),
                  buf.numel(), None, None, states.data_ptr(), out_syms.data_ptr(), None, 0, None,
                  None, 16, s)
    torch.cuda.synchronize()
    print(json.dumps({"probe": "ok", "copy_bytes": 2 * src.numel() * 4}))


def gpu_bench(args, weights16, w8a8=False, step_probe=False):
    import numpy as np
    import torch
    from krunch_amd import _lib, cpp_path, synthetic
    from krunch_amd.model import State

    dev = torch.device("cuda")
    W = cpp_path.init_weights(weights16, "cuda", w8a8=w8a8)
    P = W["prepared"]
    B, Tw = args.batch, args.window
    n_win = args.warmup + args.steps
    # one more window after the timed ones: compressed untimed, and the first
    # probe_steps of its decode run with the decode-step timing on
    # (step_timed_launches), so that measurement never touches the timed region
    probe_steps = PROBE_STEPS if step_probe else 0
    L = (n_win + (1 if step_probe else 0)) * Tw
    toks = synthetic.zipf_tokens(B, L, repeat_rate=0.05)
    inp = synthetic.model_inputs(toks)
    tok_d = torch.from_numpy(toks).to(dev)
    inp_d = torch.from_numpy(inp).to(dev)
    win_inp = [inp_d[:, w * Tw:(w + 1) * Tw].contiguous() for w in range(L // Tw)]
    win_tok = [tok_d[:, w * Tw:(w + 1) * Tw].contiguous() for w in range(L // Tw)]
    s = _lib.stream_ptr()
    PREC = 24

    # ------------------------------------------------------------- compress
    M = B * Tw
    ws, ws_bytes = cpp_path.workspace(W, M)
    x = torch.empty((M, P.C), dtype=torch.float16, device=dev)
    head_rows = min(M, args.head_rows)
    ld = cpp_path.logits_ld(P.V)
    logits = torch.empty((head_rows, ld), dtype=torch.float16, device=dev)
    # the encoder of window w overlaps the forward of window w+1 (its own
    # stream, double-buffered pairs), as in InferenceEngine.compress_tokens_batched
    main = torch.cuda.current_stream(dev)
    enc = torch.cuda.Stream(device=dev)
    pairs = [torch.empty((M, 2), dtype=torch.int32, device=dev) for _ in range(2)]
    fwd_done = [torch.cuda.Event() for _ in range(2)]
    enc_done = [torch.cuda.Event() for _ in range(2)]
    cap = 4 * L + 64
    out = torch.zeros(B * cap, dtype=torch.uint8, device=dev)
    base = (torch.arange(B, dtype=torch.int32, device=dev) * cap).contiguous()
    ac = torch.zeros((B, 4), dtype=torch.int64)
    ac[:, 1] = 0xFFFFFFFF
    ac = ac.to(torch.uint32).to(dev).contiguous()
    err = torch.zeros(1, dtype=torch.uint32, device=dev)
    cstate = State(P.n_layer, B, P.C, dev)

    def compress_window(w):
        buf = pairs[w % 2]
        if w >= 2:
            main.wait_event(enc_done[w % 2])
        _lib.call("kr_compress_window", P.ptr, win_inp[w].data_ptr(), win_tok[w].data_ptr(), B, Tw,
                  cstate.ptr, x.data_ptr(), ws.data_ptr(), ws_bytes, logits.data_ptr(), ld,
                  head_rows, buf.data_ptr(), PREC, s)
        fwd_done[w % 2].record(main)
        enc.wait_event(fwd_done[w % 2])
        _lib.call("kr_encode_pairs_batched", buf.data_ptr(), Tw, Tw, None, out.data_ptr(),
                  out.numel(), base.data_ptr(), ac.data_ptr(), B, PREC, err.data_ptr(),
                  enc.cuda_stream)
        enc_done[w % 2].record(enc)

    for w in range(args.warmup):
        compress_window(w)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for w in range(args.warmup, n_win):
        compress_window(w)
    torch.cuda.synchronize()
    t_c = time.perf_counter() - t0
    for w in range(n_win, L // Tw):
        compress_window(w)
    main.wait_stream(enc)
    _lib.call("kr_encode_finalize_batched", out.data_ptr(), out.numel(), base.data_ptr(),
              ac.data_ptr(), B, err.data_ptr(), s)
    torch.cuda.synchronize()
    assert int(err.item()) == 0, "coder output overflow"
    nbytes = ((ac[:, 3].to(torch.int64) + 7) // 8).to(torch.int32).contiguous()
    comp_bytes = int(nbytes.sum().item())

    # ----------------------------------------------------------- decompress
    del ws, x, logits, pairs, enc
    G = max(1, min(args.groups, B))
    dws_bytes = _lib.lib().kr_decode_workspace_bytes(B, G, P.C, P.F)
    dws = torch.empty(dws_bytes, dtype=torch.uint8, device=dev)
    dx = torch.empty((B, P.C), dtype=torch.float16, device=dev)
    dlogits = torch.empty((B, ld), dtype=torch.float16, device=dev)
    dac = torch.empty((B, 4), dtype=torch.uint32, device=dev)
    _lib.call("kr_decode_init_batched", out.data_ptr(), out.numel(), base.data_ptr(),
              nbytes.data_ptr(), dac.data_ptr(), B, s)
    dstate = State(P.n_layer, B, P.C, dev)
    syms = torch.zeros(B, dtype=torch.int32, device=dev)
    dtoks = torch.zeros((B, L), dtype=torch.int32, device=dev)
    cnt = torch.zeros(B, dtype=torch.int32, device=dev)

    def decode(n_steps, graph=True):
        _lib.call("kr_decode_run", P.ptr, B, dstate.ptr, syms.data_ptr(), dx.data_ptr(),
                  dws.data_ptr(), dws_bytes, dlogits.data_ptr(), ld, out.data_ptr(), out.numel(),
                  base.data_ptr(), nbytes.data_ptr(), dac.data_ptr(), dtoks.data_ptr(), L,
                  cnt.data_ptr(), None, PREC, n_steps, G, 1 if graph else 0, s)

    if args.warmup:
        decode(args.warmup * Tw)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    decode(args.steps * Tw)
    torch.cuda.synchronize()
    t_d = time.perf_counter() - t0
    in_step, used = step_timed_launches(decode, probe_steps) if step_probe else (None, 0)
    n_dec = n_win * Tw + used
    exact = bool(torch.equal(dtoks[:, :n_dec], tok_d[:, :n_dec]))
    if not exact:
        bad = (dtoks[:, :n_dec] != tok_d[:, :n_dec]).nonzero()
        raise SystemExit(f"round trip NOT byte-exact; first mismatch (stream, token) = {bad[0].tolist()}")
    ntok = args.steps * B * Tw
    return dict(t_c=t_c, t_d=t_d, ntok=ntok, comp_bytes=comp_bytes, total_tok=B * L, exact=exact,
                in_step=in_step)


# Decode-step phases (kr_phase_name) of the two roofline kernels, and the
# decode steps step_timed_launches runs after the timed region.
PHASE_FFN_RK, PHASE_FFN_V = 5, 6
PROBE_STEPS = 64


def step_timed_launches(decode, n_steps, calls=4):
    """In-step durations of the two roofline launches, from decode steps that
    continue the timed region's streams (the same kernels, state and
    bitstreams), with the channel-mix R + K launch (then the value-product
    launch) of every layer timed (kr_step_timing):
      * "events": eager steps, the timed launch through hipExtLaunchKernel
        with two HIP events that take its dispatch's start and end (the
        times a kernel trace reports). A bounded GPU sleep is queued first,
        so the host enqueues the steps ahead of the GPU and the launches run
        back to back, as a replayed graph runs them;
      * "span": graph-replayed steps exactly as timed, each launch's last
        wave end minus its first wave start on the 100 MHz steady counter
        (dispatch and teardown not included).
    Each call of n_steps / (4 * calls) steps yields one sample per layer,
    from its last step. Returns ({phase: {"events": [us...], "span": [us...],
    "span_eager": [us...]}}, steps decoded)."""
    import ctypes
    import torch
    from krunch_amd import _lib
    per_call = max(1, n_steps // (4 * calls))
    used = 0
    out = {}
    launch = (ctypes.c_double * 64)()
    span = (ctypes.c_double * 64)()
    got = ctypes.c_int(0)
    try:
        for phase in (PHASE_FFN_RK, PHASE_FFN_V):
            _lib.call("kr_step_timing", phase, None)
            r = {"events": [], "span": [], "span_eager": []}
            for graph in (True, False):
                for _ in range(calls):
                    if not graph:
                        torch.cuda._sleep(20_000_000)     # ~10 ms of GPU clock cycles
                    decode(per_call, graph)
                    used += per_call
                    _lib.call("kr_step_timing_read", launch, span, 64, ctypes.byref(got))
                    n = got.value
                    r["span" if graph else "span_eager"] += [span[i] for i in range(n)]
                    if not graph:
                        r["events"] += [launch[i] for i in range(n)]
            out[phase] = r
    finally:
        _lib.lib().kr_step_timing(-1, None)
    return out, used


def _pack(X):
    """Fragment-packed copy of a [R, K] fp16 device matrix (kr_pack_fragments)."""
    import torch
    from krunch_amd import _lib
    R, K = X.shape
    buf = torch.empty(_lib.lib().kr_fragment_bytes(R, K) // 2, dtype=torch.float16,
                      device=X.device)
    _lib.call("kr_pack_fragments", X.data_ptr(), K, R, K, buf.data_ptr(), _lib.stream_ptr())
    return buf


def _graph_launch_us(launches):
    """Average duration of one launch: a captured graph of n launches, timed
    with HIP events on the stream it replays on (host launch cost kept out)."""
    import torch
    n = launches(None)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            launches(stream)
    ms = []
    with torch.cuda.stream(stream):
        for _ in range(4):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            graph.replay()
            e1.record(stream)
            e1.synchronize()
            ms.append(e0.elapsed_time(e1))
    return min(ms[1:]) * 1000.0 / n


ROOFLINE_TRACE = os.path.join(ROOT, "profiles", "decode_step_B256_roofline.json")


def _roofline_entry(kernel, alg_bytes, us_isolated, step, phase_key, traffic_file, B):
    """`frac` from the launch's average duration inside the decode step of
    this run: its in-step wave span measured live (step_timed_launches: first
    wave start to last wave end on the steady counter, graph launches) plus
    the dispatch and teardown time a rocprofv3 kernel trace of this bench
    adds to the span (the trace's mean launch duration minus the profiled
    run's span, both recorded by `bench.py --hbm-table ... --roofline-json`
    in ROOFLINE_TRACE, at B = 256). `trace_matches_build` says whether this
    run's span is within 5% of the profiled run's. Without a live span the
    trace's mean duration is used; without the trace file, the isolated
    HIP-event figure, which is also reported beside it."""
    traffic = None
    tfile = os.path.join(ROOT, "profiles", traffic_file)
    if os.path.exists(tfile) and B == 256:
        with open(tfile) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    peak = MI355X_HBM_PEAK / 1e9
    gbs = lambda us: alg_bytes / (us * 1e-6) / 1e9
    mean = lambda v: sum(v) / len(v)
    trace = None
    if B == 256 and os.path.exists(ROOFLINE_TRACE):
        with open(ROOFLINE_TRACE) as f:
            trace = json.load(f)["phases"].get(phase_key)
    span = mean(step["span"]) if step and step.get("span") else None
    rel = os.path.relpath(ROOFLINE_TRACE, ROOT)
    if trace and span and trace.get("wave_span_us_same_run"):
        over = trace["in_step_mean_us"] - trace["wave_span_us_same_run"]
        us = span + over
        timing = ("in the decode step of this run: the launch's mean in-step wave span %.3f us "
                  "(graph launches, kr_step_timing) plus %.3f us of dispatch and teardown, the "
                  "mean launch duration %.3f us of a rocprofv3 kernel trace of this bench "
                  "minus that run's span %.3f us over its %d launches (%s)"
                  % (span, over, trace["in_step_mean_us"], trace["wave_span_us_same_run"],
                     trace["launches"], rel))
    elif trace:
        us = trace["in_step_mean_us"]
        timing = ("in the decode step: mean duration of the %d launches of this kernel inside "
                  "the decode steps of a rocprofv3 kernel trace of this bench (%s)"
                  % (trace["launches"], rel))
    else:
        us = us_isolated
        timing = "isolated: graph of 64 launches over 64 weight copies"
    out = {"kernel": kernel, "bound": "hbm", "achieved": round(gbs(us), 2), "peak": peak,
           "unit": "GB/s", "frac": round(gbs(us) / peak, 4), "traffic": traffic,
           "alg_bytes_per_launch": alg_bytes, "avg_launch_us": round(us, 3), "timing": timing,
           "isolated": {"avg_launch_us": round(us_isolated, 3),
                        "achieved": round(gbs(us_isolated), 2),
                        "frac": round(gbs(us_isolated) / peak, 4)}}
    if step:
        out["in_step_wave_span_us"] = {"graph": round(span, 3),
                                       "eager": round(mean(step["span_eager"]), 3),
                                       "eager_dispatch_events": round(mean(step["events"]), 3)}
    if trace:
        out["trace_in_step_mean_us"] = trace["in_step_mean_us"]
    if trace and span and trace.get("wave_span_us_same_run"):
        ref = trace["wave_span_us_same_run"]
        out["trace_matches_build"] = bool(abs(span / ref - 1) <= 0.05)
    return out


def dominant_kernel_roofline(weights16, B, in_step=None):
    """Live rooflines of the two heaviest kernels of the timed region, both
    stepped small-M products of the decode step (12 launches each per step),
    HBM-bound:
      * the channel-mix R and K products in one launch (M = B, K = 768,
        N = 768 sigmoid + 3072 relu^2; the top kernel by time), algorithmic
        bytes = W (768 + 3072) * 768 * 2 + A 2 * B * 768 * 2 + outputs
        B * (768 + 3072) * 2;
      * the channel-mix value product (M = B, K = 3072, N = 768, gated
        residual), W 3072 * 768 * 2 + A B * 3072 * 2 + residual, gate and
        output 3 * B * 768 * 2.
    `frac` comes from each launch's average duration inside this run's
    decode step: the live in-step wave span plus the dispatch and teardown a
    kernel trace of this bench adds to it (ROOFLINE_TRACE), with the isolated
    figure beside it (_roofline_entry). The
    isolated figure: the launch as the decode step launches it
    (fragment-packed operands), in a captured
    graph of 64 launches over 64 distinct weight copies (> the 256 MB
    memory-side cache, so weights come from HBM), timed with HIP events on
    the replay stream. `traffic` is the
    HBM bytes per launch from the committed counter summaries
    (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE on bench.py --kernel-probe,
    scaled by a 256 MiB copy calibration)."""
    import torch
    from krunch_amd import _lib

    dev = torch.device("cuda")
    C, F, M = 768, 3072, B
    g = torch.Generator(device="cpu").manual_seed(3)
    n = 64
    rnd = lambda *sh: (torch.rand(sh, generator=g) * 0.04 - 0.02).half().to(dev)

    # channel-mix R + K in one launch
    xr, xk = _pack(torch.rand((M, C), generator=g).half().to(dev)), \
        _pack(torch.rand((M, C), generator=g).half().to(dev))
    rf = torch.empty((M, C), dtype=torch.float16, device=dev)
    kf = torch.empty(_lib.lib().kr_fragment_bytes(M, F) // 2, dtype=torch.float16, device=dev)
    WR = [_pack(rnd(C, C)) for _ in range(n)]
    WK = [_pack(rnd(F, C)) for _ in range(n)]
    jobs = []
    for i in range(n):
        j = (_lib.KrPackedJob * 2)()
        j[0] = _lib.KrPackedJob(xr.data_ptr(), WR[i].data_ptr(), C, rf.data_ptr(), C, 2, None, None, 0)
        j[1] = _lib.KrPackedJob(xk.data_ptr(), WK[i].data_ptr(), F, kf.data_ptr(), F, 3, None, None, 1)
        jobs.append(j)

    def rk(stream):
        s = _lib.stream_ptr(stream)
        for i in range(n):
            _lib.call("kr_det_matmul_packed_multi", jobs[i], 2, M, C, s)
        return n

    us_rk = _graph_launch_us(rk)
    del WR, WK
    bytes_rk = (C + F) * C * 2 + 2 * M * C * 2 + M * (C + F) * 2

    # channel-mix value product
    A = _pack(torch.rand((M, F), generator=g).half().to(dev))
    res = torch.randn((M, C), generator=g).half().to(dev)
    gate = torch.rand((M, C), generator=g).half().to(dev)
    out = torch.empty((M, C), dtype=torch.float16, device=dev)
    WV = [_pack(rnd(C, F)) for _ in range(n)]

    def fv(stream):
        s = _lib.stream_ptr(stream)
        for i in range(n):
            _lib.call("kr_det_matmul_packed", A.data_ptr(), M, F, WV[i].data_ptr(), C,
                      out.data_ptr(), C, 5, res.data_ptr(), gate.data_ptr(), 0, s)
        return n

    us_v = _graph_launch_us(fv)
    del WV
    bytes_v = F * C * 2 + M * F * 2 + 3 * M * C * 2
    in_step = in_step or {}
    top = _roofline_entry(
        "gemm_panel_kernel (stepped channel-mix R + K products in one launch, "
        "M=%d K=768 N=768 sigmoid + 3072 relu^2, fragment-packed operands; top kernel by time)" % M,
        bytes_rk, us_rk, in_step.get(PHASE_FFN_RK), "rk", "gemm_panel_ffn_rk_B256_traffic.json", B)
    second = _roofline_entry(
        "gemm_panel_kernel (stepped channel-mix value product, M=%d K=3072 N=768, "
        "gated residual, fragment-packed operands; second by time)" % M,
        bytes_v, us_v, in_step.get(PHASE_FFN_V), "fv", "gemm_panel_ffn_value_B256_traffic.json", B)
    return top, second


# Algorithmic bytes of each phase of one stepped decode step (B streams,
# C = 768, F = 3072, V = 50277, fp16 activations and weights, fp32 WKV
# state): what each launch must read and write at least. Phase keys are
# assigned by step_phases.
def step_kernel_bytes(B, C=768, F=3072, V=50277):
    h = 2
    return [
        # layer 0's LN1-mix of the next step runs in the decode kernel below
        ("ln1", "LN1 + 3 mixes (layers 1-11)", 11, 6 * B * C * h + 5 * C * h),
        ("kvr", "K, V, R products + WKV", 12,
         3 * C * C * h + 3 * B * C * h + 2 * C * 4 + 2 * 3 * B * C * 4 + B * C * h),
        ("ow", "output projection (residual)", 12, C * C * h + 4 * B * C * h),
        ("ln2", "LN2 + 2 mixes", 12, 5 * B * C * h + 4 * C * h),
        ("rk", "channel-mix R + K products", 12,
         (C + F) * C * h + 2 * B * C * h + B * (C + F) * h),
        ("fv", "channel-mix value product (gated residual)", 12,
         C * F * h + B * F * h + 3 * B * C * h),
        ("lnout", "LN_out", 1, 2 * B * C * h + 2 * C * h),
        ("head", "head (M = B, N = V)", 1, V * C * h + B * C * h + B * V * h),
        ("cdf", "softmax -> CDF -> range decode + layer 0's LN1 + 3 mixes", 1,
         B * V * h + 6 * B * C * h + 5 * C * h),
    ]


def step_phases(names):
    """Phase key of each launch of a fp16 stepped decode, from the kernel
    names in launch order (None for launches outside the decode step). The
    tile shapes in the template arguments change with B, so the stepped
    products are told apart by the launch before them: the output
    projection follows the K/V/R+WKV launch, the channel-mix R + K product
    follows LN2, the value product follows R + K."""
    out, prev = [], None
    for n in names:
        if "ln_mix_kernel<3, 3, false>" in n:
            ph = "ln1"
        elif "ln_mix_kernel<3, 2, false>" in n:
            ph = "ln2"
        elif "ln_mix_kernel<3, 0, false>" in n:
            ph = "lnout"
        elif "kvr_wkv_kernel<" in n and ", false>" in n:
            ph = "kvr"
        elif "gemm_panel_kernel<" in n and "false, false>" in n:
            ph = {"kvr": "ow", "ln2": "rk", "rk": "fv"}.get(prev)
        elif "gemm_head_small_kernel" in n:
            ph = "head"
        elif "row_cdf_kernel<0, 4>" in n:
            ph = "cdf"
        else:
            ph = None
        out.append(ph)
        prev = ph
    return out


def hbm_table(csv_path, B, roofline_json=None, bench_line=None):
    """Per-phase HBM fraction of one decode step from a rocprofv3 kernel
    trace of the bench (markdown on stdout): each phase's algorithmic bytes
    per launch over its median duration in the trace's decode steps (the
    most frequent kernel and grid of that phase), against 8 TB/s."""
    import csv
    import gzip
    opener = gzip.open if csv_path.endswith(".gz") else open
    rows = []
    with opener(csv_path, "rt") as f:
        for r in csv.DictReader(f):
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"],
                         int(r["Grid_Size_X"])))
    rows.sort()
    durs = {}
    for (t0, t1, name, grid), ph in zip(rows, step_phases([r[2] for r in rows])):
        if ph is not None:
            durs.setdefault(ph, {}).setdefault((name, grid), []).append((t1 - t0) / 1000.0)
    print(f"| kernel | phase | launches / step | avg us | algorithmic MB / launch | GB/s | "
          f"fraction of 8 TB/s | us / step |")
    print("|---|---|---|---|---|---|---|---|")
    total = 0.0
    for key, phase, per_step, nbytes in step_kernel_bytes(B):
        if key not in durs:
            continue
        kn = max(durs[key], key=lambda k: len(durs[key][k]))
        d = sorted(durs[key][kn])
        us = d[len(d) // 2]                                  # median launch
        gbs = nbytes / (us * 1e-6) / 1e9
        total += us * per_step
        name = kn[0].replace("(anonymous namespace)::", "").replace("void ", "").split("(")[0]
        print(f"| `{name}` | {phase} | {per_step} | {us:.2f} | {nbytes / 1e6:.2f} | {gbs:.0f} | "
              f"{gbs / (MI355X_HBM_PEAK / 1e9):.3f} | {us * per_step:.1f} |")
    print(f"\nSum over the step: {total:.1f} us (median launches; the profiler adds ~1 us per "
          f"kernel).")
    if roofline_json:
        # in-step durations (every launch of the phase inside the trace's
        # decode steps) of the two roofline kernels
        out = {"trace": os.path.basename(csv_path), "batch": B, "phases": {}}
        spans = {}
        if bench_line:
            with open(bench_line) as f:
                line = json.loads(f.read().strip().splitlines()[-1])
            for key, name in (("rk", "roofline"), ("fv", "roofline_second_kernel")):
                span = line.get(name, {}).get("in_step_wave_span_us")
                if span:
                    spans[key] = span["graph"]
        for key in ("rk", "fv"):
            if key not in durs:
                continue
            kn = max(durs[key], key=lambda k: len(durs[key][k]))
            # the timed decode's steps: the last PROBE_STEPS steps of the trace
            # are step_timed_launches' (12 launches each), not the timed region's
            d = sorted(durs[key][kn][:-12 * PROBE_STEPS])
            name = kn[0].replace("(anonymous namespace)::", "").replace("void ", "").split("(")[0]
            out["phases"][key] = {
                "kernel": name, "grid": kn[1], "launches": len(d),
                "in_step_mean_us": round(sum(d) / len(d), 4), "in_step_median_us": d[len(d) // 2],
                "wave_span_us_same_run": spans.get(key)}
        with open(roofline_json, "w") as f:
            json.dump(out, f, indent=1)


def cpu_baseline(args):
    """BASELINE config 1 on the host cores: the oracle codec (oracle/codec.py:
    fp32 row-wise torch forward, numpy CDF, C range coder) on the 169M-shaped
    fp32 model (seed 0), one chunk of `window` Zipf(1.1) tokens: packed
    compress, then stepped decompress of the first `cpu_decode_steps` tokens
    (all of them by default), checked byte-exact."""
    import numpy as np
    import torch
    from krunch_amd import synthetic
    from oracle import codec

    torch.set_num_threads(os.cpu_count() or 1)
    w = synthetic.make_weights(dtype=torch.float32)
    T = args.window
    toks = synthetic.zipf_tokens(1, T, repeat_rate=0.05)[0]
    t0 = time.perf_counter()
    bits, c_split = codec.compress(w, toks)
    t_c = time.perf_counter() - t0
    n_dec = min(args.cpu_decode_steps, T)
    t0 = time.perf_counter()
    got, d_split = codec.decompress(w, bits, n_dec)
    t_d = time.perf_counter() - t0
    c_tok_s, d_tok_s = T / t_c, n_dec / t_d
    rt = 1.0 / (1.0 / c_tok_s + 1.0 / d_tok_s)
    cpu_model = platform.processor() or ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(rt * BYTES_PER_TOKEN / 1024, 3), "unit": "KB/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"BASELINE config 1: 1 chunk, packed compress of {T} tokens + stepped "
                      f"decompress of {n_dec} (fp32 row-wise torch forward with a fixed-order "
                      f"C GEMM, numpy CDF, C range coder)",
            "compress_tok_s": round(c_tok_s, 1), "decompress_tok_s": round(d_tok_s, 2),
            "compress_split_s": {k: round(v, 3) for k, v in c_split.items()},
            "decompress_split_s": {k: round(v, 3) for k, v in d_split.items()},
            "cpu_packed_stepped_bit_identical": bool(np.array_equal(got, toks[:n_dec])),
            "cpu_model": cpu_model}


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one MI355X only: every chunk is independent, so the path "
              "would shard as one process per GPU over chunk ranges, and this build runs one "
              "GPU. Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    if args.hbm_table:
        hbm_table(args.hbm_table, args.batch, args.roofline_json, args.bench_line)
        return
    import torch
    from krunch_amd import synthetic
    weights16 = synthetic.make_weights()
    if args.kernel_probe:
        kernel_probe(weights16, args.batch, args.head_rows)
        return
    r = gpu_bench(args, weights16, step_probe=True)
    t = r["t_c"] + r["t_d"]
    kb = r["ntok"] * BYTES_PER_TOKEN / 1024
    res = {
        "metric": "compress & decompress input KB/s per MI355X (169M shape, B=256); % of peak",
        "value": round(kb / t, 2),
        "unit": "KB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1000 * t / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (random-init RWKV-4-169M-shaped weights, Zipf(1.1) tokens, 5% repeats)",
        "config": {"workload": "config5-window: B=256 chunks x 1024-token window, packed compress "
                               "+ 1024-step stepped decompress, state carried across windows",
                   "batch_chunks": args.batch, "window_tokens": args.window,
                   "decode_groups": args.groups},
        "compress_kbps": round(kb / r["t_c"], 2),
        "decompress_kbps": round(kb / r["t_d"], 2),
        "compress_tok_s": round(r["ntok"] / r["t_c"], 1),
        "decompress_tok_s": round(r["ntok"] / r["t_d"], 1),
        "compress_pflops": round(r["ntok"] * FLOP_PER_TOKEN / r["t_c"] / 1e15, 4),
        "bits_per_token": round(8 * r["comp_bytes"] / r["total_tok"], 4),
        "roundtrip_exact": r["exact"],
    }
    if not args.no_w8a8:
        # the w8a8 codec (int8 MFMA layer products, fp16 head)
        # on the same windows; its bits/token beside the fp16 codec's.
        q = gpu_bench(args, weights16, w8a8=True)
        qkb = q["ntok"] * BYTES_PER_TOKEN / 1024
        bpt16 = 8 * r["comp_bytes"] / r["total_tok"]
        bpt8 = 8 * q["comp_bytes"] / q["total_tok"]
        res["w8a8"] = {
            "compress_kbps": round(qkb / q["t_c"], 2),
            "compress_tok_s": round(q["ntok"] / q["t_c"], 1),
            "decompress_kbps": round(qkb / q["t_d"], 2),
            "roundtrip_kbps": round(qkb / (q["t_c"] + q["t_d"]), 2),
            "bits_per_token": round(bpt8, 6),
            "bits_per_token_fp16": round(bpt16, 6),
            "bits_delta_pct_vs_fp16": round(100 * (bpt8 - bpt16) / bpt16, 5),
            "roundtrip_exact": q["exact"],
            "compress_int8_fp16_tops": round(q["ntok"] * FLOP_PER_TOKEN / q["t_c"] / 1e12, 1),
        }
    res["roofline"], res["roofline_second_kernel"] = dominant_kernel_roofline(
        weights16, args.batch, r["in_step"])
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(args)
    print(json.dumps(res))


if __name__ == "__main__":
    main()
