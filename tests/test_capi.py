"""CPU-side checks of the C ABI: the library loads without a GPU, exports
every function include/krunch_hip.h declares, and the ctypes table binds
exactly those; size queries work without a device."""
import os
import re

from krunch_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                      "include", "krunch_hip.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kr_[a-z0-9_]+)\s*\(", text)))


def test_header_symbols_exported_and_bound():
    names = declared()
    assert len(names) >= 25
    L = _lib.lib()
    for n in names:
        assert hasattr(L, n), f"{n} not exported"
    assert sorted(_lib.exported_symbols()) == names


def test_size_queries_without_device():
    L = _lib.lib()
    assert L.kr_state_bytes(12, 1, 768) == 147456          # 12 layers x 12288 B/stream
    assert L.kr_forward_workspace_bytes(1024, 768, 3072) >= 1024 * 768 * (8 * 2 + 2 * 4) + 1024 * 3072 * 2
    assert L.kr_abi_version() == 2


def test_argument_errors_are_reported():
    rc = _lib.lib().kr_probs_to_cdf(None, 1, 10, 10, None, 24, None)
    assert rc != 0
    assert b"null" in _lib.lib().kr_last_error()


def test_step_timing_argument_checks():
    """kr_step_timing takes only the panel-product phases (3, 5, 6) or -1,
    and reading before any timed step is an error (no device needed)."""
    import ctypes
    L = _lib.lib()
    prev = ctypes.c_int(7)
    assert L.kr_step_timing(2, None) != 0
    assert b"phase 2" in L.kr_last_error()
    assert L.kr_step_timing(-1, ctypes.byref(prev)) == 0 and prev.value == -1
    us = (ctypes.c_double * 4)()
    span = (ctypes.c_double * 4)()
    got = ctypes.c_int(0)
    assert L.kr_step_timing_read(us, span, 4, ctypes.byref(got)) != 0
    assert b"no timed step" in L.kr_last_error()


def test_roofline_json_from_a_trace(tmp_path):
    """bench.py --hbm-table ... --roofline-json: in-step mean and median of
    the two roofline launches from a kernel-trace CSV, the launches of the
    probe steps after the timed region left out, the profiled run's wave
    spans recorded beside them."""
    import csv
    import json
    import bench
    names = {"ln2": "void (anonymous namespace)::ln_mix_kernel<3, 2, false>(x)",
             "rk": "void (anonymous namespace)::gemm_panel_kernel<4, 2, true, 256, false, false>(x)",
             "fv": "void (anonymous namespace)::gemm_panel_kernel<1, 3, true, 768, false, false>(x)"}
    steps = 10 + bench.PROBE_STEPS
    rows, t = [], 0
    for s in range(steps):
        for layer in range(12):
            for key, dur in (("ln2", 4000), ("rk", 8000 + (500 if s >= 10 else 0)), ("fv", 7000)):
                rows.append({"Kernel_Name": names[key], "Start_Timestamp": t,
                             "End_Timestamp": t + dur, "Grid_Size_X": 1024})
                t += dur + 100
    trace = tmp_path / "trace.csv"
    with open(trace, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    line = tmp_path / "line.json"
    line.write_text(json.dumps({"roofline": {"in_step_wave_span_us": {"graph": 6.5}},
                                "roofline_second_kernel": {"in_step_wave_span_us": {"graph": 5.5}}}))
    out = tmp_path / "roofline.json"
    bench.hbm_table(str(trace), 256, str(out), str(line))
    ph = json.loads(out.read_text())["phases"]
    assert ph["rk"]["launches"] == 10 * 12 and ph["rk"]["in_step_mean_us"] == 8.0
    assert ph["fv"]["in_step_median_us"] == 7.0
    assert ph["rk"]["wave_span_us_same_run"] == 6.5 and ph["fv"]["wave_span_us_same_run"] == 5.5
