"""bench.py's decode-step table: phases told apart by launch order (CPU only)."""
import csv

import bench

NS = "void (anonymous namespace)::"


def _step(tm_rk, ns_rk, ns_v):
    """Kernel names of one fp16 decode step, in launch order."""
    layer = [
        NS + "ln_mix_kernel<3, 3, false>((anonymous namespace)::LnMixArgs)",
        NS + "kvr_wkv_kernel<3, 2, 1, false>((anonymous namespace)::KvrWkvArgs)",
        NS + "gemm_panel_kernel<1, 2, true, 256, false, false>(kr_gemm_multi)",
        NS + "ln_mix_kernel<3, 2, false>((anonymous namespace)::LnMixArgs)",
        NS + f"gemm_panel_kernel<{tm_rk}, {ns_rk}, true, 256, false, false>(kr_gemm_multi)",
        NS + f"gemm_panel_kernel<1, {ns_v}, true, 768, false, false>(kr_gemm_multi)",
    ]
    # layer 0's LN1-mix runs in the previous step's decode kernel
    return layer[1:] + layer * 11 + [
        NS + "ln_mix_kernel<3, 0, false>((anonymous namespace)::LnMixArgs)",
        "_ZN12_GLOBAL__N_122gemm_head_small_kernelILi24ELi4EEEvPKDF16_S2_PDF16_xiii",
        NS + "row_cdf_kernel<0, 4>(void const*, long long, int)",
    ]


def test_step_phases_by_launch_order():
    # the output projection and the R + K product have the same template
    # arguments here; only their place in the step separates them
    names = _step(1, 2, 2)
    ph = bench.step_phases(names)
    assert ph[:11] == ["kvr", "ow", "ln2", "rk", "fv", "ln1", "kvr", "ow", "ln2", "rk", "fv"]
    assert ph[11:17] == ph[5:11]
    assert ph[-3:] == ["lnout", "head", "cdf"]
    keys = [k for k, *_ in bench.step_kernel_bytes(128)]
    assert set(ph) == set(keys)


def test_step_phases_skip_compress_and_int8():
    names = [NS + "gemm_big_kernel<1, false>(kr_gemm_args, int)",
             NS + "row_cdf_kernel<0, 3>(void const*, long long, int)",
             NS + "kvr_wkv_kernel<3, 2, 2, true>((anonymous namespace)::KvrWkvArgs)",
             NS + "gemm_panel_kernel<2, 2, true, 256, true, true>(kr_gemm_multi)"]
    assert bench.step_phases(names) == [None] * 4


def test_hbm_table_sums_the_step(tmp_path, capsys):
    names = _step(4, 2, 2) * 3
    path = tmp_path / "trace.csv"
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Kernel_Name", "Start_Timestamp", "End_Timestamp", "Grid_Size_X"])
        t = 0
        for n in names:
            w.writerow([n, t, t + 2000, 256])          # every launch 2 us
            t += 3000
    bench.hbm_table(str(path), 256)
    out = capsys.readouterr().out
    assert out.count("\n| `") == 9
    per_step = sum(n for _, _, n, _ in bench.step_kernel_bytes(256))
    assert f"Sum over the step: {2.0 * per_step:.1f} us" in out
