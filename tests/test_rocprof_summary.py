"""The rocprofv3 CSV digests behind profiles/: per-run kernel time, copy-kernel
scaled HBM bytes, and MFMA work / utilisation from counters, on small
hand-made CSVs whose answers are known."""

from __future__ import annotations

import csv
from types import SimpleNamespace

import pytest

from spinnv2_amd import rocprof_summary as rs

PMC_COLS = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]


def _write(path, cols, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=cols)
        w.writeheader()
        for r in rows:
            w.writerow(dict(zip(cols, r)))
    return str(path)


def _result(text: str, name: str) -> float:
    for line in text.splitlines():
        if line.startswith(f"result {name} ="):
            return float(line.split("=")[1])
    raise KeyError(name)


def test_stats_per_run(tmp_path):
    p = _write(tmp_path / "s.csv", ["Name", "Calls", "TotalDurationNs", "AverageNs"],
               [["void spk::kern::conv_igemm_f32<64, 64, 16, 2, 2>(spk::kern::IgemmArgs)", 20, 2_000_000, 100_000],
                ["splitk_epilogue<4>", 10, 500_000, 50_000]])
    out = rs.stats(p, runs=10)
    line = [ln for ln in out.splitlines() if ln.startswith("conv_igemm_f32<64, 64, 16, 2, 2>")][0].split()
    # 2 calls per run, 100 us average, 0.2 ms per run, 80% of the total
    assert line[-4:] == ["2.0", "100.00", "0.200", "80.0%"]
    assert out.splitlines()[-1].split()[-1] == "0.250"


def test_traffic_copy_scaled(tmp_path):
    mib = 1 << 20
    # copy kernel of 4 MiB: FETCH_SIZE reads half of it (2048 KiB), WRITE_SIZE all (4096 KiB)
    cf = _write(tmp_path / "cf.csv", PMC_COLS, [[1, "copy_kernel(float*)", "FETCH_SIZE", 2048, 0, 1000]])
    cw = _write(tmp_path / "cw.csv", PMC_COLS, [[1, "copy_kernel(float*)", "WRITE_SIZE", 4096, 0, 1000]])
    # one conv dispatch per run, two runs: 1000 KiB fetched (x2 -> 2000 KiB), 500 KiB written, 1 us each
    f = _write(tmp_path / "f.csv", PMC_COLS, [[1, "conv_igemm_f32<64>", "FETCH_SIZE", 1000, 0, 1000],
                                             [2, "conv_igemm_f32<64>", "FETCH_SIZE", 1000, 5000, 6000]])
    w = _write(tmp_path / "w.csv", PMC_COLS, [[1, "conv_igemm_f32<64>", "WRITE_SIZE", 500, 0, 1000],
                                             [2, "conv_igemm_f32<64>", "WRITE_SIZE", 500, 5000, 6000]])
    args = SimpleNamespace(fetch=f, write=w, copy_fetch=cf, copy_write=cw, copy_bytes=4 * mib, runs=2,
                           match="conv_igemm")
    out = rs.traffic(args)
    assert _result(out, "conv_igemm_read_bytes_per_step") == pytest.approx(2000 * 1024)
    assert _result(out, "conv_igemm_write_bytes_per_step") == pytest.approx(500 * 1024)
    assert _result(out, "conv_hbm_bytes_per_step") == pytest.approx(2500 * 1024)
    # 2.56 MB in 1 us per run
    row = [ln for ln in out.splitlines() if ln.startswith("conv_igemm_f32<64>")][0].split()
    assert float(row[-1]) == pytest.approx(2500 * 1024 / 1000, rel=1e-3)


def test_traffic_group_include_exclude(tmp_path):
    """--group totals the --include kernels minus --exclude, under its own label."""
    mib = 1 << 20
    cf = _write(tmp_path / "cf.csv", PMC_COLS, [[1, "copy_kernel(float*)", "FETCH_SIZE", 2048, 0, 1000]])
    cw = _write(tmp_path / "cw.csv", PMC_COLS, [[1, "copy_kernel(float*)", "WRITE_SIZE", 4096, 0, 1000]])
    names = ["void spk::kern::conv_igemm_i8<64>(A)", "spk::kern::quantize_pad_nhwc_narrow(float const*)",
             "void spk::kern::conv_igemm_f32<64, 64, 16, 2, 2, 1>(B)"]
    f = _write(tmp_path / "f.csv", PMC_COLS, [[i + 1, n, "FETCH_SIZE", 100 * (i + 1), 0, 1000]
                                             for i, n in enumerate(names)])
    w = _write(tmp_path / "w.csv", PMC_COLS, [[i + 1, n, "WRITE_SIZE", 10 * (i + 1), 0, 1000]
                                             for i, n in enumerate(names)])
    args = SimpleNamespace(fetch=f, write=w, copy_fetch=cf, copy_write=cw, copy_bytes=4 * mib, runs=1,
                           match="conv_igemm", group="q8", include=["conv_igemm", "quantize_pad"],
                           exclude=["conv_igemm_f32"])
    out = rs.traffic(args)
    # members: the int8 conv (100 KiB x2 read, 10 KiB written) and the quantize pass (200 x2, 20)
    assert _result(out, "q8_read_bytes_per_step") == pytest.approx(600 * 1024)
    assert _result(out, "q8_write_bytes_per_step") == pytest.approx(30 * 1024)
    assert _result(out, "conv_hbm_bytes_per_step") == pytest.approx(630 * 1024)
    assert _result(out, "conv_dispatches_per_step") == 2


def test_mfma_work_and_busy(tmp_path):
    rows = []
    # two dispatches of 100 us; each counts 1e6 MOPS (x512 FLOP); GUI_ACTIVE sums 8 XCDs
    for d, t0 in ((1, 0), (2, 1_000_000)):
        rows += [[d, "conv_igemm_f32<x>", "SQ_INSTS_VALU_MFMA_MOPS_F32", 1e6, t0, t0 + 100_000],
                 [d, "conv_igemm_f32<x>", "GRBM_GUI_ACTIVE", 8 * 240_000, t0, t0 + 100_000],
                 [d, "conv_igemm_f32<x>", "SQ_VALU_MFMA_BUSY_CYCLES", 0.5 * 240_000 * 256 * 4, t0, t0 + 100_000]]
    p = _write(tmp_path / "m.csv", PMC_COLS, rows)
    out = rs.mfma(SimpleNamespace(csv=p, runs=2, match="conv_igemm", cus=256, xcds=8, peak=157.3,
                                  mops="SQ_INSTS_VALU_MFMA_MOPS_F32"))
    assert _result(out, "conv_igemm_mfma_flop_per_run") == pytest.approx(512e6)
    # 512e6 FLOP per 100 us = 5.12 TFLOP/s
    assert _result(out, "conv_igemm_mfma_tflops") == pytest.approx(5.12)
    assert _result(out, "conv_igemm_mfma_busy_frac") == pytest.approx(0.5)


def test_mfma_int8_counter(tmp_path):
    # int8 work: 2e6 units of 512 ops in one 200 us dispatch = 5.12 TOP/s of a 5000 TOP/s peak
    rows = [[1, "conv_igemm_i8<128>", "SQ_INSTS_VALU_MFMA_MOPS_I8", 2e6, 0, 200_000],
            [1, "conv_igemm_i8<128>", "GRBM_GUI_ACTIVE", 8 * 480_000, 0, 200_000],
            [1, "conv_igemm_i8<128>", "SQ_VALU_MFMA_BUSY_CYCLES", 0.25 * 480_000 * 256 * 4, 0, 200_000],
            [2, "quantize_pad_nhwc", "SQ_INSTS_VALU_MFMA_MOPS_I8", 0, 300_000, 310_000]]
    p = _write(tmp_path / "m8.csv", PMC_COLS, rows)
    out = rs.mfma(SimpleNamespace(csv=p, runs=1, match="conv_igemm_i8", cus=256, xcds=8, peak=5000.0,
                                  mops="SQ_INSTS_VALU_MFMA_MOPS_I8"))
    assert _result(out, "conv_igemm_i8_mfma_flop_per_run") == pytest.approx(1.024e9)
    assert _result(out, "conv_igemm_i8_mfma_tflops") == pytest.approx(5.12)
    assert _result(out, "conv_igemm_i8_mfma_frac_of_peak") == pytest.approx(5.12 / 5000, abs=1e-4)
    assert _result(out, "conv_igemm_i8_mfma_busy_frac") == pytest.approx(0.25)


def test_stats_group_include_exclude(tmp_path):
    p = _write(tmp_path / "s.csv", ["Name", "Calls", "TotalDurationNs", "AverageNs"],
               [["void spk::kern::conv_igemm_f32<64, 64, 16, 2, 2, 0>(spk::kern::IgemmArgs)", 20, 2_000_000, 100_000],
                ["void spk::kern::conv_igemm_f32<64, 64, 16, 2, 2, 1>(spk::kern::IgemmArgs)", 10, 100_000, 10_000],
                ["splitk_epilogue<4>", 10, 500_000, 50_000],
                ["maxpool3s2_x4", 10, 300_000, 30_000]])
    out = rs.stats(p, runs=10, group="conv_kernels", include=["conv_igemm_f32", "splitk_epilogue"],
                   exclude=["conv_igemm_f32<64, 64, 16, 2, 2, 1>"])
    # 2.0 ms + 0.5 ms over 10 runs; the KVEC Gemm and the pool are not members
    assert _result(out, "conv_kernels_ms_per_run") == pytest.approx(0.25)
    assert _result(out, "conv_kernels_calls_per_run") == pytest.approx(3.0)


def test_launches_by_grid(tmp_path):
    cols = ["Kernel_Name", "Start_Timestamp", "End_Timestamp", "Workgroup_Size_X", "Workgroup_Size_Y",
            "Workgroup_Size_Z", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z"]
    k = "void spk::kern::conv_igemm_i8x<128, 64, 64, 2, 2, 0>(spk::kern::I8Args)"
    # two runs: a 6272-workgroup launch (90 and 100 us) and two 1568-workgroup
    # launches per run (20, 22, 24, 30 us); another kernel left out by --match
    rows = [[k, 0, 90_000, 256, 1, 1, 6272 * 256, 1, 1], [k, 0, 100_000, 256, 1, 1, 6272 * 256, 1, 1],
            [k, 0, 20_000, 256, 1, 1, 1568 * 256, 1, 1], [k, 0, 22_000, 256, 1, 1, 1568 * 256, 1, 1],
            [k, 0, 24_000, 256, 1, 1, 1568 * 256, 1, 1], [k, 0, 30_000, 256, 1, 1, 1568 * 256, 1, 1],
            ["copy_kernel(float*)", 0, 5_000, 256, 1, 1, 256, 1, 1]]
    out = rs.launches(_write(tmp_path / "t.csv", cols, rows), runs=2, match="conv_igemm_i8")
    lines = out.splitlines()
    assert len(lines) == 3 and "copy_kernel" not in out
    # one dispatch per run, median of 90 and 100 us, 190 us over two runs
    assert lines[1].split()[-5:] == ["6272x1x1", "256", "1.0", "95.00", "0.095"]
    small = lines[2].split()
    # four dispatches over two runs: 2 per run, median of 20, 22, 24, 30 is 23, 96 us / 2 runs
    assert small[-5:] == ["1568x1x1", "256", "2.0", "23.00", "0.048"]
