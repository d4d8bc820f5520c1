"""The rocprofv3 summaries: dispatch matching, counter calibration and per-step durations on
synthetic rocprofv3 CSV output (no GPU)."""
import csv
import json

import pytest

from aexrt_amd import profiling


def _counters(d, rows):
    d.mkdir(parents=True)
    with open(d / "run_counter_collection.csv", "w", newline="") as f:
        w = csv.DictWriter(f, ["Dispatch_Id", "Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for i, (name, grid, counter, value) in enumerate(rows):
            # two rows per dispatch (counter instances) are summed by the loader
            w.writerow(dict(Dispatch_Id=i, Kernel_Name=name, Grid_Size=grid, Counter_Name=counter, Counter_Value=value / 2))
            w.writerow(dict(Dispatch_Id=i, Kernel_Name=name, Grid_Size=grid, Counter_Name=counter, Counter_Value=value / 2))


def _trace(d, rows):
    d.mkdir(parents=True)
    with open(d / "run_kernel_trace.csv", "w", newline="") as f:
        w = csv.DictWriter(f, ["Kernel_Name", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z", "Start_Timestamp",
                               "End_Timestamp"])
        w.writeheader()
        for name, grid, t0, t1 in rows:
            w.writerow(dict(Kernel_Name=name, Grid_Size_X=grid, Grid_Size_Y=1, Grid_Size_Z=1, Start_Timestamp=t0,
                            End_Timestamp=t1))


def test_traffic_table_calibrates_and_matches_steps(tmp_path):
    cal = 1 << 20
    log = tmp_path / "fetch.log"
    log.write_text("noise\n" + json.dumps({"pmc_pass": {"steps": ["cmd#0 A", "cmd#1 B"], "calibration_bytes": cal}}))
    # FETCH_SIZE reads half the calibration bytes (scale 2), WRITE_SIZE all of them (scale 1)
    _counters(tmp_path / "f", [("warm", 64, "FETCH_SIZE", 5.0), ("void neg_kernel(float*)", 64, "FETCH_SIZE", cal / 2048),
                               ("void aexrt::k1(P)", 128, "FETCH_SIZE", 1000.0), ("void aexrt::k2(P)", 256, "FETCH_SIZE", 10.0)])
    _counters(tmp_path / "w", [("warm", 64, "WRITE_SIZE", 1.0), ("void neg_kernel(float*)", 64, "WRITE_SIZE", cal / 1024),
                               ("void aexrt::k1(P)", 128, "WRITE_SIZE", 500.0), ("void aexrt::k2(P)", 256, "WRITE_SIZE", 20.0)])
    _trace(tmp_path / "t", [("void aexrt::k1(P)", 128, 0, 4000), ("void aexrt::k1(P)", 128, 5000, 7000),
                            ("void aexrt::k2(P)", 256, 8000, 9000)])
    t = profiling.traffic_table(str(tmp_path / "f"), str(tmp_path / "w"), str(log), str(tmp_path / "t"))
    assert t[0]["f_scale"] == pytest.approx(2.0) and t[0]["w_scale"] == pytest.approx(1.0)
    r0, r1 = t[1], t[2]
    assert r0["step"] == "cmd#0 A" and r0["kernel"] == "k1" and r0["grid"] == 128
    assert r0["read_mb"] == pytest.approx(1000 * 1024 * 2 / 1e6) and r0["write_mb"] == pytest.approx(500 * 1024 / 1e6)
    assert r0["trace_us_mean"] == pytest.approx(3.0) and r0["trace_n"] == 2
    assert r1["trace_us_mean"] == pytest.approx(1.0)


def test_traffic_table_rejects_mismatched_runs(tmp_path):
    log = tmp_path / "p.log"
    log.write_text(json.dumps({"pmc_pass": {"steps": ["cmd#0 A"], "calibration_bytes": 1024}}))
    _counters(tmp_path / "f", [("neg", 1, "FETCH_SIZE", 1.0), ("k1", 1, "FETCH_SIZE", 1.0)])
    _counters(tmp_path / "w", [("neg", 1, "WRITE_SIZE", 1.0), ("k2", 1, "WRITE_SIZE", 1.0)])
    with pytest.raises(ValueError, match="dispatch order"):
        profiling.traffic_table(str(tmp_path / "f"), str(tmp_path / "w"), str(log))


def test_kernel_stats_takes_the_last_replays(tmp_path):
    log = tmp_path / "t.log"
    log.write_text(json.dumps({"trace_pass": {"batch": 64, "replays": 2, "steps": ["s0", "s1"]}}))
    # an earlier profiled pass, then two replays of two steps
    _trace(tmp_path / "t", [("void aexrt::a(P)", 1, 0, 100000), ("void aexrt::a(P)", 1, 200000, 203000),
                            ("void aexrt::b(P)", 1, 203500, 205500), ("void aexrt::a(P)", 1, 300000, 305000),
                            ("void aexrt::b(P)", 1, 305000, 306000)])
    st = profiling.kernel_stats(str(tmp_path / "t"), str(log))
    s0, s1 = st["per_step"]
    assert (s0["step"], s0["kernel"], s0["mean_us"], s0["min_us"]) == ("s0", "a", 4.0, 3.0)
    assert (s1["mean_us"], s1["min_us"]) == (1.5, 1.0)
    assert st["wall_us"] == pytest.approx((5.5 + 6.0) / 2)
    assert st["busy_us"] == pytest.approx(5.5)
    assert st["instances"]["a"] == dict(n=1, us=4.0)


def test_mfma_table_counts_ops(tmp_path):
    log = tmp_path / "m.log"
    log.write_text(json.dumps({"pmc_pass": {"steps": ["cmd#0 A"], "calibration_bytes": 1024}}))
    _counters(tmp_path / "m", [("neg", 1, "SQ_INSTS_VALU_MFMA_MOPS_I8", 0.0), ("k", 1, "SQ_INSTS_VALU_MFMA_MOPS_I8", 4.0)])
    (row,) = profiling.mfma_table(str(tmp_path / "m"), str(log))
    assert row["ops_i8"] == 4 * 512 and row["ops_f16"] == 0


def test_insts_table_per_wave_and_valu_time(tmp_path):
    log = tmp_path / "i.log"
    log.write_text(json.dumps({"pmc_pass": {"steps": ["cmd#3 CONV_SILU x alg=int8_mfma_1x1 kernel=k"],
                                            "calibration_bytes": 1024}}))
    rows = [("neg", 1, "SQ_WAVES", 4.0), ("k", 1, "SQ_WAVES", 8.0), ("k", 1, "SQ_INSTS_VALU", 800.0),
            ("k", 1, "SQ_INSTS_LDS", 80.0)]
    # one dispatch per kernel: the loader sums a dispatch's rows, so give each row its own dispatch id
    d = tmp_path / "i"
    d.mkdir(parents=True)
    with open(d / "run_counter_collection.csv", "w", newline="") as f:
        w = csv.DictWriter(f, ["Dispatch_Id", "Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for name, grid, counter, value in rows:
            w.writerow(dict(Dispatch_Id=0 if name == "neg" else 1, Kernel_Name=name, Grid_Size=grid,
                            Counter_Name=counter, Counter_Value=value))
    (row,) = profiling.insts_table(str(d), str(log))
    assert row["waves"] == 8 and row["valu"] == 100 and row["lds"] == 10
    # 800 VALU instructions x 4 cycles over 1024 SIMDs at 2.4 GHz
    assert row["valu_us"] == pytest.approx(800 * 4 / 1024 / 2.4e9 * 1e6)
