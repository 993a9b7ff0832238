"""CPU: bench.py's host-side profile handling.

The headline's roofline.frac divides the fabric bytes in the committed PMC
summaries (their BYTES lines) by the kernels' measured times, so a summary
that lost its BYTES lines, or a parser that misreads them, would change the
figure without any GPU run noticing.  These tests read the committed
summaries, and run summarize_profile on small hand-made rocprofv3 CSV files
whose expected output is worked out by hand below."""

import csv
import importlib.util
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_committed_traffic_summaries_hold_the_dominant_kernels(bench):
    """Every configuration whose roofline reads a committed summary finds both
    D=256 GCN kernels there, each moving more than one D=256 row per node of
    the graph (read + write)."""
    nodes = {"c2": 2_449_029, "c3": 2_449_029, "c4": 10_000_000}
    for cfg, path in bench.TRAFFIC_PROFILES.items():
        found = bench.traffic_from_profile(path, list(bench.GCN_DOMINANT.values()))
        assert found is not None, f"{cfg}: {path} lacks a BYTES line of a D=256 kernel"
        for kernel, nbytes in found.items():
            assert nbytes > nodes[cfg] * 256 * 4, (cfg, kernel, nbytes)


def test_request_bytes_weights_each_request_size(bench):
    means = {"TCC_EA0_RDREQ_32B_sum": 10.0, "TCC_EA0_RDREQ_64B_sum": 3.0,
             "TCC_EA0_RDREQ_128B_sum": 2.0, "TCC_EA0_WRREQ_sum": 7.0,
             "TCC_EA0_WRREQ_64B_sum": 4.0}
    # read 32*10 + 64*3 + 128*2 = 768; write 32*(7 - 4) + 64*4 = 352
    assert bench.request_bytes(means) == (768.0, 352.0)
    del means["TCC_EA0_WRREQ_64B_sum"]
    assert bench.request_bytes(means) is None


def _write_csv(path, header, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def test_summarize_profile_busy_clock_and_bytes(bench, tmp_path, capsys):
    """One GEMM dispatch of 2 ms on a GPU of 1024 SIMDs in 8 XCDs:
    GRBM_GUI_ACTIVE 32e6 is 4e6 cycles per XCD, so 2.0 GHz; 2.048e9 busy
    cycles over 1024 SIMDs x 4e6 cycles is 0.5 busy.  One aggregation dispatch
    with request counters: read 32*100 + 64*10 + 128*1000 = 131840 bytes,
    write 32*(50 - 20) + 64*20 = 2240 bytes."""
    d = tmp_path / "run"
    d.mkdir()
    _write_csv(d / "run_agent_info.csv", ["Agent_Type", "Simd_Count", "Num_Xcc"],
               [["CPU", "0", "1"], ["GPU", "1024", "8"]])
    gemm = "void gr_gemm::gemm_nt_resident32<4, 8>(float const*)"
    agg = "void gr_agg::aggregate_units<4, 64, 1, 8>(int const*)"
    header = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value",
              "Start_Timestamp", "End_Timestamp"]
    rows = [[1, gemm, "GRBM_GUI_ACTIVE", 32e6, 1_000_000, 3_000_000],
            [1, gemm, "SQ_VALU_MFMA_BUSY_CYCLES", 2.048e9, 1_000_000, 3_000_000]]
    for name, value in (("TCC_EA0_RDREQ_32B_sum", 100), ("TCC_EA0_RDREQ_64B_sum", 10),
                        ("TCC_EA0_RDREQ_128B_sum", 1000), ("TCC_EA0_WRREQ_sum", 50),
                        ("TCC_EA0_WRREQ_64B_sum", 20)):
        rows.append([2, agg, name, value, 5_000_000, 6_000_000])
    _write_csv(d / "run_counter_collection.csv", header, rows)
    _write_csv(d / "run_kernel_stats.csv", ["Name", "Calls", "TotalDurationNs", "AverageNs"],
               [[gemm, 1, 2_000_000, 2_000_000], [agg, 1, 1_000_000, 1_000_000]])
    bench.summarize_profile(str(d))
    out = capsys.readouterr().out
    assert "MFMA busy=0.500 clock_GHz=2.000 kernel=" + gemm in out
    assert "BYTES read=131840 write=2240 kernel=" + agg in out
    # The kernel stats are sorted by total time and show the share of each.
    lines = [l for l in out.splitlines() if l.strip().startswith("1 ")]
    assert "gemm_nt_resident32" in lines[0] and "66.67" in lines[0]
    # traffic_from_profile reads the BYTES line back (read + write).
    summary = tmp_path / "summary.txt"
    summary.write_text(out)
    assert bench.traffic_from_profile(str(summary), ["aggregate_units<4, 64, 1, 8>"]) == {
        "aggregate_units<4, 64, 1, 8>": 131840.0 + 2240.0}
    assert bench.traffic_from_profile(str(summary), ["aggregate_ln_relu_units"]) is None


def test_dense_probe_table_is_well_formed(bench):
    for name, (kind, rows, cols, k) in bench.DENSE_PROBES.items():
        assert kind in ("nt", "tn", "lla"), name
        assert rows >= 1 << 16 and cols % 16 == 0 and k >= 1, name
