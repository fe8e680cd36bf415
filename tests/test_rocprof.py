"""The rocprofv3 summary pipeline (decodebench_amd.rocprof) on synthetic CSVs.

Mirrors what the reference tests for its NCU parser (round detection and
per-kernel reduction, validation/analysis/parse_ncu.py:26-148): dispatches are
assigned to workloads in launch order, warm-up calls are dropped, counters are
scaled by the calibration copy, and a profile that does not match its manifest
fails loudly instead of producing numbers.
"""

import csv

import pytest

from decodebench_amd import rocprof

MANIFEST = {
    "copy_bytes": 1 << 20, "copy_calls": 2,
    "workloads": [
        {"label": "gemv", "calls": 3, "warmup": 1, "kernels_per_call": 1,
         "algorithmic_bytes": 1000},
        {"label": "attn", "calls": 2, "warmup": 0, "kernels_per_call": 2,
         "algorithmic_bytes": 5000},
    ],
}

# (name, duration ns, FETCH KiB, WRITE KiB) in dispatch order; a foreign
# kernel sits between workloads and must be ignored.
ROWS = [
    ("__amd_rocclr_copyBuffer", 900, 512.0, 1024.0),
    ("__amd_rocclr_copyBuffer", 900, 512.0, 1024.0),
    ("void at::native::fill", 10, 0.0, 4.0),
    ("void dbk::(anonymous namespace)::gemv_kernel<1>(args)", 9000, 50.0, 1.0),  # warm-up
    ("void dbk::(anonymous namespace)::gemv_kernel<1>(args)", 2000, 0.5, 0.25),
    ("void dbk::(anonymous namespace)::gemv_kernel<1>(args)", 4000, 0.5, 0.25),
    ("void at::native::copy", 10, 1.0, 1.0),
    ("void dbk::(anonymous namespace)::f4_kernel<4, 8>(args)", 3000, 2.0, 0.5),
    ("void dbk::(anonymous namespace)::f4_combine(args, int)", 1000, 0.5, 0.0625),
    ("void dbk::(anonymous namespace)::f4_kernel<4, 8>(args)", 5000, 2.0, 0.5),
    ("void dbk::(anonymous namespace)::f4_combine(args, int)", 1000, 0.5, 0.0625),
]


def write_trace(path):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Kind", "Dispatch_Id", "Kernel_Name", "Grid_Size_X", "Workgroup_Size_X",
                    "Start_Timestamp", "End_Timestamp"])
        t = 1000
        for i, (name, dur, _, _) in enumerate(ROWS, start=1):
            w.writerow(["KERNEL_DISPATCH", i, name, 256, 256, t, t + dur])
            t += dur + 100


def write_counters(path, counter, col):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Dispatch_Id", "Grid_Size", "Kernel_Name", "Workgroup_Size",
                    "Counter_Name", "Counter_Value"])
        for i, row in enumerate(ROWS, start=1):
            w.writerow([i, 256, row[0], 256, counter, row[col]])


@pytest.fixture()
def files(tmp_path):
    write_trace(tmp_path / "t.csv")
    write_counters(tmp_path / "f.csv", "FETCH_SIZE", 2)
    write_counters(tmp_path / "w.csv", "WRITE_SIZE", 3)
    return tmp_path


def test_summary_scales_counters_by_the_calibration_copy(files):
    res = rocprof.summarize(MANIFEST, trace=rocprof.read_trace(files / "t.csv"),
                            fetch=rocprof.read_counters(files / "f.csv"),
                            write=rocprof.read_counters(files / "w.csv"))
    # 1 MiB copy: FETCH reads 512 KiB -> x2, WRITE reads 1024 KiB -> x1.
    assert res["FETCH_SIZE_scale"] == pytest.approx(2.0)
    assert res["WRITE_SIZE_scale"] == pytest.approx(1.0)
    g = res["workloads"]["gemv"]
    assert g["call_us"] == pytest.approx(3.0)            # median of 2 and 4 (warm-up dropped)
    assert g["fetch_bytes"] == pytest.approx(0.5 * 1024 * 2)
    assert g["write_bytes"] == pytest.approx(0.25 * 1024)
    assert g["traffic_bytes"] == pytest.approx(1024 + 256)
    a = res["workloads"]["attn"]
    assert a["call_us"] == pytest.approx(5.0)            # (3+1) and (5+1) -> median 5
    assert a["kernel_us"]["void dbk::(anonymous namespace)::f4_combine"] == pytest.approx(1.0)
    assert a["fetch_bytes"] == pytest.approx(2.5 * 1024 * 2)
    assert a["GB/s"] == pytest.approx(5000 / 5000.0)
    assert rocprof.short_name("void dbk::(anonymous namespace)::gemv_kernel<1, 8>"
                              "(dbk::(anonymous namespace)::GemvArgs)") == \
        "void dbk::(anonymous namespace)::gemv_kernel<1, 8>"
    text = rocprof.to_markdown(res, "rocprofv3 ... -- python3 bench.py --profile-pass m.json")
    assert "| attn |" in text and "bench.py --profile-pass" in text


def test_mismatched_profile_fails(files):
    bad = dict(MANIFEST, workloads=[dict(MANIFEST["workloads"][0], calls=4)] +
               MANIFEST["workloads"][1:])
    with pytest.raises(ValueError, match="manifest expects"):
        rocprof.summarize(bad, trace=rocprof.read_trace(files / "t.csv"))
    with pytest.raises(ValueError, match="calibration"):
        rocprof.summarize(dict(MANIFEST, copy_calls=5),
                          fetch=rocprof.read_counters(files / "f.csv"))


# ------------------------------------------------ delimited segments
# The profile pass brackets every workload between two launches of the
# library's empty kernel; warm-up calls sit outside the brackets, and an
# unfused workload is whatever torch launched inside them.
NULL = "(anonymous namespace)::null_kernel()"
SEG_MANIFEST = {
    "copy_bytes": 1 << 20, "copy_calls": 1, "delimiter": "null_kernel",
    "workloads": [
        {"label": "f1", "kind": "fused", "calls": 2, "warmup": 0, "kernels_per_call": 1,
         "algorithmic_bytes": 1000},
        {"label": "f1_unfused", "kind": "unfused", "calls": 2, "warmup": 0,
         "kernels_per_call": None, "algorithmic_bytes": 3000},
    ],
}
SEG_ROWS = [
    ("__amd_rocclr_copyBuffer", 900, 512.0, 1024.0),
    ("void dbk::(anonymous namespace)::gemv_kernel<1>(args)", 7000, 9.0, 9.0),  # warm-up
    (NULL, 5, 0.0, 0.0),
    ("void dbk::(anonymous namespace)::gemv_kernel<1>(args)", 2000, 0.5, 0.25),
    ("void dbk::(anonymous namespace)::gemv_kernel<1>(args)", 4000, 0.5, 0.25),
    (NULL, 5, 0.0, 0.0),
    ("void at::native::reduce_kernel", 9000, 5.0, 5.0),                          # warm-up
    (NULL, 5, 0.0, 0.0),
    ("void at::native::reduce_kernel", 1000, 1.0, 0.0),
    ("void at::native::elementwise_kernel", 500, 0.5, 0.5),
    ("Cijk_gemv", 3000, 1.0, 0.5),
    ("void at::native::reduce_kernel", 1000, 1.0, 0.0),
    ("void at::native::elementwise_kernel", 700, 0.5, 0.5),
    ("Cijk_gemv", 3000, 1.0, 0.5),
    (NULL, 5, 0.0, 0.0),
]


def _write_rows(tmp_path, rows):
    global ROWS
    saved, ROWS = ROWS, rows
    try:
        write_trace(tmp_path / "t.csv")
        write_counters(tmp_path / "f.csv", "FETCH_SIZE", 2)
        write_counters(tmp_path / "w.csv", "WRITE_SIZE", 3)
    finally:
        ROWS = saved
    return (rocprof.read_trace(tmp_path / "t.csv"), rocprof.read_counters(tmp_path / "f.csv"),
            rocprof.read_counters(tmp_path / "w.csv"))


def test_round_detection_matches_the_reference_examples():
    assert rocprof.find_round_size(["rmsnorm", "gemv", "rmsnorm", "gemv"]) == 2
    assert rocprof.find_round_size(["gemv", "gemv", "swiglu"] * 2) == 3
    assert rocprof.find_round_size(["f1"] * 5) == 1
    assert rocprof.find_round_size(["f1"]) == 1
    with pytest.raises(ValueError, match="not periodic"):
        rocprof.find_round_size(["a", "b", "a", "c"])


def test_delimited_segments_hold_fused_and_unfused_calls(tmp_path):
    trace, fetch, write = _write_rows(tmp_path, SEG_ROWS)
    res = rocprof.summarize(SEG_MANIFEST, trace=trace, fetch=fetch, write=write)
    f1, un = res["workloads"]["f1"], res["workloads"]["f1_unfused"]
    assert f1["call_us"] == pytest.approx(3.0) and f1["kind"] == "fused"
    # three torch kernels per call, warm-up outside the brackets ignored
    assert un["kernels_per_call"] == 3 and un["kind"] == "unfused"
    assert un["call_us"] == pytest.approx((4.5 + 4.7) / 2)
    assert un["fetch_bytes"] == pytest.approx(2.5 * 1024 * 2)
    assert un["write_bytes"] == pytest.approx(1.0 * 1024)
    assert "kernel_us" not in un
    assert "3 torch kernels" in rocprof.to_markdown(res, "cmd")


def test_segments_fail_closed(tmp_path):
    # a missing end delimiter
    trace, _, _ = _write_rows(tmp_path, SEG_ROWS[:-1])
    with pytest.raises(ValueError, match="delimiters"):
        rocprof.summarize(SEG_MANIFEST, trace=trace)
    # a stray kernel inside the unfused segment breaks its rounds
    rows = SEG_ROWS[:-1] + [("void at::native::fill", 10, 0.0, 0.0), (NULL, 5, 0.0, 0.0)]
    trace, _, _ = _write_rows(tmp_path, rows)
    with pytest.raises(ValueError, match="whole calls|not periodic|period"):
        rocprof.summarize(SEG_MANIFEST, trace=trace)
    # a fused call with an unexpected kernel count
    bad = {**SEG_MANIFEST, "workloads": [dict(SEG_MANIFEST["workloads"][0], kernels_per_call=2),
                                         SEG_MANIFEST["workloads"][1]]}
    trace, _, _ = _write_rows(tmp_path, SEG_ROWS)
    with pytest.raises(ValueError, match="kernels per call"):
        rocprof.summarize(bad, trace=trace)


def _counter_csv(path, rows):
    """rows: (name, {counter: value}) per dispatch."""
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Dispatch_Id", "Grid_Size", "Kernel_Name", "Workgroup_Size",
                    "Counter_Name", "Counter_Value"])
        for i, (name, cs) in enumerate(rows, start=1):
            for c, v in cs.items():
                w.writerow([i, 256, name, 256, c, v])


READ_MANIFEST = {"copy_bytes": 1 << 20, "copy_calls": 1, "read_bytes": 1 << 20, "read_calls": 1,
                 "workloads": [{"label": "gemv", "calls": 1, "warmup": 0,
                                "kernels_per_call": 1, "algorithmic_bytes": 1000}]}
COPY = "__amd_rocclr_copyBuffer"
PROBE = "void dbk::(anonymous namespace)::stream_read_kernel<4>(args)"
GEMV = "void dbk::(anonymous namespace)::gemv_kernel<1>(args)"


def test_read_probe_scale_must_agree_with_the_copy(tmp_path):
    ok = [(COPY, {"FETCH_SIZE": 512.0}), (PROBE, {"FETCH_SIZE": 520.0}),
          (GEMV, {"FETCH_SIZE": 1.0})]
    _counter_csv(tmp_path / "ok.csv", ok)
    res = rocprof.summarize(READ_MANIFEST, fetch=rocprof.read_counters(tmp_path / "ok.csv"))
    assert res["FETCH_SIZE_scale"] == pytest.approx(2.0)
    assert res["FETCH_SIZE_read_scale"] == pytest.approx(1024 / 520)
    # a counter whose unit changes with the access pattern is rejected
    bad = [(COPY, {"FETCH_SIZE": 512.0}), (PROBE, {"FETCH_SIZE": 1024.0}),
           (GEMV, {"FETCH_SIZE": 1.0})]
    _counter_csv(tmp_path / "bad.csv", bad)
    with pytest.raises(ValueError, match="read-only probe"):
        rocprof.summarize(READ_MANIFEST, fetch=rocprof.read_counters(tmp_path / "bad.csv"))


def test_raw_read_requests_by_size(tmp_path):
    # 1 MiB read as 8192 requests of 128 bytes, all reported in TCC_EA0_RDREQ_128B and none
    # in TCC_BUBBLE: bytes by size are exact, the FETCH_SIZE formula counts them as 64 bytes.
    req = {"TCC_EA0_RDREQ_sum": 8192, "TCC_EA0_RDREQ_32B_sum": 0, "TCC_BUBBLE_sum": 0,
           "TCC_EA0_RDREQ_128B_sum": 8192}
    mix = {"TCC_EA0_RDREQ_sum": 10, "TCC_EA0_RDREQ_32B_sum": 2, "TCC_BUBBLE_sum": 3,
           "TCC_EA0_RDREQ_128B_sum": 5}
    _counter_csv(tmp_path / "raw.csv", [(COPY, req), (PROBE, req), (GEMV, mix)])
    res = rocprof.summarize(READ_MANIFEST, raw=rocprof.read_counters(tmp_path / "raw.csv"))
    probe = res["raw_read_requests"]["read_probe"]
    assert probe["bytes_by_size"] == 1 << 20
    assert probe["fetch_size_formula_bytes"] == (1 << 20) // 2
    g = res["workloads"]["gemv"]["read_requests"]
    assert g["bytes_by_size"] == 128 * 5 + 64 * 3 + 32 * 2
    assert g["fetch_size_formula_bytes"] == 128 * 3 + 64 * 5 + 32 * 2


def test_traffic_uses_reads_by_size_when_the_raw_run_exists(tmp_path):
    # 100 requests of 128 B and 20 of 64 B: 14,080 bytes read.  FETCH_SIZE's formula counts the
    # 128-byte ones as 64 bytes (7,680 bytes = 7.5 KiB-units) and the copy calibrates x2, which
    # doubles the 64-byte ones as well (15,360 bytes).
    fetch = [(COPY, {"FETCH_SIZE": 512.0}), (PROBE, {"FETCH_SIZE": 512.0}),
             (GEMV, {"FETCH_SIZE": 7.5})]
    write = [(COPY, {"WRITE_SIZE": 1024.0}), (PROBE, {"WRITE_SIZE": 0.0}),
             (GEMV, {"WRITE_SIZE": 0.5})]
    one = {"TCC_EA0_RDREQ_sum": 8192, "TCC_EA0_RDREQ_32B_sum": 0, "TCC_BUBBLE_sum": 0,
           "TCC_EA0_RDREQ_128B_sum": 8192}
    gemv = {"TCC_EA0_RDREQ_sum": 120, "TCC_EA0_RDREQ_32B_sum": 0, "TCC_BUBBLE_sum": 0,
            "TCC_EA0_RDREQ_128B_sum": 100}
    for name, rows in (("f", fetch), ("w", write), ("r", [(COPY, one), (PROBE, one),
                                                          (GEMV, gemv)])):
        _counter_csv(tmp_path / f"{name}.csv", rows)
    rd = lambda n: rocprof.read_counters(tmp_path / f"{n}.csv")  # noqa: E731
    res = rocprof.summarize(READ_MANIFEST, fetch=rd("f"), write=rd("w"), raw=rd("r"))
    g = res["workloads"]["gemv"]
    assert g["fetch_bytes"] == pytest.approx(15360)
    assert g["traffic_fetch_scaled_bytes"] == pytest.approx(15360 + 512)
    assert g["traffic_bytes"] == pytest.approx(14080 + 512)
    assert g["traffic_over_algorithmic"] == pytest.approx((14080 + 512) / 1000)
    assert "by size" in g["traffic_source"]
    md = rocprof.to_markdown(res, "cmd")
    assert "Read B by size" in md and "14,080" in md
    # without the raw run the scaled FETCH_SIZE is the read figure
    res = rocprof.summarize(READ_MANIFEST, fetch=rd("f"), write=rd("w"))
    assert res["workloads"]["gemv"]["traffic_bytes"] == pytest.approx(15360 + 512)
    assert "FETCH_SIZE" in res["workloads"]["gemv"]["traffic_source"]


def test_traffic_columns_merge_into_a_kernel_trace_summary():
    """merge_traffic adds a counter run's byte columns to the trace summary
    by workload label, and refuses a traffic file of other algorithmic bytes."""
    from decodebench_amd import rocprof

    res = {"workloads": {"f1": {"algorithmic_bytes": 100, "call_us": 1.0, "GB/s": 0.1,
                                "kernels_per_call": 1, "kind": "fused",
                                "kernel_us": {"gemv": 1.0}},
                         "f4": {"algorithmic_bytes": 50, "call_us": 2.0, "GB/s": 0.025,
                                "kernels_per_call": 1, "kind": "fused",
                                "kernel_us": {"f4": 2.0}}}}
    traffic = {"workloads": {"f1": {"algorithmic_bytes": 100, "write_bytes": 8.0,
                                    "fetch_bytes": 96.0, "traffic_bytes": 104.0,
                                    "traffic_over_algorithmic": 1.04}}}
    rocprof.merge_traffic(res, traffic)
    assert res["workloads"]["f1"]["traffic_over_algorithmic"] == pytest.approx(1.04)
    assert "write_bytes" not in res["workloads"]["f4"]
    md = rocprof.to_markdown(res, "cmd")
    assert "| f1 |" in md and "1.040" in md
    with pytest.raises(ValueError):
        rocprof.merge_traffic(res, {"workloads": {"f4": {"algorithmic_bytes": 51}}})


def test_a_fused_segment_counts_the_library_launches_only(tmp_path):
    """A graph replay of fused calls also runs the fill kernel that zeroed
    the capture's F4 workspace (once per replay): it is not part of any call,
    so a fused segment keeps the library's dispatches only."""
    rows = list(SEG_ROWS)
    i = rows.index((NULL, 5, 0.0, 0.0))
    rows.insert(i + 1, ("void at::native::vectorized_elementwise_kernel<4, FillFunctor>", 3, 0.0, 0.5))
    trace, fetch, write = _write_rows(tmp_path, rows)
    res = rocprof.summarize(SEG_MANIFEST, trace=trace, fetch=fetch, write=write)
    f1 = res["workloads"]["f1"]
    assert f1["kernels_per_call"] == 1 and f1["call_us"] == pytest.approx(3.0)
