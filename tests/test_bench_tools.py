"""bench.py's profile tooling, on synthetic rocprofv3 output: timed regions cut at the
marker dispatches, read bytes counted by request size, and the traffic a line reports."""
import csv
import importlib.util
import os

import pytest

_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
_spec = importlib.util.spec_from_file_location("bench_tools", os.path.join(_ROOT, "bench.py"))
bench = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(bench)


def _write(path, header, rows):
    with open(path, "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(header)
        w.writerows(rows)


def _trace(tmp_path, names_and_ns):
    """A kernel_trace.csv with one row per (name, start_ns, end_ns)."""
    rows = [[n, s, e] for n, s, e in names_and_ns]
    _write(tmp_path / "run_kernel_trace.csv", ["Kernel_Name", "Start_Timestamp", "End_Timestamp"],
           rows)
    return str(tmp_path)


MARK = "void at::native::vectorized_elementwise_kernel<4, at::native::bitwise_not_kernel_cuda(x)"


def test_regions_skip_the_set_up_marker_and_leave_warm_ups_out(tmp_path):
    t = 0
    ev = []

    def k(name, dur):
        nonlocal t
        ev.append((name, t, t + dur))
        t += dur + 10

    k(MARK, 1)                       # set-up launch
    k("warm_a(int)", 100)            # warm-up of region 0: outside
    k(MARK, 1)
    k("gate_a(int)", 1000)
    k("gate_a(int)", 3000)
    k(MARK, 1)
    k("warm_b(int)", 100)            # warm-up of region 1: outside
    k(MARK, 1)
    k("down_b(int)", 2000)
    k(MARK, 1)
    out = bench._regions(_trace(tmp_path, ev))
    text = "\n".join(out)
    assert "region 0: 2 dispatches" in text and "region 1: 1 dispatches" in text
    assert "warm_a" not in text and "warm_b" not in text
    line = next(l for l in out if l.strip().startswith("gate_a"))
    assert line.split()[1:3] == ["2", "2.000"]          # 2 dispatches, 2.0 us average


def test_read_bytes_count_requests_by_size_without_a_factor(tmp_path):
    d = tmp_path / "rd"
    d.mkdir()
    hdr = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]
    rows = []
    for i, (a, b, c) in enumerate([(0, 10, 1000), (0, 30, 3000)]):
        for ctr, v in (("TCC_EA0_RDREQ_32B_sum", a), ("TCC_EA0_RDREQ_64B_sum", b),
                       ("TCC_EA0_RDREQ_128B_sum", c)):
            rows.append([i, "void vaayu::prefill_down_kernel<4, 0, 16>(int)", ctr, v])
    _write(d / "run_counter_collection.csv", hdr, rows)
    text = bench.summarize([str(d)])
    want = 64 * 20 + 128 * 2000                      # averages of the two dispatches
    assert f"traffic_bytes prefill_down_kernel READ_BYTES {want}" in text


def test_traffic_prefers_read_bytes_and_counts_each_launch(tmp_path, monkeypatch):
    prof = tmp_path / "profiles"
    prof.mkdir()
    (prof / "t.txt").write_text(
        "traffic_bytes prefill_gate_up_kernel FETCH_SIZE 1000\n"
        "traffic_bytes prefill_gate_up_kernel READ_BYTES 900\n"
        "traffic_bytes prefill_gate_up_kernel WRITE_SIZE 50\n"
        "traffic_bytes prefill_down_kernel FETCH_SIZE 400\n"
        "traffic_bytes prefill_down_kernel WRITE_SIZE 20\n")
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    monkeypatch.setitem(bench.TRAFFIC_FILES, "wl", "t.txt")
    kernels = ("prefill_gate_up_kernel", "prefill_down_kernel")
    assert bench.traffic_from_profile("wl", kernels) == 900 + 50 + 400 + 20
    assert bench.traffic_from_profile("wl", kernels, 2) == 2 * (900 + 50 + 400 + 20)
    # a kernel without a write count: no figure rather than a partial one
    assert bench.traffic_from_profile("wl", kernels + ("prefill_reduce_kernel",)) is None
    assert bench.traffic_from_profile("no-such-workload", kernels) is None


def test_more_than_one_gpu_is_refused(monkeypatch, capsys):
    monkeypatch.setattr("sys.argv", ["bench.py", "--gpus", "2"])
    with pytest.raises(SystemExit) as e:
        bench.main()
    assert e.value.code == 2
    assert "one GPU" in capsys.readouterr().err
