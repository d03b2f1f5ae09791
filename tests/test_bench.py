"""bench.py's host-side reporting, on the CPU: the single-GPU refusal, the rocprofv3 kernel-trace summary, the
HBM traffic per launch from the two counter passes (each counter scaled by what it reads for the calibration
pass over 1 GiB) and the decode kernels' code sizes in the built library.  The CSVs are written here in rocprofv3's column layout; the figures are set by hand so that
every expected number follows from the arithmetic in the docstrings."""
import csv
import importlib.util
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


GATEUP = "void k_gemv<4, 32, 0, 1, 3, 1, 1>(GemvArgs)"
HEAD = "void k_gemv<8, 32, 0, 1, 4, 2, 1>(GemvArgs)"
FILL = "void at::native::vectorized_elementwise_kernel<4, at::native::FillFunctor<float>>(int)"
MUL = "void at::native::vectorized_elementwise_kernel<4, at::native::MulFunctor<float>>(int)"


def write_counters(path, counter, rows):
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.writer(f, quoting=csv.QUOTE_NONNUMERIC)
        w.writerow(["Correlation_Id", "Dispatch_Id", "Grid_Size", "Kernel_Name", "Workgroup_Size", "Counter_Name",
                    "Counter_Value", "Start_Timestamp", "End_Timestamp"])
        for i, (name, value) in enumerate(rows):
            w.writerow([i + 1, i + 1, 1024, name, 256, counter, value, 1000 * i, 1000 * i + 500])


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_traffic_per_launch_from_the_two_counter_passes(bench, tmp_path):
    """FETCH_SIZE: the calibration multiply (reads 1 GiB) reads as 524288 KiB, half the bytes, so fetches count
    double: gate/up launches of 2514 and 2516 KiB are 2515 * 1024 / 0.5 = 5,150,720 bytes each.  WRITE_SIZE: the
    fill and the multiply (each writes 1 GiB) read as 1048576 KiB, factor 1: 10 KiB = 10,240 bytes.  The fill's
    small FETCH_SIZE does not set the scale (the largest calibration reading does)."""
    write_counters(str(tmp_path / "fetch" / "host" / "fetch_counter_collection.csv"), "FETCH_SIZE",
                   [(FILL, 21.1875), (MUL, 524288.0), (GATEUP, 2514.0), (GATEUP, 2516.0), (HEAD, 61188.0)])
    write_counters(str(tmp_path / "write" / "host" / "write_counter_collection.csv"), "WRITE_SIZE",
                   [(FILL, 1048576.0), (MUL, 1048576.0), (GATEUP, 10.0), (GATEUP, 10.0), (HEAD, 320.0)])
    r = bench.traffic_from(str(tmp_path), "gateup_gemv")
    assert r["fetch_factor"] == pytest.approx(0.5) and r["write_factor"] == pytest.approx(1.0)
    assert r["fetch"] == pytest.approx(5150720.0) and r["write"] == pytest.approx(10240.0)
    h = bench.traffic_from(str(tmp_path), "head_gemv")
    assert h["fetch"] == pytest.approx(61188.0 * 2048) and h["write"] == pytest.approx(320.0 * 1024)
    assert bench.traffic_from(str(tmp_path), "down_gemv") is None  # no dispatch of that kind
    assert bench.traffic_from(str(tmp_path / "missing"), "gateup_gemv") is None


def test_trace_summary_groups_by_kernel_and_grid(bench, tmp_path, capsys):
    """durations are end - start in ns, reported in µs: gate/up at grid 100 runs 1 and 3 µs (avg 2, 40% of the
    10 µs total), at grid 200 one 4 µs call (40%), the head one 2 µs call (20%); largest share first, ties in
    the order met"""
    p = tmp_path / "t_kernel_trace.csv"
    rows = [(GATEUP, 100, 0, 1000), (GATEUP, 200, 5000, 9000), (GATEUP, 100, 10000, 13000), (HEAD, 100, 20000, 22000)]
    with open(p, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Kernel_Name", "Grid_Size", "Workgroup_Size", "Start_Timestamp", "End_Timestamp"])
        for name, grid, t0, t1 in rows:
            w.writerow([name, grid, 256, t0, t1])
    bench.trace_summary(str(p))
    lines = capsys.readouterr().out.strip().split("\n")
    assert len(lines) == 3
    first = lines[0].split()
    assert first[0] == "40.00%" and first[2] == "2" and first[4] == "2.00" and first[8] == "1.00"
    assert first[10] == "3.00" and first[12] == "100" and lines[0].endswith(GATEUP)
    second = lines[1].split()
    assert second[0] == "40.00%" and second[2] == "1" and second[4] == "4.00" and second[12] == "200"
    third = lines[2].split()
    assert third[0] == "20.00%" and lines[2].endswith(HEAD)


def test_code_sizes_cover_every_decode_kernel_kind(bench):
    """`bench.py --code-sizes` reads the built library's gfx950 code object: every decode kernel kind has code of a
    plausible size (a few to a few tens of KB), and the kinds' instantiations carry their template arguments"""
    lib = os.path.join(ROOT, "local-llama-pynq-z2_amd", "libmatvec_hip.so")
    tools = [shutil.which("objcopy"), "/opt/rocm/llvm/bin/clang-offload-bundler", "/opt/rocm/llvm/bin/llvm-readelf"]
    if not os.path.exists(lib) or not all(t and os.path.exists(t) for t in tools):
        pytest.skip("needs the built library and the ROCm LLVM tools")
    sizes = bench.code_sizes()
    assert set(sizes) == set(bench.KERNEL_SYMBOL)
    for kind, ks in sizes.items():
        assert ks, kind
        for name, b in ks.items():
            assert bench.KERNEL_SYMBOL[kind] in name
            assert 1000 < b < 100000, (name, b)
    assert GATEUP in sizes["gateup_gemv"]
