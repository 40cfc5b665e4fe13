"""CPU tests of bench.py's host-side logic: the HBM-traffic reading of rocprofv3 counter rows
and its fallback when the profiler is absent."""
import pathlib
import sys

import pytest

sys.path.insert(0, str(pathlib.Path(__file__).resolve().parents[1]))
import bench  # noqa: E402

COPY = "__amd_rocclr_copyBuffer"
SPLIT = "void pk::(anonymous namespace)::decode_split_kernel<2, 8, 1, true, false>(pk::AttnArgs)"
COMB = "void pk::(anonymous namespace)::decode_combine_kernel<0>(pk::AttnArgs)"


def _row(kernel, counter, value):
    return {"Kernel_Name": kernel, "Counter_Name": counter, "Counter_Value": str(value)}


def test_pmc_call_bytes_scales_by_the_large_copies():
    # the copies read 1 GiB and the counter reports half of it (524288 KiB): factor 2; small
    # copies (host uploads) and other kernels are ignored; per-kernel means are summed
    rows = [_row(COPY, "FETCH_SIZE", 524288.0) for _ in range(5)]
    rows += [_row(COPY, "FETCH_SIZE", 12.0), _row(COPY, "FETCH_SIZE", 3.0)]
    rows += [_row("at::native::reduce_kernel", "FETCH_SIZE", 1e9)]
    rows += [_row(SPLIT, "FETCH_SIZE", v) for v in (1000.0, 1002.0, 998.0)]
    rows += [_row(COMB, "FETCH_SIZE", v) for v in (10.0, 10.0, 10.0)]
    rows += [_row(SPLIT, "WRITE_SIZE", 7.0)]  # another counter: ignored
    got, factor = bench.pmc_call_bytes(rows, "FETCH_SIZE")
    assert factor == 2.0
    assert got == pytest.approx((1000.0 + 10.0) * 1024 * 2.0)


def test_pmc_call_bytes_needs_path_and_copy_rows():
    assert bench.pmc_call_bytes([_row(COPY, "WRITE_SIZE", 1048576.0)], "WRITE_SIZE") is None
    assert bench.pmc_call_bytes([_row(SPLIT, "WRITE_SIZE", 5.0)], "WRITE_SIZE") is None
    rows = [_row(COPY, "WRITE_SIZE", 1048576.0), _row(SPLIT, "WRITE_SIZE", 10344.5)]
    got, factor = bench.pmc_call_bytes(rows, "WRITE_SIZE")
    assert factor == 1.0 and got == pytest.approx(10344.5 * 1024)


def test_pmc_traffic_without_profiler(monkeypatch):
    import shutil

    monkeypatch.setattr(shutil, "which", lambda name: None)
    assert bench.pmc_traffic("cfg2") == (None, "rocprofv3 not found")
