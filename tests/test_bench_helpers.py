"""bench.py's measurement arithmetic, on the CPU: the algorithmic bytes behind
roofline.achieved, the pool that keeps the logits out of the Infinity Cache,
the rocprofv3 summaries behind roofline.traffic and roofline.per_kernel, and
the one-GPU guard."""
import csv
import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_algorithmic_bytes_config2():
    # per row: the logits, the 512-id window, token + status + uniform + kept
    # count (16 B), the 26-dword config (104 B), and 8 B per kept id
    per_row = 128256 * 4 + 512 * 4 + 16 + 104
    assert bench.algorithmic_bytes(64, 128256, 512, 0) == 64 * per_row == 32_972_288
    assert bench.algorithmic_bytes(64, 128256, 512, 50) - bench.algorithmic_bytes(64, 128256, 512, 0) == 64 * 50 * 8
    # bf16 logits (config 4) count two bytes each; a packed mask (config 3) one word per 32 ids
    assert bench.algorithmic_bytes(256, 151936, 1024, 0, esz=2) == 256 * (151936 * 2 + 1024 * 4 + 120)
    mw = (128256 + 31) // 32
    assert bench.algorithmic_bytes(128, 128256, 512, 0, mask_words=mw) == \
        bench.algorithmic_bytes(128, 128256, 512, 0) + 128 * mw * 4


def test_pool_exceeds_twice_the_infinity_cache():
    for B, V, esz in ((64, 128256, 4), (1, 32000, 4), (256, 151936, 2), (512, 262144, 4)):
        batch = B * V * esz
        n = bench.pool_batches(batch)
        assert n >= 2 and n * batch > 2 * bench.MALL_BYTES, (B, V)
        assert (n - 1) * batch <= 2 * bench.MALL_BYTES or n == 2  # no larger than needed
    assert bench.pool_batches(64 * 128256 * 4) == 17  # the headline's 17 batches (558 MB)


def _write_csv(path, header, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def test_summarize_trace_takes_the_sampler_kernels(tmp_path):
    hdr = ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs", "StdDev"]
    _write_csv(tmp_path / "t_kernel_stats.csv", hdr, [
        ["void oxs::stream_kernel<0, 8, true, false, false>(...)", 8000, 0, 9393.3, 0, 0, 0, 0],
        ["void oxs::stream_kernel<0, 8, true, false, false>(...)", 1, 0, 20000.0, 0, 0, 0, 0],  # an eager call
        ["void oxs::stream_kernel<1, 4, true, false, false>(...)", 9000, 0, 29000.0, 0, 0, 0, 0],  # bf16: not config 2
        ["void oxs::tail_kernel<0, 8>(...)", 8000, 0, 8512.0, 0, 0, 0, 0],
        ["void at::native::normal_kernel(...)", 16, 0, 100.0, 0, 0, 0, 0],
    ])
    s = bench.summarize_trace(tmp_path)
    assert set(s) == {"stream_kernel", "tail_kernel"}
    assert s["stream_kernel"]["avg_ns"] == 9393.3 and s["stream_kernel"]["calls"] == 8000
    assert s["tail_kernel"]["avg_ns"] == 8512.0


def _pmc(folder, counter, rows):
    folder.mkdir()
    hdr = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]
    _write_csv(folder / "x_counter_collection.csv", hdr, [[i, n, counter, v] for i, (n, v) in enumerate(rows)])


def test_summarize_pmc_pairs_launches_and_scales_by_the_copy(tmp_path):
    st, tl = "void oxs::stream_kernel<0, 8, true, false, false>", "void oxs::tail_kernel<0, 8>"
    other = "void at::native::fill_kernel"
    _pmc(tmp_path / "f", "FETCH_SIZE", [(other, 5.0), (st, 100.0), (tl, 10.0), (st, 104.0), (tl, 10.0),
                                        (st, 300.0), (tl, 12.0)])
    _pmc(tmp_path / "w", "WRITE_SIZE", [(st, 7.0), (tl, 1.0), (st, 7.0), (tl, 1.0)])
    _pmc(tmp_path / "cf", "FETCH_SIZE", [("__amd_rocclr_copyBuffer", 131072.0)] * 3)  # reads half of 256 MiB
    _pmc(tmp_path / "cw", "WRITE_SIZE", [("__amd_rocclr_copyBuffer", 262144.0)] * 3)
    s = bench.summarize_pmc(tmp_path / "f", tmp_path / "w", tmp_path / "cf", tmp_path / "cw")
    assert s["launches_fetch"] == 3 and s["launches_write"] == 2
    assert s["fetch_kib_raw"] == 114.0  # the median of 110, 114, 312 KiB per (stream, tail) pair
    assert s["copy_scale_fetch"] == 2.0 and s["copy_scale_write"] == 1.0
    assert s["traffic_bytes_per_launch"] == 114.0 * 1024 * 2.0 + 8.0 * 1024


def test_committed_summaries_agree_with_the_algorithmic_bytes():
    traffic, src = bench.read_traffic(ROOT / "profiles" / "config2_pmc_traffic.json")
    assert src is not None
    algo = bench.algorithmic_bytes(64, 128256, 512, 0)
    # every logit is read once: traffic at least the logits, within 1.2x of the algorithmic bytes
    assert 64 * 128256 * 4 <= traffic <= 1.2 * algo
    trace, src = bench.read_kernel_trace(ROOT / "profiles" / "config2_kernel_trace.json")
    assert src is not None
    stream_ns = trace["stream_kernel"]["avg_ns"]
    assert "stream_kernel<0, 8" in trace["stream_kernel"]["name"] and "tail_kernel<0, 8" in trace["tail_kernel"]["name"]
    # the stream kernel cannot beat the 8 TB/s peak over the logits it reads
    assert 64 * 128256 * 4 / (stream_ns * 1e-9) < 8e12
    md = (ROOT / "profiles" / "config2_sample_batch_kernel_trace.md").read_text()
    assert f"| {round(stream_ns)} |" in md and f"| {round(trace['tail_kernel']['avg_ns'])} |" in md


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120, cwd=ROOT)
    assert r.returncode == 2 and "one GPU" in r.stderr and r.stdout == ""


@pytest.mark.parametrize("bad", [["--workload", "nope"], ["--gpus", "x"]])
def test_bad_arguments_are_refused(bad):
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), *bad], capture_output=True, text=True, timeout=120,
                       cwd=ROOT)
    assert r.returncode == 2 and r.stdout == ""
