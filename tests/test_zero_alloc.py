"""The C ABI allocates nothing per call, checked as the reference checks its
decode loop (crates/oxide-engine/tests/test_zero_alloc_forward_decode.rs:9-85,
with the counting allocator of crates/oxide-core/src/zero_alloc_guard.rs:9-41).

tests/cpp/zero_alloc_test.cpp defines malloc, calloc, realloc, the aligned
allocators and operator new itself, so every library in the process resolves
to its counters; a call counts against the sampler when its return address
lies in liboxide_sampler.so's mapped range. Over 1000 oxs_sample_batch,
1000 oxs_decode_step and 1000 oxs_sample_batch_static calls on a config-2
shaped batch (after a warm-up) the library must make no host allocation, and hipMemGetInfo's free device bytes
must not change. The binary is built in-tree by the package build
(tests/cpp/Makefile).
"""
import json
import subprocess
from pathlib import Path

import pytest

BIN = Path(__file__).resolve().parent / "cpp" / "_bin" / "zero_alloc_test"


@pytest.mark.gpu
def test_sample_and_decode_allocate_nothing(torch_gpu):
    if not BIN.exists():
        pytest.skip("tests/cpp not built (run __graft_entry__.build())")
    print("\n[case] zero_alloc_test: 1000 oxs_sample_batch + 1000 oxs_decode_step + 1000 oxs_sample_batch_static,"
          " B=64 V=128256", flush=True)
    r = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=180)
    print(r.stdout, r.stderr, flush=True)
    line = [x for x in r.stdout.splitlines() if x.startswith("{")]
    assert line, "no result line"
    d = json.loads(line[-1])
    assert d["rc_sample"] == 0 and d["rc_decode"] == 0 and d["rc_static"] == 0, d
    assert d["library_host_allocations"] == 0, d
    assert d["device_free_bytes_before"] == d["device_free_bytes_after"], d
    assert r.returncode == 0
