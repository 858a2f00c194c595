"""oxs_sample_batch_static (the no-allocation entry point) against
oxs_sample_batch on the same inputs: every output identical, over two calls
in a row on one device, the second smaller than the first (the static
workspace keeps the first call's contents)."""
import pytest

from harness import compare, run_gpu
from oxide_sampler import _abi
from oxide_sampler import workloads as wl
from test_gpu_parity import mixed_workload

pytestmark = pytest.mark.gpu


def banner(msg):
    print(f"\n[case] {msg}", flush=True)


def test_static_matches_sampler_two_calls(torch_gpu):
    big = wl.config2()  # B=64 x V=128256, full chain
    small = mixed_workload(40, 50001, seed=4242)  # every chain shape, DRY rows, ragged histories
    for w, kw in ((big, dict(logits_out=True)), (small, dict(kept_ld=1024, logits_out=True, max_top_k=1024))):
        banner(f"static vs sampler: {w.name} B={w.batch} V={w.vocab}")
        want = run_gpu(w, torch_gpu, **kw)
        got = run_gpu(w, torch_gpu, no_alloc=True, **kw)
        compare(got, want, 0.0, f"static {w.name}")


def test_static_rejects_oversize(torch_gpu):
    lib = _abi.load_library()
    b = _abi.OxsBatch()
    b.batch, b.vocab = _abi.OXS_STATIC_MAX_BATCH + 1, 1000
    assert lib.oxs_sample_batch_static(b, None) == _abi.OXS_ERR_LIMITS
    b.batch, b.vocab = 1, _abi.OXS_STATIC_MAX_VOCAB + 1
    assert lib.oxs_sample_batch_static(b, None) == _abi.OXS_ERR_LIMITS
    assert lib.oxs_sample_batch_static(None, None) == _abi.OXS_ERR_INVALID_ARGUMENT
    b.batch, b.vocab = 0, 1000  # nothing to do
    assert lib.oxs_sample_batch_static(b, None) == _abi.OXS_OK
