"""The model's final logit softcap applied by the sampler as it reads the logits.

Reference: the backend's softcap pass, logits[i] = cap * tanhf(logits[i] / cap)
(crates/oxide-hardware/oxide-backend-cuda/src/kernels/vec_ops_activations.cu:131-136,
launched before sampling at oxide-backend-cuda/src/lib.rs:3243-3255). Here it is
a field of the batch descriptor, fused into the sampler's read of the logits,
so the separate read and write of [B, V] logits disappears.
"""
import numpy as np
import pytest

from harness import compare, run_gpu, run_oracle
from oxide_sampler import workloads as wl
from test_gpu_parity import RTOL_F32, banner, mixed_workload


def test_oracle_softcap_closed_form():
    # cap * tanh(l / cap) with glibc's tanhf (within a few ulp of tanh) and the
    # special values: +-inf -> +-cap, NaN stays NaN (then not a candidate)
    V = 4000
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((1, V)) * 20).astype(np.float32)
    x[0, :4] = [np.inf, -np.inf, np.nan, 0.0]
    for cap in (30.0, 0.5, 7.25):
        w = wl.Workload("softcap", x.copy(), "f32", [wl.disabled_config(temperature=0.0)], np.zeros((1, 2), np.uint32),
                        np.zeros(1, np.uint32), np.zeros(1, np.float32), extra={"softcap": cap})
        got = run_oracle(w, logits_out=True).logits_out[0]
        c = np.float32(cap)
        exact = (np.float64(c) * np.tanh(np.float64((x[0] / c).astype(np.float32)))).astype(np.float32)
        fin = np.isfinite(x[0])
        # glibc's tanhf is within 2 ulp of tanh and the product rounds once more
        np.testing.assert_allclose(got[fin], exact[fin], rtol=5e-7, atol=0)
        assert got[0] == c and got[1] == -c and np.isnan(got[2]) and got[3] == 0.0
        assert np.all(np.abs(got[fin]) <= c)
        # the sampled token is the first largest capped logit
        t = run_oracle(w).tokens[0]
        capped = np.where(np.isnan(got), -np.inf, got)
        assert t == int(np.argmax(capped))


def test_oracle_softcap_off_values():
    # 0, negative and NaN caps leave the logits alone (lib.rs:3244: cap > 0.0)
    x = np.array([[1.0, 5.0, -3.0, 40.0]], np.float32)
    for cap in (0.0, -2.0, float("nan")):
        w = wl.Workload("off", x.copy(), "f32", [wl.disabled_config(temperature=0.0)], np.zeros((1, 2), np.uint32),
                        np.zeros(1, np.uint32), np.zeros(1, np.float32), extra={"softcap": cap})
        np.testing.assert_array_equal(run_oracle(w, logits_out=True).logits_out, x)


@pytest.mark.gpu
@pytest.mark.parametrize("cap,V,dtype,masked", [(30.0, 50001, "f32", False), (0.5, 32000, "f32", True),
                                                (15.0, 131072, "bf16", False), (2.0, 4097, "f32", True)])
def test_gpu_softcap_matches_oracle(torch_gpu, cap, V, dtype, masked):
    B = 40
    w = mixed_workload(B, V, seed=int(cap * 10) + V)
    w.extra["softcap"] = cap  # cap 0.5 saturates tanh to exactly 1: long runs of equal capped logits
    if dtype == "bf16":
        w.logits = wl.f32_to_bf16_bits(w.logits)
        w.dtype = "bf16"
    if masked:
        rng = np.random.default_rng(V)
        bits = rng.random((B, V)) < 0.4
        bits[:, :64] = True
        w.mask = wl.pack_mask(bits, V)
    banner(f"softcap {cap} B={B} V={V} {dtype} mask={masked}")
    compare(run_gpu(w, torch_gpu, kept_ld=1024, logits_out=True, max_top_k=1024),
            run_oracle(w, kept_ld=1024, logits_out=True), RTOL_F32, f"softcap {cap} V={V}")
