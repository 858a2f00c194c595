"""GPU sampler vs the CPU oracle on identical seeded inputs.

Bar: selected token ids and kept-index sets match
exactly (ties by lower index); post-filter probabilities and Mirostat mu agree
within 1e-5 relative for f32 logits and 1e-3 for bf16 logits. The device
reproduces the oracle's float operations one for one (glibc-exact exp/ln/log2,
reference summation order), so these tests also require bit-identical
probabilities; the tolerance is checked first so a failure says which bar broke.
"""
import numpy as np
import pytest

from harness import compare, run_gpu, run_oracle
from oxide_sampler import MirostatMode, _abi
from oxide_sampler import workloads as wl

pytestmark = pytest.mark.gpu

RTOL_F32 = 1e-5
RTOL_BF16 = 1e-3


def banner(msg):
    print(f"\n[case] {msg}", flush=True)


def test_config1_full(torch_gpu):
    w = wl.config1()
    banner("config1 B=1 V=32000")
    compare(run_gpu(w, torch_gpu), run_oracle(w), RTOL_F32, "config1")


def test_config1_batched(torch_gpu):
    w = wl.config1(batch=32)
    banner("config1 B=32 V=32000")
    compare(run_gpu(w, torch_gpu), run_oracle(w), RTOL_F32, "config1x32")


def test_config2_full(torch_gpu):
    w = wl.config2()
    banner("config2 B=64 V=128256")
    compare(run_gpu(w, torch_gpu, logits_out=True), run_oracle(w, logits_out=True), RTOL_F32, "config2")


def test_config3_full(torch_gpu):
    w = wl.config3()
    banner("config3 B=128 V=128256 masked")
    g = run_gpu(w, torch_gpu)
    compare(g, run_oracle(w), RTOL_F32, "config3")
    words = w.mask
    for b in range(w.batch):  # every sampled token is allowed by the mask
        t = int(g.tokens[b])
        assert (words[b, t >> 5] >> (t & 31)) & 1


def test_config4_full(torch_gpu):
    w = wl.config4()
    banner("config4 B=256 V=151936 bf16 typical+tfs")
    compare(run_gpu(w, torch_gpu), run_oracle(w), RTOL_BF16, "config4")


def test_config5_eight_steps(torch_gpu):
    w = wl.config5(batch=64)
    banner("config5 B=64 V=262144 mirostat v2 x8 steps")
    g_hist, g_len, g_mu = w.history.copy(), w.history_len.copy(), w.mu.copy()
    r_hist, r_len, r_mu = w.history.copy(), w.history_len.copy(), w.mu.copy()
    for step in range(w.steps):
        w.logits = wl.config5_step_logits(w.batch, w.vocab, wl.SEED_BASE + 5, step)
        w.history, w.history_len, w.mu = g_hist, g_len, g_mu
        g = run_gpu(w, torch_gpu)
        w.history, w.history_len, w.mu = r_hist, r_len, r_mu
        r = run_oracle(w)
        compare(g, r, RTOL_F32, f"config5 step {step}")
        g_hist, g_len, g_mu = g.history, g.history_len, g.mu
        r_hist, r_len, r_mu = r.history, r.history_len, r.mu
    assert int(r_len[0]) == 256 + 2 * w.steps  # two records per Mirostat step (sampler.rs:301, :307)
