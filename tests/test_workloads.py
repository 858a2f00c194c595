"""The seeded workloads against BASELINE.json's five configs, on the CPU: shapes,
dtypes, distributions, histories, masks and the chain each row's config asks
for. The GPU parity tests and bench.py both draw on these builders, so a drift
here would move every measured line away from the configuration it names."""
import math

import numpy as np
import pytest

from oxide_sampler import MirostatMode
from oxide_sampler import workloads as wl

U24 = np.float32(2.0 ** -24)


def _uniforms_ok(u):
    assert u.dtype == np.float32 and ((u >= 0) & (u < 1)).all()
    assert (np.floor(u / U24) * U24 == u).all()  # on the 24-bit grid of next_f32 (sampler.rs:150-153)


def _chain(c, **want):
    for k, v in want.items():
        got = getattr(c, k)
        assert (got == pytest.approx(v)) if isinstance(v, float) else got == v, (k, got, v)


def test_config1():
    w = wl.config1()
    assert (w.batch, w.vocab, w.dtype) == (1, 32000, "f32") and w.logits.dtype == np.float32
    x = w.logits[0]
    spikes = x == np.float32(8.0)
    assert spikes.sum() == 5  # five random spikes at +8
    assert abs(float(x[~spikes].std()) - 2.0) < 0.05 and abs(float(x[~spikes].mean())) < 0.05
    assert int(w.history_len[0]) == 64 and (w.history[0, :64] < 32000).all()
    _chain(w.configs[0], repeat_penalty=1.1, temperature=0.8, top_k=40, top_p=0.95, min_p=0.0,
           mirostat_mode=MirostatMode.Disabled, frequency_penalty=0.0, presence_penalty=0.0)
    assert w.configs[0].repeat_last_n in (0, 64)  # the whole 64-id history
    _uniforms_ok(w.uniforms)


def test_config2():
    w = wl.config2()
    assert (w.batch, w.vocab, w.dtype) == (64, 128256, "f32")
    # N(0, 3) plus -1.1 ln(rank) over a permutation: each row's mean is the prior's
    prior_mean = -1.1 * float(np.log(np.arange(1, 128257, dtype=np.float64)).mean())
    means = w.logits.mean(axis=1)
    assert np.abs(means - prior_mean).max() < 0.05
    # the prior is a permutation per row: rows differ in where the largest values sit
    assert len({int(np.argmax(r)) for r in w.logits}) > 32
    assert (w.history_len == 512).all() and (w.history[:, :512] < 128256).all()
    for c in w.configs:
        _chain(c, frequency_penalty=0.3, presence_penalty=0.2, repeat_penalty=1.05, temperature=0.7, top_k=50,
               top_p=0.9, min_p=0.05, mirostat_mode=MirostatMode.Disabled, dry_multiplier=0.0)
        assert c.repeat_last_n in (0, 512)
    _uniforms_ok(w.uniforms)


def test_config3():
    w = wl.config3()
    assert (w.batch, w.vocab, w.dtype) == (128, 128256, "f32")
    words = (128256 + 31) // 32
    assert w.mask.shape == (128, words) and w.mask.dtype == np.uint32
    bits = np.unpackbits(w.mask.view(np.uint8), axis=1, bitorder="little")
    assert not bits[:, 128256:].any()  # no bit past the vocabulary
    density = bits[:, :128256].mean(axis=1)
    assert (density > 0.027).all() and (density < 0.033).all()  # ~3% allowed
    assert (bits.sum(axis=1) >= 1).all()
    for c in w.configs:
        _chain(c, temperature=1.0, top_p=0.95, top_k=0, min_p=0.0, repeat_penalty=1.0,
               mirostat_mode=MirostatMode.Disabled)
    _uniforms_ok(w.uniforms)


def test_config4_small_batch():
    w = wl.config4(batch=8)
    assert (w.batch, w.vocab, w.dtype) == (8, 151936, "bf16") and w.logits.dtype == np.uint16
    x = wl.bf16_bits_to_f32(w.logits)
    heavy = x >= np.float32(6.0)
    # 1% of entries drawn in [6, 10], plus the N(0, 2.5) entries at or above 6 (P(Z >= 2.4))
    want = 0.01 + 0.99 * 0.5 * math.erfc(2.4 / math.sqrt(2.0))
    assert abs(heavy.mean() - want) < 0.001
    q1, q3 = np.percentile(x, [25, 75])
    assert abs((q3 - q1) / 1.349 - 2.5) < 0.05  # the N(0, 2.5) body, from its interquartile range
    assert (w.history_len == 1024).all() and (w.history[:, :1024] < 151936).all()
    for c in w.configs:
        _chain(c, repeat_penalty=1.1, temperature=0.9, typical_p=0.95, tfs_z=0.95, top_k=0, top_p=1.0,
               mirostat_mode=MirostatMode.Disabled)
        assert c.repeat_last_n in (0, 1024)


def test_bf16_rounding_is_nearest_even():
    x = np.array([1.0, 1.00390625, 1.01171875, -2.5, 3.0e38, 1.0 + 2.0 ** -8 + 2.0 ** -20], np.float32)
    b = wl.f32_to_bf16_bits(x)
    # 1 + 2^-8 is halfway between bf16 1.0 and 1 + 2^-7: ties go to the even 1.0; 1 + 3*2^-8 goes up
    assert list(wl.bf16_bits_to_f32(b)[:4]) == [1.0, 1.0, 1.015625, -2.5]
    assert wl.bf16_bits_to_f32(b)[5] == np.float32(1.0078125)  # just above halfway rounds up


def test_config5_small_batch():
    w = wl.config5(batch=16, vocab=4096)
    assert (w.batch, w.vocab, w.dtype, w.steps) == (16, 4096, "f32", 8)
    assert (w.mu == np.float32(10.0)).all() and (w.history_len == 256).all()
    assert w.history.shape[1] >= 256 + 8  # room for the 8 steps' records
    temps = np.array([c.temperature for c in w.configs])
    assert ((temps >= 0.5) & (temps <= 1.5)).all() and len(set(temps.tolist())) == 16
    for c in w.configs:
        _chain(c, presence_penalty=0.5, mirostat_mode=MirostatMode.V2, mirostat_tau=5.0, mirostat_eta=0.1,
               frequency_penalty=0.0, repeat_penalty=1.0)
    # fresh seeded logits each step, the same on every call
    s1, s1b, s2 = (wl.config5_step_logits(16, 4096, 7, s) for s in (1, 1, 2))
    assert np.array_equal(s1, s1b) and not np.array_equal(s1, s2)
    assert np.array_equal(w.logits, wl.config5_step_logits(16, 4096, wl.SEED_BASE + 5, 0))
    assert abs(float(s2.std()) - 2.0) < 0.05


def test_builders_are_seeded():
    a, b = wl.config1(), wl.config1()
    assert np.array_equal(a.logits, b.logits) and np.array_equal(a.history, b.history)
    assert np.array_equal(a.uniforms, b.uniforms)
    c = wl.config1(seed=wl.SEED_BASE + 99)
    assert not np.array_equal(a.logits, c.logits)
