"""Seeded synthetic inputs for the five BASELINE configurations.

Each builder returns a `Workload` of host numpy arrays (logits, per-row
configs, histories, masks, uniforms, Mirostat state) that the GPU sampler and
the CPU oracle both consume, so the two see identical bytes. Data is synthetic
(there are no datasets or checkpoints offline); shapes and distributions follow
BASELINE.json's `configs`:

1. B=1,   V=32000  f32 N(0,2) + 5 spikes at +8, history 64;
   repeat 1.1 -> temp 0.8 -> top-k 40 -> top-p 0.95 -> draw.
2. B=64,  V=128256 f32 N(0,3) + Zipf(1.1)-shaped prior -1.1*ln(rank) over a
   per-row random permutation, history 512; freq 0.3 + presence 0.2 +
   repeat 1.05 -> temp 0.7 -> top-k 50 -> top-p 0.9 -> min-p 0.05 -> draw.
3. B=128, V=128256 f32 as (2) + packed allowed-mask with ~3% bits and one
   guaranteed id; mask -> temp 1.0 -> top-p 0.95 -> draw.
4. B=256, V=151936 bf16 N(0,2.5), 1% of entries U[6,10], history 1024;
   repeat 1.1 -> temp 0.9 -> tail-free 0.95 -> typical 0.95 -> draw
   (the reference runs tail-free before typical, sampler.rs:336-343).
5. B=512, V=262144 f32 N(0,2), per-row temperature U[0.5,1.5] (inert under
   Mirostat, sampler.rs:249), history 256; presence 0.5 -> Mirostat v2
   (tau 5, eta 0.1, mu0 10) for 8 steps with fresh logits each step.

Uniforms are 24-bit-grid values from a per-row xorshift64 stream (exactly
representable, identical on CPU and GPU).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

from .engine import MirostatMode, SamplingConfig, configs_to_array

SEED_BASE = 0x5EED0000


def disabled_config(**kw) -> SamplingConfig:
    """A SamplingConfig with every stage at its disabled value, then `kw`."""
    c = SamplingConfig(temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, tfs_z=1.0, typical_p=1.0,
                       xtc_probability=0.0, mirostat_mode=MirostatMode.Disabled, dry_multiplier=0.0,
                       repeat_penalty=1.0, repeat_last_n=0, frequency_penalty=0.0, presence_penalty=0.0,
                       penalize_nl=False)
    for k, v in kw.items():
        setattr(c, k, v)
    return c


@dataclass
class Workload:
    name: str
    logits: np.ndarray            # [B, V] float32, or uint16 bf16 bits
    dtype: str                    # "f32" | "bf16"
    configs: List[SamplingConfig]
    history: np.ndarray           # [B, cap] uint32
    history_len: np.ndarray       # [B] uint32
    uniforms: np.ndarray          # [B] float32
    mask: Optional[np.ndarray] = None   # [B, ceil(V/32)] uint32
    mu: Optional[np.ndarray] = None     # [B] float32
    steps: int = 1
    newline_token_id: int = 10
    extra: dict = field(default_factory=dict)

    @property
    def batch(self) -> int:
        return int(self.logits.shape[0])

    @property
    def vocab(self) -> int:
        return int(self.logits.shape[1])

    def packed_configs(self):
        return configs_to_array(self.configs, self.newline_token_id)


def xorshift_uniforms(n: int, seed: int) -> np.ndarray:
    """n values of SamplerState::next_f32 (sampler.rs:139-153), one per row stream."""
    out = np.empty(n, dtype=np.float32)
    mask = (1 << 64) - 1
    for i in range(n):
        x = (seed * 0x9E3779B97F4A7C15 + i * 0xBF58476D1CE4E5B9 + 1) & mask or 1
        for _ in range(3):  # decorrelate nearby seeds
            x ^= (x << 13) & mask
            x ^= x >> 7
            x ^= (x << 17) & mask
        out[i] = np.float32(np.uint32(x >> 40)) / np.float32(16777216.0)
    return out


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit patterns."""
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return rounded.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def pack_mask(allowed: np.ndarray, vocab: int) -> np.ndarray:
    """[B, V] bool -> [B, ceil(V/32)] uint32 with bit (i % 32) of word i // 32 = allowed[i]."""
    B = allowed.shape[0]
    words = (vocab + 31) // 32
    bits = np.zeros((B, words * 32), dtype=bool)
    bits[:, :vocab] = allowed[:, :vocab]
    packed = np.packbits(bits.reshape(B, words, 32), axis=-1, bitorder="little")
    return np.ascontiguousarray(packed).view("<u4").reshape(B, words).astype(np.uint32)


def zipf_prior_logits(rng: np.random.Generator, B: int, V: int, sigma: float) -> np.ndarray:
    """N(0, sigma) plus -1.1*ln(rank) over a per-row random permutation of ranks."""
    prior = (-1.1 * np.log(np.arange(1, V + 1, dtype=np.float64))).astype(np.float32)
    out = rng.standard_normal((B, V), dtype=np.float32) * np.float32(sigma)
    for b in range(B):
        out[b] += prior[rng.permutation(V)]
    return out


def config1(batch: int = 1, vocab: int = 32000, seed: int = SEED_BASE + 1) -> Workload:
    rng = np.random.default_rng(seed)
    logits = rng.standard_normal((batch, vocab), dtype=np.float32) * np.float32(2.0)
    for b in range(batch):
        logits[b, rng.choice(vocab, 5, replace=False)] = np.float32(8.0)
    H = 64
    hist = rng.integers(0, vocab, (batch, H + 2), dtype=np.uint32)
    cfg = disabled_config(repeat_penalty=1.1, repeat_last_n=64, temperature=0.8, top_k=40, top_p=0.95, min_p=0.0)
    return Workload("config1", logits, "f32", [cfg] * batch, hist, np.full(batch, H, np.uint32),
                    xorshift_uniforms(batch, seed))


def config2(batch: int = 64, vocab: int = 128256, seed: int = SEED_BASE + 2) -> Workload:
    rng = np.random.default_rng(seed)
    logits = zipf_prior_logits(rng, batch, vocab, 3.0)
    H = 512
    hist = rng.integers(0, vocab, (batch, H + 2), dtype=np.uint32)
    cfg = disabled_config(frequency_penalty=0.3, presence_penalty=0.2, repeat_penalty=1.05, repeat_last_n=512,
                          temperature=0.7, top_k=50, top_p=0.9, min_p=0.05)
    return Workload("config2", logits, "f32", [cfg] * batch, hist, np.full(batch, H, np.uint32),
                    xorshift_uniforms(batch, seed))


def config2_dry(batch: int = 64, vocab: int = 128256, seed: int = SEED_BASE + 22) -> Workload:
    """Config 2 with DRY on every row (multiplier 0.8, base 1.75, allowed length 2, range 1024) over
    histories that end in a repeated motif of high-logit ids, so that DRY penalises candidates."""
    w = config2(batch, vocab, seed)
    rng = np.random.default_rng(seed + 1)
    x = w.logits
    H = int(w.history_len[0])
    for b in range(batch):
        top = np.argsort(-x[b])[:32].astype(np.uint32)
        motif = rng.choice(top, 6, replace=False)
        w.history[b, H - 48:H] = np.tile(motif, 8)
        w.history[b, rng.integers(0, H - 100, 6)] = motif[0]
    cfg = disabled_config(frequency_penalty=0.3, presence_penalty=0.2, repeat_penalty=1.05, repeat_last_n=512,
                          temperature=0.7, top_k=50, top_p=0.9, min_p=0.05, dry_multiplier=0.8, dry_base=1.75,
                          dry_allowed_length=2, dry_range=1024)
    w.configs = [cfg] * batch
    w.name = "config2_dry"
    return w


def config3(batch: int = 128, vocab: int = 128256, seed: int = SEED_BASE + 3) -> Workload:
    rng = np.random.default_rng(seed)
    logits = zipf_prior_logits(rng, batch, vocab, 3.0)
    words = (vocab + 31) // 32
    bits = rng.random((batch, words * 32)) < 0.03
    bits[:, vocab:] = False
    guaranteed = rng.integers(0, vocab, batch)
    bits[np.arange(batch), guaranteed] = True
    mask = pack_mask(bits[:, :vocab], vocab)
    cfg = disabled_config(temperature=1.0, top_p=0.95)
    return Workload("config3", logits, "f32", [cfg] * batch, np.zeros((batch, 2), np.uint32),
                    np.zeros(batch, np.uint32), xorshift_uniforms(batch, seed), mask=mask,
                    extra={"guaranteed": guaranteed})


def config4(batch: int = 256, vocab: int = 151936, seed: int = SEED_BASE + 4) -> Workload:
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((batch, vocab), dtype=np.float32) * np.float32(2.5)
    heavy = rng.random((batch, vocab)) < 0.01
    x[heavy] = rng.uniform(6.0, 10.0, int(heavy.sum())).astype(np.float32)
    logits = f32_to_bf16_bits(x)
    H = 1024
    hist = rng.integers(0, vocab, (batch, H + 2), dtype=np.uint32)
    cfg = disabled_config(repeat_penalty=1.1, repeat_last_n=1024, temperature=0.9, typical_p=0.95, tfs_z=0.95)
    return Workload("config4", logits, "bf16", [cfg] * batch, hist, np.full(batch, H, np.uint32),
                    xorshift_uniforms(batch, seed))


def config5(batch: int = 512, vocab: int = 262144, seed: int = SEED_BASE + 5, steps: int = 8) -> Workload:
    """Step 0's logits; `config5_step_logits` gives the logits of later steps."""
    rng = np.random.default_rng(seed)
    logits = config5_step_logits(batch, vocab, seed, 0)
    H = 256
    cap = H + 2 * steps
    hist = np.zeros((batch, cap), np.uint32)
    hist[:, :H] = rng.integers(0, vocab, (batch, H), dtype=np.uint32)
    temps = rng.uniform(0.5, 1.5, batch).astype(np.float32)
    cfgs = [disabled_config(presence_penalty=0.5, repeat_last_n=0, mirostat_mode=MirostatMode.V2,
                            mirostat_tau=5.0, mirostat_eta=0.1, temperature=float(t)) for t in temps]
    return Workload("config5", logits, "f32", cfgs, hist, np.full(batch, H, np.uint32),
                    xorshift_uniforms(batch, seed), mu=np.full(batch, 10.0, np.float32), steps=steps)


def config5_step_logits(batch: int, vocab: int, seed: int, step: int) -> np.ndarray:
    rng = np.random.default_rng([seed, step])
    return rng.standard_normal((batch, vocab), dtype=np.float32) * np.float32(2.0)


BUILDERS = {1: config1, 2: config2, 3: config3, 4: config4, 5: config5}
