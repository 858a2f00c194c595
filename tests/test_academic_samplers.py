"""The reference's known-answer tests for the sampling chain, run on both the
CPU oracle and the GPU sampler.

Each test restates one test of crates/oxide-core/tests/academic_samplers_test.rs
(or crates/oxide-server/tests/server_api_test.rs:100-121) with the same inputs
and assertions. The `gpu` variants go through the product's single-row API
(oxide_sampler.AcademicSamplerEngine -> oxs_sample_batch); the `oracle`
variants pin the CPU restatement that every other parity test trusts.
"""
import math

import numpy as np
import pytest

import oxs_oracle_ctypes as oracle
from oxide_sampler import AcademicSamplerEngine, MirostatMode, SamplerState, SamplingConfig, _abi
from oxide_sampler.engine import configs_to_array

BACKENDS = [pytest.param("oracle", id="oracle"), pytest.param("gpu", id="gpu", marks=pytest.mark.gpu)]


def engine(backend, config):
    if backend == "oracle":
        return oracle.OracleEngine(config, _abi, configs_to_array)
    return AcademicSamplerEngine(config)


@pytest.mark.parametrize("backend", BACKENDS)
def test_academic_sampler_temperature_and_top_k(backend):
    # academic_samplers_test.rs:6-20
    logits = [1.0, 2.0, 5.0, 3.0, 0.5]
    sampler = engine(backend, SamplingConfig(temperature=0.5, top_k=2))
    state = SamplerState.new(5.0)
    picked = sampler.sample_token(logits, state, 13)
    assert picked == 2
    assert state.generated_tokens == [2]


@pytest.mark.parametrize("backend", BACKENDS)
def test_academic_sampler_min_p_and_xtc(backend):
    # academic_samplers_test.rs:22-37: XTC drops the top choice, leaving token 1.
    logits = [10.0, 9.5, 2.0, 1.0]
    sampler = engine(backend, SamplingConfig(min_p=0.1, xtc_threshold=0.5, xtc_probability=1.0))
    state = SamplerState.new(5.0)
    assert sampler.sample_token(logits, state, 13) == 1


@pytest.mark.parametrize("backend", BACKENDS)
def test_dry_repetition_penalty(backend):
    # academic_samplers_test.rs:39-56
    logits = [5.0, 5.0, 5.0]
    sampler = engine(backend, SamplingConfig(dry_multiplier=2.0, dry_base=1.5, dry_allowed_length=2, dry_range=16))
    state = SamplerState.new(5.0)
    state.generated_tokens = [0, 1, 0, 1, 0, 1]
    assert sampler.sample_token(logits, state, 13) != 0


@pytest.mark.parametrize("backend", BACKENDS)
def test_sliding_window_repetition_penalty(backend):
    # academic_samplers_test.rs:58-76: 10.0 / 2.0 is left in logits[0].
    logits = [10.0, 5.0, 2.0]
    sampler = engine(backend, SamplingConfig(repeat_penalty=2.0, repeat_last_n=4, temperature=0.0))
    state = SamplerState.new(5.0)
    state.generated_tokens = [0]
    sampler.sample_token(logits, state, 13)
    assert logits[0] == 5.0


@pytest.mark.parametrize("backend", BACKENDS)
def test_mirostat_v2_sampling(backend):
    # academic_samplers_test.rs:78-92
    logits = [1.0, 2.0, 3.0, 4.0, 5.0]
    sampler = engine(backend, SamplingConfig(mirostat_mode=MirostatMode.V2, mirostat_tau=3.0, mirostat_eta=0.1))
    state = SamplerState.new(3.0)
    assert sampler.sample_token(logits, state, 13) == 4


@pytest.mark.parametrize("backend", BACKENDS)
def test_logit_bias_and_token_bans(backend):
    # academic_samplers_test.rs:125-137
    logits = [10.0, 5.0, 1.0]
    config = SamplingConfig()
    config.banned_tokens.add(0)
    config.logit_biases[2] = 20.0
    sampler = engine(backend, config)
    state = SamplerState.new(5.0)
    assert sampler.sample_token(logits, state, 13) == 2


@pytest.mark.parametrize("backend", BACKENDS)
def test_penalize_newline(backend):
    # academic_samplers_test.rs:139-153
    logits = [5.0, 5.0, 5.0]
    sampler = engine(backend, SamplingConfig(penalize_nl=True, newline_penalty=10.0))
    state = SamplerState.new(5.0)
    assert sampler.sample_token(logits, state, 1) != 1


@pytest.mark.parametrize("backend", BACKENDS)
def test_multinomial_seed_determinism_and_temperature(backend):
    # academic_samplers_test.rs:155-214
    logits_greedy = [1.0, 2.0, 8.0, 3.0]
    sampler_greedy = engine(backend, SamplingConfig(temperature=0.0))
    assert sampler_greedy.sample_token(logits_greedy, SamplerState.new(5.0), 0) == 2

    def draws():
        sampler = engine(backend, SamplingConfig(temperature=1.0, seed=42))
        state = SamplerState.new_with_seed(5.0, 42)
        out = []
        for _ in range(50):
            out.append(sampler.sample_token([2.0, 2.0, 2.0], state, 99))
        return out

    draws1, draws2 = draws(), draws()
    assert draws1 == draws2
    assert 0 in draws1 and 1 in draws1 and 2 in draws1


@pytest.mark.parametrize("backend", BACKENDS)
def test_academic_sampler_integration_with_logits(backend):
    # crates/oxide-server/tests/server_api_test.rs:100-121
    sampler = engine(backend, SamplingConfig(temperature=0.5, top_k=10, top_p=0.9, min_p=0.05))
    state = SamplerState.new(5.0)
    logits = [0.0] * 100
    logits[42] = 15.0
    logits[43] = 12.0
    sampled = sampler.sample_token(logits, state, 10)
    assert sampled in (42, 43)
    assert len(state.generated_tokens) == 1


@pytest.mark.parametrize("backend", BACKENDS)
def test_grammar_mask_disallowed_become_neg_inf(backend):
    # academic_samplers_test.rs:94-123 masks tokens 0 and 2 of four equal
    # logits. The device applies the same mask as a packed bitmask; the
    # oracle gets the -inf row the reference's masker would have written.
    if backend == "oracle":
        logits = [-math.inf, 10.0, -math.inf, 10.0]
        sampler = engine(backend, SamplingConfig(temperature=0.0))
        tok = sampler.sample_token(logits, SamplerState.new(5.0), 13)
    else:
        import torch
        from oxide_sampler import BatchSampler
        from oxide_sampler.workloads import pack_mask
        s = BatchSampler(1, 4)
        cfg, _, _, _ = configs_to_array([SamplingConfig(temperature=0.0)], 13)
        mask = pack_mask(np.array([[False, True, False, True]]), 4)
        d = torch.device("cuda")
        x = torch.full((1, 4), 10.0, device=d)
        lo = torch.empty(1, 4, device=d)
        out = s.sample(x, torch.from_numpy(cfg).to(d), mask=torch.from_numpy(mask.view(np.int32)).to(d),
                       uniforms=torch.zeros(1, device=d), logits_out=lo)
        torch.cuda.synchronize()
        logits = lo[0].cpu().tolist()
        tok = int(out["tokens"][0])
    assert logits[0] == -math.inf and logits[2] == -math.inf
    assert logits[1] == 10.0 and logits[3] == 10.0
    assert tok == 1  # greedy, ties to the lower id


@pytest.mark.parametrize("backend", BACKENDS)
def test_empty_logits_is_shape_mismatch(backend):
    # sampler.rs:179-181
    sampler = engine(backend, SamplingConfig())
    with pytest.raises(ValueError):
        sampler.sample_token([], SamplerState.new(5.0), 0)


@pytest.mark.parametrize("backend", BACKENDS)
def test_all_neg_inf_returns_zero_without_recording(backend):
    # sampler.rs:267-270
    sampler = engine(backend, SamplingConfig())
    state = SamplerState.new(5.0)
    rng0 = state.rng_state
    assert sampler.sample_token([-math.inf, float("nan"), -math.inf], state, 0) == 0
    assert state.generated_tokens == []
    assert state.rng_state == rng0  # no draw happened
