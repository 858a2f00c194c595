"""The reference's sampler tests through the C++ mirror of its API.

tests/cpp/academic_samplers_test.cpp ports every case of
crates/oxide-core/tests/academic_samplers_test.rs (and the sampler case of
oxide-server/tests/server_api_test.rs:100-121) onto
oxide-tech-llm-engine_amd/cpp/oxide_sampler.hpp: SamplingConfig, SamplerState,
AcademicSamplerEngine::sample_token and GbnfGrammarEngine in C++, each call
running on the GPU through liboxide_sampler.so. The binary is built in-tree by
the package build (tests/cpp/Makefile).
"""
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CPP = ROOT / "tests" / "cpp"
BIN = CPP / "_bin" / "academic_samplers_test"

# cases that need no device: host-side SamplerState and the empty-row check
HOST_CASES = ["sampler_state_rng", "empty_row_is_shape_mismatch"]
GPU_CASES = ["temperature_and_top_k", "min_p_and_xtc", "dry_repetition_penalty",
             "sliding_window_repetition_penalty", "mirostat_v2_sampling", "logit_bias_and_token_bans",
             "penalize_newline", "multinomial_seed_determinism_and_temperature", "server_api_sampling",
             "gbnf_grammar_constrained_masking", "all_masked_row"]


def _binary() -> Path:
    if not BIN.exists():
        pytest.skip("tests/cpp not built (run __graft_entry__.build())")
    return BIN


def _run(cases, timeout):
    r = subprocess.run([str(_binary()), *cases], capture_output=True, text=True, timeout=timeout)
    print(r.stdout, r.stderr, flush=True)
    return r


def test_cpp_mirror_builds_and_links(tmp_path):
    # compiles the header and the test against the C ABI with warnings as errors
    lib = ROOT / "oxide-tech-llm-engine_amd" / "lib" / "liboxide_sampler.so"
    if not lib.exists():
        pytest.skip("liboxide_sampler.so not built")
    out = tmp_path / "t"
    subprocess.run(["make", "-s", "-C", str(CPP), f"OUT={out}",
                    "CXXFLAGS=-O0 -std=c++17 -Wall -Wextra -Werror -D__HIP_PLATFORM_AMD__ -I/opt/rocm/include"],
                   check=True, timeout=300)
    assert out.exists()


def test_cpp_mirror_host_cases():
    r = _run(HOST_CASES, 60)
    assert r.returncode == 0
    for c in HOST_CASES:
        assert f"ok {c}" in r.stdout


@pytest.mark.gpu
def test_cpp_mirror_reference_cases(torch_gpu):
    print("\n[case] C++ mirror: academic_samplers_test.rs cases", flush=True)
    r = _run([], 120)
    for c in HOST_CASES + GPU_CASES:
        assert f"ok {c}" in r.stdout, c
    assert r.returncode == 0
