"""The device's expf/logf/log2f/powf/tanhf (oxs_libm.h) against the host glibc, bit for bit.

The GPU kernels reproduce the reference's f32::{exp, ln, log2}
(sampler.rs:289, :424, :440, :451, :496, :502) and f32::powf (:409, DRY), and f32::tanh for the logit softcap, which
lower to glibc on
x86_64-linux-gnu. oxs_libm.h compiles as plain host C++ too, so this test
builds tests/libm_sweep.cpp with g++ and compares every 197th float bit
pattern plus dense sweeps of the softmax and probability ranges. glibc picks
its FMA build on CPUs with FMA and AVX2; the fused form must match it there.
"""
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


def _host_has_fma() -> bool:
    try:
        flags = Path("/proc/cpuinfo").read_text().split()
    except OSError:
        return False
    return "fma" in flags and "avx2" in flags


@pytest.fixture(scope="module")
def sweep_bin(tmp_path_factory):
    out = tmp_path_factory.mktemp("libm") / "libm_sweep"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-fno-fast-math", "-o", str(out),
                    str(HERE / "libm_sweep.cpp"), "-lm"], check=True)
    return out


@pytest.mark.parametrize("fused", [1, 0])
def test_device_libm_matches_host_glibc(sweep_bin, fused):
    if fused == 0 and _host_has_fma():
        # glibc runs its FMA build here; the generic form is still swept and
        # reported, and must agree except where fusing changes the last bit.
        pass
    res = subprocess.run([str(sweep_bin), str(fused), "197"], capture_output=True, text=True, timeout=300)
    lines = dict((l.split()[0], l.split()[1:]) for l in res.stdout.strip().splitlines())
    assert set(lines) == {"expf", "logf", "log2f", "powf", "tanhf"}, res.stdout + res.stderr
    for fn, (checked, bad, first) in lines.items():
        assert int(checked) > (500_000 if fn == "powf" else 10_000_000), f"{fn}: sweep too small"
        if fused == 1 or not _host_has_fma():
            assert int(bad) == 0, f"{fn}: {bad} of {checked} differ from glibc (first input bits {first})"
