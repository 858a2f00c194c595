"""The C ABI on a CPU host: the library loads and exports every entry point
that include/oxide_sampler.h declares, and its host-only helpers return the
reference's defaults. No call here touches a GPU.
"""
import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from oxide_sampler import SamplingConfig, _abi

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "oxide_sampler.h"


def _declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b(oxs_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not _abi.LIB_PATH.exists():
        subprocess.run(["make", "-j8", "-C", str(ROOT / "oxide-tech-llm-engine_amd")], check=True)
    return _abi.load_library()


def test_header_declares_the_entry_points():
    names = _declared_functions()
    for want in ("oxs_sampler_create", "oxs_sampler_destroy", "oxs_sample_batch", "oxs_sampler_workspace_bytes",
                 "oxs_sampling_config_default", "oxs_rng_state_from_seed", "oxs_mirostat_mu_from_tau",
                 "oxs_status_string", "oxs_abi_version"):
        assert want in names


def test_library_exports_every_declared_symbol(lib):
    dyn = subprocess.run(["nm", "-D", "--defined-only", str(_abi.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {l.split()[-1] for l in dyn.splitlines() if l.strip()}
    for name in _declared_functions():
        assert name in exported, f"{name} is declared in oxide_sampler.h but not exported"
        assert hasattr(lib, name)


def test_abi_version_and_struct_sizes(lib):
    assert lib.oxs_abi_version() == _abi.OXS_ABI_VERSION
    assert ctypes.sizeof(_abi.OxsSamplingConfig) == 26 * 4


def test_status_strings(lib):
    for code in (_abi.OXS_OK, _abi.OXS_ERR_INVALID_ARGUMENT, _abi.OXS_ERR_UNSUPPORTED):
        s = lib.oxs_status_string(code)
        assert s and len(s.decode()) >= 2
    assert lib.oxs_status_string(_abi.OXS_OK) != lib.oxs_status_string(_abi.OXS_ERR_UNSUPPORTED)


def test_config_default_matches_reference_defaults(lib):
    # sampler.rs:44-73, which the Python mirror's SamplingConfig also carries.
    c = _abi.OxsSamplingConfig()
    lib.oxs_sampling_config_default(ctypes.byref(c))
    ref = SamplingConfig()
    for name in ("temperature", "top_p", "min_p", "tfs_z", "typical_p", "xtc_threshold", "xtc_probability",
                 "mirostat_tau", "mirostat_eta", "dry_multiplier", "dry_base", "repeat_penalty",
                 "frequency_penalty", "presence_penalty", "newline_penalty"):
        assert getattr(c, name) == float(np.float32(getattr(ref, name))), name
    assert c.top_k == 40 and c.repeat_last_n == 64 and c.dry_allowed_length == 2 and c.dry_range == 1024
    assert c.mirostat_mode == _abi.OXS_MIROSTAT_DISABLED and c.penalize_nl == 0
    assert c.bias_count == 0 and c.ban_count == 0


def test_rng_seed_and_mu_helpers(lib):
    # SamplerState::new / new_with_seed (sampler.rs:104-128): the default state, seed 0 maps to it.
    default = 0x853C49E6748FEA9B
    assert lib.oxs_rng_state_from_seed(0, 123) == default
    assert lib.oxs_rng_state_from_seed(1, 0) == default
    assert lib.oxs_rng_state_from_seed(1, 42) == 42
    assert lib.oxs_mirostat_mu_from_tau(5.0) == 10.0
    assert lib.oxs_mirostat_mu_from_tau(3.0) == 6.0


def test_create_rejects_bad_arguments_without_a_device(lib):
    # Argument checks run before any HIP call.
    h = ctypes.c_void_p()
    assert lib.oxs_sampler_create(None, None, 0) == _abi.OXS_ERR_INVALID_ARGUMENT
    lim = _abi.OxsLimits(0, 1000, 256)
    assert lib.oxs_sampler_create(ctypes.byref(h), ctypes.byref(lim), 0) == _abi.OXS_ERR_INVALID_ARGUMENT
    assert lib.oxs_sample_batch(None, None, None) == _abi.OXS_ERR_INVALID_ARGUMENT
    assert lib.oxs_sampler_destroy(None) in (_abi.OXS_OK, _abi.OXS_ERR_INVALID_ARGUMENT)


_STRUCTS = ("oxs_sampling_config", "oxs_limits", "oxs_batch", "oxs_decode_io", "oxs_dfa", "oxs_token_bytes",
            "oxs_gbnf_rule")


def _c_layouts(tmp_path):
    """sizeof and every field's offset of the header's structs, from a C compiler."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    fields = {}
    for name in _STRUCTS:
        body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (name, name), text, flags=re.S).group(1)
        fields[name] = re.findall(r"(\w+)\s*;", body)
    lines = ["#include <stddef.h>", "#include <stdio.h>", f'#include "{HEADER}"', "int main(void) {"]
    for name, fs in fields.items():
        lines.append(f'  printf("{name} sizeof %zu\\n", sizeof({name}));')
        for f in fs:
            lines.append(f'  printf("{name} {f} %zu\\n", offsetof({name}, {f}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-o", str(exe), str(src)], check=True)
    out = {}
    for l in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines():
        s, f, v = l.split()
        out[(s, f)] = int(v)
    return fields, out


def test_ctypes_structs_match_the_header_layout(tmp_path):
    # every struct the Python binding passes through the ABI, field by field
    py = {"oxs_sampling_config": _abi.OxsSamplingConfig, "oxs_limits": _abi.OxsLimits, "oxs_batch": _abi.OxsBatch,
          "oxs_decode_io": _abi.OxsDecodeIo, "oxs_dfa": _abi.OxsDfa, "oxs_token_bytes": _abi.OxsTokenBytes,
          "oxs_gbnf_rule": _abi.OxsGbnfRule}
    fields, c = _c_layouts(tmp_path)
    for name, cls in py.items():
        assert [f for f, _ in cls._fields_] == fields[name], name
        assert ctypes.sizeof(cls) == c[(name, "sizeof")], name
        for f in fields[name]:
            assert getattr(cls, f).offset == c[(name, f)], (name, f)
