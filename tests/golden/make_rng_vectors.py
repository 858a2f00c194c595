"""Writes rng_vectors.json: SamplerState's xorshift64 stream and next_f32 values.

The generator restates crates/oxide-core/src/sampler.rs:139-153 with Python
integers (no fixed-width types to overflow), independently of the C++ oracle
and of the device code. The seeds cover SamplerState::default / new
(0x853c_49e6_748f_ea9b, sampler.rs:98 and :110), new_with_seed(42), seed 1
(whose first step is derived by hand in the test) and a value with high bits
set. Run: python tests/golden/make_rng_vectors.py
"""
import json
import struct
from pathlib import Path

MASK = (1 << 64) - 1
SEEDS = [0x853C49E6748FEA9B, 42, 1, 0xDEADBEEFCAFEF00D]
STEPS = 16


def f32(x: float) -> float:
    """Rounds a Python float to the nearest binary32 value."""
    return struct.unpack("<f", struct.pack("<f", x))[0]


def main() -> None:
    out = []
    for seed in SEEDS:
        x = seed
        u64, f = [], []
        for _ in range(STEPS):
            x ^= (x << 13) & MASK
            x ^= x >> 7
            x ^= (x << 17) & MASK
            u64.append(x)
            # (x >> 40) fits in 24 bits, so both the u32 -> f32 conversion and
            # the division by 2^24 are exact.
            f.append(f32((x >> 40) / 16777216.0))
        out.append({"seed": f"{seed:#018x}", "next_u64": [f"{v:#018x}" for v in u64], "next_f32": f})
    path = Path(__file__).with_name("rng_vectors.json")
    path.write_text(json.dumps({"source": "sampler.rs:139-153", "vectors": out}, indent=1) + "\n")
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
