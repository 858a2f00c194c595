"""The float identity behind the stream kernel's survivor mask.

Each wavefront keeps the values at or above its threshold t. The kernel reads
that bit as the inverted sign bit of v - tq (tq = -0.0 when t is +0.0 or -0.0,
else t), computed in f32 with round to nearest and IEEE denormals, as the
kernel is compiled. For every v that is not NaN and every t that is not
infinite or NaN (the kernel keeps a plain comparison for those), the sign bit
is 0 exactly when v >= t. A NaN v may set its bit; the kernel drops it when
the value's key is formed. These checks compare the sign rule with the
comparison itself, over the f32 edge cases and random values, and show that
using +0.0 for a zero threshold would miss v = -0.0.
"""
import numpy as np

F32 = np.float32
EDGES = np.array([0.0, -0.0, 1e-45, -1e-45, 1.17549435e-38, -1.17549435e-38, 1e-30, -1e-30, 0.5, -0.5, 1.0,
                  -1.0, 1.0000001, 3.4028235e38, -3.4028235e38, np.inf, -np.inf], dtype=F32)


def sign_rule(v, t):
    tq = np.where(t == 0, F32(-0.0), t).astype(F32)
    with np.errstate(over="ignore", invalid="ignore"):
        d = (v - tq).astype(F32)
    return ~np.signbit(d)


def check(v, t):
    keep = sign_rule(v, t)
    want = v >= t
    bad = keep != want
    assert not bad.any(), (v[bad][:5], t[bad][:5] if np.ndim(t) else t)


def test_edge_values_against_every_finite_threshold():
    thresholds = EDGES[np.isfinite(EDGES)]
    for t in thresholds:
        check(EDGES, np.full(EDGES.shape, t, F32))


def test_random_values_and_thresholds():
    rng = np.random.default_rng(11)
    for scale in (1e-40, 1e-3, 1.0, 1e30):
        v = (rng.standard_normal(200_000) * scale).astype(F32)
        t = (rng.standard_normal(200_000) * scale).astype(F32)
        t[::7] = v[::7]  # equal pairs
        check(v, t)


def test_random_bit_patterns():
    rng = np.random.default_rng(12)
    v = rng.integers(0, 2**32, 400_000, dtype=np.uint64).astype(np.uint32).view(F32)
    t = rng.integers(0, 2**32, 400_000, dtype=np.uint64).astype(np.uint32).view(F32)
    ok = ~np.isnan(v) & np.isfinite(t)
    check(v[ok], t[ok])


def test_plus_zero_threshold_would_drop_minus_zero():
    v = np.array([-0.0], F32)
    with np.errstate(invalid="ignore"):
        plain = ~np.signbit((v - F32(0.0)).astype(F32))
    assert not plain[0] and v[0] >= F32(0.0)  # the reason for tq = -0.0
    assert sign_rule(v, np.array([0.0], F32))[0]
