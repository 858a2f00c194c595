"""The LM head in the reference's Q8_0 x q8_1 formats: oracle pins and GPU parity.

Reference: launch_cuda_quantize_q8_1 (quantize_f32_to_q8_1_cuda_kernel,
oxide-backend-cuda/src/kernels/norms_rope.cu:2-29) and launch_cuda_mmvq_q8_0
(mmvq_q8_0_cuda_kernel, quant_gemv_standard.cu:425-513), called by the batched
decode at oxide-backend-cuda/src/lib.rs:4013-4035. The reference ships no test
vectors for these kernels; the oracle is pinned by:
- IEEE half conversions: every half against numpy, and float->half rounding
  against numpy on random and edge values;
- q8_1: the butterfly-order sum on a hand-worked block where it differs from
  a left-to-right sum, the dequantisation bound |x - q d| <= d / 2 and
  q = +-127 at the largest magnitude;
- Q8_0 x q8_1: a single block's value in closed form, the (A0 + A2) + (A1 + A3)
  order and the fused multiply-add on hand-worked blocks where the other
  orders and an unfused product give different floats, and a float64 bound.
The GPU path is then compared with the oracle bit for bit.
"""
import math
from fractions import Fraction

import numpy as np
import pytest

import oxs_oracle_ctypes as oracle


def f16(v):
    return np.float16(v).view(np.uint16)


def q8_0_rows(scales, quants):
    """GGUF Q8_0 bytes from scales [m, nb] (float) and quants [m, nb, 32] (int8)."""
    m, nb = scales.shape
    blocks = np.zeros((m, nb, 34), np.uint8)
    blocks[:, :, 0:2] = np.asarray(scales, np.float16).view(np.uint8).reshape(m, nb, 2)
    blocks[:, :, 2:] = np.asarray(quants, np.int8).view(np.uint8)
    return blocks.reshape(-1)


def q8_1_rows(scales, quants, sums=None):
    """q8_1 bytes from d [batch, nb], quants [batch, nb, 32] (and optional sums)."""
    batch, nb = scales.shape
    blocks = np.zeros((batch, nb, 36), np.uint8)
    blocks[:, :, 0:2] = np.asarray(scales, np.float16).view(np.uint8).reshape(batch, nb, 2)
    if sums is not None:
        blocks[:, :, 2:4] = np.asarray(sums, np.float16).view(np.uint8).reshape(batch, nb, 2)
    blocks[:, :, 4:] = np.asarray(quants, np.int8).view(np.uint8)
    return blocks.reshape(-1)


def random_case(rng, m, k, batch):
    nb = k // 32
    ws = rng.uniform(0.002, 0.05, size=(m, nb)) * rng.choice([-1, 1], size=(m, nb))
    wq = rng.integers(-128, 128, size=(m, nb, 32))
    x = rng.normal(0, 1.5, size=(batch, k)).astype(np.float32)
    return q8_0_rows(ws, wq), x


# ----------------------------------------------------------------------------- oracle pins

def test_half_to_float_every_half():
    h = np.arange(65536, dtype=np.uint16)
    got = oracle.f16_to_f32_host(h)
    want = h.view(np.float16).astype(np.float32)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all()


def test_float_to_half_rounding():
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.normal(0, 100, 20000).astype(np.float32),
        rng.uniform(-1e-4, 1e-4, 20000).astype(np.float32),      # subnormal halves
        np.float32(2.0) ** rng.integers(-30, 17, 5000).astype(np.float32) * rng.uniform(1, 2, 5000).astype(np.float32),
        np.array([0.0, -0.0, 65504, 65519.99, 65520, 1e9, -1e9, np.inf, -np.inf, 2.0 ** -24, 2.0 ** -25,
                  2.0 ** -25 * 1.0000001, 3 * 2.0 ** -26, 1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, 6.1e-5], np.float32),
    ])
    got = oracle.f32_to_f16_host(vals)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, want)


def test_quantize_butterfly_sum_known_answer():
    # x0 = 2^24, x16 = -2^24, x1 = 1: the butterfly adds x0 + x16 first (offset 16),
    # so lane 0 ends with 0 + 1 = 1; a left-to-right sum would lose the 1 (2^24 + 1 = 2^24)
    x = np.zeros(32, np.float32)
    x[0], x[16], x[1] = 2.0 ** 24, -(2.0 ** 24), 1.0
    out = oracle.quantize_q8_1_host(x)
    assert out[2:4].view(np.float16)[0] == 1.0
    assert out[0:2].view(np.uint16)[0] == 0x7C00  # d = 2^24 / 127 overflows half: +inf, as __float2half gives
    q = out[4:].view(np.int8)
    assert q[0] == 127 and q[16] == -127 and q[1] == 0


def test_quantize_bounds_and_zero_block():
    rng = np.random.default_rng(1)
    x = rng.normal(0, 3, size=64 * 32).astype(np.float32)
    x[:32] = 0.0  # amax 0: d = 0, id = 0, every q 0
    out = oracle.quantize_q8_1_host(x).reshape(-1, 36)
    assert (out[0] == 0).all()
    for blk in range(1, 64):
        v = x[blk * 32:(blk + 1) * 32]
        q = out[blk, 4:].view(np.int8).astype(np.int32)
        d = np.float32(np.abs(v).max()) / np.float32(127)
        assert abs(int(q[np.abs(v).argmax()])) == 127
        assert np.all(np.abs(v - q * d) <= d * (0.5 + 1e-5))
        assert out[blk, 0:2].view(np.float16)[0] == np.float16(d)
        assert abs(float(out[blk, 2:4].view(np.float16)[0]) - float(v.astype(np.float64).sum())) <= \
            1e-3 * (1 + abs(float(v.sum())))


def test_mmvq_single_block_closed_form():
    # one nonzero block: y = round(d_w * d_x * dot), the product d_w * d_x rounded first
    k, nb = 128, 4
    ws = np.zeros((1, nb)); ws[0, 2] = 0.0123
    wq = np.zeros((1, nb, 32), np.int64); wq[0, 2] = np.arange(32) - 16
    xs = np.full((1, nb), 0.377)
    xq = np.zeros((1, nb, 32), np.int64); xq[0, 2] = 3 * (np.arange(32) % 7) - 9
    y = oracle.mmvq_q8_0_host(q8_0_rows(ws, wq), q8_1_rows(xs, xq), 1, k, 1)
    dot = int(np.dot(wq[0, 2], xq[0, 2]))
    dd = np.float32(np.float16(0.0123)) * np.float32(np.float16(0.377))
    assert y[0, 0] == np.float32(float(Fraction(float(dd)) * dot))


def _blocks_with(products):
    """Blocks b = 0.. whose d_w * d_x * dot are the given (d_w, d_x, dot) triples."""
    nb = len(products)
    ws, xs = np.zeros((1, nb)), np.zeros((1, nb))
    wq, xq = np.zeros((1, nb, 32), np.int64), np.zeros((1, nb, 32), np.int64)
    for b, (dw, dx, dot) in enumerate(products):
        ws[0, b], xs[0, b] = dw, dx
        # dot as a sum of 32 int8 products: 127 * 127 terms and one remainder term
        rem, e = dot, 0
        sign = 1 if dot >= 0 else -1
        while abs(rem) > 127 * 127:
            wq[0, b, e], xq[0, b, e] = 127, 127 * sign
            rem -= 127 * 127 * sign
            e += 1
        # the remainder as one product of int8 values (-128 for w allows 128 * 126)
        for w in list(range(127, 0, -1)) + [-128]:
            if rem % w == 0 and -128 <= rem // w <= 127:
                wq[0, b, e], xq[0, b, e] = w, rem // w
                break
        else:
            raise AssertionError(f"cannot write {rem} as one int8 product")
        assert int(np.dot(wq[0, b].astype(np.int8).astype(np.int64), xq[0, b].astype(np.int8).astype(np.int64))) == dot
    return q8_0_rows(ws, wq), q8_1_rows(xs, xq)


def test_mmvq_reduction_order_known_answer():
    # A0 = 2^24, A1 = 1, A2 = -2^24, A3 = 0.5:
    #   (A0 + A2) + (A1 + A3) = 1.5 (the reference's shuffle order)
    #   ((A0 + A1) + A2) + A3 = 0.5 and (A0 + A1) + (A2 + A3) = 0 in float32
    w, x = _blocks_with([(256.0, 256.0, 256), (1.0, 1.0, 1), (256.0, 256.0, -256), (0.5, 1.0, 1)])
    assert oracle.mmvq_q8_0_host(w, x, 1, 128, 1)[0, 0] == 1.5


def test_mmvq_fused_multiply_add_known_answer():
    # block 0 leaves A0 = 2^-6; block 4 adds (1 + 2^-10) * 516127 = 516631.0302734375 exactly.
    # fmaf rounds 516631.0458984375 once: 516631.03125; a rounded product then an
    # add gives 516631.03125 + 0.015625 = 516631.046875, a tie that rounds to 516631.0625.
    prods = [(2.0 ** -6, 1.0, 1), (0.0, 0.0, 0), (0.0, 0.0, 0), (0.0, 0.0, 0),
             (1 + 2.0 ** -10, 1.0, 516127), (0.0, 0.0, 0), (0.0, 0.0, 0), (0.0, 0.0, 0)]
    w, x = _blocks_with(prods)
    got = oracle.mmvq_q8_0_host(w, x, 1, 256, 1)[0, 0]
    exact = Fraction(1, 64) + Fraction(1025, 1024) * 516127
    assert got == np.float32(float(exact)) == np.float32(516631.03125)
    unfused = np.float32(np.float32(float(Fraction(1025, 1024) * 516127)) + np.float32(2.0 ** -6))
    assert unfused == np.float32(516631.0625) != got


@pytest.mark.parametrize("m,k,batch", [(37, 128, 3), (64, 896, 2)])
def test_mmvq_against_float64(m, k, batch):
    rng = np.random.default_rng(m * k + batch)
    w, x = random_case(rng, m, k, batch)
    xq = oracle.quantize_q8_1_host(x)
    y = oracle.mmvq_q8_0_host(w, xq, m, k, batch)
    nb = k // 32
    wb = w.reshape(m, nb, 34)
    xb = xq.reshape(batch, nb, 36)
    wd = wb[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    xd = xb[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    wqv = wb[:, :, 2:].view(np.int8).astype(np.float64)
    xqv = xb[:, :, 4:].view(np.int8).astype(np.float64)
    dots = np.einsum("mbe,cbe->cmb", wqv, xqv)
    terms = dots * wd[None, :, :] * xd[:, None, :]
    exact = terms.sum(axis=2)
    bound = np.abs(terms).sum(axis=2) * 2.0 ** -22 + 1e-30
    assert np.all(np.abs(y - exact) <= bound)


# ----------------------------------------------------------------------------- GPU

def _to_dev(torch, arr):
    return torch.from_numpy(np.ascontiguousarray(arr)).cuda()


@pytest.mark.gpu
@pytest.mark.parametrize("batch,k", [(1, 128), (3, 4096), (77, 896)])
def test_gpu_quantize_matches_oracle(torch_gpu, batch, k):
    from oxide_sampler import quantize_q8_1
    rng = np.random.default_rng(batch * 7 + k)
    x = rng.normal(0, 2, size=(batch, k)).astype(np.float32)
    x[0, :32] = 0.0  # a zero block
    x[-1, 32:64] *= 1e-30  # subnormal-scale block
    print(f"\n[case] quantize_q8_1 batch={batch} k={k}", flush=True)
    got = quantize_q8_1(_to_dev(torch_gpu, x)).cpu().numpy().reshape(-1)
    np.testing.assert_array_equal(got, oracle.quantize_q8_1_host(x))


@pytest.mark.gpu
@pytest.mark.parametrize("m,k,batch", [(1, 128, 1), (33, 128, 3), (130, 256, 64), (1001, 896, 65),
                                       (4099, 512, 130), (2050, 4096, 7), (517, 4096, 1), (300, 1024, 2),
                                       (129, 4096, 4), (70, 16384, 4), (64, 16384, 5), (257, 4096, 6), (96, 4096, 8),
                                       (40, 8192, 8), (33, 128, 9)])
def test_gpu_mmvq_matches_oracle(torch_gpu, m, k, batch):
    # batch <= 4 with x (staged for 1, 2 or 4 columns) within 64 KB of LDS takes the
    # small-batch kernel; (70, 16384, 4) and batch > 4 take the MFMA kernel
    from oxide_sampler import LmHeadQ8_0, quantize_q8_1
    rng = np.random.default_rng(m + 3 * k + 7 * batch)
    w, x = random_case(rng, m, k, batch)
    print(f"\n[case] mmvq_q8_0 m={m} k={k} batch={batch}", flush=True)
    head = LmHeadQ8_0(w, m, k)
    xq = quantize_q8_1(_to_dev(torch_gpu, x))
    got = head.project(xq.view(batch, -1)).cpu().numpy()
    want = oracle.mmvq_q8_0_host(w, oracle.quantize_q8_1_host(x), m, k, batch)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.gpu
def test_gpu_mmvq_known_answers(torch_gpu):
    from oxide_sampler import LmHeadQ8_0
    print("\n[case] mmvq_q8_0 hand-worked blocks", flush=True)
    w, x = _blocks_with([(256.0, 256.0, 256), (1.0, 1.0, 1), (256.0, 256.0, -256), (0.5, 1.0, 1)])
    y = LmHeadQ8_0(w, 1, 128).project(_to_dev(torch_gpu, x).view(1, -1)).cpu().numpy()
    assert y[0, 0] == 1.5
    prods = [(2.0 ** -6, 1.0, 1), (0.0, 0.0, 0), (0.0, 0.0, 0), (0.0, 0.0, 0),
             (1 + 2.0 ** -10, 1.0, 516127), (0.0, 0.0, 0), (0.0, 0.0, 0), (0.0, 0.0, 0)]
    w, x = _blocks_with(prods)
    y = LmHeadQ8_0(w, 1, 256).project(_to_dev(torch_gpu, x).view(1, -1)).cpu().numpy()
    assert y[0, 0] == np.float32(516631.03125)


@pytest.mark.gpu
def test_gpu_mmvq_full_vocab_sampled_rows(torch_gpu):
    # config-2 shape: 128256 tokens x hidden 4096, a decode batch of 64; the
    # oracle checks every column on a sample of token rows (rows are independent)
    from oxide_sampler import LmHeadQ8_0, quantize_q8_1
    m, k, batch = 128256, 4096, 64
    nb = k // 32
    rng = np.random.default_rng(42)
    print(f"\n[case] mmvq_q8_0 m={m} k={k} batch={batch} (sampled rows)", flush=True)
    ws = (rng.uniform(0.002, 0.05, size=(m, nb)) * rng.choice([-1, 1], size=(m, nb)))
    wq = rng.integers(-128, 128, size=(m, nb, 32), dtype=np.int8)
    w = q8_0_rows(ws, wq)
    x = rng.normal(0, 1.5, size=(batch, k)).astype(np.float32)
    head = LmHeadQ8_0(w, m, k)
    y = head.project(quantize_q8_1(_to_dev(torch_gpu, x)).view(batch, -1)).cpu().numpy()
    rows = np.unique(np.concatenate([rng.integers(0, m, 200), [0, 31, 32, m - 33, m - 1]]))
    sub = w.reshape(m, nb * 34)[rows].reshape(-1)
    want = oracle.mmvq_q8_0_host(sub, oracle.quantize_q8_1_host(x), len(rows), k, batch)
    np.testing.assert_array_equal(y[:, rows].view(np.uint32), want.view(np.uint32))
    assert np.isfinite(y).all()


@pytest.mark.gpu
def test_gpu_lm_head_errors(torch_gpu):
    import ctypes
    from oxide_sampler import LmHeadQ8_0, load_library
    lib = load_library()
    assert lib.oxs_q8_0_packed_bytes(10, 96) == 0
    assert lib.oxs_pack_q8_0(None, 10, 96, None, None) == -5  # k not a multiple of 128
    assert lib.oxs_mmvq_q8_0(None, None, None, 0, 128, 4, None) == 0  # m == 0: nothing to do
    assert lib.oxs_mmvq_q8_0(None, None, None, 10, 128, 4, None) == -1
    assert lib.oxs_quantize_q8_1(None, 31, None, None) == 0  # fewer than 32 values: no block
    with pytest.raises(ValueError):
        LmHeadQ8_0(np.zeros(10 * 3 * 34, np.uint8), 10, 96)
    # misaligned pointers are refused before any launch
    buf = torch_gpu.zeros(4096, dtype=torch_gpu.uint8, device="cuda")
    p = buf.data_ptr()
    assert lib.oxs_mmvq_q8_0(ctypes.c_void_p(p), ctypes.c_void_p(p + 8), ctypes.c_void_p(p), 1, 128, 1, None) == -1
    assert lib.oxs_mmvq_q8_0(ctypes.c_void_p(p), ctypes.c_void_p(p), ctypes.c_void_p(p + 2), 1, 128, 1, None) == -1
    assert lib.oxs_pack_q8_0(ctypes.c_void_p(p), 1, 128, ctypes.c_void_p(p + 4), None) == -1
    assert lib.oxs_quantize_q8_1(ctypes.c_void_p(p + 1), 32, ctypes.c_void_p(p), None) == -1


@pytest.mark.gpu
def test_gpu_mmvq_unaligned_output_rows(torch_gpu):
    # y at an offset of one float (4-byte aligned only) and m % 4 == 0: the scalar store path
    import ctypes
    from oxide_sampler import LmHeadQ8_0, load_library, quantize_q8_1
    m, k, batch = 96, 128, 3
    rng = np.random.default_rng(5)
    w, x = random_case(rng, m, k, batch)
    print("\n[case] mmvq_q8_0 into y + 1 float", flush=True)
    head = LmHeadQ8_0(w, m, k)
    xq = quantize_q8_1(_to_dev(torch_gpu, x))
    y = torch_gpu.full((batch * m + 4,), -7.0, dtype=torch_gpu.float32, device="cuda")
    lib = load_library()
    assert lib.oxs_mmvq_q8_0(ctypes.c_void_p(y.data_ptr() + 4), ctypes.c_void_p(head.packed.data_ptr()),
                             ctypes.c_void_p(xq.data_ptr()), m, k, batch, None) == 0
    torch_gpu.cuda.synchronize()
    got = y.cpu().numpy()
    want = oracle.mmvq_q8_0_host(w, oracle.quantize_q8_1_host(x), m, k, batch).reshape(-1)
    np.testing.assert_array_equal(got[1:1 + batch * m].view(np.uint32), want.view(np.uint32))
    assert got[0] == -7.0 and (got[1 + batch * m:] == -7.0).all()


@pytest.mark.gpu
@pytest.mark.parametrize("batch,softcap", [(3, 0.0), (40, 0.0), (40, 30.0)])
def test_gpu_decode_head_chain_matches_oracle(torch_gpu, batch, softcap):
    # hidden states -> q8_1 -> LM head -> sampler (config 2's chain), every step on the
    # device with no host copy between them, against the oracle's chain on the same inputs
    from harness import compare, run_gpu, run_oracle
    from oxide_sampler import LmHeadQ8_0, quantize_q8_1
    from oxide_sampler import workloads as wl
    m, k = 5003, 512
    rng = np.random.default_rng(100 + batch)
    w8, x = random_case(rng, m, k, batch)
    print(f"\n[case] decode head chain batch={batch} softcap={softcap}", flush=True)
    head = LmHeadQ8_0(w8, m, k)
    logits_dev = head.project(quantize_q8_1(_to_dev(torch_gpu, x)))
    w = wl.config2(batch=batch, vocab=m)
    w.logits = oracle.mmvq_q8_0_host(w8, oracle.quantize_q8_1_host(x), m, k, batch)
    if softcap:
        w.extra["softcap"] = softcap
    gpu = run_gpu(w, torch_gpu, logits_dev=logits_dev)
    ref = run_oracle(w)
    compare(gpu, ref, 1e-5, "decode head chain")
    assert (gpu.status == 0).all()
