"""The LM head that produces the sampler's logits, in the reference's Q8_0 format.

The reference's batched decode quantizes the final hidden states to q8_1 and
projects them through a Q8_0 LM head (oxide-backend-cuda/src/lib.rs:4013-4035;
launch_cuda_quantize_q8_1 and launch_cuda_mmvq_q8_0). `quantize_q8_1` and
`LmHeadQ8_0.project` run the same two steps on the GPU and give the same
bytes and floats as the reference kernels. The weights are repacked once, at
construction, into the layout the matrix cores read.
"""
from __future__ import annotations

import ctypes

import numpy as np

from ._abi import check, load_library

Q8_1_BYTES = 36  # {f16 d, f16 sum, int8 qs[32]} per 32 values
Q8_0_BYTES = 34  # {f16 d, int8 qs[32]} per 32 weights


def _torch():
    import torch  # noqa: PLC0415 — torch is plumbing for device memory

    if not torch.cuda.is_available():
        raise RuntimeError("no HIP device visible to torch: the LM head runs on the GPU only")
    return torch


def _stream(t, device, stream):
    s = stream if stream is not None else t.cuda.current_stream(device)
    return ctypes.c_void_p(s.cuda_stream)


def quantize_q8_1(x, out=None, stream=None):
    """launch_cuda_quantize_q8_1 over a float32 device tensor [..., k]: uint8 [..., k / 32 * 36]."""
    t = _torch()
    if x.dtype != t.float32 or not x.is_cuda:
        raise TypeError("x must be a float32 device tensor")
    if not x.is_contiguous():  # a copy here would run on the current stream, not on `stream`
        raise ValueError("x must be contiguous")
    k = x.shape[-1]
    if k % 32:
        raise ValueError("the last dimension must be a multiple of 32")
    shape = tuple(x.shape[:-1]) + (k // 32 * Q8_1_BYTES,)
    if out is None:
        out = t.empty(shape, dtype=t.uint8, device=x.device)
    elif tuple(out.shape) != shape or out.dtype != t.uint8 or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous uint8 tensor of shape {shape}")
    lib = load_library()
    check(lib.oxs_quantize_q8_1(ctypes.c_void_p(x.data_ptr()), x.numel(), ctypes.c_void_p(out.data_ptr()),
                                _stream(t, x.device, stream)), "oxs_quantize_q8_1")
    return out


class LmHeadQ8_0:
    """A Q8_0 LM head of `m` tokens over hidden size `k` (a multiple of 128)
    on the GPU. `weights` holds the GGUF rows ([m][k / 32] 34-byte blocks) as
    bytes: a numpy array, or a uint8 device tensor."""

    def __init__(self, weights, m: int, k: int, device: int = 0):
        t = _torch()
        self.torch = t
        self.m, self.k = int(m), int(k)
        if self.k <= 0 or self.k % 128:
            raise ValueError("k must be a positive multiple of 128")
        dev = t.device("cuda", device)
        self.device = dev
        nbytes = self.m * (self.k // 32) * Q8_0_BYTES
        if isinstance(weights, np.ndarray):
            if weights.nbytes != nbytes:
                raise ValueError(f"weights hold {weights.nbytes} bytes, expected {nbytes}")
            src = t.from_numpy(np.ascontiguousarray(weights).view(np.uint8).reshape(-1)).to(dev)
        else:
            if weights.numel() * weights.element_size() != nbytes:
                raise ValueError(f"weights hold {weights.numel() * weights.element_size()} bytes, expected {nbytes}")
            src = weights.contiguous().view(t.uint8).reshape(-1).to(dev)
        lib = load_library()
        self.lib = lib
        self.packed = t.empty(int(lib.oxs_q8_0_packed_bytes(self.m, self.k)), dtype=t.uint8, device=dev)
        check(lib.oxs_pack_q8_0(ctypes.c_void_p(src.data_ptr()), self.m, self.k,
                                ctypes.c_void_p(self.packed.data_ptr()), _stream(t, dev, None)), "oxs_pack_q8_0")
        t.cuda.current_stream(dev).synchronize()  # src is freed on return

    def project(self, x_q8_1, out=None, stream=None):
        """launch_cuda_mmvq_q8_0: q8_1 activations (uint8 device tensor [batch, k / 32 * 36]) -> float32 [batch, m]."""
        t = self.torch
        row_bytes = self.k // 32 * Q8_1_BYTES
        if x_q8_1.dtype != t.uint8 or not x_q8_1.is_cuda or x_q8_1.dim() != 2 or x_q8_1.shape[1] != row_bytes:
            raise ValueError(f"x_q8_1 must be a uint8 device tensor [batch, {row_bytes}]")
        if not x_q8_1.is_contiguous():
            raise ValueError("x_q8_1 must be contiguous")
        x = x_q8_1
        batch = x.shape[0]
        if out is None:
            out = t.empty(batch, self.m, dtype=t.float32, device=x.device)
        elif tuple(out.shape) != (batch, self.m) or out.dtype != t.float32 or not out.is_contiguous():
            raise ValueError(f"out must be a contiguous float32 tensor [{batch}, {self.m}]")
        check(self.lib.oxs_mmvq_q8_0(ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(self.packed.data_ptr()),
                                     ctypes.c_void_p(x.data_ptr()), self.m, self.k, batch,
                                     _stream(t, x.device, stream)), "oxs_mmvq_q8_0")
        return out
