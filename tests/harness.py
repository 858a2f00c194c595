"""Runs one Workload through the GPU sampler and through the CPU oracle.

Both paths get the same bytes: logits, packed configs, bias/ban CSR arrays,
history, mask, uniforms and Mirostat mu. The GPU path calls the C ABI
(oxs_sample_batch) through oxide_sampler.BatchSampler.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import numpy as np

import oxs_oracle_ctypes as oracle
from oxide_sampler import _abi
from oxide_sampler.workloads import Workload


@dataclass
class Result:
    tokens: np.ndarray
    status: np.ndarray
    kept_count: np.ndarray
    kept_ids: np.ndarray
    kept_probs: np.ndarray
    history: np.ndarray
    history_len: np.ndarray
    mu: Optional[np.ndarray]
    rng_state: Optional[np.ndarray]
    logits_out: Optional[np.ndarray]


def run_oracle(w: Workload, kept_ld: int = 256, record: bool = True, use_rng: bool = False,
               rng_state: Optional[np.ndarray] = None, logits_out: bool = False, n_threads: int = 1,
               shared_mask: bool = False) -> Result:
    cfg, bias_ids, bias_vals, ban_ids = w.packed_configs()
    history = w.history.copy()
    hist_len = w.history_len.copy()
    mu = w.mu.copy() if w.mu is not None else None
    rng = rng_state.copy() if rng_state is not None else None
    lo = np.zeros((w.batch, w.vocab), np.float32) if logits_out else None
    out = oracle.sample_batch_host(
        _abi, logits=np.ascontiguousarray(w.logits), dtype=w.dtype, configs_bytes=cfg, bias_ids=bias_ids,
        bias_values=bias_vals, ban_ids=ban_ids, mask=w.mask, history=history, history_len=hist_len,
        history_cap=history.shape[1], record=record, uniforms=None if use_rng else w.uniforms,
        rng_state=rng, mu=mu, kept_ld=kept_ld, logits_out=lo, n_threads=n_threads,
        softcap=float(w.extra.get("softcap", 0.0)), shared_mask=shared_mask)
    return Result(out["tokens"], out["status"], out["kept_count"], out["kept_ids"][:, :kept_ld],
                  out["kept_probs"][:, :kept_ld], history, hist_len, mu, rng, lo)


_SAMPLERS = {}


def gpu_sampler(max_batch: int, max_vocab: int, max_top_k: int = 256, exact_limits: bool = False,
                max_dry_ids: int = 0):
    """A cached BatchSampler at least this large (exactly these limits with exact_limits)."""
    from oxide_sampler import BatchSampler
    key = (max_batch, max_vocab, max_top_k, max_dry_ids)
    if key not in _SAMPLERS:
        for (b, v, k, d), s in _SAMPLERS.items():
            if exact_limits:
                break
            if b >= max_batch and v >= max_vocab and k >= max_top_k and d == max_dry_ids:
                return s
        _SAMPLERS[key] = BatchSampler(max_batch, max_vocab, max_top_k, max_dry_ids=max_dry_ids)
    return _SAMPLERS[key]


def to_device(w: Workload, torch):
    d = torch.device("cuda")
    if w.dtype == "bf16":
        logits = torch.from_numpy(np.ascontiguousarray(w.logits).view(np.int16)).to(d).view(torch.bfloat16)
    else:
        logits = torch.from_numpy(np.ascontiguousarray(w.logits)).to(d)
    return logits


def run_gpu(w: Workload, torch, kept_ld: int = 256, record: bool = True, use_rng: bool = False,
            rng_state: Optional[np.ndarray] = None, logits_out: bool = False, logits_dev=None,
            max_top_k: int = 256, shared_mask: bool = False, no_alloc: bool = False,
            exact_limits: bool = False, max_dry_ids: int = 0) -> Result:
    d = torch.device("cuda")
    cfg, bias_ids, bias_vals, ban_ids = w.packed_configs()
    s = gpu_sampler(w.batch, w.vocab, max_top_k, exact_limits, max_dry_ids)
    logits = logits_dev if logits_dev is not None else to_device(w, torch)
    hist = torch.from_numpy(w.history.view(np.int32).copy()).to(d)
    hlen = torch.from_numpy(w.history_len.view(np.int32).copy()).to(d)
    mu = torch.from_numpy(w.mu.copy()).to(d) if w.mu is not None else None
    rng = torch.from_numpy(rng_state.view(np.int64).copy()).to(d) if rng_state is not None else None
    mask = torch.from_numpy(w.mask.view(np.int32)).to(d) if w.mask is not None else None
    if mask is not None and shared_mask:
        mask = mask[0].contiguous()  # 1-D: one mask for every row (mask_ld = 0)
    lo = torch.empty(w.batch, w.vocab, dtype=torch.float32, device=d) if logits_out else None
    out = s.sample(
        logits, torch.from_numpy(cfg).to(d),
        bias_ids=torch.from_numpy(bias_ids.view(np.int32)).to(d) if bias_ids.size else None,
        bias_values=torch.from_numpy(bias_vals).to(d) if bias_vals.size else None,
        ban_ids=torch.from_numpy(ban_ids.view(np.int32)).to(d) if ban_ids.size else None,
        mask=mask, history=hist, history_len=hlen, history_cap=w.history.shape[1], record=record,
        uniforms=None if use_rng else torch.from_numpy(w.uniforms).to(d), rng_state=rng,
        mirostat_mu=mu, kept_ld=kept_ld, logits_out=lo, softcap=float(w.extra.get("softcap", 0.0)),
        no_alloc=no_alloc)
    torch.cuda.synchronize()
    return Result(
        out["tokens"].cpu().numpy().view(np.uint32), out["status"].cpu().numpy(),
        out["kept_count"].cpu().numpy().view(np.uint32), out["kept_ids"].cpu().numpy().view(np.uint32),
        out["kept_probs"].cpu().numpy(), hist.cpu().numpy().view(np.uint32), hlen.cpu().numpy().view(np.uint32),
        mu.cpu().numpy() if mu is not None else None,
        rng.cpu().numpy().view(np.uint64) if rng is not None else None,
        lo.cpu().numpy() if lo is not None else None)


def compare(gpu: Result, ref: Result, rtol: float, what: str = "", exact_probs: bool = True) -> dict:
    """Asserts parity; returns counts of bit-inexact probabilities."""
    B = len(ref.tokens)
    bad_rows = np.nonzero(gpu.tokens != ref.tokens)[0]
    assert bad_rows.size == 0, f"{what}: token mismatch in rows {bad_rows[:10]} gpu={gpu.tokens[bad_rows[:5]]} ref={ref.tokens[bad_rows[:5]]}"
    np.testing.assert_array_equal(gpu.status, ref.status, err_msg=f"{what}: status")
    np.testing.assert_array_equal(gpu.kept_count, ref.kept_count, err_msg=f"{what}: kept_count")
    inexact = 0
    kl = ref.kept_ids.shape[1]
    for b in range(B):
        n = min(int(ref.kept_count[b]), kl)
        np.testing.assert_array_equal(gpu.kept_ids[b, :n], ref.kept_ids[b, :n], err_msg=f"{what}: kept ids row {b}")
        gp, rp = gpu.kept_probs[b, :n], ref.kept_probs[b, :n]
        np.testing.assert_allclose(gp, rp, rtol=rtol, atol=0, err_msg=f"{what}: kept probs row {b}")
        inexact += int(np.count_nonzero(gp.view(np.uint32) != rp.view(np.uint32)))
    np.testing.assert_array_equal(gpu.history_len, ref.history_len, err_msg=f"{what}: history_len")
    for b in range(B):
        n = int(ref.history_len[b])
        np.testing.assert_array_equal(gpu.history[b, :n], ref.history[b, :n], err_msg=f"{what}: history row {b}")
    if ref.mu is not None:
        np.testing.assert_allclose(gpu.mu, ref.mu, rtol=rtol, atol=0, err_msg=f"{what}: mu")
        inexact += int(np.count_nonzero(gpu.mu.view(np.uint32) != ref.mu.view(np.uint32)))
    if ref.rng_state is not None:
        np.testing.assert_array_equal(gpu.rng_state, ref.rng_state, err_msg=f"{what}: rng_state")
    if ref.logits_out is not None:
        np.testing.assert_array_equal(gpu.logits_out.view(np.uint32), ref.logits_out.view(np.uint32),
                                      err_msg=f"{what}: logits_out")
    if exact_probs:
        assert inexact == 0, f"{what}: {inexact} probabilities/mu differ from the oracle in the last bits"
    return {"inexact": inexact}
