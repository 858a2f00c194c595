"""The reference sampler's API over the GPU sampler.

`SamplingConfig`, `MirostatMode`, `SamplerState` and
`AcademicSamplerEngine.sample_token` keep the names, defaults, argument
meaning and error behaviour of crates/oxide-core/src/sampler.rs:15-390, so
code (and tests) written against the reference read the same. Every
`sample_token` call runs one row through `oxs_sample_batch` on the GPU; the
batched form is `BatchSampler.sample`.
"""
from __future__ import annotations

import ctypes
import enum
from dataclasses import dataclass, field
from typing import Dict, Iterable, List, Optional, Sequence, Set, Tuple

import numpy as np

from . import _abi
from ._abi import OxsBatch, OxsDecodeIo, OxsLimits, OxsSamplingConfig, check, load_library

_DEFAULT_RNG = 0x853C49E6748FEA9B  # SamplerState::default() (sampler.rs:98)
_MASK64 = (1 << 64) - 1


class ShapeMismatch(ValueError):
    """EngineError::ShapeMismatch (crates/oxide-core/src/error.rs:52)."""


class MirostatMode(enum.IntEnum):
    """sampler.rs:77-82."""

    Disabled = _abi.OXS_MIROSTAT_DISABLED
    V1 = _abi.OXS_MIROSTAT_V1
    V2 = _abi.OXS_MIROSTAT_V2


@dataclass
class SamplingConfig:
    """sampler.rs:17-42 with the defaults of sampler.rs:44-73."""

    temperature: float = 0.8
    top_k: int = 40
    top_p: float = 0.95
    min_p: float = 0.05
    tfs_z: float = 1.0
    typical_p: float = 1.0
    xtc_threshold: float = 0.1
    xtc_probability: float = 0.0
    mirostat_mode: MirostatMode = MirostatMode.Disabled
    mirostat_tau: float = 5.0
    mirostat_eta: float = 0.1
    dry_multiplier: float = 0.0
    dry_base: float = 1.75
    dry_allowed_length: int = 2
    dry_range: int = 1024
    repeat_penalty: float = 1.1
    repeat_last_n: int = 64
    frequency_penalty: float = 0.0
    presence_penalty: float = 0.0
    penalize_nl: bool = False
    newline_penalty: float = 0.5
    logit_biases: Dict[int, float] = field(default_factory=dict)
    banned_tokens: Set[int] = field(default_factory=set)
    seed: Optional[int] = None

    def to_c(self, newline_token_id: int = 0, bias_offset: int = 0, ban_offset: int = 0) -> OxsSamplingConfig:
        c = OxsSamplingConfig()
        for name in (
            "temperature", "top_p", "min_p", "tfs_z", "typical_p", "xtc_threshold", "xtc_probability",
            "mirostat_tau", "mirostat_eta", "dry_multiplier", "dry_base", "repeat_penalty",
            "frequency_penalty", "presence_penalty", "newline_penalty",
        ):
            setattr(c, name, float(getattr(self, name)))
        c.top_k = int(self.top_k)
        c.mirostat_mode = int(self.mirostat_mode)
        c.dry_allowed_length = int(self.dry_allowed_length)
        c.dry_range = int(self.dry_range)
        c.repeat_last_n = int(self.repeat_last_n)
        c.penalize_nl = 1 if self.penalize_nl else 0
        c.newline_token_id = int(newline_token_id)
        c.bias_offset = bias_offset
        c.bias_count = len(self.logit_biases)
        c.ban_offset = ban_offset
        c.ban_count = len(self.banned_tokens)
        return c


def configs_to_array(configs: Sequence[SamplingConfig], newline_token_ids: Sequence[int] | int = 0):
    """Packs per-row configs into the C array plus the bias/ban CSR arrays.

    Returns (config_bytes: np.ndarray[uint8], bias_ids: np.ndarray[uint32],
    bias_values: np.ndarray[float32], ban_ids: np.ndarray[uint32]).
    """
    n = len(configs)
    if isinstance(newline_token_ids, int):
        newline_token_ids = [newline_token_ids] * n
    arr = (OxsSamplingConfig * n)()
    bias_ids: List[int] = []
    bias_vals: List[float] = []
    ban_ids: List[int] = []
    for i, cfg in enumerate(configs):
        arr[i] = cfg.to_c(newline_token_ids[i], len(bias_ids), len(ban_ids))
        for k, v in cfg.logit_biases.items():
            bias_ids.append(int(k))
            bias_vals.append(float(v))
        ban_ids.extend(int(t) for t in sorted(cfg.banned_tokens))
    raw = np.frombuffer(bytes(arr), dtype=np.uint8).copy()
    return (raw, np.asarray(bias_ids, dtype=np.uint32), np.asarray(bias_vals, dtype=np.float32),
            np.asarray(ban_ids, dtype=np.uint32))


class SamplerState:
    """sampler.rs:86-158."""

    def __init__(self, mirostat_mu: float = 10.0, generated_tokens: Optional[List[int]] = None,
                 rng_state: int = _DEFAULT_RNG):
        self.mirostat_mu = float(np.float32(mirostat_mu))
        self.generated_tokens: List[int] = list(generated_tokens or [])
        self.rng_state = int(rng_state) & _MASK64
        self.candidates_buffer: List[Tuple[int, float]] = []

    @classmethod
    def default(cls) -> "SamplerState":
        return cls()

    @classmethod
    def new(cls, target_tau: float) -> "SamplerState":
        return cls(mirostat_mu=float(np.float32(2.0) * np.float32(target_tau)))

    @classmethod
    def new_with_seed(cls, target_tau: float, seed: int) -> "SamplerState":
        return cls(mirostat_mu=float(np.float32(2.0) * np.float32(target_tau)),
                   rng_state=_DEFAULT_RNG if seed == 0 else seed)

    @classmethod
    def from_config(cls, config: SamplingConfig) -> "SamplerState":
        if config.seed is not None:
            return cls.new_with_seed(config.mirostat_tau, config.seed)
        return cls.new(config.mirostat_tau)

    def next_u64(self) -> int:
        x = self.rng_state
        x ^= (x << 13) & _MASK64
        x ^= x >> 7
        x ^= (x << 17) & _MASK64
        self.rng_state = x
        return x

    def next_f32(self) -> float:
        val = np.uint32(self.next_u64() >> 40)
        return float(np.float32(val) / np.float32(16777216.0))

    def record_token(self, token: int) -> None:
        self.generated_tokens.append(int(token))


def _torch():
    import torch  # noqa: PLC0415 — torch is plumbing for device memory

    if not torch.cuda.is_available():
        raise RuntimeError("no HIP device visible to torch: the sampler runs on the GPU only")
    return torch


class BatchSampler:
    """One `oxs_sampler` handle: preallocated workspace, batched launches."""

    def __init__(self, max_batch: int, max_vocab: int, max_top_k: int = 256, device: int = 0,
                 max_dry_ids: int = 0):
        self.lib = load_library()
        self.torch = _torch()
        self.device = device
        lim = OxsLimits(max_batch, max_vocab, max_top_k, max_dry_ids)
        h = ctypes.c_void_p()
        check(self.lib.oxs_sampler_create(ctypes.byref(h), ctypes.byref(lim), device), "oxs_sampler_create")
        self.handle = h
        self.limits = (max_batch, max_vocab, max_top_k, max_dry_ids)

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.torch.cuda.synchronize(self.device)
            self.lib.oxs_sampler_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def workspace_bytes(self) -> int:
        return int(self.lib.oxs_sampler_workspace_bytes(self.handle))

    def count_paths(self, enable: bool = True) -> None:
        """Turns the per-row top-M path counters on or off and zeroes them (synchronises)."""
        check(self.lib.oxs_sampler_count_paths(self.handle, 1 if enable else 0), "oxs_sampler_count_paths")

    def path_counts(self) -> dict:
        """Rows per top-M selection path since the counters were zeroed: buckets, sort, exact, none."""
        c = (ctypes.c_uint32 * 4)()
        check(self.lib.oxs_sampler_path_counts(self.handle, c), "oxs_sampler_path_counts")
        return {"buckets": int(c[0]), "sort": int(c[1]), "exact": int(c[2]), "none": int(c[3])}

    def launch(self, batch: OxsBatch, stream=None, decode: Optional[OxsDecodeIo] = None,
               no_alloc: bool = False) -> None:
        """Raw launch of a prepared descriptor on `stream` (torch stream or None);
        with `decode`, a decode step (oxs_decode_step); with `no_alloc`, through
        oxs_sample_batch_static (the library's fixed workspace, not this sampler's)."""
        s = stream if stream is not None else self.torch.cuda.current_stream(self.device)
        if no_alloc:
            if decode is not None:
                raise ValueError("oxs_sample_batch_static has no decode-step form")
            check(self.lib.oxs_sample_batch_static(ctypes.byref(batch), ctypes.c_void_p(s.cuda_stream)),
                  "oxs_sample_batch_static")
        elif decode is None:
            check(self.lib.oxs_sample_batch(self.handle, ctypes.byref(batch), ctypes.c_void_p(s.cuda_stream)),
                  "oxs_sample_batch")
        else:
            check(self.lib.oxs_decode_step(self.handle, ctypes.byref(batch), ctypes.byref(decode),
                                           ctypes.c_void_p(s.cuda_stream)), "oxs_decode_step")

    def sample(self, logits, configs, *, bias_ids=None, bias_values=None, ban_ids=None, shared_config=False,
               mask=None, history=None, history_len=None, history_cap: Optional[int] = None,
               record: bool = False, uniforms=None, rng_state=None, mirostat_mu=None,
               kept_ld: int = 0, logits_out=None, stream=None, decode: Optional[OxsDecodeIo] = None,
               out: Optional[dict] = None, softcap: float = 0.0, no_alloc: bool = False):
        """Samples every row of `logits` ([B, V] f32/bf16 CUDA tensor).

        `configs` is a uint8 CUDA tensor holding B (or 1 with shared_config)
        packed `oxs_sampling_config` records. Returns a dict of output tensors
        (tokens, status, kept_count and, with kept_ld > 0, kept_ids/kept_probs),
        the ones of `out` when given. With `decode` (an OxsDecodeIo) the call
        is a decode step (oxs_decode_step). `softcap` > 0 applies the model's
        final logit softcap as the logits are read. `no_alloc` runs the call
        through oxs_sample_batch_static.
        """
        t = self.torch
        dev = logits.device
        B, V = int(logits.shape[0]), int(logits.shape[1])
        if logits.dtype == t.float32:
            dtype = _abi.OXS_DTYPE_F32
        elif logits.dtype == t.bfloat16:
            dtype = _abi.OXS_DTYPE_BF16
        else:
            raise TypeError(f"logits dtype {logits.dtype} is not float32 or bfloat16")
        out = dict(out) if out is not None else {}
        for k in ("tokens", "status", "kept_count"):
            if k not in out:
                out[k] = t.empty(B, dtype=t.int32, device=dev)
        b = OxsBatch()
        b.batch, b.vocab, b.logits_dtype = B, V, dtype
        b.flags = (_abi.OXS_FLAG_RECORD_HISTORY if record else 0) | (_abi.OXS_FLAG_SHARED_CONFIG if shared_config else 0)
        b.logits_ld = int(logits.stride(0))
        b.logits = logits.data_ptr()
        b.configs = configs.data_ptr()
        if bias_ids is not None and bias_ids.numel() > 0:
            b.bias_ids = bias_ids.data_ptr()
            b.bias_values = bias_values.data_ptr()
        if ban_ids is not None and ban_ids.numel() > 0:
            b.ban_ids = ban_ids.data_ptr()
        if mask is not None:
            b.allowed_mask = mask.data_ptr()
            b.mask_ld = int(mask.stride(0)) if mask.dim() == 2 else 0  # a 1-D mask is shared by every row
        if history is not None:
            b.history = history.data_ptr()
            b.history_ld = int(history.stride(0))
            b.history_len = history_len.data_ptr()
            b.history_cap = int(history_cap if history_cap is not None else history.shape[1])
        if uniforms is not None:
            b.uniforms = uniforms.data_ptr()
        if rng_state is not None:
            b.rng_state = rng_state.data_ptr()
        if mirostat_mu is not None:
            b.mirostat_mu = mirostat_mu.data_ptr()
        b.out_tokens = out["tokens"].data_ptr()
        b.out_status = out["status"].data_ptr()
        b.out_kept_count = out["kept_count"].data_ptr()
        if kept_ld > 0:
            if "kept_ids" not in out:
                out["kept_ids"] = t.empty(B, kept_ld, dtype=t.int32, device=dev)
            if "kept_probs" not in out:
                out["kept_probs"] = t.empty(B, kept_ld, dtype=t.float32, device=dev)
            b.out_kept_ids = out["kept_ids"].data_ptr()
            b.out_kept_probs = out["kept_probs"].data_ptr()
            b.kept_ld = kept_ld
        if logits_out is not None:
            b.logits_out = logits_out.data_ptr()
            b.logits_out_ld = int(logits_out.stride(0))
        b.logit_softcap = float(softcap)
        self.launch(b, stream, decode, no_alloc)
        return out


_ENGINE_SAMPLERS: Dict[Tuple[int, int], BatchSampler] = {}


def _row_sampler(vocab: int, top_k: int) -> BatchSampler:
    need_k = max(256, int(top_k))
    for (v, k), s in _ENGINE_SAMPLERS.items():
        if v >= vocab and k >= need_k:
            return s
    s = BatchSampler(1, max(vocab, 1), need_k)
    _ENGINE_SAMPLERS[(max(vocab, 1), need_k)] = s
    return s


class AcademicSamplerEngine:
    """sampler.rs:161-390, one row per call, executed on the GPU."""

    def __init__(self, config: SamplingConfig):
        self.config = config

    @classmethod
    def new(cls, config: SamplingConfig) -> "AcademicSamplerEngine":
        return cls(config)

    def sample_token(self, logits, state: SamplerState, newline_token_id: int) -> int:
        """sample_token(&self, logits: &mut [f32], state: &mut SamplerState, newline_token_id: u32).

        `logits` (a list, numpy array or torch tensor of f32) is updated in
        place with the penalised, temperature-scaled values, as in the
        reference; `state` gains the recorded token(s), the new mu, the
        advanced rng_state and the candidates_buffer. Raises ShapeMismatch for
        an empty row. An all -inf row returns 0 without recording (:267-270).
        """
        host = np.asarray(logits.detach().cpu() if hasattr(logits, "detach") else logits, dtype=np.float32)
        host = host.reshape(-1)
        V = int(host.shape[0])
        if V == 0:
            raise ShapeMismatch("Tensor shape or dimension mismatch")
        t = _torch()
        cfg = self.config
        sampler = _row_sampler(V, cfg.top_k)
        dev = t.device("cuda", sampler.device)
        cfg_bytes, bias_ids, bias_vals, ban_ids = configs_to_array([cfg], newline_token_id)
        hist_np = np.asarray(state.generated_tokens, dtype=np.uint32)
        cap = int(hist_np.shape[0]) + 2
        hist = t.zeros(1, cap, dtype=t.int32, device=dev)
        if hist_np.size:
            hist[0, : hist_np.size] = t.from_numpy(hist_np.view(np.int32)).to(dev)
        hist_len = t.tensor([hist_np.size], dtype=t.int32, device=dev)
        rng = t.tensor([np.uint64(state.rng_state).view(np.int64)], dtype=t.int64, device=dev)
        mu = t.tensor([state.mirostat_mu], dtype=t.float32, device=dev)
        d_logits = t.from_numpy(host.copy()).to(dev).reshape(1, V)
        d_out_logits = t.empty(1, V, dtype=t.float32, device=dev)
        kept_ld = max(256, int(cfg.top_k))
        out = sampler.sample(
            d_logits, t.from_numpy(cfg_bytes).to(dev),
            bias_ids=t.from_numpy(bias_ids.view(np.int32)).to(dev) if bias_ids.size else None,
            bias_values=t.from_numpy(bias_vals).to(dev) if bias_vals.size else None,
            ban_ids=t.from_numpy(ban_ids.view(np.int32)).to(dev) if ban_ids.size else None,
            history=hist, history_len=hist_len, history_cap=cap, record=True,
            rng_state=rng, mirostat_mu=mu, kept_ld=kept_ld, logits_out=d_out_logits)
        t.cuda.synchronize(dev)
        status = int(out["status"][0])
        if status in (_abi.OXS_ROW_UNSUPPORTED, _abi.OXS_ROW_MISSING_STATE):
            raise _abi.OxsError(_abi.OXS_ERR_UNSUPPORTED, f"row status {status}")
        new_logits = d_out_logits[0].cpu().numpy()
        if hasattr(logits, "copy_"):
            logits.copy_(t.from_numpy(new_logits).to(logits.device).reshape(logits.shape))
        elif isinstance(logits, np.ndarray):
            logits.reshape(-1)[:] = new_logits
        elif isinstance(logits, list):
            logits[:] = [float(x) for x in new_logits]
        n_hist = int(hist_len[0])
        state.generated_tokens = [int(x) for x in hist[0, :n_hist].cpu().numpy().view(np.uint32)]
        state.mirostat_mu = float(mu[0])
        state.rng_state = int(np.int64(rng[0].item()).view(np.uint64))
        kc = int(out["kept_count"][0])
        ids = out["kept_ids"][0, : min(kc, kept_ld)].cpu().numpy().view(np.uint32)
        probs = out["kept_probs"][0, : min(kc, kept_ld)].cpu().numpy()
        state.candidates_buffer = [(int(i), float(p)) for i, p in zip(ids, probs)]
        return int(np.int32(out["tokens"][0].item()).view(np.uint32))
