"""ctypes binding of liboxs_oracle.so — TEST INFRASTRUCTURE ONLY.

The CPU restatement of crates/oxide-core/src/sampler.rs (oxs_oracle.cpp).
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, as the checker and the CPU baseline.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
ORACLE_LIB = ORACLE_DIR / "liboxs_oracle.so"

OXO_OK = 0
OXO_EMPTY = 1
OXO_HISTORY_FULL = 2
OXO_SHAPE_MISMATCH = -2

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)
    return ORACLE_LIB


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not ORACLE_LIB.exists():
        build()
    lib = ctypes.CDLL(str(ORACLE_LIB))
    vp = ctypes.c_void_p
    lib.oxo_next_u64.restype = ctypes.c_uint64
    lib.oxo_next_u64.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
    lib.oxo_next_f32.restype = ctypes.c_float
    lib.oxo_next_f32.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
    lib.oxo_sample_token.restype = ctypes.c_int
    lib.oxo_sample_token.argtypes = [vp, vp, vp, vp, vp, ctypes.c_uint32, vp, vp, ctypes.c_uint32, vp, vp, vp,
                                     vp, vp, vp, vp, ctypes.c_uint32]
    lib.oxo_sample_batch.restype = ctypes.c_int
    lib.oxo_sample_batch.argtypes = [vp, ctypes.c_int]
    for f in ("oxo_expf", "oxo_logf", "oxo_log2f"):
        getattr(lib, f).restype = ctypes.c_float
        getattr(lib, f).argtypes = [ctypes.c_float]
    lib.oxo_powf.restype = ctypes.c_float
    lib.oxo_powf.argtypes = [ctypes.c_float, ctypes.c_float]
    lib.oxo_decode_step.restype = ctypes.c_int
    lib.oxo_decode_step.argtypes = [vp, vp, ctypes.c_int]
    lib.oxo_argmax_floor.restype = None
    lib.oxo_argmax_floor.argtypes = [vp, ctypes.c_uint32, ctypes.c_uint32, vp, vp]
    lib.oxo_raw_argmax.restype = ctypes.c_uint32
    lib.oxo_raw_argmax.argtypes = [vp, ctypes.c_uint32]
    lib.oxo_gbnf_mask.restype = None
    lib.oxo_gbnf_mask.argtypes = [vp, ctypes.c_uint32, vp, vp, ctypes.c_uint32, vp, vp, ctypes.c_uint32,
                                  ctypes.c_uint32, vp]
    lib.oxo_ascii_mask.restype = None
    lib.oxo_ascii_mask.argtypes = [vp, vp, ctypes.c_uint32, vp]
    lib.oxo_f16_to_f32.argtypes = [ctypes.c_uint16]
    lib.oxo_f16_to_f32.restype = ctypes.c_float
    lib.oxo_f32_to_f16.argtypes = [ctypes.c_float]
    lib.oxo_f32_to_f16.restype = ctypes.c_uint16
    lib.oxo_quantize_q8_1.argtypes = [vp, ctypes.c_uint32, vp]
    lib.oxo_mmvq_q8_0.argtypes = [vp, vp, vp, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]
    lib.oxo_dfa_mask.restype = None
    lib.oxo_dfa_mask.argtypes = [vp, ctypes.c_uint32, vp, vp, ctypes.c_uint32, ctypes.c_uint32, vp, ctypes.c_uint32,
                                 vp, ctypes.c_int64]
    _lib = lib
    return lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def sample_batch_host(abi, *, logits, dtype, configs_bytes, bias_ids, bias_values, ban_ids, mask, history,
                      history_len, history_cap, record, uniforms, rng_state, mu, kept_ld, logits_out=None,
                      shared_config=False, n_threads=1, decode=None, kept_fill=0, softcap=0.0, shared_mask=False):
    """Runs the oracle over host numpy arrays with the oxs_batch descriptor.

    `abi` is the product's ctypes module (for the OxsBatch layout). Mutable
    arrays (history, history_len, rng_state, mu) are updated in place.
    Returns dict(tokens, status, kept_count, kept_ids, kept_probs).
    With `decode` (a dict of current_token, current_position, generated_count
    arrays, updated in place) it runs oxo_decode_step instead. The kept arrays
    start filled with `kept_fill`.
    """
    lib = load()
    B, V = logits.shape
    out = {
        "tokens": np.zeros(B, np.uint32),
        "status": np.zeros(B, np.int32),
        "kept_count": np.full(B, kept_fill, np.uint32),
        "kept_ids": np.full((B, max(kept_ld, 1)), kept_fill, np.uint32),
        "kept_probs": np.full((B, max(kept_ld, 1)), kept_fill, np.uint32).view(np.float32),
    }
    b = abi.OxsBatch()
    b.batch, b.vocab = B, V
    b.logits_dtype = abi.OXS_DTYPE_BF16 if dtype == "bf16" else abi.OXS_DTYPE_F32
    b.flags = (abi.OXS_FLAG_RECORD_HISTORY if record else 0) | (abi.OXS_FLAG_SHARED_CONFIG if shared_config else 0)
    b.logits_ld = logits.shape[1]
    b.logits = logits.ctypes.data
    b.configs = configs_bytes.ctypes.data
    b.bias_ids = _ptr(bias_ids) if bias_ids is not None and bias_ids.size else None
    b.bias_values = _ptr(bias_values) if bias_values is not None and bias_values.size else None
    b.ban_ids = _ptr(ban_ids) if ban_ids is not None and ban_ids.size else None
    if mask is not None:
        b.allowed_mask = mask.ctypes.data
        b.mask_ld = 0 if shared_mask else mask.shape[1]  # 0: row 0 for every row
    if history is not None:
        b.history = history.ctypes.data
        b.history_ld = history.shape[1]
        b.history_len = history_len.ctypes.data
        b.history_cap = history_cap
    b.uniforms = _ptr(uniforms)
    b.rng_state = _ptr(rng_state)
    b.mirostat_mu = _ptr(mu)
    b.out_tokens = out["tokens"].ctypes.data
    b.out_status = out["status"].ctypes.data
    b.out_kept_count = out["kept_count"].ctypes.data
    b.out_kept_ids = out["kept_ids"].ctypes.data
    b.out_kept_probs = out["kept_probs"].ctypes.data
    b.kept_ld = max(kept_ld, 1)
    if logits_out is not None:
        b.logits_out = logits_out.ctypes.data
        b.logits_out_ld = logits_out.shape[1]
    b.logit_softcap = softcap
    if decode is None:
        rc = lib.oxo_sample_batch(ctypes.byref(b), n_threads)
    else:
        io = abi.OxsDecodeIo()
        io.current_token = _ptr(decode.get("current_token"))
        io.current_position = _ptr(decode.get("current_position"))
        io.generated_count = _ptr(decode.get("generated_count"))
        rc = lib.oxo_decode_step(ctypes.byref(b), ctypes.byref(io), n_threads)
    if rc != 0:
        raise ValueError(f"oracle returned {rc}")
    return out


class OracleEngine:
    """AcademicSamplerEngine over the CPU oracle: the same call shape as the
    product's Python mirror, so one test body can drive either."""

    def __init__(self, config, abi, configs_to_array):
        self.config = config
        self._abi = abi
        self._pack = configs_to_array

    def sample_token(self, logits, state, newline_token_id):
        lib = load()
        arr = np.asarray(logits, dtype=np.float32).reshape(-1).copy()
        V = arr.shape[0]
        cfg_bytes, bias_ids, bias_vals, ban_ids = self._pack([self.config], newline_token_id)
        hist = np.zeros(len(state.generated_tokens) + 2, np.uint32)
        hist[: len(state.generated_tokens)] = np.asarray(state.generated_tokens, np.uint32)
        hlen = np.array([len(state.generated_tokens)], np.uint32)
        mu = np.array([state.mirostat_mu], np.float32)
        rng = np.array([state.rng_state], np.uint64)
        tok = np.zeros(1, np.uint32)
        kept_cap = max(256, int(self.config.top_k))
        kids = np.zeros(kept_cap, np.uint32)
        kp = np.zeros(kept_cap, np.float32)
        kc = np.zeros(1, np.uint32)
        st = lib.oxo_sample_token(_ptr(cfg_bytes), _ptr(bias_ids) if bias_ids.size else None,
                                  _ptr(bias_vals) if bias_vals.size else None,
                                  _ptr(ban_ids) if ban_ids.size else None, _ptr(arr), V, _ptr(hist), _ptr(hlen),
                                  hist.shape[0], _ptr(mu), _ptr(rng), None, _ptr(tok), _ptr(kids), _ptr(kp),
                                  _ptr(kc), kept_cap)
        if st == OXO_SHAPE_MISMATCH:
            raise ValueError("ShapeMismatch")
        if isinstance(logits, np.ndarray):
            logits.reshape(-1)[:] = arr
        elif isinstance(logits, list):
            logits[:] = [float(x) for x in arr]
        state.generated_tokens = [int(x) for x in hist[: int(hlen[0])]]
        state.mirostat_mu = float(mu[0])
        state.rng_state = int(rng[0])
        n = min(int(kc[0]), kept_cap)
        state.candidates_buffer = [(int(i), float(p)) for i, p in zip(kids[:n], kp[:n])]
        return int(tok[0])


def dfa_mask_host(transitions, num_states, offsets, byte_arr, states):
    """The oracle's packed grammar masks: [batch, ceil(vocab / 32)] uint32."""
    lib = load()
    transitions = np.ascontiguousarray(transitions, dtype=np.uint32)
    offsets = np.ascontiguousarray(offsets, dtype=np.uint32)
    byte_arr = np.ascontiguousarray(byte_arr, dtype=np.uint8)
    states = np.ascontiguousarray(states, dtype=np.uint32)
    vocab = offsets.shape[0] - 1
    words = (vocab + 31) // 32
    mask = np.zeros((states.shape[0], max(words, 1)), np.uint32)
    lib.oxo_dfa_mask(_ptr(transitions) if transitions.size else None, num_states, _ptr(offsets),
                     _ptr(byte_arr) if byte_arr.size else None, byte_arr.shape[0], vocab, _ptr(states),
                     states.shape[0], _ptr(mask), mask.shape[1])
    return mask[:, :words]


def raw_argmax_host(row) -> int:
    """oxo_raw_argmax on one f32 row (continuous_batching.rs:961-970)."""
    row = np.ascontiguousarray(row, dtype=np.float32)
    return int(load().oxo_raw_argmax(_ptr(row), row.shape[0]))


def _pack_strings(items):
    data = [bytes(x) for x in items]
    off = np.zeros(len(data) + 1, np.uint32)
    if data:
        off[1:] = np.cumsum([len(d) for d in data])
    flat = np.frombuffer(b"".join(data), np.uint8).copy() if data else np.zeros(0, np.uint8)
    return off, flat


def gbnf_mask_host(ranges, literals, offsets, byte_arr):
    """The oracle's GBNF start-rule mask: ranges [(lo, hi) code points], literals [bytes]."""
    lib = load()
    r = np.asarray(ranges, np.uint32).reshape(-1)
    loff, lbytes = _pack_strings(literals)
    offsets = np.ascontiguousarray(offsets, dtype=np.uint32)
    byte_arr = np.ascontiguousarray(byte_arr, dtype=np.uint8)
    vocab = offsets.shape[0] - 1
    mask = np.zeros(max((vocab + 31) // 32, 1), np.uint32)
    lib.oxo_gbnf_mask(_ptr(r) if r.size else None, r.size // 2, _ptr(loff), _ptr(lbytes) if lbytes.size else None,
                      len(literals), _ptr(offsets), _ptr(byte_arr) if byte_arr.size else None, byte_arr.shape[0],
                      vocab, _ptr(mask))
    return mask[: (vocab + 31) // 32]


def ascii_mask_host(allowed, token_ascii):
    """The oracle's ASCII masker row: allowed [256] bools, token_ascii [vocab] (>= 256 for None)."""
    lib = load()
    a = np.ascontiguousarray(allowed, dtype=np.uint8)
    ta = np.ascontiguousarray(token_ascii, dtype=np.uint16)
    vocab = ta.shape[0]
    mask = np.zeros(max((vocab + 31) // 32, 1), np.uint32)
    lib.oxo_ascii_mask(_ptr(a), _ptr(ta), vocab, _ptr(mask))
    return mask[: (vocab + 31) // 32]


def argmax_floor_host(row, batch=2):
    """oxo_argmax_floor: (token, value) of one f32 row of a launch over `batch` rows."""
    row = np.ascontiguousarray(row, dtype=np.float32)
    tok = np.zeros(1, np.uint32)
    val = np.zeros(1, np.float32)
    load().oxo_argmax_floor(_ptr(row), row.shape[0], batch, _ptr(tok), _ptr(val))
    return int(tok[0]), float(val[0])


def f16_to_f32_host(h):
    lib = load()
    return np.array([lib.oxo_f16_to_f32(int(v)) for v in np.asarray(h, np.uint16).ravel()], np.float32)


def f32_to_f16_host(f):
    lib = load()
    return np.array([lib.oxo_f32_to_f16(float(v)) for v in np.asarray(f, np.float32).ravel()], np.uint16)


def quantize_q8_1_host(x):
    """oxo_quantize_q8_1: float32 [..., n] -> uint8 [n / 32 blocks x 36 bytes] (flattened input)."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.zeros((x.size // 32) * 36, np.uint8)
    load().oxo_quantize_q8_1(_ptr(x), x.size, _ptr(out))
    return out


def mmvq_q8_0_host(w, x_q8_1, m, k, batch):
    """oxo_mmvq_q8_0: GGUF Q8_0 bytes [m][k / 32][34] and q8_1 bytes [batch][k / 32][36] -> y [batch, m]."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x_q8_1, dtype=np.uint8)
    assert w.size == m * (k // 32) * 34 and x.size == batch * (k // 32) * 36
    y = np.zeros((batch, m), np.float32)
    load().oxo_mmvq_q8_0(_ptr(y), _ptr(w), _ptr(x), m, k, batch)
    return y
