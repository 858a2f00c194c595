"""The scheduler's decode stage with the sampler state on the GPU.

`DecodeLoop` mirrors Stage 2 of ContinuousBatchingEngine::step
(crates/oxide-engine/src/continuous_batching.rs:940-1040) for a fixed set of
slots. Each active slot holds one sequence with the loop's sampler, a
`SamplingConfig { temperature, top_p, ..Default }`, and a
`SamplerState::new(5.0)` (:446-452). All of that state stays on the device:
the config, history, mu, rng_state, current token, position and generated
count.

One `oxs_decode_step` launch per step then does every slot's work:
- the raw argmax for temperature <= 1e-6;
- otherwise sample_token with newline id 10, giving 0 on error;
- the advance of current_token, position and count.

Each row's token lands directly in host-mapped memory, tagged with the row's
step count in the same 8-byte store. The host polls the tags instead of
copying logits back and synchronising the stream. The
per-token bookkeeping stays on the host, as in the reference (:986-1030):
stop tokens, the DFA state walk, accepting states and max_tokens. It is a few
comparisons per sequence.

The step can be captured once in a HIP graph (`capture`) and replayed, since
it issues only kernels.
"""
from __future__ import annotations

import ctypes
import time
from dataclasses import dataclass
from typing import Callable, Dict, Iterable, List, Optional

import numpy as np

from . import _abi
from ._abi import OxsDecodeIo, check
from .engine import BatchSampler, SamplerState, SamplingConfig, _torch
from .grammar import DFA_ERROR_STATE, DfaSchemaGrammar, SchemaMismatch

# Stop tokens without a tokenizer (continuous_batching.rs:990-1000).
STOP_TOKENS = frozenset((0, 2, 128_001, 128_008, 128_009, 151_643, 151_645))
# The newline id the decode loop passes to sample_token (:972).
NEWLINE_TOKEN_ID = 10

_CFG_BYTES = ctypes.sizeof(_abi.OxsSamplingConfig)


@dataclass
class TokenEvent:
    """TokenEvent (continuous_batching.rs:1021-1025)."""

    token_id: int
    is_terminal: bool
    finish_reason: Optional[str]


@dataclass
class Sequence:
    """The host-side part of ActiveSequence (continuous_batching.rs:59-75)."""

    max_tokens: int
    temperature: float
    generated_count: int = 0
    dfa: Optional[DfaSchemaGrammar] = None
    dfa_state: int = 0


def next_event(seq: Sequence, token: int, token_bytes: Optional[Callable[[int], bytes]] = None,
               is_stop_token: Optional[Callable[[int], bool]] = None) -> TokenEvent:
    """The loop's bookkeeping after a sampled token (continuous_batching.rs:975-1030).

    `seq.generated_count` has already counted the token.
    """
    is_eos = is_stop_token(token) if is_stop_token else token in STOP_TOKENS
    is_accepting = False
    if seq.dfa is not None:
        # the token's bytes, or its low byte without a tokenizer (:1007-1011);
        # bytes with no transition leave the state where it is (:1012-1018)
        data = token_bytes(token) if token_bytes else bytes([token & 0xFF])
        for b in data:
            try:
                nxt = seq.dfa.transition(seq.dfa_state, b)
            except SchemaMismatch:
                continue
            if nxt != DFA_ERROR_STATE:
                seq.dfa_state = nxt
        acc = seq.dfa.accepting_states
        is_accepting = bool(acc[seq.dfa_state]) if seq.dfa_state < len(acc) else False
    reached_max = seq.generated_count >= seq.max_tokens
    is_terminal = is_eos or reached_max or is_accepting
    if is_eos or is_accepting:
        reason = "stop"
    elif reached_max:
        reason = "length"
    else:
        reason = None
    return TokenEvent(int(token), is_terminal, reason)


class DecodeLoop:
    """`max_slots` decode slots sampled together by `oxs_decode_step`."""

    def __init__(self, max_slots: int, vocab: int, history_cap: int = 4096, max_top_k: int = 256,
                 device: int = 0, token_bytes: Optional[Callable[[int], bytes]] = None,
                 is_stop_token: Optional[Callable[[int], bool]] = None):
        t = _torch()
        self.torch = t
        self.sampler = BatchSampler(max_slots, vocab, max_top_k, device)
        self.lib = self.sampler.lib
        self.max_slots, self.vocab, self.history_cap = int(max_slots), int(vocab), int(history_cap)
        self.max_top_k = int(max_top_k)
        self.token_bytes = token_bytes
        self.is_stop_token = is_stop_token
        dev = t.device("cuda", device)
        self.device = dev
        S = self.max_slots
        idle = np.frombuffer(bytes(self._idle_config()), np.uint8)
        self.configs = t.from_numpy(np.tile(idle, S).copy()).to(dev)
        self.history = t.zeros(S, self.history_cap, dtype=t.int32, device=dev)
        self.history_len = t.zeros(S, dtype=t.int32, device=dev)
        self.mirostat_mu = t.zeros(S, dtype=t.float32, device=dev)
        self.rng_state = t.zeros(S, dtype=t.int64, device=dev)
        self.current_token = t.zeros(S, dtype=t.int32, device=dev)
        self.current_position = t.zeros(S, dtype=t.int32, device=dev)
        self.generated_count = t.zeros(S, dtype=t.int32, device=dev)
        self.out = {k: t.zeros(S, dtype=t.int32, device=dev) for k in ("tokens", "status", "kept_count")}
        host = ctypes.c_void_p()
        check(self.lib.oxs_host_alloc(8 * S, ctypes.byref(host)), "oxs_host_alloc")
        self._host = host.value
        # slot b: (steps row b has completed << 32) | its last token
        self._slots = np.frombuffer((ctypes.c_uint64 * S).from_address(self._host), dtype=np.uint64)
        self.io = OxsDecodeIo(self.current_token.data_ptr(), self.current_position.data_ptr(),
                              self.generated_count.data_ptr(), self._host)
        self.launched = 0  # steps launched; every step covers every slot
        self._tokens = np.zeros(S, np.uint32)
        self.active: Dict[int, Sequence] = {}
        self._graph = None

    # ------------------------------------------------------------ slots

    @staticmethod
    def _idle_config() -> _abi.OxsSamplingConfig:
        # a free slot runs as a raw-argmax row: it changes no sampler state
        return SamplingConfig(temperature=0.0).to_c(NEWLINE_TOKEN_ID)

    def add_sequence(self, slot: int, *, temperature: float, top_p: float, current_token: int,
                     current_position: int, max_tokens: int, dfa: Optional[DfaSchemaGrammar] = None,
                     config: Optional[SamplingConfig] = None, state: Optional[SamplerState] = None) -> None:
        """Admits a sequence (continuous_batching.rs:446-470): config
        `SamplingConfig { temperature, top_p, ..Default }` unless `config` is
        given, and state `SamplerState::new(5.0)` unless `state` is given."""
        if not 0 <= slot < self.max_slots:
            raise IndexError(f"slot {slot} outside 0..{self.max_slots}")
        cfg = config if config is not None else SamplingConfig(temperature=temperature, top_p=top_p)
        if cfg.logit_biases or cfg.banned_tokens:
            raise ValueError("the decode loop's configs carry no bias or ban lists")
        if max(cfg.top_k, 256) > max(self.max_top_k, 256):
            raise ValueError(f"top_k {cfg.top_k} above the loop's max_top_k {self.max_top_k}")
        st = state if state is not None else SamplerState.new(5.0)
        if len(st.generated_tokens) > self.history_cap:
            raise ValueError("the state's history exceeds history_cap")
        t = self.torch
        raw = np.frombuffer(bytes(cfg.to_c(NEWLINE_TOKEN_ID)), np.uint8).copy()
        self.configs[slot * _CFG_BYTES:(slot + 1) * _CFG_BYTES].copy_(t.from_numpy(raw))
        n = len(st.generated_tokens)
        if n:
            self.history[slot, :n].copy_(t.tensor(np.asarray(st.generated_tokens, np.uint32).view(np.int32)))
        self.history_len[slot] = n
        self.mirostat_mu[slot] = float(st.mirostat_mu)
        self.rng_state[slot] = int(np.uint64(st.rng_state).view(np.int64))
        self.current_token[slot] = int(np.uint32(current_token).view(np.int32))
        self.current_position[slot] = int(current_position)
        self.generated_count[slot] = 0
        self.active[slot] = Sequence(int(max_tokens), float(temperature), 0, dfa, 0)

    def remove_sequence(self, slot: int) -> None:
        raw = np.frombuffer(bytes(self._idle_config()), np.uint8).copy()
        self.configs[slot * _CFG_BYTES:(slot + 1) * _CFG_BYTES].copy_(self.torch.from_numpy(raw))
        self.active.pop(slot, None)

    def state(self, slot: int) -> SamplerState:
        """The slot's SamplerState, read back from the device."""
        n = int(self.history_len[slot])
        hist = self.history[slot, :n].cpu().numpy().view(np.uint32).tolist()
        return SamplerState(float(self.mirostat_mu[slot]), hist,
                            int(np.int64(int(self.rng_state[slot])).view(np.uint64)))

    # ------------------------------------------------------------ steps

    def _launch(self, logits, mask=None, stream=None) -> None:
        if tuple(logits.shape) != (self.max_slots, self.vocab):
            raise ValueError(f"logits must be [{self.max_slots}, {self.vocab}]")
        self.sampler.sample(logits, self.configs, mask=mask, history=self.history, history_len=self.history_len,
                            history_cap=self.history_cap, record=True, rng_state=self.rng_state,
                            mirostat_mu=self.mirostat_mu, stream=stream, decode=self.io, out=self.out)

    def launch(self, logits, mask=None, stream=None) -> int:
        """Queues one decode step over every slot; returns its step number."""
        self._launch(logits, mask, stream)
        self.launched += 1
        return self.launched

    def capture(self, logits, mask=None) -> None:
        """Captures one decode step over these (static) logits in a HIP graph."""
        t = self.torch
        g = t.cuda.CUDAGraph()
        with t.cuda.graph(g):
            self._launch(logits, mask)
        self._graph = g

    def replay(self) -> int:
        if self._graph is None:
            raise RuntimeError("no captured step")
        self._graph.replay()
        self.launched += 1
        return self.launched

    def completed(self) -> int:
        """Steps the device has finished for every slot (the smallest tag)."""
        return int((self._slots.copy() >> np.uint64(32)).min())

    def wait(self, step: Optional[int] = None, timeout: float = 30.0) -> np.ndarray:
        """Polls the host slots (oxs_host_wait, in C) until every row carries
        step `step` (default: the last launched), then returns the tokens of
        every slot; no stream sync. Each slot is one 8-byte store, so its
        token belongs to its tag."""
        want = (self.launched if step is None else int(step)) & 0xFFFFFFFF
        deadline = time.monotonic() + timeout
        out = self._tokens
        while True:
            rc = self.lib.oxs_host_wait(ctypes.c_void_p(self._host), self.max_slots, want,
                                        out.ctypes.data_as(ctypes.c_void_p), 1 << 20)
            if rc == _abi.OXS_OK:
                return out.copy()
            if rc != _abi.OXS_ERR_TIMEOUT:
                check(rc, "oxs_host_wait")
            if time.monotonic() > deadline:
                raise TimeoutError(f"decode step {want} not finished after {timeout} s")

    def step(self, logits=None, mask=None) -> Dict[int, TokenEvent]:
        """One decode step: launches (or replays the captured step when
        `logits` is None), waits for the tokens and returns each active
        slot's TokenEvent; finished sequences leave their slots."""
        if logits is None:
            self.replay()
        else:
            self.launch(logits, mask)
        tokens = self.wait()
        events: Dict[int, TokenEvent] = {}
        for slot, seq in list(self.active.items()):
            seq.generated_count += 1
            ev = next_event(seq, int(tokens[slot]), self.token_bytes, self.is_stop_token)
            events[slot] = ev
            if ev.is_terminal:
                self.remove_sequence(slot)
        return events

    def close(self) -> None:
        if getattr(self, "_host", None):
            self.torch.cuda.synchronize(self.device)
            self._graph = None
            self.lib.oxs_host_free(ctypes.c_void_p(self._host))
            self._host = None
        self.sampler.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
