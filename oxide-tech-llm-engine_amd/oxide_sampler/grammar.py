"""The reference's DFA grammar API over the GPU mask kernel.

`DfaSchemaGrammar` keeps the names, constructors and behaviour of
crates/oxide-core/src/dfa.rs:4-190 (the same type is re-exported by
crates/oxide-server/src/dfa.rs). Its token masks run on the GPU through
`oxs_dfa_mask` (the C ABI in include/oxide_sampler.h):

- `DfaSchemaGrammar.token_masks(token_bytes, states)`: packed allowed-token
  masks for a batch of rows, ready for `oxs_sample_batch`'s allowed_mask
  (StructuredOutputEngine::compute_token_mask, grammar_engine.rs:42-65);
- `DfaSchemaGrammar.apply_dfa_mask(state, vocab_bytes, logits)`: the reference's
  in-place -inf masking of one row (dfa.rs:130-148);
- `DfaSchemaGrammar.state_masks(token_bytes)` then `.gather_masks(compiled,
  states)`: the same masks from a per-state table computed once per grammar and
  vocabulary (`oxs_dfa_mask_gather`), for decode loops.

The two static maskers of the reference are mirrored the same way:
`GbnfGrammarEngine` (sampler.rs:523-585; `oxs_gbnf_mask`) and
`GrammarLogitMasker` (grammar_mask.rs:17-66; `oxs_ascii_mask`).

`transition`, `deterministic_transition` and `find_jump_forward_bytes` walk the
table on the host, as the reference does (dfa.rs:110-190): they are single
lookups, not a data-parallel path.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

from . import _abi
from ._abi import OxsDfa, OxsGbnfRule, OxsTokenBytes, check, load_library

DFA_ERROR_STATE = _abi.OXS_DFA_ERROR_STATE


class SchemaMismatch(ValueError):
    """EngineError::SchemaMismatch { state, byte } (crates/oxide-core/src/error.rs)."""

    def __init__(self, state: int, byte: int):
        super().__init__(f"schema mismatch at state {state}, byte {byte}")
        self.state = state
        self.byte = byte


def _torch():
    import torch  # noqa: PLC0415 — torch is plumbing for device memory

    if not torch.cuda.is_available():
        raise RuntimeError("no HIP device visible to torch: the grammar masks run on the GPU only")
    return torch


class TokenBytes:
    """A vocabulary's token byte strings on the device, as offsets + bytes."""

    def __init__(self, vocab: Sequence[bytes], device: int = 0):
        t = _torch()
        lens = np.fromiter((len(b) for b in vocab), dtype=np.int64, count=len(vocab))
        total = int(lens.sum()) if len(vocab) else 0
        if total >= 1 << 32 or len(vocab) >= 1 << 31:
            raise ValueError("token bytes are indexed with 32-bit offsets: at most 4 GiB and 2^31 tokens")
        offsets = np.zeros(len(vocab) + 1, np.uint32)
        if len(vocab):
            offsets[1:] = np.cumsum(lens).astype(np.uint32)
        flat = np.frombuffer(b"".join(bytes(b) for b in vocab), dtype=np.uint8)
        dev = t.device("cuda", device)
        self.vocab = len(vocab)
        self.num_bytes = int(flat.shape[0])
        self.offsets = t.from_numpy(offsets.view(np.int32).copy()).to(dev)
        self.bytes = t.from_numpy(flat.copy() if flat.size else np.zeros(1, np.uint8)).to(dev)

    def as_c(self) -> OxsTokenBytes:
        return OxsTokenBytes(self.vocab, self.num_bytes, self.offsets.data_ptr(), self.bytes.data_ptr())


class StateMasks:
    """Packed masks of every state of one grammar over one vocabulary:
    `table` is int32 [num_states + 1, ceil(vocab / 32)] on the GPU."""

    def __init__(self, num_states: int, vocab: int, table):
        self.num_states = int(num_states)
        self.vocab = int(vocab)
        self.words = (self.vocab + 31) // 32
        self.table = table


class DfaSchemaGrammar:
    """dfa.rs:4-12: num_states, a flat [num_states * 256] transition table, accepting states."""

    def __init__(self, num_states: int, transitions: Sequence[int], accepting_states: Sequence[bool]):
        self.num_states = int(num_states)
        self.transitions = np.asarray(transitions, dtype=np.uint32).reshape(-1)
        self.accepting_states = [bool(a) for a in accepting_states]
        if self.transitions.shape[0] != self.num_states * 256:
            raise ValueError("transitions must hold num_states * 256 entries")
        self._dev = None

    @classmethod
    def new_simple_json_validator(cls) -> "DfaSchemaGrammar":
        """dfa.rs:16-63: an 8-state JSON object validator."""
        n = 8
        t = np.full(n * 256, DFA_ERROR_STATE, np.uint32)
        acc = [False] * n
        t[ord("{")] = 1
        t[256 + ord('"')] = 2
        t[256 + ord("}")] = 7
        t[2 * 256:3 * 256] = 2
        t[2 * 256 + ord('"')] = 3
        t[3 * 256 + ord(":")] = 4
        for b in range(ord("0"), ord("9") + 1):
            t[4 * 256 + b] = 5
            t[5 * 256 + b] = 5
        t[4 * 256 + ord('"')] = 6
        t[5 * 256 + ord(",")] = 1
        t[5 * 256 + ord("}")] = 7
        t[6 * 256:7 * 256] = 6
        t[6 * 256 + ord('"')] = 5
        acc[7] = True
        return cls(n, t, acc)

    @classmethod
    def new_json_with_fixed_prefix(cls, prefix: str) -> "DfaSchemaGrammar":
        """dfa.rs:66-106: the prefix as a chain of states, then a number or string value and '}'."""
        pb = prefix.encode()
        plen = len(pb)
        n = plen + 4
        t = np.full(n * 256, DFA_ERROR_STATE, np.uint32)
        acc = [False] * n
        for i, b in enumerate(pb):
            t[i * 256 + b] = i + 1
        val, end, strv, term = plen, plen + 1, plen + 2, plen + 3
        for b in range(ord("0"), ord("9") + 1):
            t[val * 256 + b] = end
            t[end * 256 + b] = end
        t[val * 256 + ord('"')] = strv
        t[end * 256 + ord("}")] = term
        t[strv * 256:(strv + 1) * 256] = strv
        t[strv * 256 + ord('"')] = end
        acc[term] = True
        return cls(n, t, acc)

    def transition(self, current_state: int, byte: int) -> int:
        """dfa.rs:110-126."""
        if current_state >= self.num_states:
            raise SchemaMismatch(current_state, byte)
        nxt = int(self.transitions[current_state * 256 + byte])
        if nxt == DFA_ERROR_STATE:
            raise SchemaMismatch(current_state, byte)
        return nxt

    def deterministic_transition(self, current_state: int) -> Optional[int]:
        """dfa.rs:151-168: the only byte with a transition, if there is exactly one."""
        if current_state >= self.num_states:
            return None
        row = self.transitions[current_state * 256:(current_state + 1) * 256]
        live = np.nonzero(row != DFA_ERROR_STATE)[0]
        return int(live[0]) if live.shape[0] == 1 else None

    def find_jump_forward_bytes(self, current_state: int, max_lookahead: int) -> Tuple[List[int], int]:
        """dfa.rs:170-190: follow unambiguous arcs up to max_lookahead bytes."""
        out: List[int] = []
        while len(out) < max_lookahead:
            b = self.deterministic_transition(current_state)
            if b is None:
                break
            out.append(b)
            current_state = int(self.transitions[current_state * 256 + b])
            if current_state >= self.num_states or current_state == DFA_ERROR_STATE:
                break
        return out, current_state

    def _device_table(self, device: int):
        if self._dev is None:
            t = _torch()
            self._dev = t.from_numpy(self.transitions.view(np.int32).copy()).to(t.device("cuda", device))
        return self._dev

    def token_masks(self, token_bytes: TokenBytes, states, device: int = 0, stream=None):
        """Packed masks [len(states), ceil(vocab / 32)] (int32 tensor on the GPU; bit set = allowed)."""
        t = _torch()
        lib = load_library()
        dev = t.device("cuda", device)
        st = states if hasattr(states, "data_ptr") else t.tensor(np.asarray(states, np.uint32).view(np.int32), device=dev)
        st = st.to(dev).contiguous()
        B = int(st.shape[0])
        words = (token_bytes.vocab + 31) // 32
        mask = t.empty(B, max(words, 1), dtype=t.int32, device=dev)
        table = self._device_table(device)
        dfa = OxsDfa(self.num_states, table.data_ptr() if self.num_states else 0)
        tb = token_bytes.as_c()
        s = stream if stream is not None else t.cuda.current_stream(dev)
        check(lib.oxs_dfa_mask(ctypes.byref(dfa), ctypes.byref(tb), ctypes.c_void_p(st.data_ptr()), B,
                               ctypes.c_void_p(mask.data_ptr()), mask.stride(0), ctypes.c_void_p(s.cuda_stream)),
              "oxs_dfa_mask")
        return mask[:, :words]

    def state_masks(self, token_bytes: TokenBytes, device: int = 0, stream=None) -> "StateMasks":
        """The masks of every state, once: rows 0 .. num_states - 1, and row
        num_states for any state outside the table."""
        t = _torch()
        states = t.arange(self.num_states + 1, dtype=t.int32, device=t.device("cuda", device))
        m = self.token_masks(token_bytes, states, device, stream)
        return StateMasks(self.num_states, token_bytes.vocab, m.contiguous())

    def gather_masks(self, compiled: "StateMasks", states, out=None, device: int = 0, stream=None):
        """token_masks(states) from a StateMasks table (int32 [len(states), ceil(vocab / 32)])."""
        t = _torch()
        lib = load_library()
        if compiled.num_states != self.num_states:
            raise ValueError("the table was compiled for another grammar")
        dev = t.device("cuda", device)
        st = states if hasattr(states, "data_ptr") else t.tensor(np.asarray(states, np.uint32).view(np.int32), device=dev)
        st = st.to(dev).contiguous()
        B = int(st.shape[0])
        words = compiled.words
        if out is None:
            out = t.empty(B, max(words, 1), dtype=t.int32, device=dev)
        s = stream if stream is not None else t.cuda.current_stream(dev)
        check(lib.oxs_dfa_mask_gather(ctypes.c_void_p(compiled.table.data_ptr()), self.num_states,
                                      compiled.table.stride(0), compiled.vocab, ctypes.c_void_p(st.data_ptr()), B,
                                      ctypes.c_void_p(out.data_ptr()), out.stride(0), ctypes.c_void_p(s.cuda_stream)),
              "oxs_dfa_mask_gather")
        return out[:, :words]

    def apply_dfa_mask(self, current_state: int, token_bytes, logits) -> None:
        """dfa.rs:130-148: tokens whose bytes do not walk from current_state get -inf (in place)."""
        tb = token_bytes if isinstance(token_bytes, TokenBytes) else TokenBytes(list(token_bytes))
        _mask_in_place(logits, self.token_masks(tb, [current_state])[0], tb.vocab)


def _mask_in_place(logits, words, vocab: int) -> None:
    """-inf into `logits` (list, numpy array or torch tensor) where the packed row `words` has a 0 bit."""
    t = _torch()
    w = words.cpu().numpy().view(np.uint32)
    bits = np.unpackbits(w.view(np.uint8), bitorder="little")[:vocab].astype(bool)
    n = min(vocab, len(logits))
    if hasattr(logits, "masked_fill_"):
        allowed = t.from_numpy(bits[:n].copy()).to(logits.device)
        logits[:n].masked_fill_(~allowed, float("-inf"))
    else:
        for i in range(n):
            if not bits[i]:
                logits[i] = float("-inf")


@dataclass
class GbnfRule:
    """GbnfRule (crates/oxide-core/src/sampler.rs:523-529)."""

    rule_name: str
    allowed_char_ranges: List[Tuple[str, str]] = field(default_factory=list)
    literal_strings: List[str] = field(default_factory=list)


class GbnfGrammarEngine:
    """GbnfGrammarEngine (sampler.rs:531-585): rules by name and a start rule.
    Its mask is one static row (oxs_gbnf_mask on the GPU)."""

    def __init__(self, rules: Dict[str, GbnfRule], start_rule: str):
        self.rules = dict(rules)
        self.start_rule = start_rule

    @classmethod
    def new_json_grammar(cls) -> "GbnfGrammarEngine":
        """sampler.rs:539-553."""
        root = GbnfRule("root", [("{", "{"), ("[", "["), ('"', '"')], ["true", "false", "null"])
        return cls({"root": root}, "root")

    def token_mask(self, vocab_tokens, device: int = 0, stream=None):
        """Packed mask (int32 [ceil(vocab / 32)] on the GPU) of the start rule,
        or None when the start rule is missing (the reference then masks nothing)."""
        rule = self.rules.get(self.start_rule)
        if rule is None:
            return None
        t = _torch()
        lib = load_library()
        dev = t.device("cuda", device)
        tb = vocab_tokens if isinstance(vocab_tokens, TokenBytes) else TokenBytes(
            [str(x).encode("utf-8") for x in vocab_tokens], device)
        ranges = np.array([[ord(a), ord(b)] for a, b in rule.allowed_char_ranges], np.uint32).reshape(-1)
        lits = [x.encode("utf-8") for x in rule.literal_strings]
        loff = np.zeros(len(lits) + 1, np.uint32)
        if lits:
            loff[1:] = np.cumsum([len(x) for x in lits])
        lbytes = np.frombuffer(b"".join(lits), np.uint8).copy() if lits else np.zeros(1, np.uint8)
        d_ranges = t.from_numpy(ranges.view(np.int32).copy() if ranges.size else np.zeros(2, np.int32)).to(dev)
        d_loff = t.from_numpy(loff.view(np.int32).copy()).to(dev)
        d_lbytes = t.from_numpy(lbytes if lbytes.size else np.zeros(1, np.uint8)).to(dev)
        words = (tb.vocab + 31) // 32
        mask = t.zeros(max(words, 1), dtype=t.int32, device=dev)
        r = OxsGbnfRule(ranges.size // 2, d_ranges.data_ptr(), len(lits), d_loff.data_ptr(), d_lbytes.data_ptr())
        s = stream if stream is not None else t.cuda.current_stream(dev)
        check(lib.oxs_gbnf_mask(ctypes.byref(r), ctypes.byref(tb.as_c()), ctypes.c_void_p(mask.data_ptr()),
                                ctypes.c_void_p(s.cuda_stream)), "oxs_gbnf_mask")
        s.synchronize()  # the argument buffers above are freed on return
        return mask[:words]

    def apply_grammar_mask(self, logits, vocab_tokens) -> None:
        """sampler.rs:556-584: disallowed tokens' logits become -inf (in place)."""
        m = self.token_mask(vocab_tokens)
        if m is not None:
            _mask_in_place(logits, m, len(vocab_tokens) if not isinstance(vocab_tokens, TokenBytes)
                           else vocab_tokens.vocab)


class GrammarLogitMasker:
    """GrammarLogitMasker (crates/oxide-core/src/grammar_mask.rs:17-66): an
    allowed-byte table over token ASCII bytes. Its mask runs on the GPU
    (oxs_ascii_mask)."""

    def __init__(self):
        mask = [False] * 256  # Default (grammar_mask.rs:23-35): printable ASCII, newline and tab
        for b in range(0x20, 0x7F):
            mask[b] = True
        mask[ord("\n")] = True
        mask[ord("\t")] = True
        self.allowed_ascii_mask = mask
        self.is_active = True

    @classmethod
    def new(cls) -> "GrammarLogitMasker":
        return cls()

    def restrict_to_numbers(self) -> None:
        """grammar_mask.rs:43-52."""
        self.allowed_ascii_mask = [False] * 256
        for b in b"0123456789.-,}]":
            self.allowed_ascii_mask[b] = True

    def token_mask(self, vocab_ascii_bytes: Sequence[Optional[int]], device: int = 0, stream=None):
        """Packed mask (int32 [ceil(n / 32)] on the GPU) of the first n tokens."""
        t = _torch()
        lib = load_library()
        dev = t.device("cuda", device)
        n = len(vocab_ascii_bytes)
        codes = np.array([256 if b is None else int(b) for b in vocab_ascii_bytes], np.uint16)
        allowed = t.tensor([1 if a else 0 for a in self.allowed_ascii_mask], dtype=t.uint8, device=dev)
        d_codes = t.from_numpy(codes.view(np.int16).copy() if n else np.zeros(1, np.int16)).to(dev)
        words = (n + 31) // 32
        mask = t.zeros(max(words, 1), dtype=t.int32, device=dev)
        s = stream if stream is not None else t.cuda.current_stream(dev)
        check(lib.oxs_ascii_mask(ctypes.c_void_p(allowed.data_ptr()), ctypes.c_void_p(d_codes.data_ptr()), n,
                                 ctypes.c_void_p(mask.data_ptr()), ctypes.c_void_p(s.cuda_stream)), "oxs_ascii_mask")
        s.synchronize()
        return mask[:words]

    def mask_logits(self, vocab_ascii_bytes: Sequence[Optional[int]], logits) -> None:
        """grammar_mask.rs:55-65: tokens with a disallowed byte get -inf (in place)."""
        if not self.is_active:
            return
        n = min(len(vocab_ascii_bytes), len(logits))
        _mask_in_place(logits, self.token_mask(list(vocab_ascii_bytes)[:n]), n)


class GrammarConstraintType:
    """GrammarConstraintType (crates/oxide-server/src/grammar_engine.rs:10-15)."""

    def __init__(self, kind: str, text: str):
        if kind not in ("JsonSchema", "Regex", "Ebnf"):
            raise ValueError(f"unknown constraint type {kind}")
        self.kind, self.text = kind, text

    @classmethod
    def JsonSchema(cls, schema: str) -> "GrammarConstraintType":
        return cls("JsonSchema", schema)

    @classmethod
    def Regex(cls, pattern: str) -> "GrammarConstraintType":
        return cls("Regex", pattern)

    @classmethod
    def Ebnf(cls, rules: str) -> "GrammarConstraintType":
        return cls("Ebnf", rules)


class StructuredOutputEngine:
    """StructuredOutputEngine (grammar_engine.rs:17-75): every constraint type
    compiles to DfaSchemaGrammar::new_simple_json_validator (:26-38, :67-75);
    compute_token_mask runs on the GPU (oxs_dfa_mask)."""

    def __init__(self, grammar: DfaSchemaGrammar):
        self.grammar = grammar

    @classmethod
    def compile(cls, constraint: GrammarConstraintType) -> "StructuredOutputEngine":
        return cls(DfaSchemaGrammar.new_simple_json_validator())

    def compute_token_mask(self, current_state: int, vocab) -> List[bool]:
        """grammar_engine.rs:40-65: True where the token's bytes walk from current_state."""
        tb = vocab if isinstance(vocab, TokenBytes) else TokenBytes([bytes(v) for v in vocab])
        words = self.grammar.token_masks(tb, [current_state])[0].cpu().numpy().view(np.uint32)
        return np.unpackbits(words.view(np.uint8), bitorder="little")[: tb.vocab].astype(bool).tolist()
