"""The reference's static maskers on the GPU, against the oracle and the reference's tests.

GbnfGrammarEngine::apply_grammar_mask (crates/oxide-core/src/sampler.rs:555-583;
KAT academic_samplers_test.rs:94-123) and GrammarLogitMasker::mask_logits
(crates/oxide-core/src/grammar_mask.rs:55-65; KAT grammar_mask.rs:82-96).
"""
import math

import numpy as np
import pytest

import oxs_oracle_ctypes as oracle
from oxide_sampler.grammar import GbnfGrammarEngine, GbnfRule, GrammarLogitMasker


def pack(tokens):
    data = [t if isinstance(t, bytes) else t.encode("utf-8") for t in tokens]
    off = np.zeros(len(data) + 1, np.uint32)
    off[1:] = np.cumsum([len(d) for d in data])
    return off, np.frombuffer(b"".join(data), np.uint8).copy()


def bits(words, n):
    return np.unpackbits(np.asarray(words, np.uint32).view(np.uint8), bitorder="little")[:n].astype(bool).tolist()


def brute_gbnf(ranges, literals, tokens):
    """sampler.rs:558-580 in Python: str.startswith and the first character of a lossy UTF-8 decode."""
    out = []
    for raw in tokens:
        raw = raw if isinstance(raw, bytes) else raw.encode("utf-8")
        if not raw:
            out.append(True)
            continue
        first = ord(raw.decode("utf-8", errors="replace")[0])
        ok = any(lo <= first <= hi for lo, hi in ranges)
        for lit in literals:
            ok = ok or lit.startswith(raw) or raw.startswith(lit)
        out.append(ok)
    return out


def gbnf_host(ranges, literals, tokens):
    off, by = pack(tokens)
    return bits(oracle.gbnf_mask_host(ranges, literals, off, by), len(tokens))


# ----------------------------------------------------------------------------- the oracle

def test_oracle_gbnf_known_answer():
    # academic_samplers_test.rs:94-123: '"key"' and '123' masked, '{' and 'true' kept
    got = gbnf_host([(ord("{"), ord("{"))], [b"true"], ['"key"', "{", "123", "true"])
    assert got == [False, True, False, True]


def test_oracle_gbnf_json_grammar_cases():
    # new_json_grammar (sampler.rs:539-553): '{', '[', '"' start a value; prefixes of true/false/null
    # either way round; the empty token is never masked; the first character counts, not the first byte
    rule = GbnfGrammarEngine.new_json_grammar().rules["root"]
    ranges = [(ord(a), ord(b)) for a, b in rule.allowed_char_ranges]
    lits = [x.encode() for x in rule.literal_strings]
    toks = ["{", "[1", '"a', "tr", "true", "trueish", "nul", "nulx", "f", "x", "", "5", "€", " {"]
    want = [True, True, True, True, True, True, True, False, True, False, True, False, False, False]
    assert gbnf_host(ranges, lits, toks) == want == brute_gbnf(ranges, lits, toks)


@pytest.mark.parametrize("seed", range(4))
def test_oracle_gbnf_matches_brute_force(seed):
    rng = np.random.default_rng(seed)
    alphabet = ["{", "[", '"', "t", "r", "u", "e", "n", "l", "a", "1", " ", "é", "€", "\U0001f600"]
    toks = ["".join(rng.choice(alphabet, size=int(rng.integers(0, 6)))).encode() for _ in range(400)]
    # malformed UTF-8: truncated, bad continuation, overlong, surrogate, beyond U+10FFFF, lone continuation
    toks += [b"\xe2\x82", b"\xe2(\xa1", b"\xc0\x80", b"\xed\xa0\x80x", b"\xf4\x90\x80\x80", b"\x80a", b"\xff"]
    ranges = [(0x7B, 0x7B), (0x20AC, 0x20AC), (0xFFFD, 0xFFFD)] if seed % 2 else [(0x30, 0x39), (0x1F600, 0x1F64F)]
    lits = [b"true", b"nul", b""] if seed == 3 else [b"true", b"null", "été".encode()]
    assert gbnf_host(ranges, lits, toks) == brute_gbnf(ranges, lits, toks)


def test_oracle_ascii_masker_known_answer():
    # grammar_mask.rs:82-96 with restrict_to_numbers; None is never masked
    m = GrammarLogitMasker.new()
    m.restrict_to_numbers()
    codes = [ord("5"), ord("a"), ord("."), ord("Z"), 256]
    got = bits(oracle.ascii_mask_host(m.allowed_ascii_mask, codes), 5)
    assert got == [True, False, True, False, True]
    d = GrammarLogitMasker.new()  # Default: printable ASCII, newline and tab (grammar_mask.rs:23-35)
    got = bits(oracle.ascii_mask_host(d.allowed_ascii_mask, [0x20, 0x7E, 0x7F, 10, 9, 13, 0]), 7)
    assert got == [True, True, False, True, True, False, False]


# ----------------------------------------------------------------------------- the GPU

@pytest.mark.gpu
def test_gpu_gbnf_known_answer(torch_gpu):
    # academic_samplers_test.rs:94-123 through the mirror's apply_grammar_mask
    g = GbnfGrammarEngine({"root": GbnfRule("root", [("{", "{")], ["true"])}, "root")
    logits = [10.0, 10.0, 10.0, 10.0]
    g.apply_grammar_mask(logits, ['"key"', "{", "123", "true"])
    assert logits == [-math.inf, 10.0, -math.inf, 10.0]
    missing = GbnfGrammarEngine({}, "root")  # no start rule: nothing masked (sampler.rs:557)
    logits = [1.0, 2.0]
    missing.apply_grammar_mask(logits, ["x", "y"])
    assert logits == [1.0, 2.0]


@pytest.mark.gpu
def test_gpu_ascii_masker_known_answer(torch_gpu):
    m = GrammarLogitMasker.new()
    m.restrict_to_numbers()
    logits = [0.0] * 4
    m.mask_logits([ord("5"), ord("a"), ord("."), ord("Z")], logits)
    assert logits == [0.0, -math.inf, 0.0, -math.inf]
    logits = [1.0, 1.0, 1.0]  # more logits than bytes: only the first two are looked at
    m.mask_logits([ord("a"), None], logits)
    assert logits == [-math.inf, 1.0, 1.0]
    m.is_active = False
    logits = [1.0]
    m.mask_logits([ord("a")], logits)
    assert logits == [1.0]


@pytest.mark.gpu
@pytest.mark.parametrize("V", [1, 63, 5000, 50001])
def test_gpu_static_masks_match_oracle(torch_gpu, V):
    from oxide_sampler.grammar import TokenBytes
    rng = np.random.default_rng(V)
    alphabet = ["{", "[", '"', "t", "r", "u", "e", "n", "l", "1", " ", "é", "€", "\U0001f600"]
    toks = ["".join(rng.choice(alphabet, size=int(rng.integers(0, 7)))).encode() for _ in range(V)]
    for i, bad in zip(range(0, V, 97), [b"\xe2\x82", b"\xc0\x80", b"\xed\xa0\x80", b"\x80", b"\xff\xfe"] * V):
        toks[i] = bad
    print(f"\n[case] static masks V={V}", flush=True)
    g = GbnfGrammarEngine.new_json_grammar()
    rule = g.rules["root"]
    got = g.token_mask(TokenBytes(toks)).cpu().numpy().view(np.uint32)
    off, by = pack(toks)
    want = oracle.gbnf_mask_host([(ord(a), ord(b)) for a, b in rule.allowed_char_ranges],
                                 [x.encode() for x in rule.literal_strings], off, by)
    np.testing.assert_array_equal(got, want)
    m = GrammarLogitMasker.new()
    codes = [None if rng.random() < 0.1 else int(x) for x in rng.integers(0, 256, size=V)]
    got = m.token_mask(codes).cpu().numpy().view(np.uint32)
    want = oracle.ascii_mask_host(m.allowed_ascii_mask, [256 if c is None else c for c in codes])
    np.testing.assert_array_equal(got, want)


@pytest.mark.gpu
def test_gpu_shared_static_mask_feeds_the_sampler(torch_gpu):
    # one GBNF mask for every row (mask_ld = 0), against the oracle with the same shared mask
    from harness import run_gpu, run_oracle
    from oxide_sampler import workloads as wl
    rng = np.random.default_rng(3)
    V, B = 6000, 16
    alphabet = ["{", "[", '"', "t", "r", "u", "e", "x", "1", " "]
    toks = ["".join(rng.choice(alphabet, size=int(rng.integers(1, 5)))) for _ in range(V)]
    g = GbnfGrammarEngine.new_json_grammar()
    row = g.token_mask(toks).cpu().numpy().view(np.uint32)
    w = wl.config3(batch=B, vocab=V)
    w.mask = np.ascontiguousarray(row[None, :])  # [1, words]: the harness passes it as shared
    gpu = run_gpu(w, torch_gpu, shared_mask=True)
    ref = run_oracle(w, shared_mask=True)
    np.testing.assert_array_equal(gpu.tokens, ref.tokens)
    np.testing.assert_array_equal(gpu.status, ref.status)
    allowed = bits(row, V)
    assert all(allowed[int(t)] for t in gpu.tokens)
