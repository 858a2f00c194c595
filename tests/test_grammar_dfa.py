"""Grammar masks from a DFA: the reference's known answers, the oracle against a
brute-force walk, and the GPU kernel (oxs_dfa_mask) against the oracle, bit for bit.

Known answers: crates/oxide-server/tests/dfa_grammar_tests.rs:4-51 and the unit
tests of crates/oxide-core/src/dfa.rs:193-223.
"""
import numpy as np
import pytest

import oxs_oracle_ctypes as oracle
from oxide_sampler.grammar import DFA_ERROR_STATE, DfaSchemaGrammar, SchemaMismatch

ERR = DFA_ERROR_STATE


def pack(vocab):
    lens = np.array([len(b) for b in vocab], np.int64)
    offsets = np.zeros(len(vocab) + 1, np.uint32)
    offsets[1:] = np.cumsum(lens)
    return offsets, np.frombuffer(b"".join(vocab), np.uint8).copy()


def brute_mask(table, num_states, vocab, states):
    """Walks every (row, token) in Python, straight from dfa.rs:110-126 and grammar_engine.rs:42-65."""
    words = (len(vocab) + 31) // 32
    out = np.zeros((len(states), words), np.uint32)
    for b, s0 in enumerate(states):
        for t, tok in enumerate(vocab):
            s, ok = int(s0), True
            for byte in tok:
                if s >= num_states or table[s * 256 + byte] == ERR:
                    ok = False
                    break
                s = int(table[s * 256 + byte])
            if ok:
                out[b, t // 32] |= np.uint32(1 << (t % 32))
    return out


def random_dfa(rng, n, density):
    t = np.full(n * 256, ERR, np.uint32)
    live = rng.random(n * 256) < density
    t[live] = rng.integers(0, n + 2, size=int(live.sum()))  # some next states outside the table
    return t


def random_vocab(rng, V, alphabet, max_len):
    alpha = np.frombuffer(alphabet, np.uint8)
    out = []
    for _ in range(V):
        L = int(rng.integers(0, max_len + 1)) if rng.random() < 0.97 else int(rng.integers(17, 45))
        out.append(bytes(alpha[rng.integers(0, alpha.shape[0], size=L)]))
    return out


JSON_ALPHA = b'{}":,0123456789abcxyz "'


# ----------------------------------------------------------------------------- host logic (the reference's tests)

def test_dfa_json_validator_walk():
    # dfa_grammar_tests.rs:4-19
    dfa = DfaSchemaGrammar.new_simple_json_validator()
    state = 0
    for b in b'{"key":123}':
        state = dfa.transition(state, b)
    assert dfa.accepting_states[state]
    with pytest.raises(SchemaMismatch):
        dfa.transition(0, ord("5"))


def test_dfa_jump_forward():
    # dfa_grammar_tests.rs:39-51 and dfa.rs:197-213
    dfa = DfaSchemaGrammar.new_simple_json_validator()
    assert dfa.find_jump_forward_bytes(0, 4) == ([ord("{")], 1)
    assert dfa.find_jump_forward_bytes(3, 4) == ([ord(":")], 4)
    assert dfa.find_jump_forward_bytes(1, 10) == ([], 1)


def test_dfa_fixed_prefix_jump_forward():
    # dfa.rs:216-222
    dfa = DfaSchemaGrammar.new_json_with_fixed_prefix('{"answer": ')
    jump, state = dfa.find_jump_forward_bytes(0, 32)
    assert bytes(jump) == b'{"answer": ' and state == 11


# ----------------------------------------------------------------------------- the oracle

def test_oracle_logit_masking_known_answer():
    # dfa_grammar_tests.rs:21-37: from state 0 only '{"' is allowed
    dfa = DfaSchemaGrammar.new_simple_json_validator()
    vocab = [b'{"', b"123", b"hello"]
    off, by = pack(vocab)
    m = oracle.dfa_mask_host(dfa.transitions, dfa.num_states, off, by, np.array([0], np.uint32))
    assert m.tolist() == [[0b001]]


@pytest.mark.parametrize("seed", range(6))
def test_oracle_matches_brute_force(seed):
    rng = np.random.default_rng(seed)
    n = [1, 3, 8, 20, 47, 60][seed]
    table = random_dfa(rng, n, 0.5)
    vocab = random_vocab(rng, 150 + 37 * seed, JSON_ALPHA, 6)
    vocab[3] = b""  # an empty token is allowed from any state
    states = np.concatenate([rng.integers(0, n, size=5), [n, n + 7, ERR]]).astype(np.uint32)  # and from outside
    off, by = pack(vocab)
    got = oracle.dfa_mask_host(table, n, off, by, states)
    np.testing.assert_array_equal(got, brute_mask(table, n, vocab, states))
    assert all((got[b, 0] >> 3) & 1 for b in range(len(states)))


def test_oracle_rejects_ranges_outside_the_bytes():
    off = np.array([0, 2, 1, 9], np.uint32)  # token 1 runs backwards, token 2 past the 4 bytes
    by = np.frombuffer(b"{{{{", np.uint8).copy()
    dfa = DfaSchemaGrammar.new_simple_json_validator()
    m = oracle.dfa_mask_host(dfa.transitions, dfa.num_states, off, by, np.array([0], np.uint32))
    assert m.tolist() == [[0]]  # token 0 "{{" fails too: state 1 has no '{'


# ----------------------------------------------------------------------------- the GPU kernel

def gpu_mask(torch, table, n, vocab, states, offsets=None, by=None):
    import ctypes
    from oxide_sampler import _abi
    from oxide_sampler._abi import OxsDfa, OxsTokenBytes, check, load_library
    lib = load_library()
    d = torch.device("cuda")
    if offsets is None:
        offsets, by = pack(vocab)
    V = offsets.shape[0] - 1
    t_table = torch.from_numpy(np.asarray(table, np.uint32).view(np.int32).copy()).to(d)
    t_off = torch.from_numpy(offsets.view(np.int32).copy()).to(d)
    t_by = torch.from_numpy(by.copy() if by.size else np.zeros(1, np.uint8)).to(d)
    t_st = torch.from_numpy(np.asarray(states, np.uint32).view(np.int32).copy()).to(d)
    words = (V + 31) // 32
    mask = torch.full((len(states), words + 3), -1, dtype=torch.int32, device=d)  # padding words must stay
    dfa = OxsDfa(n, t_table.data_ptr())
    tb = OxsTokenBytes(V, int(by.shape[0]), t_off.data_ptr(), t_by.data_ptr())
    check(lib.oxs_dfa_mask(ctypes.byref(dfa), ctypes.byref(tb), ctypes.c_void_p(t_st.data_ptr()), len(states),
                           ctypes.c_void_p(mask.data_ptr()), mask.stride(0), None), "oxs_dfa_mask")
    torch.cuda.synchronize()
    m = mask.cpu().numpy().view(np.uint32)
    assert (m[:, words:] == 0xFFFFFFFF).all(), "wrote past ceil(vocab / 32) words"
    return m[:, :words]


@pytest.mark.gpu
def test_gpu_logit_masking_known_answer(torch_gpu):
    dfa = DfaSchemaGrammar.new_simple_json_validator()
    logits = [10.0, 10.0, 10.0]
    dfa.apply_dfa_mask(0, [b'{"', b"123", b"hello"], logits)  # dfa_grammar_tests.rs:21-37 on the GPU
    assert logits == [10.0, float("-inf"), float("-inf")]


@pytest.mark.gpu
@pytest.mark.parametrize("n,V,B", [(8, 1, 3), (8, 63, 5), (1, 64, 17), (20, 65, 16), (47, 1000, 33),
                                   (60, 2049, 7), (64, 3000, 9), (65, 3000, 9), (120, 700, 20),
                                   (8, 128256, 128)])
def test_gpu_dfa_mask_matches_oracle(torch_gpu, n, V, B):
    rng = np.random.default_rng(n * 1000 + V)
    table = random_dfa(rng, n, 0.4 if n > 2 else 0.9)
    vocab = random_vocab(rng, V, JSON_ALPHA, 8)
    states = rng.integers(0, n, size=B).astype(np.uint32)
    states[::5] = n + 1  # outside the table
    if B > 2:
        states[2] = ERR
    off, by = pack(vocab)
    print(f"\n[case] dfa mask states={n} vocab={V} rows={B}", flush=True)
    got = gpu_mask(torch_gpu, table, n, vocab, states)
    want = oracle.dfa_mask_host(table, n, off, by, states)
    np.testing.assert_array_equal(got, want)


@pytest.mark.gpu
def test_gpu_dfa_mask_empty_table(torch_gpu):
    # no states: every state is outside the table, so only tokens with no bytes are allowed
    vocab = [b"", b"a", b"", b"{}", b"x" * 40]
    off, by = pack(vocab)
    states = np.array([0, 3, ERR], np.uint32)
    got = gpu_mask(torch_gpu, np.zeros(0, np.uint32), 0, vocab, states)
    np.testing.assert_array_equal(got, oracle.dfa_mask_host(np.zeros(0, np.uint32), 0, off, by, states))
    assert got.tolist() == [[0b00101]] * 3


@pytest.mark.gpu
def test_gpu_dfa_mask_json_grammar_and_malformed_ranges(torch_gpu):
    dfa = DfaSchemaGrammar.new_json_with_fixed_prefix('{"answer": ')
    rng = np.random.default_rng(5)
    vocab = random_vocab(rng, 3000, b'{"answer: }0123456789', 5)
    off, by = pack(vocab)
    off[100] = off[101] + 3  # token 99 runs past token 100's start... and token 100 backwards
    off[2000] = by.shape[0] + 50  # tokens 1999 and 2000 leave the byte array
    states = np.arange(dfa.num_states + 2, dtype=np.uint32)
    got = gpu_mask(torch_gpu, dfa.transitions, dfa.num_states, None, states, off, by)
    np.testing.assert_array_equal(got, oracle.dfa_mask_host(dfa.transitions, dfa.num_states, off, by, states))


@pytest.mark.gpu
def test_gpu_dfa_mask_feeds_the_sampler(torch_gpu):
    # masks from oxs_dfa_mask as oxs_sample_batch's allowed_mask: every sampled token walks the DFA
    from harness import run_gpu, run_oracle
    from oxide_sampler import workloads as wl
    from oxide_sampler.grammar import TokenBytes
    dfa = DfaSchemaGrammar.new_simple_json_validator()
    rng = np.random.default_rng(11)
    V, B = 4096, 24
    vocab = random_vocab(rng, V, JSON_ALPHA, 4)
    states = rng.integers(0, dfa.num_states, size=B).astype(np.uint32)
    mask = dfa.token_masks(TokenBytes(vocab), states).cpu().numpy().view(np.uint32)
    w = wl.config3(batch=B, vocab=V)
    w.mask = np.ascontiguousarray(mask)
    g = run_gpu(w, torch_gpu)
    ref = run_oracle(w)
    np.testing.assert_array_equal(g.tokens, ref.tokens)
    np.testing.assert_array_equal(g.status, ref.status)
    for b in range(B):
        t = int(g.tokens[b])
        if g.status[b] == 0:
            assert (mask[b, t >> 5] >> (t & 31)) & 1
            s = int(states[b])
            for byte in vocab[t]:
                s = dfa.transition(s, byte)


@pytest.mark.gpu
@pytest.mark.parametrize("n,V", [(8, 1000), (47, 4097), (70, 20000)])
def test_gpu_state_mask_gather_matches_direct_walk(torch_gpu, n, V):
    # per-state masks computed once, gathered per step: equal to the direct walk and the oracle
    from oxide_sampler.grammar import TokenBytes
    rng = np.random.default_rng(n + V)
    table = random_dfa(rng, n, 0.4)
    vocab = random_vocab(rng, V, JSON_ALPHA, 6)
    g = DfaSchemaGrammar(n, table, [False] * n)
    tb = TokenBytes(vocab)
    print(f"\n[case] state-mask gather states={n} vocab={V}", flush=True)
    compiled = g.state_masks(tb)
    off, by = pack(vocab)
    for step in range(3):
        states = rng.integers(0, n, size=37).astype(np.uint32)
        states[::7] = n + 3
        states[5] = ERR
        got = g.gather_masks(compiled, states).cpu().numpy().view(np.uint32)
        direct = g.token_masks(tb, states).cpu().numpy().view(np.uint32)
        np.testing.assert_array_equal(got, direct)
        np.testing.assert_array_equal(got, oracle.dfa_mask_host(table, n, off, by, states))


@pytest.mark.gpu
def test_gpu_structured_output_engine_token_mask(torch_gpu):
    # grammar_engine.rs:40-65: every constraint type falls back to the JSON validator (:67-75)
    from oxide_sampler.grammar import GrammarConstraintType, StructuredOutputEngine
    vocab = [b'{"', b"123", b"hello", b"", b"{", b'{"a":1}', b"}"]
    for c in (GrammarConstraintType.JsonSchema("{}"), GrammarConstraintType.Regex(".*"),
              GrammarConstraintType.Ebnf("root ::= x")):
        eng = StructuredOutputEngine.compile(c)
        assert eng.compute_token_mask(0, vocab) == [True, False, False, True, True, True, False]
        off, by = pack(vocab)
        for state in (0, 1, 4, 5, 9):
            want = oracle.dfa_mask_host(eng.grammar.transitions, eng.grammar.num_states, off, by,
                                        np.array([state], np.uint32))
            assert eng.compute_token_mask(state, vocab) == [bool((want[0, t // 32] >> (t % 32)) & 1)
                                                            for t in range(len(vocab))]
