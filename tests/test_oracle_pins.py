"""Pins the CPU oracle (oracle/oxs_oracle.cpp) before any GPU result is trusted.

Each test checks one stage of crates/oxide-core/src/sampler.rs against
something the oracle's code does not share: the golden RNG vectors and a step
derived by hand, brute force over tiny vocabularies (full sort with the
lower-index tie rule, float64 softmax), hand-built probability lists whose
answers are worked out in the comments, closed forms for the Mirostat update,
and exhaustive sweeps of the draw. A plausible slip in the oracle (a dropped
-inf/NaN filter, a wrong cutoff index, tail-free and typical swapped, min-p /
XTC / top-k out of order, a shift in the window, a fused multiply-add in the
penalties) fails at least one of them.
"""
import json
import math
from pathlib import Path

import numpy as np
import pytest

import oxs_oracle_ctypes as oracle
from harness import run_oracle
from oxide_sampler import MirostatMode, SamplerState
from oxide_sampler.workloads import Workload, disabled_config

GOLDEN = Path(__file__).resolve().parent / "golden"
F32 = np.float32


def row(logits, cfg, history=(), u=0.5, mu=None, newline=0, logits_out=False, use_rng=False, rng=None):
    """Runs one row through the oracle's batch entry point (the descriptor the GPU path takes)."""
    lg = np.asarray(logits, np.float32).reshape(1, -1)
    V = lg.shape[1]
    hist = np.zeros((1, len(history) + 4), np.uint32)
    hist[0, : len(history)] = np.asarray(history, np.uint32)
    w = Workload(name="pin", logits=lg, dtype="f32", configs=[cfg], history=hist,
                 history_len=np.array([len(history)], np.uint32), uniforms=np.array([u], np.float32),
                 mu=None if mu is None else np.array([mu], np.float32), newline_token_id=newline)
    rs = None if rng is None else np.array([rng], np.uint64)
    return run_oracle(w, kept_ld=max(256, int(cfg.top_k), V), logits_out=logits_out, use_rng=use_rng, rng_state=rs)


def kept(r):
    n = int(r.kept_count[0])
    return r.kept_ids[0, :n].tolist(), r.kept_probs[0, :n]


# ----------------------------------------------------------------------------- a3: SamplerState RNG

def _golden_rng():
    return json.loads((GOLDEN / "rng_vectors.json").read_text())["vectors"]


def test_rng_first_step_by_hand():
    # sampler.rs:139-146 from x = 1: x ^= x << 13 -> 0x2001 (8193); x ^= x >> 7 -> 8193 ^ 64 = 8257;
    # x ^= x << 17 -> 8257 ^ (8257 << 17) = 8257 + 1082261504 = 1082269761.
    s = np.array([1], np.uint64)
    lib = oracle.load()
    import ctypes
    assert lib.oxo_next_u64(s.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64))) == 1082269761
    assert int(s[0]) == 1082269761


@pytest.mark.parametrize("vec", _golden_rng(), ids=lambda v: v["seed"])
def test_rng_golden_vectors(vec):
    import ctypes
    lib = oracle.load()
    seed = int(vec["seed"], 16)
    s = np.array([seed], np.uint64)
    p = s.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64))
    got = [lib.oxo_next_u64(p) for _ in vec["next_u64"]]
    assert got == [int(v, 16) for v in vec["next_u64"]]
    s[0] = seed
    got_f = [lib.oxo_next_f32(p) for _ in vec["next_f32"]]
    assert got_f == vec["next_f32"]
    # next_f32 lies on the 2^-24 grid in [0, 1 - 2^-24] (sampler.rs:150-153).
    for f in got_f:
        assert 0.0 <= f <= 1.0 - 2.0 ** -24 and (f * 16777216.0).is_integer()
    # The product's host mirror of SamplerState agrees.
    st = SamplerState(rng_state=seed)
    assert [st.next_u64() for _ in vec["next_u64"]] == [int(v, 16) for v in vec["next_u64"]]


def test_rng_is_linear_over_gf2():
    # Every xorshift step is a linear map over GF(2)^64: next(a ^ b) == next(a) ^ next(b).
    # An add in place of an xor, or an arithmetic right shift, breaks this.
    import ctypes
    lib = oracle.load()
    rng = np.random.default_rng(3)
    for _ in range(64):
        a, b = (int(x) for x in rng.integers(1, 2 ** 63, size=2, dtype=np.int64))
        a |= 1 << 63
        sa, sb, sab = (np.array([v], np.uint64) for v in (a, b, a ^ b))
        f = lambda s: lib.oxo_next_u64(s.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)))
        assert f(sab) == f(sa) ^ f(sb)


def test_draw_consumes_one_rng_step_and_greedy_none():
    # sampler.rs:371-389: a draw calls next_f32 once; temperature <= 1e-6 never touches the RNG.
    vec = _golden_rng()[0]
    seed = int(vec["seed"], 16)
    lg = [0.5, 2.0, 1.0, -1.0]
    r = row(lg, disabled_config(temperature=1.0), use_rng=True, rng=seed)
    assert int(r.rng_state[0]) == int(vec["next_u64"][0], 16)
    ids, probs = kept(r)
    u = vec["next_f32"][0]
    acc, want = F32(0), ids[0]
    for i, p in zip(ids, probs):
        acc = F32(acc + p)
        if F32(u) <= acc:
            want = i
            break
    assert int(r.tokens[0]) == want
    r = row(lg, disabled_config(temperature=0.0), use_rng=True, rng=seed)
    assert int(r.rng_state[0]) == seed and int(r.tokens[0]) == 1


# ----------------------------------------------------------------------------- a5, a7-a9: pre-softmax stages

def _brute_penalties(lg, cfg, history, newline):
    """sampler.rs:184-254 written directly from the reference's statements, one float32 op at a time."""
    x = [F32(v) for v in lg]
    V = len(x)
    for t in cfg.banned_tokens:
        if t < V:
            x[t] = F32(-np.inf)
    for t, b in cfg.logit_biases.items():
        if t < V:
            x[t] = F32(x[t] + F32(b))
    if cfg.penalize_nl and newline < V:
        x[newline] = F32(x[newline] - F32(cfg.newline_penalty))
    if history:
        n = cfg.repeat_last_n if cfg.repeat_last_n > 0 else len(history)
        window = list(history[max(0, len(history) - n):])
        rp = F32(cfg.repeat_penalty)
        if abs(float(rp) - 1.0) > 1e-5 and rp > 0:
            seen = set()
            for t in window:
                if t in seen:
                    continue
                seen.add(t)
                if t < V:
                    x[t] = F32(x[t] / rp) if x[t] > 0 else F32(x[t] * rp)
        f, p = F32(cfg.frequency_penalty), F32(cfg.presence_penalty)
        if abs(float(f)) > 1e-5 or abs(float(p)) > 1e-5:
            for t in sorted(set(window)):
                if t < V:
                    c = F32(window.count(t))
                    x[t] = F32(x[t] - F32(F32(c * f) + p))  # two roundings, no fused multiply-add
    if cfg.temperature > 0 and cfg.mirostat_mode == MirostatMode.Disabled:
        inv = F32(F32(1.0) / F32(cfg.temperature))
        x = [F32(v * inv) for v in x]
    return np.array(x, np.float32)


@pytest.mark.parametrize("repeat_last_n", [0, 1, 5, 8, 100])
def test_penalties_bias_ban_newline_temperature_brute_force(repeat_last_n):
    V = 48
    rng = np.random.default_rng(7 + repeat_last_n)
    lg = (rng.standard_normal(V) * 3).astype(np.float32)
    lg[5], lg[6], lg[12] = -2.5, 0.0, 7.25  # the divide branch, the multiply branch at 0, a large positive
    history = [3, 5, 5, 9, 6, 12, 5, 40, 3, 17, 9, 9, 77, 12]  # 77 is out of range: skipped
    cfg = disabled_config(repeat_penalty=1.3, repeat_last_n=repeat_last_n, frequency_penalty=0.4,
                          presence_penalty=0.25, temperature=0.7, logit_biases={3: 1.5, 20: -0.75, 99: 4.0, 17: 2.0},
                          banned_tokens={17, 30, 1000}, penalize_nl=True, newline_penalty=0.5)
    r = row(lg, cfg, history, newline=9, logits_out=True)
    want = _brute_penalties(lg, cfg, history, 9)
    np.testing.assert_array_equal(r.logits_out[0].view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("prefix", [[], [2], [2, 2, 1]])
def test_dry_penalty_by_hand(prefix):
    # sampler.rs:393-415 over the last dry_range = 6 ids [0, 1, 0, 1, 0, 1] (ids before them are
    # out of range), multiplier 2, base 1.5, allowed length 2. Matches of the suffix and the id after them:
    #   L=4: [0,1,0,1] at i=0 -> id 0, penalty 2 * 1.5^2 = 4.5
    #   L=3: [1,0,1]   at i=1 -> id 0, penalty 3
    #   L=2: [0,1]     at i=0 and i=2 -> id 0 twice, penalty 2 each
    # so logit 0 goes 5 - 4.5 - 3 - 2 - 2 = -6.5 and ids 1, 2 keep 5.
    history = prefix + [0, 1, 0, 1, 0, 1]
    cfg = disabled_config(dry_multiplier=2.0, dry_base=1.5, dry_allowed_length=2, dry_range=6, temperature=0.0)
    r = row([5.0, 5.0, 5.0], cfg, history, logits_out=True)
    assert r.logits_out[0].tolist() == [-6.5, 5.0, 5.0]
    assert int(r.tokens[0]) == 1  # greedy: ids 1 and 2 tie, the lower id wins


def test_temperature_skipped_under_mirostat():
    # sampler.rs:249: no temperature scaling when Mirostat is on.
    lg = np.array([1.0, 2.5, -3.0, 0.25], np.float32)
    r = row(lg, disabled_config(temperature=0.37, mirostat_mode=MirostatMode.V2), mu=10.0, logits_out=True)
    np.testing.assert_array_equal(r.logits_out[0], lg)


# ----------------------------------------------------------------------------- a10-a11: pool, top-M, softmax

@pytest.mark.parametrize("V,top_k,seed", [(2000, 0, 1), (1999, 40, 2), (300, 0, 3), (100, 0, 4), (700, 300, 5)])
def test_top_m_select_brute_force(V, top_k, seed):
    rng = np.random.default_rng(seed)
    lg = (np.round(rng.standard_normal(V) * 4) / 4).astype(np.float32)  # a quarter-step grid: many ties
    lg[rng.choice(V, 7, replace=False)] = -np.inf
    lg[rng.choice(V, 3, replace=False)] = np.nan  # NaN is not > -inf: dropped from the pool (sampler.rs:257-265)
    r = row(lg, disabled_config(top_k=top_k))
    pool = np.nonzero(lg > -np.inf)[0]
    order = pool[np.lexsort((pool, -lg[pool].astype(np.float64)))]  # descending logit, then lower id
    M = min(max(top_k, 256), pool.size)
    K = min(top_k, M) if top_k > 0 else M
    ids, probs = kept(r)
    assert ids == order[:K].tolist()
    # softmax over the top-M only (sampler.rs:286-295), then renormalised over the kept K
    z = lg[order[:M]].astype(np.float64)
    p = np.exp(z - z[0])
    p /= p.sum()
    q = p[:K] / p[:K].sum()
    np.testing.assert_allclose(probs, q, rtol=1e-5, atol=1e-12)


def test_all_masked_and_nan_rows_are_empty():
    r = row([np.nan, -np.inf, np.nan], disabled_config())
    assert int(r.tokens[0]) == 0 and int(r.history_len[0]) == 0 and int(r.status[0]) == 1


# ----------------------------------------------------------------------------- a13-a19: filters on hand-built lists

P4 = np.log(np.array([0.5, 0.3, 0.15, 0.05]))  # softmax gives back p = [0.5, 0.3, 0.15, 0.05]


@pytest.mark.parametrize("cfg_kw,want_ids", [
    # top-p (sampler.rs:346-357): cum 0.5, 0.8 >= 0.75 -> keep 2; 0.85 -> cum 0.95 at i=2 -> keep 3
    (dict(top_p=0.75), [0, 1]),
    (dict(top_p=0.85), [0, 1, 2]),
    (dict(top_p=1.0), [0, 1, 2, 3]),
    # min-p (:315-319): threshold 0.5 * 0.5 = 0.25 keeps 0.5, 0.3
    (dict(min_p=0.5), [0, 1]),
    (dict(min_p=0.0), [0, 1, 2, 3]),
    # XTC (:322-328): 0.4 <= p0 = 0.5 < 0.98 removes id 0; threshold 0.6 > p0 keeps it
    (dict(xtc_threshold=0.4, xtc_probability=1.0), [1, 2, 3]),
    (dict(xtc_threshold=0.6, xtc_probability=1.0), [0, 1, 2, 3]),
    # min-p -> XTC -> top-k: min-p 0.2 keeps 3, XTC drops id 0, top-k 1 keeps id 1.
    # (top-k before XTC would keep [0]; XTC before min-p would keep [1, 2].)
    (dict(min_p=0.2, xtc_threshold=0.4, xtc_probability=1.0, top_k=1), [1]),
    # tail-free (:459-490): d1 = [.2, .15, .1], d2 = [.05, .05], S = .1, cum = .5, 1.0;
    # z = 0.4 -> cutoff 1; z = 0.7 -> cutoff 2 (i + 1, not i + 2)
    (dict(tfs_z=0.4), [0]),
    (dict(tfs_z=0.7), [0, 1]),
    (dict(top_k=2, tfs_z=0.1), [0, 1]),  # two candidates: tail-free needs > 2 (:336) and is a no-op
])
def test_filters_on_hand_built_list(cfg_kw, want_ids):
    r = row(P4, disabled_config(**cfg_kw), u=0.0)
    ids, probs = kept(r)
    assert ids == want_ids
    p = np.array([0.5, 0.3, 0.15, 0.05])[want_ids]
    np.testing.assert_allclose(probs, p / p.sum(), rtol=1e-6)
    assert int(r.tokens[0]) == want_ids[0]  # u = 0 picks the first kept candidate


def test_typical_reorders_by_score():
    # p = [0.6, 0.3, 0.1]: H = -sum p ln p = 0.8979; |-ln p - H| = [0.3871, 0.3061, 1.4046];
    # a stable ascending sort gives [1, 0, 2] (sampler.rs:493-520).
    lg = np.log(np.array([0.6, 0.3, 0.1]))
    r = row(lg, disabled_config(typical_p=0.25), u=0.999)
    assert kept(r)[0] == [1] and int(r.tokens[0]) == 1        # cum 0.3 >= 0.25
    r = row(lg, disabled_config(typical_p=0.5), u=0.0)
    ids, probs = kept(r)
    assert ids == [1, 0]                                       # cum 0.3, then 0.9 >= 0.5
    np.testing.assert_allclose(probs, [1 / 3, 2 / 3], rtol=1e-6)
    assert int(r.tokens[0]) == 1


def test_tail_free_runs_before_typical():
    # sampler.rs:336-343. p = [0.5, 0.3, 0.15, 0.05]: tail-free z = 0.7 keeps [0, 1] (p = .5, .3, not
    # renormalised); typical then sees H = 0.7078, scores [0.0147, 0.4962] -> order [0, 1]; typical_p 0.4
    # keeps [0]. Typical first would score all four (H = 1.1468: [0.4537, 0.0572, 0.7503, 1.8489]),
    # keep [1, 0] and tail-free would leave that two-element list alone.
    r = row(P4, disabled_config(tfs_z=0.7, typical_p=0.4), u=0.999)
    assert kept(r)[0] == [0]


@pytest.mark.parametrize("u_num", range(0, 65))
def test_draw_inverse_cdf_sweep(u_num):
    # sampler.rs:371-389: acc += p in order; the first r <= acc wins; falling off the end picks cand[0].
    u = min(u_num / 64.0, 1.0 - 2.0 ** -24)
    lg = np.array([0.3, 1.7, -0.4, 1.1, 0.9], np.float32)
    r = row(lg, disabled_config(temperature=1.3), u=u)
    ids, probs = kept(r)
    acc, want = F32(0), ids[0]
    for i, p in zip(ids, probs):
        acc = F32(acc + p)
        if F32(u) <= acc:
            want = i
            break
    assert int(r.tokens[0]) == want


def test_greedy_lower_index_on_ties():
    r = row([1.0, 3.0, 3.0, 2.0], disabled_config(temperature=0.0), u=0.99)
    assert int(r.tokens[0]) == 1


# ----------------------------------------------------------------------------- a12: Mirostat

P3 = np.log(np.array([0.7, 0.2, 0.1]))


def test_mirostat_v2_small_mu_closed_form():
    # mu = 1: surprise(p1 = 0.2) = 2.32 > 1 stops at i = 1, so cum = p0 and prob = p0 / p0 = 1 exactly;
    # mu' = 1 - 0.1f * (0 - 5) = 1.5 exactly. The token is top-1 and is recorded twice (:301/:307, :454).
    r = row(P3, disabled_config(mirostat_mode=MirostatMode.V2, mirostat_tau=5.0, mirostat_eta=0.1), [4], mu=1.0, u=0.9)
    assert int(r.tokens[0]) == 0
    assert float(r.mu[0]) == 1.5
    assert r.history[0, : int(r.history_len[0])].tolist() == [4, 0, 0]
    # no filters after Mirostat: the buffer keeps the whole top-M
    assert kept(r)[0] == [0, 1, 2]


def test_mirostat_v2_large_mu_closed_form():
    # mu = 10: every surprise <= 10, cutoff 3, cum = 1, prob = p0 = 0.7: mu' = 10 - 0.1 (-log2 0.7 - 5).
    r = row(P3, disabled_config(mirostat_mode=MirostatMode.V2, mirostat_tau=5.0, mirostat_eta=0.1), mu=10.0)
    assert math.isclose(float(r.mu[0]), 10.0 - 0.1 * (-math.log2(0.7) - 5.0), rel_tol=1e-6)


def test_mirostat_v1_closed_form():
    # sampler.rs:418-429: mu' = mu - eta (-log2(max(p0, 1e-6)) - tau), token = top-1 recorded twice.
    r = row(P3, disabled_config(mirostat_mode=MirostatMode.V1, mirostat_tau=3.0, mirostat_eta=0.25), mu=6.0)
    assert int(r.tokens[0]) == 0 and int(r.history_len[0]) == 2
    assert math.isclose(float(r.mu[0]), 6.0 - 0.25 * (-math.log2(0.7) - 3.0), rel_tol=1e-6)
