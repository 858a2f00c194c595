"""The decode stage: oxs_decode_step and DecodeLoop against the oracle.

Reference: crates/oxide-engine/src/continuous_batching.rs:940-1040 (the
scheduler's decode stage) and megakernel_ops.cu:331-347 (the device-side
advance and host hand-off).
"""
import ctypes

import numpy as np
import pytest

import oxs_oracle_ctypes as oracle
from oxide_sampler import _abi
from oxide_sampler.decode import STOP_TOKENS, Sequence, next_event
from oxide_sampler.engine import MirostatMode, SamplerState, SamplingConfig, configs_to_array
from oxide_sampler.grammar import DfaSchemaGrammar

SENT = 0xA5A5A5A5  # fills the kept arrays: a raw-argmax row must leave them as they were


# ----------------------------------------------------------------------------- the oracle's raw argmax

def test_raw_argmax_special_cases():
    # continuous_batching.rs:961-970: strict '>' from -inf at index 0
    inf, nan = np.inf, np.nan
    cases = [
        ([1.0, 3.0, 3.0, 2.0], 1),       # first of equal maxima
        ([-inf, -inf], 0),               # nothing above -inf: the initial index
        ([nan, nan, nan], 0),            # NaN is never larger
        ([nan, 1.0, nan, 0.5], 1),
        ([-inf, nan, -5.0], 2),
        ([2.0, inf, 7.0, inf], 1),       # first +inf
        ([-0.0, 0.0], 0),                # 0.0 > -0.0 is false
        ([-3e38, -inf, -2e38], 2),
    ]
    for row, want in cases:
        assert oracle.raw_argmax_host(np.array(row, np.float32)) == want, row


def test_raw_argmax_matches_numpy():
    rng = np.random.default_rng(7)
    for n in (1, 2, 17, 1000, 32000):
        x = rng.standard_normal(n).astype(np.float32)
        x[rng.random(n) < 0.1] = np.nan
        x[rng.random(n) < 0.1] = -np.inf
        if n > 3:
            x[n // 3] = x[2 * n // 3] = np.float32(9.0)  # a tie for the maximum
        y = np.where(np.isnan(x), -np.inf, x)
        want = int(np.argmax(y))  # numpy's argmax returns the first maximum
        assert oracle.raw_argmax_host(x) == want


# ----------------------------------------------------------------------------- a decode-step workload

def decode_configs():
    C = SamplingConfig
    rows = [
        C(temperature=0.8, top_p=0.95),                           # the loop's own config (:446-450)
        C(temperature=0.0, top_p=0.9),                            # raw argmax (:961)
        C(temperature=1e-6, repeat_penalty=2.0),                  # raw: penalties do not apply
        C(temperature=2e-6, top_k=0, min_p=0.0),                  # sampled, scaled by 1/T
        C(temperature=float("nan")),                              # NaN <= 1e-6 is false: sampled, no scaling
        C(temperature=1.0, top_k=0, mirostat_mode=MirostatMode.V2),
        C(temperature=0.7, frequency_penalty=0.3, presence_penalty=0.2, repeat_penalty=1.05, repeat_last_n=0,
          top_k=50, top_p=0.9),
        C(temperature=0.9, dry_multiplier=0.8, dry_allowed_length=2, top_k=0, min_p=0.0, top_p=0.97),
        C(temperature=1.2, typical_p=0.9, tfs_z=0.95, top_k=0, min_p=0.0),
        C(temperature=0.5, xtc_probability=0.5, xtc_threshold=0.05, min_p=0.0),
        C(temperature=1.0, mirostat_mode=MirostatMode.V1),
        C(temperature=-1.0, penalize_nl=True),                    # raw
    ]
    return rows + rows


def decode_state(B, cap, seed):
    rng = np.random.default_rng(seed)
    history = np.zeros((B, cap), np.uint32)
    hlen = rng.integers(0, 24, size=B).astype(np.uint32)
    motif = rng.integers(0, 50, size=6)
    for b in range(B):
        h = np.concatenate([motif, rng.integers(0, 400, size=40), motif])[: hlen[b]]
        history[b, : hlen[b]] = h
    hlen[5] = cap - 1  # the Mirostat row records twice per step: its history fills
    mu = np.full(B, 10.0, np.float32)  # SamplerState::new(5.0)
    rng_state = np.array([0x853C49E6748FEA9B + 977 * b for b in range(B)], np.uint64)
    dec = {"current_token": rng.integers(0, 1000, size=B).astype(np.uint32),
           "current_position": rng.integers(0, 5000, size=B).astype(np.int32),
           "generated_count": rng.integers(0, 50, size=B).astype(np.uint32)}
    return history, hlen, mu, rng_state, dec


def decode_logits(B, V, step, history, hlen):
    rng = np.random.default_rng(1000 + step)
    x = (rng.standard_normal((B, V), dtype=np.float32) * np.float32(2.0))
    for b in range(B):  # recent history ids strong, so the penalties matter
        n = int(hlen[b])
        if n:
            ids = history[b, max(0, n - 8):n]
            x[b, ids] += np.float32(4.0)
    x[1, 10:14] = np.float32(50.0)         # a tie for the raw argmax
    if step == 2:
        x[2, :] = -np.inf                   # raw row with no candidate: token 0
        x[0, :] = -np.inf                   # sampled row with no candidate: EMPTY, nothing recorded
    if step == 3:
        x[1, ::3] = np.nan
        x[6, ::5] = np.nan
    return x


def oracle_decode(cfg_bytes, logits, history, hlen, mu, rng_state, dec, cap):
    return oracle.sample_batch_host(
        _abi, logits=logits, dtype="f32", configs_bytes=cfg_bytes, bias_ids=None, bias_values=None, ban_ids=None,
        mask=None, history=history, history_len=hlen, history_cap=cap, record=True, uniforms=None,
        rng_state=rng_state, mu=mu, kept_ld=256, decode=dec, kept_fill=SENT)


def test_oracle_decode_step_is_sample_batch_plus_raw_rows():
    B, V, cap = 24, 3001, 64
    cfgs = decode_configs()
    cfg_bytes = configs_to_array(cfgs, 10)[0]
    history, hlen, mu, rng_state, dec = decode_state(B, cap, 3)
    logits = decode_logits(B, V, 1, history, hlen)
    h2, l2, m2, r2 = history.copy(), hlen.copy(), mu.copy(), rng_state.copy()
    d0 = {k: v.copy() for k, v in dec.items()}
    got = oracle_decode(cfg_bytes, logits, history, hlen, mu, rng_state, dec, cap)
    ref = oracle.sample_batch_host(
        _abi, logits=logits, dtype="f32", configs_bytes=cfg_bytes, bias_ids=None, bias_values=None, ban_ids=None,
        mask=None, history=h2, history_len=l2, history_cap=cap, record=True, uniforms=None, rng_state=r2, mu=m2,
        kept_ld=256, kept_fill=SENT)
    raw = np.array([c.temperature <= 1e-6 for c in cfgs])
    for b in range(B):
        if raw[b]:
            assert got["tokens"][b] == oracle.raw_argmax_host(logits[b])
            assert got["kept_count"][b] == SENT and (got["kept_ids"][b] == SENT).all()
        else:
            assert got["tokens"][b] == ref["tokens"][b] and got["status"][b] == ref["status"][b]
            np.testing.assert_array_equal(got["kept_ids"][b], ref["kept_ids"][b])
    # raw rows: the sampler state is untouched; sampled rows: as sample_batch left it
    assert (history[raw] == decode_state(B, cap, 3)[0][raw]).all()
    np.testing.assert_array_equal(hlen[~raw], l2[~raw])
    np.testing.assert_array_equal(rng_state[~raw], r2[~raw])
    np.testing.assert_array_equal(rng_state[raw], decode_state(B, cap, 3)[3][raw])
    np.testing.assert_array_equal(dec["current_token"], got["tokens"])
    np.testing.assert_array_equal(dec["current_position"], d0["current_position"] + 1)
    np.testing.assert_array_equal(dec["generated_count"], d0["generated_count"] + 1)


# ----------------------------------------------------------------------------- the host bookkeeping

def test_next_event_stop_length_and_dfa():
    # :986-1030 — stop tokens without a tokenizer, max_tokens, DFA accepting states
    ev = next_event(Sequence(3, 0.8, 1), 128_009)
    assert ev.is_terminal and ev.finish_reason == "stop"
    ev = next_event(Sequence(3, 0.8, 3), 500)
    assert ev.is_terminal and ev.finish_reason == "length"
    ev = next_event(Sequence(3, 0.8, 2), 500)
    assert not ev.is_terminal and ev.finish_reason is None
    assert all(t in STOP_TOKENS for t in (0, 2, 128_001, 128_008, 128_009, 151_643, 151_645))
    # a DFA walk over the token's low byte; bytes with no transition keep the state
    dfa = DfaSchemaGrammar.new_simple_json_validator()
    seq = Sequence(100, 0.8, 1, dfa, 0)
    for tok in (ord("{"), ord("x"), ord('"'), ord("k"), ord('"'), ord(":"), ord("7")):
        assert not next_event(seq, tok + 256).is_terminal  # + 256: only the low byte counts
    assert seq.dfa_state == 5
    ev = next_event(seq, ord("}"))
    assert ev.is_terminal and ev.finish_reason == "stop" and seq.dfa_state == 7
    # with a tokenizer's bytes
    seq = Sequence(100, 0.8, 1, dfa, 0)
    next_event(seq, 9999, token_bytes=lambda t: b'{"ab"')
    assert seq.dfa_state == 3


# ----------------------------------------------------------------------------- the GPU

def _to_dev(torch, a, dtype=None):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    elif a.dtype == np.uint64:
        a = a.view(np.int64)
    return torch.from_numpy(a.copy()).to("cuda")


def _u32(t):
    return t.cpu().numpy().view(np.uint32)


@pytest.mark.gpu
def test_gpu_decode_steps_match_oracle(torch_gpu):
    from oxide_sampler import BatchSampler
    from oxide_sampler._abi import OxsDecodeIo
    t = torch_gpu
    B, V, cap, steps = 24, 50001, 64, 5
    cfgs = decode_configs()
    cfg_bytes = configs_to_array(cfgs, 10)[0]
    history, hlen, mu, rng_state, dec = decode_state(B, cap, 11)
    d_cfg = _to_dev(t, cfg_bytes)
    d_hist, d_hlen, d_mu, d_rng = (_to_dev(t, a) for a in (history, hlen, mu, rng_state))
    d_dec = {k: _to_dev(t, v) for k, v in dec.items()}
    lib = _abi.load_library()
    host = ctypes.c_void_p()
    _abi.check(lib.oxs_host_alloc(8 * B, ctypes.byref(host)), "oxs_host_alloc")
    try:
        io = OxsDecodeIo(d_dec["current_token"].data_ptr(), d_dec["current_position"].data_ptr(),
                         d_dec["generated_count"].data_ptr(), host.value)
        s = BatchSampler(B, V, 256)
        out = {"tokens": t.zeros(B, dtype=t.int32, device="cuda"),
               "status": t.zeros(B, dtype=t.int32, device="cuda"),
               "kept_count": t.zeros(B, dtype=t.int32, device="cuda"),
               "kept_ids": t.zeros(B, 256, dtype=t.int32, device="cuda"),
               "kept_probs": t.zeros(B, 256, dtype=t.float32, device="cuda")}
        sent = int(np.uint32(SENT).view(np.int32))
        for step in range(steps):
            print(f"\n[case] decode step {step} B={B} V={V}", flush=True)
            logits = decode_logits(B, V, step, history, hlen)
            for k in ("kept_count", "kept_ids"):
                out[k].fill_(sent)
            out["kept_probs"].view(t.int32).fill_(sent)
            s.sample(_to_dev(t, logits), d_cfg, history=d_hist, history_len=d_hlen, history_cap=cap, record=True,
                     rng_state=d_rng, mirostat_mu=d_mu, kept_ld=256, decode=io, out=out)
            t.cuda.synchronize()
            ref = oracle_decode(cfg_bytes, logits, history, hlen, mu, rng_state, dec, cap)
            np.testing.assert_array_equal(_u32(out["tokens"]), ref["tokens"])
            np.testing.assert_array_equal(out["status"].cpu().numpy(), ref["status"])
            np.testing.assert_array_equal(_u32(out["kept_count"]), ref["kept_count"])
            kc = ref["kept_count"]
            kid, kpr = _u32(out["kept_ids"]), out["kept_probs"].cpu().numpy().view(np.uint32)
            for b in range(B):
                n = 256 if kc[b] == SENT else int(kc[b])
                np.testing.assert_array_equal(kid[b, :n], ref["kept_ids"][b, :n])
                np.testing.assert_array_equal(kpr[b, :n], ref["kept_probs"][b, :n].view(np.uint32))
            np.testing.assert_array_equal(_u32(d_hlen), hlen)
            np.testing.assert_array_equal(_u32(d_hist), history)
            np.testing.assert_array_equal(d_mu.cpu().numpy().view(np.uint32), mu.view(np.uint32))
            np.testing.assert_array_equal(d_rng.cpu().numpy().view(np.uint64), rng_state)
            for k in dec:
                np.testing.assert_array_equal(d_dec[k].cpu().numpy().view(dec[k].dtype), dec[k])
            slots = np.frombuffer((ctypes.c_uint64 * B).from_address(host.value), dtype=np.uint64).copy()
            np.testing.assert_array_equal((slots & np.uint64(0xFFFFFFFF)).astype(np.uint32), ref["tokens"])
            assert ((slots >> np.uint64(32)) == step + 1).all()  # every row's step count
        raw = np.array([c.temperature <= 1e-6 for c in cfgs])
        assert (ref["status"][~raw] == _abi.OXS_ROW_HISTORY_FULL).any()  # the filled history was reached
        s.close()
    finally:
        t.cuda.synchronize()
        lib.oxs_host_free(host)


def _loop_with(torch, cfgs, V, cap=128):
    from oxide_sampler import DecodeLoop
    loop = DecodeLoop(len(cfgs), V, history_cap=cap)
    for slot, c in enumerate(cfgs):
        loop.add_sequence(slot, temperature=c.temperature, top_p=c.top_p, current_token=slot, current_position=7,
                          max_tokens=1000, config=c)
    return loop


@pytest.mark.gpu
def test_gpu_decode_loop_host_poll_and_graph_replays(torch_gpu):
    t = torch_gpu
    cfgs = decode_configs()[:12]
    B, V = len(cfgs), 32000
    eager = _loop_with(t, cfgs, V)
    graphed = _loop_with(t, cfgs, V)
    static = t.zeros(B, V, dtype=t.float32, device="cuda")
    graphed.capture(static)
    hist = np.zeros((B, 1), np.uint32)
    for step in range(6):
        print(f"\n[case] decode loop step {step}: eager, then graph replay", flush=True)
        x = decode_logits(B, V, step + 10, hist, np.zeros(B, np.uint32))
        n = eager.launch(_to_dev(t, x))
        tok_e = eager.wait(n)  # polled from host memory, no stream sync
        static.copy_(_to_dev(t, x))
        m = graphed.replay()
        tok_g = graphed.wait(m)
        assert eager.completed() == step + 1 and graphed.completed() == step + 1
        np.testing.assert_array_equal(tok_g, tok_e)
        t.cuda.synchronize()
        np.testing.assert_array_equal(_u32(eager.out["tokens"]), tok_e)
        for name in ("history", "history_len", "mirostat_mu", "rng_state", "current_token", "current_position",
                     "generated_count"):
            a, b = getattr(eager, name), getattr(graphed, name)
            assert t.equal(a, b), (step, name)
    # raw slots (temperature <= 1e-6) kept their state; the others recorded
    for slot, c in enumerate(cfgs):
        st = eager.state(slot)
        if c.temperature <= 1e-6:
            assert st.generated_tokens == [] and st.rng_state == SamplerState.new(5.0).rng_state
        assert int(eager.current_position[slot]) == 7 + 6 and int(eager.generated_count[slot]) == 6
    eager.close()
    graphed.close()


@pytest.mark.gpu
def test_gpu_decode_loop_events_match_reference_loop(torch_gpu):
    # DecodeLoop.step against the reference loop run on the oracle, sequence by sequence
    t = torch_gpu
    V, B, steps = 4096, 8, 12
    from oxide_sampler import DecodeLoop
    loop = DecodeLoop(B, V, history_cap=64)
    dfa = DfaSchemaGrammar.new_simple_json_validator()
    specs = [(0.8, 0.95, 5, None), (0.0, 1.0, 100, None), (1.0, 0.9, 100, dfa), (0.5, 0.5, 3, None),
             (0.9, 0.95, 100, dfa), (1e-7, 0.95, 4, dfa)]
    ref_state = {}
    for slot, (temp, top_p, max_tok, g) in enumerate(specs):
        loop.add_sequence(slot, temperature=temp, top_p=top_p, current_token=1, current_position=0,
                          max_tokens=max_tok, dfa=g)
        ref_state[slot] = (SamplerState.new(5.0), Sequence(max_tok, temp, 0, g, 0),
                           SamplingConfig(temperature=temp, top_p=top_p))
    rng = np.random.default_rng(5)
    for step in range(steps):
        x = (rng.standard_normal((B, V), dtype=np.float32) * np.float32(3.0))
        x[:, [0, 2]] -= np.float32(6.0)          # stop tokens possible but rare
        x[:, [ord("{"), ord('"'), ord("}")]] += np.float32(5.0)
        print(f"\n[case] decode loop events step {step}", flush=True)
        active = dict(loop.active)
        events = loop.step(_to_dev(t, x))
        assert set(events) == set(active)
        for slot in active:
            st, seq, cfg = ref_state[slot]
            row = x[slot].copy()
            if cfg.temperature <= 1e-6:
                tok = oracle.raw_argmax_host(row)
            else:
                eng = oracle.OracleEngine(cfg, _abi, configs_to_array)
                tok = eng.sample_token(row, st, 10)
            seq.generated_count += 1
            want = next_event(seq, tok)
            assert events[slot] == want, (step, slot)
        if not loop.active:
            break
    loop.close()


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,softcap", [("bf16", 0.0), ("f32", 20.0), ("bf16", 3.0)])
def test_gpu_decode_step_bf16_softcap_mask(torch_gpu, dtype, softcap):
    # the decode step's kernel kinds with bf16 logits, the softcap and a grammar mask
    from oxide_sampler import BatchSampler
    from oxide_sampler import workloads as wl
    from oxide_sampler._abi import OxsDecodeIo
    t = torch_gpu
    B, V, cap = 24, 20001, 64
    cfgs = decode_configs()
    cfg_bytes = configs_to_array(cfgs, 10)[0]
    history, hlen, mu, rng_state, dec = decode_state(B, cap, 21)
    x = decode_logits(B, V, 1, history, hlen)
    rng = np.random.default_rng(4)
    bits = rng.random((B, V)) < 0.5
    bits[:, :64] = True
    mask = wl.pack_mask(bits, V)
    if dtype == "bf16":
        logits = wl.f32_to_bf16_bits(x)
        d_logits = t.from_numpy(logits.view(np.int16).copy()).to("cuda").view(t.bfloat16)
    else:
        logits = x
        d_logits = _to_dev(t, x)
    d_hist, d_hlen, d_mu, d_rng = (_to_dev(t, a) for a in (history, hlen, mu, rng_state))
    d_dec = {k: _to_dev(t, v) for k, v in dec.items()}
    lib = _abi.load_library()
    host = ctypes.c_void_p()
    _abi.check(lib.oxs_host_alloc(8 * B, ctypes.byref(host)), "oxs_host_alloc")
    try:
        io = OxsDecodeIo(d_dec["current_token"].data_ptr(), d_dec["current_position"].data_ptr(),
                         d_dec["generated_count"].data_ptr(), host.value)
        s = BatchSampler(B, V, 256)
        print(f"\n[case] decode step {dtype} softcap={softcap} masked", flush=True)
        out = s.sample(d_logits, _to_dev(t, cfg_bytes), mask=_to_dev(t, mask), history=d_hist, history_len=d_hlen,
                       history_cap=cap, record=True, rng_state=d_rng, mirostat_mu=d_mu, decode=io, softcap=softcap)
        t.cuda.synchronize()
        ref = oracle.sample_batch_host(
            _abi, logits=logits, dtype=dtype, configs_bytes=cfg_bytes, bias_ids=None, bias_values=None,
            ban_ids=None, mask=mask, history=history, history_len=hlen, history_cap=cap, record=True, uniforms=None,
            rng_state=rng_state, mu=mu, kept_ld=1, decode=dec, softcap=softcap)
        np.testing.assert_array_equal(_u32(out["tokens"]), ref["tokens"])
        np.testing.assert_array_equal(out["status"].cpu().numpy(), ref["status"])
        np.testing.assert_array_equal(_u32(d_hlen), hlen)
        np.testing.assert_array_equal(_u32(d_hist), history)
        np.testing.assert_array_equal(d_mu.cpu().numpy().view(np.uint32), mu.view(np.uint32))
        np.testing.assert_array_equal(d_rng.cpu().numpy().view(np.uint64), rng_state)
        for k in dec:
            np.testing.assert_array_equal(d_dec[k].cpu().numpy().view(dec[k].dtype), dec[k])
        slots = np.frombuffer((ctypes.c_uint64 * B).from_address(host.value), dtype=np.uint64).copy()
        np.testing.assert_array_equal((slots & np.uint64(0xFFFFFFFF)).astype(np.uint32), ref["tokens"])
        for b in range(B):  # every token allowed by the mask (or 0 for an empty row)
            tok = int(ref["tokens"][b])
            assert bits[b, tok] or ref["status"][b] == _abi.OXS_ROW_EMPTY
        s.close()
    finally:
        t.cuda.synchronize()
        lib.oxs_host_free(host)


def test_host_wait_reads_tagged_slots():
    # oxs_host_wait makes no HIP call: plain host memory stands in for the mapped slots
    lib = _abi.load_library()
    tokens = np.zeros(4, np.uint32)
    slots = np.array([(5 << 32) | 11, (5 << 32) | 22, (6 << 32) | 33, (5 << 32) | 44], np.uint64)
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    assert lib.oxs_host_wait(ptr(slots), 4, 5, ptr(tokens), 0) == _abi.OXS_OK
    assert tokens.tolist() == [11, 22, 33, 44]
    slots[1] = (4 << 32) | 99  # one row behind: times out after the spin limit
    assert lib.oxs_host_wait(ptr(slots), 4, 5, ptr(tokens), 1000) == _abi.OXS_ERR_TIMEOUT
    # step counts wrap modulo 2^32: 0xffffffff is behind 0, 1 is ahead of it
    slots[:] = [(1 << 32) | 7, (0 << 32) | 8, (1 << 32) | 9, (0 << 32) | 10]
    assert lib.oxs_host_wait(ptr(slots), 4, 0, ptr(tokens), 0) == _abi.OXS_OK
    assert tokens.tolist() == [7, 8, 9, 10]
    slots[2] = (0xFFFFFFFF << 32) | 9
    assert lib.oxs_host_wait(ptr(slots), 4, 0, ptr(tokens), 10) == _abi.OXS_ERR_TIMEOUT
    assert lib.oxs_host_wait(None, 4, 0, ptr(tokens), 10) == _abi.OXS_ERR_INVALID_ARGUMENT


# ----------------------------------------------------------------------------- the CUDA backend's argmax

def _rev5(x):
    return int(f"{x:05b}"[::-1], 2)


def _argmax_closed_form(row, batch):
    """launch_cuda_argmax's winner written from its reduction's structure, not
    by simulating it: among the ids holding the largest value above -1e30, the
    thread whose warp (then lane; with one row, block then warp then lane)
    index has the smallest bit reversal, and that thread's first such id. A
    left-biased strict-'>' tree over lanes l, l + 16, l + 8, ... compares bit 0
    of the lane index last, bit 4 first (sampling_dfa.cu:26-33)."""
    v = np.asarray(row, np.float32)
    ok = v > np.float32(-1e30)
    if not ok.any():
        return 0
    idx = np.nonzero(ok & (v == v[ok].max()))[0]

    def prio(i):
        i = int(i)
        if batch == 1:
            g = i % 6144
            return (_rev5(g >> 8), _rev5((g >> 5) & 7), _rev5(g & 31), i)
        t = i % 1024
        return (_rev5(t >> 5), _rev5(t & 31), i)

    return int(min(idx, key=prio))


def test_oracle_argmax_floor_cases():
    # launch_cuda_argmax's floor: only values strictly above -1e30 are taken
    inf, nan = np.inf, np.nan
    # [1, 3, 3]: ids 1 and 2 are lanes 1 and 2 of warp 0; the tree's offset-2
    # step hands lane 2's 3.0 to lane 0, and lane 1's equal 3.0 never replaces
    # it at offset 1, so id 2 wins (not the lower id)
    cases = [([1.0, 3.0, 3.0], (2, 3.0)), ([-inf, nan], (0, -1e30)), ([-1e30, -2e30], (0, -1e30)),
             ([-1e30, -9.9e29], (1, -9.9e29)), ([nan, 2.0, inf, inf], (2, inf)), ([-5.0], (0, -5.0))]
    for batch in (1, 2):
        for row, (tok, val) in cases:
            got = oracle.argmax_floor_host(np.array(row, np.float32), batch)
            assert got[0] == tok and got[1] == np.float32(val), (row, batch)
    rng = np.random.default_rng(3)
    x = rng.standard_normal(5000).astype(np.float32)
    x[[10, 4000]] = 7.0  # warp 0 (reversal 0) beats warp 29 (reversal 23)
    assert oracle.argmax_floor_host(x) == (10, 7.0)
    # -0.0 equals +0.0: the layout's winner keeps its own sign bit (id 2, lane 2)
    tok, val = oracle.argmax_floor_host(np.array([-1.0, -0.0, 0.0, -3.0], np.float32))
    assert tok == 2 and np.float32(val).view(np.uint32) == 0
    tok, val = oracle.argmax_floor_host(np.array([-1.0, 0.0, -0.0], np.float32))
    assert tok == 2 and np.float32(val).view(np.uint32) == 0x80000000


def test_oracle_argmax_tie_rule_is_the_reference_layouts():
    # ties at 42752 (thread 768 = warp 24) and 85504 (thread 512 = warp 16) of a
    # 128256-id row: warp 16's reversal (1) beats warp 24's (3); with one row,
    # 42752 = block 23 (reversal 29) of the 24-block layout, 85504 = block 21
    # (reversal 21)
    x = np.random.default_rng(7).standard_normal(128256).astype(np.float32)
    x[[42752, 85504]] = 9.0
    assert oracle.argmax_floor_host(x, 2) == (85504, 9.0)
    assert oracle.argmax_floor_host(x, 1) == (85504, 9.0)
    # lanes 8 and 16 of warp 0: reversal 2 against 1, so the higher thread wins
    # (a lowest-thread rule would give 8)
    y = np.full(64, -1.0, np.float32)
    y[[8, 16]] = 2.0
    assert oracle.argmax_floor_host(y, 2)[0] == 16
    # one row: blocks 1 and 2 (ids 256 and 512) have reversals 16 and 8
    z = np.full(7000, -1.0, np.float32)
    z[[256, 512]] = 2.0
    assert oracle.argmax_floor_host(z, 1)[0] == 512
    assert oracle.argmax_floor_host(z, 2)[0] == 512  # (warps 8 and 16 of one block: reversals 2 and 1)
    # one thread's ids: its first maximum (ids 5 and 1029 are both thread 5)
    w = np.full(3000, -1.0, np.float32)
    w[[5, 1029]] = 4.0
    assert oracle.argmax_floor_host(w, 2)[0] == 5


def test_oracle_argmax_against_closed_form():
    rng = np.random.default_rng(11)
    for trial in range(200):
        V = int(rng.integers(1, 30000))
        batch = int(rng.choice([1, 2]))
        x = rng.standard_normal(V).astype(np.float32)
        pos = rng.integers(0, V, int(rng.integers(1, 7)))
        if trial % 3 == 0:  # ties at zero, signs mixed
            x = -np.abs(x) - np.float32(0.5)
            x[pos] = np.float32(0.0)
            x[pos[::2]] = np.float32(-0.0)
        else:
            x[pos] = np.float32(6.0)
        got = oracle.argmax_floor_host(x, batch)
        assert got[0] == _argmax_closed_form(x, batch), (V, batch, pos.tolist())
        assert np.float32(got[1]).view(np.uint32) == x[got[0]].view(np.uint32)


@pytest.mark.gpu
@pytest.mark.parametrize("B,V,ld", [(1, 1, 1), (1, 128256, 128256), (5, 1001, 1003), (64, 32000, 32000),
                                    (3, 7, 8), (64, 128256, 128256), (2, 300001, 300004), (1, 7000, 7000),
                                    (16390, 12, 12)])
def test_gpu_argmax_matches_oracle(torch_gpu, B, V, ld):
    t = torch_gpu
    rng = np.random.default_rng(B * V)
    x = rng.standard_normal((B, ld)).astype(np.float32)
    x[:, V // 3] = x[:, (2 * V) // 3] = np.float32(9.0)  # ties: the reference layout's winner
    if V >= 85505:
        x[0, [42752, 85504]] = np.float32(12.0)  # the two rules differ here (85504 wins)
    if V >= 513:
        x[-1, [256, 512]] = np.float32(15.0)  # one row: block 2 beats block 1 (512)
    if V >= 17:
        x[min(B - 1, 1), [8, 16]] = np.float32(20.0)  # lanes 8 and 16: 16 wins
    if B > 2:
        x[1, :] = -np.inf
        x[2, : V // 2] = np.nan
        x[2, V // 2:] = np.float32(-2e30)
    if B > 3:  # the maximum is zero, both signs: the winner's bits come back
        x[3, :] = np.float32(-1.0)
        x[3, V // 5] = np.float32(-0.0)
        x[3, V // 2] = np.float32(0.0)
    print(f"\n[case] argmax B={B} V={V} ld={ld}", flush=True)
    d = t.from_numpy(x).to("cuda")
    tok = t.zeros(B, dtype=t.int32, device="cuda")
    val = t.zeros(B, dtype=t.float32, device="cuda")
    lib = _abi.load_library()
    for call in range(2):  # the second call finds the row slots cleared by the first
        _abi.check(lib.oxs_argmax(ctypes.c_void_p(d.data_ptr()), V, ld, B, ctypes.c_void_p(tok.data_ptr()),
                                  ctypes.c_void_p(val.data_ptr()), None), "oxs_argmax")
        t.cuda.synchronize()
        got_tok = tok.cpu().numpy()
        got_bits = val.cpu().numpy().view(np.uint32)
        rows = range(B) if B <= 64 else list(range(8)) + list(range(B - 8, B))
        for b in rows:
            want = oracle.argmax_floor_host(x[b, :V], B)
            assert int(got_tok[b]) == want[0] and got_bits[b] == np.float32(want[1]).view(np.uint32), \
                (call, b, int(got_tok[b]), want)
        if B > 64:  # the middle rows: all equal shape, the ties at V // 3 and 2V // 3
            mid = np.array([oracle.argmax_floor_host(x[b, :V], B)[0] for b in range(8, B - 8, 997)])
            assert (got_tok[8:B - 8:997] == mid).all()
