"""Randomised parity sweep: every SamplingConfig stage switched on at random, per row.

Each case draws a batch shape, a logits dtype (f32 or bf16), a logit
distribution (Gaussian, heavy spikes, long runs of equal values, -inf rows), a
grammar mask (none, per row or shared), a softcap, histories of random
length, and for every row a SamplingConfig whose fields are each enabled with
probability 1/2 at random values (sampler.rs:16-73), top_k up to 50000 (the
wide kernel past 1024), DRY ranges up to 4096
over histories up to 4400 ids. The HIP path must match
the oracle exactly: tokens, status, kept ids and probabilities, history, mu.
`test_random_configs_large_vocab` draws vocabularies above 131072 (more than 16
stream chunks per row, the 4096-key candidate union) with batches divisible by 8
(rows grouped by XCD).
"""
import numpy as np
import pytest

from harness import compare, run_gpu, run_oracle
from oxide_sampler import MirostatMode
from oxide_sampler import workloads as wl

RTOL_F32 = 1e-5
RTOL_BF16 = 1e-3


def banner(msg):
    print(f"\n[case] {msg}", flush=True)


def random_config(rng, V):
    kw = {}
    coin = lambda: rng.random() < 0.5  # noqa: E731
    kw["temperature"] = float(rng.choice([0.0, 1e-7, 0.3, 0.7, 1.0, 1.6])) if coin() else 1.0
    if coin():
        kw["top_k"] = int(rng.choice([1, 2, 40, 50, 255, 256, 300, 1024, 2000, 50000]))
    if coin():
        kw["top_p"] = float(rng.choice([0.5, 0.9, 0.95, 0.999]))
    if coin():
        kw["min_p"] = float(rng.choice([0.01, 0.05, 0.2]))
    if coin():
        kw["tfs_z"] = float(rng.choice([0.5, 0.9, 0.99]))
    if coin():
        kw["typical_p"] = float(rng.choice([0.2, 0.8, 0.95]))
    if coin():
        kw["xtc_threshold"] = float(rng.choice([0.01, 0.1, 0.3]))
        kw["xtc_probability"] = float(rng.choice([0.3, 1.0]))
    if rng.random() < 0.2:
        kw["mirostat_mode"] = MirostatMode.V1 if coin() else MirostatMode.V2
        kw["mirostat_tau"] = float(rng.choice([2.0, 5.0]))
        kw["mirostat_eta"] = float(rng.choice([0.1, 0.3]))
    if rng.random() < 0.25:
        kw["dry_multiplier"] = float(rng.choice([0.5, 1.5]))
        kw["dry_base"] = float(rng.choice([1.1, 1.75, -1.2]))  # (< 0: alternating-sign penalties)
        kw["dry_allowed_length"] = int(rng.choice([0, 2, 3]))
        kw["dry_range"] = int(rng.choice([16, 128, 1024, 4096]))
    if coin():
        kw["repeat_penalty"] = float(rng.choice([0.9, 1.1, 1.3]))
        kw["repeat_last_n"] = int(rng.choice([0, 8, 64, 512]))
    if coin():
        kw["frequency_penalty"] = float(rng.choice([-0.3, 0.2, 0.6]))
    if coin():
        kw["presence_penalty"] = float(rng.choice([-0.2, 0.3]))
    if coin():
        kw["penalize_nl"] = True
        kw["newline_penalty"] = float(rng.choice([0.5, 2.0]))
    if coin():
        ids = rng.integers(0, V + 3, size=int(rng.integers(1, 6)))
        kw["logit_biases"] = {int(i): float(rng.choice([-5.0, -0.5, 0.75, 4.0])) for i in ids}
    if coin():
        kw["banned_tokens"] = {int(i) for i in rng.integers(0, V + 3, size=int(rng.integers(1, 6)))}
    return wl.disabled_config(**kw)


def random_workload(seed, large_vocab=False):
    rng = np.random.default_rng(seed)
    if large_vocab:
        B = int(rng.choice([8, 16, 24, 40]))
        V = int(rng.choice([151936, 262144]))
    else:
        B = int(rng.choice([1, 3, 8, 17, 33]))
        V = int(rng.choice([5, 100, 1000, 4097, 20000, 65537]))
    kind = rng.integers(0, 3)
    x = rng.standard_normal((B, V)).astype(np.float32) * np.float32(rng.choice([0.5, 2.0, 4.0]))
    if kind == 1:  # a heavy tail of spikes
        x[rng.random((B, V)) < 0.01] += np.float32(8.0)
    elif kind == 2 and V > 20:  # long runs of equal values: ties broken by the lower id
        x[:, V // 4: V // 2] = np.float32(1.5)
    if B > 2 and rng.random() < 0.5:
        x[1, :] = -np.inf
    bf16 = rng.random() < 0.3
    logits = wl.f32_to_bf16_bits(x) if bf16 else x
    cap = 4500
    history = rng.integers(0, V, size=(B, cap), dtype=np.uint32)
    history[:, ::9] = np.uint32(min(10, V - 1))
    hlen = rng.integers(0, 1090, size=B).astype(np.uint32)
    long_rows = rng.random(B) < 0.3  # DRY slices past the 1024 ids an LDS copy holds
    hlen[long_rows] = rng.integers(1100, 4400, size=int(long_rows.sum())).astype(np.uint32)
    for b in range(B):
        n = int(hlen[b])
        if n >= 30 and rng.random() < 0.5:  # repeated motifs: DRY n-gram matches
            history[b, n - 30:n] = np.tile(rng.integers(0, V, size=3, dtype=np.uint32), 10)
    mask = None
    mchoice = rng.integers(0, 3)
    if mchoice:
        words = (V + 31) // 32
        bits = rng.random((1 if mchoice == 2 else B, words * 32)) < rng.choice([0.03, 0.5])
        bits[:, int(rng.integers(0, V))] = True
        mask = np.packbits(bits.astype(np.uint8), axis=1, bitorder="little").view(np.uint32)[:, :words].copy()
    configs = [random_config(rng, V) for _ in range(B)]
    w = wl.Workload(name=f"random seed={seed} B={B} V={V}", logits=logits, dtype="bf16" if bf16 else "f32",
                    configs=configs, history=history, history_len=hlen, uniforms=wl.xorshift_uniforms(B, seed),
                    mask=mask, mu=np.full(B, 10.0, np.float32))
    if rng.random() < 0.3:
        w.extra["softcap"] = float(rng.choice([5.0, 30.0]))
    return w, mchoice == 2


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(24))
def test_random_configs(torch_gpu, seed):
    w, shared = random_workload(1000 + seed)
    banner(f"{w.name} {w.dtype} mask={'shared' if shared else w.mask is not None} "
           f"softcap={w.extra.get('softcap', 0)}")
    g = run_gpu(w, torch_gpu, kept_ld=1024, logits_out=True, max_top_k=50000, shared_mask=shared)
    r = run_oracle(w, kept_ld=1024, logits_out=True, shared_mask=shared)
    compare(g, r, RTOL_BF16 if w.dtype == "bf16" else RTOL_F32, w.name)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(8))
def test_random_configs_large_vocab(torch_gpu, seed):
    w, shared = random_workload(2000 + seed, large_vocab=True)
    banner(f"{w.name} {w.dtype} mask={'shared' if shared else w.mask is not None} "
           f"softcap={w.extra.get('softcap', 0)}")
    g = run_gpu(w, torch_gpu, kept_ld=1024, logits_out=True, max_top_k=50000, shared_mask=shared)
    r = run_oracle(w, kept_ld=1024, logits_out=True, shared_mask=shared, n_threads=8)
    compare(g, r, RTOL_BF16 if w.dtype == "bf16" else RTOL_F32, w.name)


@pytest.mark.gpu
def test_logits_out_when_penalty_ids_overflow_the_chunk_hash(torch_gpu):
    # V = 1000 is one stream chunk; a whole-history window of 900 distinct ids overflows its
    # 256-slot LDS hash, so the row goes to the exact path, which must write every id of
    # logits_out with its penalties (sampler.rs:207-245)
    rng = np.random.default_rng(77)
    B, V = 4, 1000
    logits = (rng.standard_normal((B, V)) * 2.0).astype(np.float32)
    history = np.stack([rng.permutation(V)[:900].astype(np.uint32) for _ in range(B)])
    configs = [wl.disabled_config(frequency_penalty=0.6, presence_penalty=0.2, repeat_last_n=0),
               wl.disabled_config(repeat_penalty=1.3, repeat_last_n=0, temperature=0.7),
               wl.disabled_config(presence_penalty=-0.2, top_k=40, top_p=0.9),
               wl.disabled_config(frequency_penalty=0.3, repeat_penalty=1.1, repeat_last_n=900, min_p=0.05)]
    w = wl.Workload(name="hash overflow", logits=logits, dtype="f32", configs=configs, history=history,
                    history_len=np.full(B, 900, np.uint32), uniforms=wl.xorshift_uniforms(B, 77))
    banner("logits_out with 900 distinct penalty ids in one chunk")
    g = run_gpu(w, torch_gpu, logits_out=True, record=False)
    r = run_oracle(w, logits_out=True, record=False)
    compare(g, r, RTOL_F32, w.name)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(5000, 5008))
def test_random_decode_steps(torch_gpu, seed):
    # oxs_decode_step over three steps with random configs (raw-argmax rows included) and
    # the device rng: tokens, kept sets, history, mu, rng state and the per-row advance
    import ctypes
    import test_decode_loop as td
    from oxide_sampler import BatchSampler, _abi, configs_to_array
    from oxide_sampler._abi import OxsDecodeIo
    t = torch_gpu
    rng = np.random.default_rng(seed)
    B, V, cap = int(rng.choice([3, 17, 40])), int(rng.choice([1000, 50001])), 1200
    cfgs = []
    for _ in range(B):
        c = random_config(rng, V)
        c.logit_biases, c.banned_tokens = {}, set()  # the decode loop's configs carry no lists
        if rng.random() < 0.25:
            c.temperature = float(rng.choice([0.0, 1e-6, -1.0]))
        cfgs.append(c)
    cfg_bytes = configs_to_array(cfgs, 10)[0]
    history = rng.integers(0, V, size=(B, cap), dtype=np.uint32)
    hlen = rng.integers(0, 1100, size=B).astype(np.uint32)
    mu = np.full(B, 10.0, np.float32)
    rng_state = np.array([(0x853C49E6748FEA9B + 977 * b * seed) & (2**64 - 1) or 1 for b in range(B)], np.uint64)
    dec = {"current_token": rng.integers(0, V, size=B).astype(np.uint32),
           "current_position": rng.integers(0, 5000, size=B).astype(np.int32),
           "generated_count": rng.integers(0, 50, size=B).astype(np.uint32)}
    d_cfg = td._to_dev(t, cfg_bytes)
    d_hist, d_hlen, d_mu, d_rng = (td._to_dev(t, a) for a in (history, hlen, mu, rng_state))
    d_dec = {k: td._to_dev(t, v) for k, v in dec.items()}
    lib = _abi.load_library()
    host = ctypes.c_void_p()
    _abi.check(lib.oxs_host_alloc(8 * B, ctypes.byref(host)), "oxs_host_alloc")
    s = BatchSampler(B, V, 50000)  # rows with top_k > 1024 take the wide kernel's decode form
    try:
        io = OxsDecodeIo(d_dec["current_token"].data_ptr(), d_dec["current_position"].data_ptr(),
                         d_dec["generated_count"].data_ptr(), host.value)
        out = {"tokens": t.zeros(B, dtype=t.int32, device="cuda"), "status": t.zeros(B, dtype=t.int32, device="cuda"),
               "kept_count": t.zeros(B, dtype=t.int32, device="cuda"),
               "kept_ids": t.zeros(B, 256, dtype=t.int32, device="cuda"),
               "kept_probs": t.zeros(B, 256, dtype=t.float32, device="cuda")}
        sent = int(np.uint32(td.SENT).view(np.int32))
        for step in range(3):
            banner(f"random decode seed={seed} B={B} V={V} step {step}")
            x = (rng.standard_normal((B, V)) * 2.0).astype(np.float32)
            x[rng.random((B, V)) < 0.003] += np.float32(6.0)
            for k in ("kept_count", "kept_ids"):
                out[k].fill_(sent)
            out["kept_probs"].view(t.int32).fill_(sent)
            s.sample(td._to_dev(t, x), d_cfg, history=d_hist, history_len=d_hlen, history_cap=cap, record=True,
                     rng_state=d_rng, mirostat_mu=d_mu, kept_ld=256, decode=io, out=out)
            t.cuda.synchronize()
            ref = td.oracle_decode(cfg_bytes, x, history, hlen, mu, rng_state, dec, cap)
            np.testing.assert_array_equal(td._u32(out["tokens"]), ref["tokens"])
            np.testing.assert_array_equal(out["status"].cpu().numpy(), ref["status"])
            np.testing.assert_array_equal(td._u32(out["kept_count"]), ref["kept_count"])
            kid, kpr = td._u32(out["kept_ids"]), out["kept_probs"].cpu().numpy().view(np.uint32)
            for b in range(B):
                n = 256 if ref["kept_count"][b] == td.SENT else min(int(ref["kept_count"][b]), 256)
                np.testing.assert_array_equal(kid[b, :n], ref["kept_ids"][b, :n])
                np.testing.assert_array_equal(kpr[b, :n], ref["kept_probs"][b, :n].view(np.uint32))
            np.testing.assert_array_equal(td._u32(d_hlen), hlen)
            np.testing.assert_array_equal(td._u32(d_hist), history)
            np.testing.assert_array_equal(d_mu.cpu().numpy().view(np.uint32), mu.view(np.uint32))
            np.testing.assert_array_equal(d_rng.cpu().numpy().view(np.uint64), rng_state)
            for k in dec:
                np.testing.assert_array_equal(d_dec[k].cpu().numpy().view(dec[k].dtype), dec[k])
    finally:
        t.cuda.synchronize()
        s.close()
        lib.oxs_host_free(host)
