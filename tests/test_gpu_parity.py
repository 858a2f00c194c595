"""GPU sampler vs the CPU oracle on identical seeded inputs.

Bar: selected token ids and kept-index sets match
exactly (ties by lower index); post-filter probabilities and Mirostat mu agree
within 1e-5 relative for f32 logits and 1e-3 for bf16 logits. The device
reproduces the oracle's float operations one for one (glibc-exact exp/ln/log2,
reference summation order), so these tests also require bit-identical
probabilities; the tolerance is checked first so a failure says which bar broke.
"""
import numpy as np
import pytest

from harness import compare, run_gpu, run_oracle
from oxide_sampler import MirostatMode, _abi
from oxide_sampler import workloads as wl

pytestmark = pytest.mark.gpu

RTOL_F32 = 1e-5
RTOL_BF16 = 1e-3


def banner(msg):
    print(f"\n[case] {msg}", flush=True)


def test_config1_full(torch_gpu):
    w = wl.config1()
    banner("config1 B=1 V=32000")
    compare(run_gpu(w, torch_gpu), run_oracle(w), RTOL_F32, "config1")


def test_config1_batched(torch_gpu):
    w = wl.config1(batch=32)
    banner("config1 B=32 V=32000")
    compare(run_gpu(w, torch_gpu), run_oracle(w), RTOL_F32, "config1x32")


def test_config2_full(torch_gpu):
    w = wl.config2()
    banner("config2 B=64 V=128256")
    compare(run_gpu(w, torch_gpu, logits_out=True), run_oracle(w, logits_out=True), RTOL_F32, "config2")


def test_config3_full(torch_gpu):
    w = wl.config3()
    banner("config3 B=128 V=128256 masked")
    g = run_gpu(w, torch_gpu)
    compare(g, run_oracle(w), RTOL_F32, "config3")
    words = w.mask
    for b in range(w.batch):  # every sampled token is allowed by the mask
        t = int(g.tokens[b])
        assert (words[b, t >> 5] >> (t & 31)) & 1


def test_config4_full(torch_gpu):
    w = wl.config4()
    banner("config4 B=256 V=151936 bf16 typical+tfs")
    compare(run_gpu(w, torch_gpu), run_oracle(w), RTOL_BF16, "config4")


def oracle_threads():
    """Host threads for the oracle: the GPU box's CPU share is 16 cores, whatever os.cpu_count() shows."""
    import os
    return max(1, min(16, len(os.sched_getaffinity(0))))


@pytest.mark.parametrize("batch", [64, 512])
def test_config5_eight_steps(torch_gpu, batch):
    # batch 512 is config 5 itself: B=512 x V=262144 (537 MB of logits per step, rows grouped
    # 64 per XCD, 16384 stream blocks); batch 64 is the smaller grouping (8 rows per XCD)
    w = wl.config5(batch=batch)
    nt = oracle_threads()
    g_hist, g_len, g_mu = w.history.copy(), w.history_len.copy(), w.mu.copy()
    r_hist, r_len, r_mu = w.history.copy(), w.history_len.copy(), w.mu.copy()
    for step in range(w.steps):
        banner(f"config5 B={batch} V=262144 mirostat v2 step {step} (oracle on {nt} threads)")
        w.logits = wl.config5_step_logits(w.batch, w.vocab, wl.SEED_BASE + 5, step)
        w.history, w.history_len, w.mu = g_hist, g_len, g_mu
        g = run_gpu(w, torch_gpu)
        w.history, w.history_len, w.mu = r_hist, r_len, r_mu
        r = run_oracle(w, n_threads=nt)
        compare(g, r, RTOL_F32, f"config5 B={batch} step {step}")
        g_hist, g_len, g_mu = g.history, g.history_len, g.mu
        r_hist, r_len, r_mu = r.history, r.history_len, r.mu
    assert (r_len == 256 + 2 * w.steps).all()  # two records per Mirostat step (sampler.rs:301, :307)


@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5])
def test_baseline_configs_take_the_candidate_path(torch_gpu, cfg):
    # the exact re-scan gives the same answers (parity cannot see it) at many times the cost:
    # every row of a BASELINE config must find its top M among the stream phase's candidates
    from harness import gpu_sampler
    w = wl.BUILDERS[cfg]()
    banner(f"config{cfg} B={w.batch} V={w.vocab}: top-M selection paths")
    s = gpu_sampler(w.batch, w.vocab)
    s.count_paths(True)
    try:
        run_gpu(w, torch_gpu)
        counts = s.path_counts()
    finally:
        s.count_paths(False)
    print(f"config{cfg} paths: {counts}", flush=True)
    assert counts["exact"] == 0 and counts["none"] == 0, counts
    assert counts["buckets"] + counts["sort"] == w.batch, counts


def test_dry_rows_take_the_candidate_path(torch_gpu):
    # config 2 with DRY on every row over histories ending in a repeated motif of high-logit ids:
    # DRY lowers some candidates, and every row still finds its top M among the stream's candidates
    from harness import gpu_sampler
    w = wl.config2_dry()
    banner(f"config2_dry B={w.batch} V={w.vocab}: parity and top-M paths")
    s = gpu_sampler(w.batch, w.vocab)
    s.count_paths(True)
    try:
        g = run_gpu(w, torch_gpu, logits_out=True)
        counts = s.path_counts()
    finally:
        s.count_paths(False)
    print(f"config2_dry paths: {counts}", flush=True)
    compare(g, run_oracle(w, logits_out=True, n_threads=oracle_threads()), RTOL_F32, "config2_dry")
    assert counts["exact"] == 0 and counts["buckets"] + counts["sort"] == w.batch, counts


def mixed_workload(B, V, seed):
    """B rows cycling through every chain shape the config API offers, with ragged histories,
    empty (all -inf) rows and a row whose history is already full."""
    from oxide_sampler import SamplingConfig
    rng = np.random.default_rng(seed)
    logits = (rng.standard_normal((B, V)) * 2.5).astype(np.float32)
    spikes = rng.choice(V, min(V, 20), replace=False)
    logits[:, spikes] += 6.0
    if V > 64:
        logits[:, 40:64] = np.float32(3.25)  # a run of equal logits: the lower id ranks first
    base = [
        wl.disabled_config(temperature=0.0),
        wl.disabled_config(mirostat_mode=MirostatMode.V1, mirostat_tau=3.0, mirostat_eta=0.2, presence_penalty=0.3),
        wl.disabled_config(mirostat_mode=MirostatMode.V2, repeat_penalty=1.2, repeat_last_n=32),
        wl.disabled_config(min_p=0.02, xtc_threshold=0.05, xtc_probability=0.5, top_k=20),
        wl.disabled_config(temperature=0.9, logit_biases={7 % V: 3.0, 11 % V: -2.0, V - 1: 5.0, V + 5: 1.0},
                           banned_tokens={0, 3 % V, V + 2}, penalize_nl=True, newline_penalty=0.75),
        wl.disabled_config(temperature=1.1, tfs_z=0.9, typical_p=0.8),
        wl.disabled_config(temperature=0.8, top_k=300, top_p=0.97),
        wl.disabled_config(temperature=1.5, top_k=1024),
        SamplingConfig(),
        wl.disabled_config(temperature=0.6, frequency_penalty=-0.5, presence_penalty=-0.2, repeat_penalty=0.8,
                           repeat_last_n=0),
        # DRY (sampler.rs:393-415) with the other sparse stages, and with allowed_length 0
        wl.disabled_config(temperature=0.8, dry_multiplier=0.8, dry_base=1.75, dry_allowed_length=2, dry_range=64,
                           repeat_penalty=1.1, repeat_last_n=16, logit_biases={7 % V: 2.0}, banned_tokens={3 % V},
                           penalize_nl=True),
        wl.disabled_config(temperature=1.0, dry_multiplier=1.5, dry_base=1.1, dry_allowed_length=0, dry_range=300,
                           top_k=30),
        # dry_base < 0: penalties of alternating sign (powf of a negative base, integer exponents), so DRY
        # can raise a value and the row takes the exact re-scan
        wl.disabled_config(temperature=0.9, dry_multiplier=0.7, dry_base=-1.3, dry_allowed_length=1, dry_range=200,
                           top_k=60, repeat_penalty=1.05, repeat_last_n=24),
    ]
    configs = [base[i % len(base)] for i in range(B)]
    cap = 300
    history = rng.integers(0, V, size=(B, cap), dtype=np.uint32)
    history[:, ::7] = np.uint32(min(10, V - 1))  # the newline id recurs
    hlen = rng.integers(0, 200, size=B).astype(np.uint32)
    hlen[min(5, B - 1)] = cap  # no room to record: OXS_ROW_HISTORY_FULL
    for b in range(B):  # a repeated motif at the end of each history: n-gram matches for DRY
        n = int(hlen[b])
        if n >= 40:
            history[b, n - 40:n] = np.tile(rng.integers(0, V, size=5, dtype=np.uint32), 8)
    if B > 13:
        logits[13, :] = -np.inf  # OXS_ROW_EMPTY
    mu = np.full(B, 10.0, np.float32)
    return wl.Workload(name=f"mixed B={B} V={V}", logits=logits, dtype="f32", configs=configs, history=history,
                       history_len=hlen, uniforms=wl.xorshift_uniforms(B, seed), mu=mu)


@pytest.mark.parametrize("V", [1, 3, 257, 4097, 50001, 131072, 151936, 262144])
def test_mixed_configs_ragged_vocab(torch_gpu, V):
    # B = 40 groups rows by XCD (5 per XCD); vocabularies past 131072 take the 4096-key union
    B = 40 if V >= 4097 else 12
    w = mixed_workload(B, V, seed=100 + V)
    banner(f"mixed configs B={B} V={V}")
    compare(run_gpu(w, torch_gpu, kept_ld=1024, logits_out=True, max_top_k=1024),
            run_oracle(w, kept_ld=1024, logits_out=True), RTOL_F32, f"mixed V={V}")


def wide_workload(B, V, seed, dtype="f32"):
    """Rows whose pool max(top_k, 256) exceeds 1024 (the wide kernel), among ordinary rows."""
    from oxide_sampler import SamplingConfig
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((B, V)) * 1.5).astype(np.float32)
    x[:, rng.choice(V, 30, replace=False)] += 5.0
    if V > 3000:
        x[:, 2000:2600] = np.float32(0.75)  # equal values inside the pool: the lower id ranks first
    logits = wl.f32_to_bf16_bits(x) if dtype == "bf16" else x
    ks = [1025, 2000, 50000, 40, 0, 1100]
    base = [
        dict(temperature=0.8),
        dict(temperature=1.1, top_p=0.999, min_p=0.0001),
        dict(temperature=1.3, tfs_z=0.99, typical_p=0.99),
        dict(temperature=0.7, xtc_threshold=0.001, xtc_probability=1.0, top_p=0.95),
        dict(mirostat_mode=MirostatMode.V2, mirostat_tau=9.0, mirostat_eta=0.1),
        dict(mirostat_mode=MirostatMode.V1, mirostat_tau=8.0, mirostat_eta=0.2),
        dict(temperature=0.9, dry_multiplier=0.8, dry_base=1.75, dry_allowed_length=2, dry_range=2048,
             repeat_penalty=1.1, repeat_last_n=64, logit_biases={3: 2.0}, banned_tokens={5}),
        dict(temperature=0.0),
    ]
    configs = []
    for b in range(B):
        kw = dict(base[b % len(base)])
        kw["top_k"] = ks[b % len(ks)]
        configs.append(wl.disabled_config(**kw) if b % 9 else SamplingConfig(top_k=kw["top_k"]))
    cap = 3000
    history = rng.integers(0, V, size=(B, cap), dtype=np.uint32)
    hlen = rng.integers(0, 2900, size=B).astype(np.uint32)
    for b in range(B):
        n = int(hlen[b])
        if n >= 40:
            history[b, n - 40:n] = np.tile(rng.integers(0, V, size=5, dtype=np.uint32), 8)
    return wl.Workload(name=f"wide top_k B={B} V={V}", logits=logits, dtype=dtype, configs=configs,
                       history=history, history_len=hlen, uniforms=wl.xorshift_uniforms(B, seed),
                       mu=np.full(B, 18.0, np.float32))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_signed_zero_threshold(torch_gpu, dtype):
    # rows of negative logits with one +0.0 or -0.0 every 80 ids: each stream wavefront's
    # threshold is exactly zero, and -0.0 must count as >= it (a -0.0 of lower id ranks
    # before a later +0.0 among the tied top 50)
    B, V = 16, 128256
    rng = np.random.default_rng(77)
    x = (-1.0 - 4.0 * rng.random((B, V))).astype(np.float32)
    for b in range(B):
        at = np.arange(b % 80, V, 80)
        x[b, at] = np.where(rng.random(at.size) < 0.5, np.float32(-0.0), np.float32(0.0))
    logits = wl.f32_to_bf16_bits(x) if dtype == "bf16" else x
    # (temperature 1: at another temperature a key equal to a wavefront's threshold lies below the
    # scaled bound that proves the top M, and those rows take the exact re-scan by design)
    configs = [wl.disabled_config(top_k=50, top_p=0.95) if b % 2 else
               wl.disabled_config(top_k=200, min_p=0.01, repeat_penalty=1.2, repeat_last_n=64)
               for b in range(B)]
    history = rng.integers(0, V, size=(B, 64), dtype=np.uint32)
    w = wl.Workload(name=f"signed zeros {dtype}", logits=logits, dtype=dtype, configs=configs, history=history,
                    history_len=np.full(B, 64, np.uint32), uniforms=wl.xorshift_uniforms(B, 78))
    banner(f"signed-zero thresholds B={B} V={V} {dtype}")
    from harness import gpu_sampler
    s = gpu_sampler(w.batch, w.vocab)
    s.count_paths(True)
    try:
        g = run_gpu(w, torch_gpu, kept_ld=512, logits_out=True)
        counts = s.path_counts()
    finally:
        s.count_paths(False)
    compare(g, run_oracle(w, kept_ld=512, logits_out=True), RTOL_BF16 if dtype == "bf16" else RTOL_F32,
            f"signed zeros {dtype}")
    # about 26 zeros per wavefront fit its 32-key list: every row is proven from the candidates
    # (so a dropped -0.0 key would show as a wrong kept set, not hide behind the exact re-scan)
    assert counts["exact"] == 0 and counts["buckets"] + counts["sort"] == B, counts


@pytest.mark.parametrize("V,dtype", [(60000, "f32"), (151936, "bf16"), (1500, "f32")])
def test_wide_top_k(torch_gpu, V, dtype):
    # top_k 1025, 2000 and 50000 (kept to V when larger) beside ordinary rows: the wide kernel's
    # exact top-M select, its sort in global memory and the chain over up to 50000 candidates
    B = 24
    w = wide_workload(B, V, seed=500 + V, dtype=dtype)
    banner(f"wide top_k B={B} V={V} {dtype}")
    compare(run_gpu(w, torch_gpu, kept_ld=2048, logits_out=True, max_top_k=50000),
            run_oracle(w, kept_ld=2048, logits_out=True, n_threads=oracle_threads()),
            RTOL_BF16 if dtype == "bf16" else RTOL_F32, f"wide V={V}")


def test_wide_top_k_beyond_the_sampler_limit(torch_gpu):
    # a sampler created with max_top_k = 2000 runs top_k 2000 and reports top_k 5000 unsupported
    from harness import gpu_sampler
    w = wide_workload(8, 60000, seed=77)
    for b in range(8):
        w.configs[b].top_k = 5000 if b == 2 else 2000
    s = gpu_sampler(8, 60000, 2000, exact_limits=True)
    assert s.limits[2] == 2000
    banner("wide top_k beyond max_top_k")
    g = run_gpu(w, torch_gpu, kept_ld=256, max_top_k=2000, exact_limits=True)
    r = run_oracle(w, kept_ld=256)
    assert g.status[2] == _abi.OXS_ROW_UNSUPPORTED and g.tokens[2] == 0
    keep = np.arange(8) != 2
    np.testing.assert_array_equal(g.tokens[keep], r.tokens[keep])
    np.testing.assert_array_equal(g.kept_count[keep], r.kept_count[keep])


def dry_long_workload(B, V, seed):
    """DRY rows whose slices (1500 and 4096 ids) are longer than the 1024 ids the tail copies into LDS."""
    rng = np.random.default_rng(seed)
    logits = (rng.standard_normal((B, V)) * 2.0).astype(np.float32)
    cap = 5000
    history = rng.integers(0, V, size=(B, cap), dtype=np.uint32)
    hlen = rng.integers(3000, 4900, size=B).astype(np.uint32)
    for b in range(B):  # repeated motifs spread over the slice: matches of several lengths
        n = int(hlen[b])
        motif = rng.integers(0, V, size=int(rng.integers(3, 9)), dtype=np.uint32)
        for start in rng.integers(0, n - 200, size=12):
            history[b, start:start + 4 * len(motif)] = np.tile(motif, 4)
        history[b, n - 2 * len(motif):n] = np.tile(motif, 2)
    configs = [wl.disabled_config(temperature=0.9, dry_multiplier=float(rng.choice([0.5, 1.2])),
                                  dry_base=1.75, dry_allowed_length=int(rng.choice([0, 2, 3])),
                                  dry_range=int(rng.choice([1500, 4096])), top_k=int(rng.choice([0, 40])),
                                  repeat_penalty=1.1, repeat_last_n=64)
               for _ in range(B)]
    return wl.Workload(name=f"dry long B={B} V={V}", logits=logits, dtype="f32", configs=configs,
                       history=history, history_len=hlen, uniforms=wl.xorshift_uniforms(B, seed),
                       mu=np.full(B, 10.0, np.float32))


def test_dry_long_slices(torch_gpu):
    w = dry_long_workload(24, 32000, seed=31)
    banner("DRY slices of 1500 and 4096 ids B=24 V=32000")
    compare(run_gpu(w, torch_gpu, kept_ld=256, logits_out=True), run_oracle(w, kept_ld=256, logits_out=True),
            RTOL_F32, "dry long")


def dry_many_ids_workload(n_ids: int, seed: int, dry_base: float = 1.75):
    """dry_long_workload(8, 32000) whose row 3 has the history [A, B, x_i] x n_ids with distinct x_i,
    ending in [A, B]: the length-2 suffix matches before every x_i, so n_ids distinct ids take a DRY
    penalty."""
    V = 32000
    w = dry_long_workload(8, V, seed=seed)
    a, b = 7, 11
    xs = np.arange(100, 100 + n_ids, dtype=np.uint32)
    trip = np.stack([np.full(len(xs), a, np.uint32), np.full(len(xs), b, np.uint32), xs], axis=1).reshape(-1)
    seq = np.concatenate([trip, np.array([a, b], np.uint32)])
    hist = np.zeros((8, max(len(seq) + 100, w.history.shape[1])), np.uint32)
    hist[:, :w.history.shape[1]] = w.history
    hist[3, :len(seq)] = seq
    w.history = hist
    w.history_len = w.history_len.copy()
    w.history_len[3] = len(seq)
    w.configs[3] = wl.disabled_config(temperature=0.9, dry_multiplier=0.8, dry_base=dry_base, dry_allowed_length=2,
                                      dry_range=30000)
    return w


def test_dry_more_penalised_ids_than_the_list_holds(torch_gpu):
    # 9000 distinct penalised ids: more than the default max_dry_ids (8192), so with the default
    # limits that row reports OXS_ROW_UNSUPPORTED (token 0) and the other rows are unaffected
    w = dry_many_ids_workload(9000, seed=32)
    banner("DRY row with 9000 distinct penalised ids, default max_dry_ids")
    g = run_gpu(w, torch_gpu, kept_ld=256)
    r = run_oracle(w, kept_ld=256)
    assert g.status[3] == _abi.OXS_ROW_UNSUPPORTED and g.tokens[3] == 0
    keep = np.arange(8) != 3
    np.testing.assert_array_equal(g.tokens[keep], r.tokens[keep])
    np.testing.assert_array_equal(g.status[keep], r.status[keep])
    np.testing.assert_array_equal(g.history_len[keep], r.history_len[keep])


@pytest.mark.parametrize("dry_base", [1.75, -1.2])
def test_dry_many_ids_with_max_dry_ids(torch_gpu, dry_base):
    # the same row on a sampler created with max_dry_ids = V (every row fits): full parity, the
    # logits write-back included; dry_base < 0 sends the row to the exact re-scan, which reads
    # every penalised id's DRY value from the row's list
    w = dry_many_ids_workload(9000, seed=32, dry_base=dry_base)
    banner(f"DRY row with 9000 distinct penalised ids, max_dry_ids = V, dry_base {dry_base}")
    g = run_gpu(w, torch_gpu, kept_ld=256, logits_out=True, max_dry_ids=w.vocab)
    assert g.status[3] == _abi.OXS_ROW_OK
    compare(g, run_oracle(w, kept_ld=256, logits_out=True), RTOL_F32, "dry many ids")


def test_mixed_configs_device_rng(torch_gpu):
    # rng_state instead of uniforms: each drawing row advances its xorshift state by one step
    w = mixed_workload(40, 32000, seed=7)
    banner("mixed configs B=40 V=32000 device rng")
    states = np.array([0x853C49E6748FEA9B ^ (i * 0x9E3779B97F4A7C15 & (2**64 - 1)) or 1 for i in range(40)],
                      np.uint64)
    compare(run_gpu(w, torch_gpu, kept_ld=1024, use_rng=True, rng_state=states, max_top_k=1024),
            run_oracle(w, kept_ld=1024, use_rng=True, rng_state=states), RTOL_F32, "mixed rng")
