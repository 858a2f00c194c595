#!/usr/bin/env python3
"""bench.py — throughput of the MI355X batched token sampler.

Metric: sampled rows/s and achieved HBM GB/s for the full
sampling chain at batch 64 x vocab 128256, fp32 logits (config 2: frequency
0.3 + presence 0.2 + repetition 1.05 over a 512-token history -> temperature
0.7 -> top-k 50 -> top-p 0.9 -> min-p 0.05 -> draw with a supplied uniform).

One step = one `oxs_sample_batch` launch over one batch of 64 rows. Inputs are
resident in HBM before timing. Steps rotate over a pool of distinct batches
larger than twice the 256 MiB Infinity Cache, so the logits come from HBM.
Launches are replayed from a captured HIP graph (the decode-loop form: a
host-side Python loop cannot issue launches as fast as the GPU runs them).

Prints one JSON line (see `main`). `--gpus N` with N > 1 exits: this build
runs on one GPU.

Two secondary measurements print their own JSON line instead:
  --workload decode    one decode step of the scheduler's decode stage for the
                       config-2 batch (oxs_decode_step: sample, advance, tokens
                       into host memory), host-observed latency, beside a
                       device-to-host copy of the tokens and the reference's
                       copy of the whole logits to the host;
  --workload dfa_mask  grammar masks (oxs_dfa_mask) for 128 rows over a
                       128256-token vocabulary;
  --workload configs   oxs_sample_batch on each of the five BASELINE configs;
  --workload lm_head   the Q8_0 LM head that produces the logits (64 columns x
                       128256 tokens x hidden 4096), and the chain quantize ->
                       LM head -> sampler of one decode step.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "oxide-tech-llm-engine_amd"))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E


def algorithmic_bytes(B, V, H, kept_avg, esz=4, mask_words=0):
    """Bytes a perfect single pass must move per launch (reads + writes)."""
    per_row = V * esz + H * 4 + mask_words * 4 + 4 + 4 + 4 + 4 + kept_avg * 8 + 104
    return B * per_row


def make_pool(torch, w, n_pool, seed=0x5EED0002):
    """Pool entry 0 is the seeded CPU workload; the rest are drawn on the GPU
    from the same distribution (N(0,3) + -1.1 ln(rank) over a random permutation)."""
    d = torch.device("cuda")
    B, V = w.batch, w.vocab
    pool = [torch.from_numpy(np.ascontiguousarray(w.logits)).to(d)]
    g = torch.Generator(device=d)
    g.manual_seed(seed)
    prior = (-1.1 * torch.log(torch.arange(1, V + 1, device=d, dtype=torch.float64))).to(torch.float32)
    for _ in range(1, n_pool):
        x = torch.randn(B, V, device=d, generator=g) * 3.0
        perm = torch.argsort(torch.rand(B, V, device=d, generator=g), dim=1)
        x += prior[perm]
        pool.append(x.contiguous())
    return pool


def cpu_baseline(w, gpu_tokens, seconds):
    """The CPU oracle (a restatement of sampler.rs) on this host, 1 thread, rows
    in series as the reference decode loop does, over a bounded sample."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oxs_oracle_ctypes as oracle  # noqa: PLC0415 — baseline leg only
    from oxide_sampler import _abi  # noqa: PLC0415

    oracle.load()
    cfg, bias_ids, bias_vals, ban_ids = w.packed_configs()

    def run(rows, n_threads=1):
        hist = w.history[:rows].copy()
        hlen = w.history_len[:rows].copy()
        return oracle.sample_batch_host(
            _abi, logits=np.ascontiguousarray(w.logits[:rows]), dtype=w.dtype, configs_bytes=cfg,
            bias_ids=bias_ids, bias_values=bias_vals, ban_ids=ban_ids, mask=None, history=hist, history_len=hlen,
            history_cap=hist.shape[1], record=False, uniforms=w.uniforms[:rows], rng_state=None, mu=None,
            kept_ld=64, n_threads=n_threads)

    t0 = time.perf_counter()
    out = run(w.batch)  # warm-up and parity spot check on the whole batch
    t_batch = time.perf_counter() - t0
    match = bool(np.array_equal(out["tokens"], gpu_tokens)) if gpu_tokens is not None else None
    reps = max(5, int(seconds / max(t_batch, 1e-6)))
    passes = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run(w.batch)
        passes.append(time.perf_counter() - t0)
    dt = float(sum(passes))
    rows = reps * w.batch
    ncores = len(os.sched_getaffinity(0))
    run(w.batch, n_threads=min(ncores, w.batch))  # warm-up of the thread pool
    passes_all = []
    for _ in range(5):
        t0 = time.perf_counter()
        run(w.batch, n_threads=min(ncores, w.batch))
        passes_all.append(time.perf_counter() - t0)
    dt_all = float(np.median(passes_all))
    cpu_model = platform.processor() or platform.machine()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": rows / dt,
        "unit": "rows/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{rows} rows ({reps} passes over config-2 batch 0: B=64, V=128256 f32), 1 thread, rows in series",
        "us_per_row": dt / rows * 1e6,
        "median_pass_s": float(np.median(passes)),
        "all_cores": {"value": w.batch / dt_all, "unit": "rows/s", "cores": min(ncores, w.batch),
                      "sample": "median of 5 passes over config-2 batch 0, rows split statically"},
        "cpu_model": cpu_model,
        "libc": " ".join(platform.libc_ver()),
        "tokens_match_gpu": match,
    }


def _percentiles(xs):
    a = np.sort(np.asarray(xs, dtype=np.float64))
    return {"median": float(np.median(a)), "p10": float(a[len(a) // 10]), "p90": float(a[(9 * len(a)) // 10])}


def bench_decode(args, torch):
    """Host-observed latency of one decode step over the config-2 batch."""
    from oxide_sampler import BatchSampler, DecodeLoop, SamplerState  # noqa: PLC0415
    from oxide_sampler import workloads as wl  # noqa: PLC0415

    d = torch.device("cuda")
    w = wl.config2()
    B, V = w.batch, w.vocab
    H = int(w.history_len[0])
    n = max(50, args.steps)
    pool = make_pool(torch, w, pool_batches(B * V * 4))
    loop = DecodeLoop(B, V, history_cap=H + 3 * n + 64)
    for slot in range(B):
        st = SamplerState(10.0, w.history[slot, :H].tolist())
        loop.add_sequence(slot, temperature=w.configs[slot].temperature, top_p=w.configs[slot].top_p,
                          current_token=1, current_position=H, max_tokens=1 << 30, config=w.configs[slot], state=st)

    def timed(fn, reps):
        out = []
        for i in range(reps):
            t0 = time.perf_counter()
            fn(i)
            out.append((time.perf_counter() - t0) * 1e6)
        return out

    def eager(i):
        loop.launch(pool[i % len(pool)])
        loop.wait()

    timed(eager, 20)
    t_eager = timed(eager, n)
    static = pool[0].clone()
    loop.capture(static)

    def replay(i):
        loop.replay()
        loop.wait()

    timed(replay, 20)
    t_graph = timed(replay, n)
    # GPU time of the step itself, replayed back to back
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ev0.record()
    for _ in range(n):
        loop.replay()
    ev1.record()
    torch.cuda.synchronize()
    gpu_us = ev0.elapsed_time(ev1) * 1e3 / n
    loop.wait()

    # the conventional form: sample, then copy the tokens back and synchronise
    sampler = BatchSampler(B, V, 256)
    cfg, _, _, _ = w.packed_configs()
    d_cfg = torch.from_numpy(cfg).to(d)
    d_hist = torch.from_numpy(w.history.view(np.int32).copy()).to(d)
    d_hlen = torch.from_numpy(w.history_len.view(np.int32).copy()).to(d)
    d_u = torch.from_numpy(w.uniforms).to(d)

    def copy_back(i):
        out = sampler.sample(pool[i % len(pool)], d_cfg, history=d_hist, history_len=d_hlen, uniforms=d_u)
        out["tokens"].cpu()

    timed(copy_back, 20)
    t_copy = timed(copy_back, n)
    # the CUDA backend's greedy path (launch_cuda_argmax) as oxs_argmax, 50 calls per graph replay
    lib = sampler.lib
    tok = torch.zeros(B, dtype=torch.int32, device=d)
    val = torch.zeros(B, dtype=torch.float32, device=d)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g_arg = torch.cuda.CUDAGraph()
    n_arg = 3 * len(pool)  # a rotation over the whole pool: read from HBM
    with torch.cuda.graph(g_arg, stream=side):
        for i in range(n_arg):
            lib.oxs_argmax(ctypes.c_void_p(pool[i % len(pool)].data_ptr()), V, V, B, ctypes.c_void_p(tok.data_ptr()),
                           ctypes.c_void_p(val.data_ptr()), ctypes.c_void_p(side.cuda_stream))
    g_arg.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(20):
        g_arg.replay()
    e1.record()
    torch.cuda.synchronize()
    argmax_us = e0.elapsed_time(e1) * 1e3 / (20 * n_arg)
    # the reference's hand-off: the whole logits to pinned host memory
    # (oxide-backend-cuda/src/lib.rs:6037-6041), before any CPU sampling
    host = torch.empty(B, V, dtype=torch.float32, pin_memory=True)

    def logits_back(i):
        host.copy_(pool[i % len(pool)], non_blocking=True)
        torch.cuda.synchronize()

    timed(logits_back, 5)
    t_logits = timed(logits_back, max(20, n // 10))
    result = {
        "metric": "decode step latency, config-2 batch (64 x 128256 f32), sample + advance + tokens on the host",
        "value": _percentiles(t_graph)["median"],
        "unit": "us/step",
        "higher_is_better": False,
        "n_gpus": 1,
        "steps": n,
        "dtype": "f32",
        "data": f"synthetic (config-2 batch and {len(pool) - 1} GPU-drawn batches of the same distribution)",
        "config": {"workload": "decode: 64 sequences, config-2 SamplingConfig and a 512-token history each, "
                               "device xorshift draws; DecodeLoop over oxs_decode_step"},
        "graph_replay_us": _percentiles(t_graph),
        "graph_replay_inputs": "one captured batch, replayed: cache-resident (32.8 MB < 256 MiB Infinity Cache)",
        "pool_bytes": len(pool) * B * V * 4,
        "eager_launch_us": _percentiles(t_eager),
        "gpu_us_per_step": gpu_us,
        "sample_then_copy_tokens_us": _percentiles(t_copy),
        "reference_logits_to_host_us": _percentiles(t_logits),
        "greedy_argmax_us": argmax_us,
        "greedy_argmax_GBps": B * V * 4 / (argmax_us * 1e-6) / 1e9,
        "reference_logits_bytes": B * V * 4,
    }
    if not args.no_cpu:
        base = cpu_baseline(w, None, args.cpu_seconds)
        base["note"] = "CPU sampling the reference runs after the logits copy, per step, rows in series"
        base["us_per_step"] = base["us_per_row"] * B
        result["cpu_baseline"] = base
    print(json.dumps(result), flush=True)
    loop.close()


def bench_dfa_mask(args, torch):
    """oxs_dfa_mask over 128 rows x a 128256-token synthetic vocabulary."""
    from oxide_sampler import DfaSchemaGrammar, TokenBytes  # noqa: PLC0415

    B, V = 128, 128256
    rng = np.random.default_rng(0x5EED00DF)
    alphabet = np.frombuffer(b'{}[]":,0123456789abcdefghijklmnopqrstuvwxyz _-.', np.uint8)
    lens = np.minimum(rng.geometric(0.25, size=V), 24)  # mean ~4 bytes, a few long tokens
    vocab = [bytes(alphabet[rng.integers(0, alphabet.shape[0], size=int(L))]) for L in lens]
    tb = TokenBytes(vocab)
    grammars = {"json_validator_8_states": DfaSchemaGrammar.new_simple_json_validator(),
                "fixed_prefix_68_states": DfaSchemaGrammar.new_json_with_fixed_prefix('{"' + "k" * 60 + '": ')}
    n = max(20, args.steps // 10)
    lines = {}
    for name, g in grammars.items():
        states = rng.integers(0, g.num_states, size=B).astype(np.uint32)
        d_states = torch.from_numpy(states.view(np.int32)).cuda()
        for _ in range(5):
            g.token_masks(tb, d_states)
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        ev0.record()
        for _ in range(n):
            g.token_masks(tb, d_states)
        ev1.record()
        torch.cuda.synchronize()
        us = ev0.elapsed_time(ev1) * 1e3 / n
        # the decode-loop form: per-state masks once, then one gather per step
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        compiled = g.state_masks(tb)
        torch.cuda.synchronize()
        compile_us = (time.perf_counter() - t0) * 1e6
        out = torch.empty(B, compiled.words, dtype=torch.int32, device="cuda")
        for _ in range(5):
            g.gather_masks(compiled, d_states, out=out)
        # replayed from a graph of 50 gathers: a Python loop launches slower than one gather runs
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            for _ in range(50):
                g.gather_masks(compiled, d_states, out=out)
        reps = max(1, n // 50)
        torch.cuda.synchronize()
        ev0.record()
        for _ in range(reps):
            graph.replay()
        ev1.record()
        torch.cuda.synchronize()
        gather_us = ev0.elapsed_time(ev1) * 1e3 / (50 * reps)
        assert torch.equal(out, g.token_masks(tb, d_states)), "gathered masks differ from the direct walk"
        lookups = float(B) * float(lens.sum())  # upper bound: every walk runs to the token's end
        lines[name] = {"us_per_call": us, "gather_us_per_call": gather_us, "state_masks_compile_us": compile_us,
                       "state_masks_bytes": compiled.table.numel() * 4,
                       "gather_GBps": 2.0 * B * compiled.words * 4 / (gather_us * 1e-6) / 1e9,
                       "rows": B, "vocab": V, "states": g.num_states,
                       "token_bytes": int(lens.sum()), "row_token_pairs_per_s": B * V / (us * 1e-6),
                       "table_lookups_upper_bound_per_s": lookups / (us * 1e-6),
                       "table": "LDS" if g.num_states <= 48 else "global (L2)"}
    result = {
        "metric": "grammar mask latency per decode step (per-state table gather), 128 rows x 128256-token vocabulary",
        "value": lines["json_validator_8_states"]["gather_us_per_call"],
        "unit": "us/call",
        "higher_is_better": False,
        "n_gpus": 1,
        "steps": n,
        "dtype": "u8/u32",
        "data": "synthetic vocabulary (geometric token lengths, mean 4 bytes, JSON-ish alphabet), random states",
        "config": {"workload": "dfa_mask: oxs_dfa_mask_gather from per-state masks (oxs_dfa_mask over the states "
                               "once), 128 rows, V=128256; us_per_call is the direct walk of every row"},
        "grammars": lines,
    }
    if not args.no_cpu:
        sys.path.insert(0, str(ROOT / "oracle"))
        import oxs_oracle_ctypes as oracle  # noqa: PLC0415 — baseline leg only

        g = grammars["json_validator_8_states"]
        offsets = tb.offsets.cpu().numpy().view(np.uint32)
        flat = tb.bytes.cpu().numpy()[: tb.num_bytes]
        rows = 8
        states = rng.integers(0, g.num_states, size=rows).astype(np.uint32)
        t0 = time.perf_counter()
        reps = 0
        while time.perf_counter() - t0 < args.cpu_seconds or reps == 0:
            oracle.dfa_mask_host(g.transitions, g.num_states, offsets, flat, states)
            reps += 1
        dt = time.perf_counter() - t0
        result["cpu_baseline"] = {"value": reps * rows / dt, "unit": "rows/s", "cores": 1, "kind": "port",
                                  "sample": f"{reps} x {rows} rows of the 8-state grammar over the same vocabulary",
                                  "us_per_call_128_rows": dt / (reps * rows) * 128 * 1e6}
    print(json.dumps(result), flush=True)


def bench_lm_head(args, torch):
    """The Q8_0 LM head of the batched decode (oxs_quantize_q8_1 + oxs_mmvq_q8_0)
    at config 2's shape: 64 columns x 128256 tokens x hidden 4096, then the
    chain quantize -> LM head -> oxs_sample_batch that one decode step runs."""
    from oxide_sampler import BatchSampler, LmHeadQ8_0, _abi, quantize_q8_1  # noqa: PLC0415
    from oxide_sampler import workloads as wl  # noqa: PLC0415

    m, k, B = 128256, 4096, args.lm_batch
    nb = k // 32
    rng = np.random.default_rng(0x5EED0011)
    blocks = np.empty((m, nb, 34), np.uint8)
    blocks[:, :, 2:] = rng.integers(-128, 128, size=(m, nb, 32), dtype=np.int8).view(np.uint8)
    blocks[:, :, 0:2] = rng.uniform(0.002, 0.05, size=(m, nb)).astype(np.float16).view(np.uint8).reshape(m, nb, 2)
    w_host = blocks.reshape(-1)
    del blocks
    head = LmHeadQ8_0(w_host, m, k)
    x = torch.from_numpy(rng.normal(0, 1.5, size=(B, k)).astype(np.float32)).cuda()
    xq = quantize_q8_1(x).view(B, -1)
    y = torch.empty(B, m, dtype=torch.float32, device="cuda")
    head.project(xq, out=y)
    torch.cuda.synchronize()
    y_eager = y.clone()

    # the decode step's sampler on these logits: config 2's chain and history
    w = wl.config2(batch=B, vocab=m)
    sampler = BatchSampler(B, m, 256)
    cfg, _, _, _ = w.packed_configs()
    d_cfg = torch.from_numpy(cfg).cuda()
    d_hist = torch.from_numpy(w.history.view(np.int32).copy()).cuda()
    d_hlen = torch.from_numpy(w.history_len.view(np.int32).copy()).cuda()
    d_u = torch.from_numpy(w.uniforms).cuda()
    tokens = torch.empty(B, dtype=torch.int32, device="cuda")
    status = torch.empty(B, dtype=torch.int32, device="cuda")
    b = _abi.OxsBatch()
    b.batch, b.vocab, b.logits_dtype, b.flags = B, m, _abi.OXS_DTYPE_F32, 0
    b.logits_ld, b.logits, b.configs = m, y.data_ptr(), d_cfg.data_ptr()
    b.history, b.history_ld, b.history_len = d_hist.data_ptr(), d_hist.stride(0), d_hlen.data_ptr()
    b.uniforms, b.out_tokens, b.out_status = d_u.data_ptr(), tokens.data_ptr(), status.data_ptr()

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    reps = 10
    g_head, g_chain = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_head, stream=stream):
        for _ in range(reps):
            head.project(xq, out=y)
    with torch.cuda.graph(g_chain, stream=stream):
        for _ in range(reps):
            quantize_q8_1(x, out=xq, stream=stream)
            head.project(xq, out=y, stream=stream)
            sampler.launch(b, stream)
    torch.cuda.synchronize()

    def timed(graph, n):
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
        with torch.cuda.stream(stream):
            evs[0].record(stream)
            for i in range(n):
                graph.replay()
                evs[i + 1].record(stream)
        torch.cuda.synchronize()
        return [evs[i].elapsed_time(evs[i + 1]) * 1e3 / reps for i in range(n)]

    n = max(5, args.steps // 400)
    timed(g_head, 3)
    head_us = timed(g_head, n)
    assert torch.equal(y, y_eager), "graph replay of the LM head differs from the eager launch"
    timed(g_chain, 3)
    chain_us = timed(g_chain, n)
    assert (status == 0).all().item(), "sampler reported a non-OK row status"
    med = float(np.median(head_us))
    alg = m * nb * 34 + B * nb * 36 + B * m * 4
    achieved = alg / (med * 1e-6) / 1e9
    result = {
        "metric": f"Q8_0 LM head logits/s (batch {B} x vocab 128256 x hidden 4096), bit-exact with launch_cuda_mmvq_q8_0",
        "value": B * m / (med * 1e-6),
        "unit": "logits/s",
        "higher_is_better": True,
        "n_gpus": 1,
        "steps": n * reps,
        "median_us_per_step": med,
        "dtype": "int8 x int8 -> i32 (MFMA), f32 accumulation in the reference's order",
        "data": "synthetic Q8_0 weights (uniform int8 quants, f16 scales in [0.002, 0.05]), hidden ~ N(0, 1.5)",
        "config": {"workload": f"lm_head: oxs_mmvq_q8_0, m=128256, k=4096, batch={B} (64: config 2's decode batch); "
                               "chain = oxs_quantize_q8_1 + oxs_mmvq_q8_0 + oxs_sample_batch (config-2 chain)",
                   "m": m, "k": k, "batch": B, "launch": "hip_graph"},
        "chain_us_per_step": float(np.median(chain_us)),
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None, "algorithmic_bytes_per_launch": alg,
                     "kernel": "mmvq_q8_0_kernel",
                     "note": "batch >= 5: MFMA kernel, VALU-bound (48 VALU instructions per 32 tokens x 32 "
                             "columns x k block beside one MFMA); batch <= 4: dot4 kernel, HBM-bound"},
    }
    tpath = ROOT / "profiles" / "lm_head_pmc_traffic.json"
    if tpath.exists() and B == 64:  # the committed counters were taken at batch 64
        t = json.loads(tpath.read_text())
        result["roofline"]["traffic"] = t["traffic_bytes_per_launch"]
        result["roofline"]["traffic_source"] = str(tpath.relative_to(ROOT))
    if not args.no_cpu:
        sys.path.insert(0, str(ROOT / "oracle"))
        import oxs_oracle_ctypes as oracle  # noqa: PLC0415 — baseline leg only

        rows = 512  # a bounded sample: 512 token rows x every column
        sub = w_host[: rows * nb * 34]
        xq_host = oracle.quantize_q8_1_host(x.cpu().numpy())
        t0 = time.perf_counter()
        done = 0
        while time.perf_counter() - t0 < args.cpu_seconds or done == 0:
            want = oracle.mmvq_q8_0_host(sub, xq_host, rows, k, B)
            done += 1
        dt = time.perf_counter() - t0
        assert np.array_equal(want.view(np.uint32), y_eager[:, :rows].cpu().numpy().view(np.uint32)), \
            "the GPU logits differ from the oracle's"
        result["cpu_baseline"] = {"value": done * rows * B / dt, "unit": "logits/s", "cores": 1, "kind": "port",
                                  "sample": f"{done} passes of the first {rows} tokens x {B} columns"}
    print(json.dumps(result), flush=True)


MALL_BYTES = 256 << 20  # MI355X Infinity Cache


def bench_argmax(args, torch):
    """oxs_argmax, the greedy path (launch_cuda_argmax, sampling_dfa.cu:2-178), per batch shape: graph replays
    over a pool of distinct logits batches larger than the 256 MiB MALL, so every launch reads from HBM; HIP
    events on the launch stream; tokens checked against torch.argmax on rows without a tied maximum."""
    from oxide_sampler import _abi  # noqa: PLC0415
    d = torch.device("cuda")
    lib = _abi.load_library()
    lines = {}
    for B, V in ((1, 128256), (8, 128256), (64, 128256), (256, 151936)):
        n_pool = max(2, int(600e6 // (B * V * 4)) + 1)
        g = torch.Generator(device=d)
        g.manual_seed(0x5EED0300 + B)
        pool = torch.randn(n_pool, B, V, device=d, generator=g)
        tok = torch.zeros(B, dtype=torch.int32, device=d)
        val = torch.zeros(B, dtype=torch.float32, device=d)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        n = 3 * n_pool
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            for i in range(n):
                _abi.check(lib.oxs_argmax(ctypes.c_void_p(pool[i % n_pool].data_ptr()), V, V, B,
                                          ctypes.c_void_p(tok.data_ptr()), ctypes.c_void_p(val.data_ptr()),
                                          ctypes.c_void_p(side.cuda_stream)), "oxs_argmax")
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 20
        with torch.cuda.stream(side):
            e0.record(side)
            for _ in range(reps):
                graph.replay()
            e1.record(side)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (reps * n)
        last = pool[(n - 1) % n_pool]
        single = (last == last.max(dim=1, keepdim=True).values).sum(dim=1) == 1  # rows without a tied maximum
        ok = bool(((tok.long() == torch.argmax(last, dim=1)) | ~single).all())
        gbs = B * V * 4 / (us * 1e-6) / 1e9
        lines[f"B{B}xV{V}"] = {"batch": B, "vocab": V, "us_per_launch": us, "GBps": gbs,
                               "frac_of_hbm_peak": gbs / HBM_PEAK_GBS, "tokens_match_torch_argmax": ok,
                               "pool_batches": n_pool}
        print(f"[argmax] B={B} V={V}: {us:.2f} us per launch, {gbs:.0f} GB/s, tokens ok {ok}",
              file=sys.stderr, flush=True)
        assert ok, "oxs_argmax differs from torch.argmax on a tie-free batch"
        del pool
        torch.cuda.empty_cache()
    print(json.dumps({"metric": "oxs_argmax (greedy decode path) per batch shape", "unit": "us/launch",
                      "higher_is_better": False, "n_gpus": 1, "dtype": "f32",
                      "data": "synthetic N(0,1) logits, pools larger than 600 MB", "shapes": lines}), flush=True)


def bench_read_floor(args, torch):
    """The read floor of the stream phase on config 2: oxs_read_floor (the
    stream kernel's grid and 16-byte non-temporal loads over the same
    [64, 128256] f32 logits, nothing else) graph-replayed over the headline's
    pool of distinct batches, timed with HIP events on the launch stream."""
    import ctypes  # noqa: PLC0415
    from oxide_sampler import _abi  # noqa: PLC0415
    from oxide_sampler import workloads as wl  # noqa: PLC0415
    lib = _abi.load_library()
    w = wl.config2()
    B, V = w.batch, w.vocab
    P = pool_batches(B * V * 4)
    pool = make_pool(torch, w, P)
    d = torch.device("cuda")
    sink = torch.empty(B * ((V + 8191) // 8192), dtype=torch.int32, device=d)
    stream = torch.cuda.Stream()

    def call(i):
        _abi.check(lib.oxs_read_floor(ctypes.c_void_p(pool[i].data_ptr()), V, V, B, ctypes.c_void_p(sink.data_ptr()),
                                      ctypes.c_void_p(stream.cuda_stream)), "oxs_read_floor")

    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for i in range(P):
            call(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(P):
            call(i)
    reps = max(3, args.steps // P)
    with torch.cuda.stream(stream):
        for _ in range(max(1, args.warmup // P)):
            graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        e0.record(stream)
        for _ in range(reps):
            graph.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (reps * P)
    nbytes = B * V * 4
    gbs = nbytes / (us * 1e-6) / 1e9
    result = {
        "metric": "read floor of the stream phase: one pass over config 2's logits",
        "value": gbs, "unit": "GB/s", "higher_is_better": True, "n_gpus": 1, "steps": reps * P,
        "us_per_launch": us, "bytes_per_launch": nbytes, "frac_of_peak": gbs / HBM_PEAK_GBS,
        "dtype": "f32", "data": f"synthetic: the headline's pool of {P} distinct config-2 batches",
        "config": {"workload": "read_floor: oxs_read_floor over [64, 128256] f32, the stream kernel's grid "
                               "(1024 blocks of 8192 logits, eight 16-byte non-temporal loads per thread)"},
    }
    print(json.dumps(result), flush=True)


def pool_batches(batch_bytes, at_least=2):
    """Distinct input batches whose total exceeds twice the Infinity Cache, so
    a rotation over them streams from HBM."""
    return max(at_least, (2 * MALL_BYTES) // batch_bytes + 1)


def config_pool(torch, w, n_pool, seed):
    """[n_pool, B, V] logits for workload w: entry 0 is the seeded CPU workload,
    the rest are drawn on the GPU from the same distribution
    (oxide_sampler.workloads: config 1 N(0,2) + 5 spikes at +8; configs 2-3
    N(0,3) + -1.1 ln(rank) over a random permutation; config 4 N(0,2.5) with 1%
    of entries U[6,10], as bf16; config 5 N(0,2))."""
    d = torch.device("cuda")
    B, V = w.batch, w.vocab
    g = torch.Generator(device=d)
    g.manual_seed(seed)
    dt = torch.bfloat16 if w.dtype == "bf16" else torch.float32
    pool = torch.empty(n_pool, B, V, dtype=dt, device=d)
    if w.dtype == "bf16":
        pool[0] = torch.from_numpy(w.logits.view(np.int16)).to(d).view(torch.bfloat16)
    else:
        pool[0] = torch.from_numpy(w.logits).to(d)
    prior = (-1.1 * torch.log(torch.arange(1, V + 1, device=d, dtype=torch.float64))).to(torch.float32)
    for i in range(1, n_pool):
        if w.name == "config1":
            x = torch.randn(B, V, device=d, generator=g) * 2.0
            spikes = torch.randint(0, V, (B, 5), device=d, generator=g)
            x.scatter_(1, spikes, 8.0)
        elif w.name in ("config2", "config3", "config2_dry"):
            x = torch.randn(B, V, device=d, generator=g) * 3.0
            x += prior[torch.argsort(torch.rand(B, V, device=d, generator=g), dim=1)]
        elif w.name == "config4":
            x = torch.randn(B, V, device=d, generator=g) * 2.5
            heavy = torch.rand(B, V, device=d, generator=g) < 0.01
            x = torch.where(heavy, 6.0 + 4.0 * torch.rand(B, V, device=d, generator=g), x)
        else:
            x = torch.randn(B, V, device=d, generator=g) * 2.0
        pool[i] = x.to(dt)
    return pool


def config_masks(torch, w, n_pool, seed):
    """[n_pool, B, ceil(V/32)] packed masks for config 3: entry 0 the seeded one,
    the rest with each bit set with probability 0.03 and one guaranteed id."""
    d = torch.device("cuda")
    B, V = w.batch, w.vocab
    words = (V + 31) // 32
    g = torch.Generator(device=d)
    g.manual_seed(seed)
    out = torch.empty(n_pool, B, words, dtype=torch.int32, device=d)
    out[0] = torch.from_numpy(w.mask.view(np.int32)).to(d)
    weights = (2 ** torch.arange(32, device=d, dtype=torch.int64))
    for i in range(1, n_pool):
        bits = torch.rand(B, words * 32, device=d, generator=g) < 0.03
        bits[:, V:] = False
        bits[torch.arange(B, device=d), torch.randint(0, V, (B,), device=d, generator=g)] = True
        packed = (bits.view(B, words, 32).to(torch.int64) * weights).sum(-1)
        out[i] = packed.to(torch.uint32).view(torch.int32) if hasattr(torch, "uint32") else \
            ((packed + 2**31) % 2**32 - 2**31).to(torch.int32)
    return out


def bench_configs(args, torch):
    """oxs_sample_batch on each of BASELINE.json's five configs, and config 2
    with DRY on every row (oxide_sampler.workloads.config2_dry). Each config
    rotates over its own pool of distinct input batches larger than twice the
    Infinity Cache (graph replays of the whole rotation), so every figure is
    streamed from HBM: us per call, rows/s, algorithmic GB/s with its roofline
    fraction, and how each row's top M was found (path counters)."""
    from oxide_sampler import BatchSampler  # noqa: PLC0415
    from oxide_sampler import workloads as wl  # noqa: PLC0415

    d = torch.device("cuda")
    lines = {}
    ids = [c if c == "2dry" else int(c) for c in args.config_ids.split(",")]
    for cfg_id in ids:
        w = wl.config2_dry() if cfg_id == "2dry" else wl.BUILDERS[cfg_id]()
        name = w.name
        cfg, bias_ids, bias_vals, ban_ids = w.packed_configs()
        sampler = BatchSampler(w.batch, w.vocab, 256)
        esz = 2 if w.dtype == "bf16" else 4
        words = (w.vocab + 31) // 32 if w.mask is not None else 0
        batch_bytes = w.batch * (w.vocab * esz + words * 4)
        P = pool_batches(batch_bytes)
        seed_id = 22 if cfg_id == "2dry" else cfg_id
        pool = config_pool(torch, w, P, 0x5EED0100 + seed_id)
        masks = config_masks(torch, w, P, 0x5EED0200 + seed_id) if w.mask is not None else None
        hist = torch.from_numpy(w.history.view(np.int32).copy()).to(d)
        hlen = torch.from_numpy(w.history_len.view(np.int32).copy()).to(d)
        mu = torch.from_numpy(w.mu.copy()).to(d) if w.mu is not None else None
        dcfg = torch.from_numpy(cfg).to(d)
        u = torch.from_numpy(w.uniforms).to(d)
        out = {k: torch.empty(w.batch, dtype=torch.int32, device=d) for k in ("tokens", "status", "kept_count")}
        stream = torch.cuda.Stream()

        def call(i):
            sampler.sample(pool[i], dcfg, mask=None if masks is None else masks[i], history=hist, history_len=hlen,
                           history_cap=0, record=False, uniforms=u, mirostat_mu=mu, stream=stream, out=out)

        stream.wait_stream(torch.cuda.current_stream())
        sampler.count_paths(True)
        with torch.cuda.stream(stream):
            call(0)
        torch.cuda.synchronize()
        paths = sampler.path_counts()
        sampler.count_paths(False)
        assert (out["status"] == 0).all().item(), f"{name}: a row reported a non-OK status"
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(P):
                call(i)
        reps = max(3, min(50, 4000 // P))
        with torch.cuda.stream(stream):
            graph.replay()
        torch.cuda.synchronize()
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
        with torch.cuda.stream(stream):
            evs[0].record(stream)
            for i in range(reps):
                graph.replay()
                evs[i + 1].record(stream)
        torch.cuda.synchronize()
        us = float(np.median([evs[i].elapsed_time(evs[i + 1]) * 1e3 / P for i in range(reps)]))
        H = int(w.history_len[0])
        alg = algorithmic_bytes(w.batch, w.vocab, H, 0.0, esz=esz, mask_words=words)
        gbs = alg / (us * 1e-6) / 1e9
        lines[name] = {"batch": w.batch, "vocab": w.vocab, "dtype": w.dtype, "us_per_call": us,
                       "rows_per_s": w.batch / (us * 1e-6), "algorithmic_bytes": alg,
                       "pool_batches": P, "pool_bytes": P * batch_bytes,
                       "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                    "frac": gbs / HBM_PEAK_GBS},
                       "top_m_paths": paths}
        print(f"[configs] {name}: {us:.2f} us per call, {gbs:.0f} GB/s, paths {paths}", file=sys.stderr, flush=True)
        sampler.close()
        del pool, masks
        torch.cuda.empty_cache()
    result = {
        "metric": "oxs_sample_batch per BASELINE config (config 5: one of its 8 steps)",
        "value": lines["config2"]["rows_per_s"] if "config2" in lines else None,
        "unit": "rows/s",
        "higher_is_better": True,
        "n_gpus": 1,
        "dtype": "f32 / bf16 (config 4)",
        "data": "synthetic: the seeded workloads of oxide_sampler.workloads plus GPU-drawn batches of each "
                "config's distribution",
        "config": {"workload": "configs: configs 1-5 of BASELINE.json, each rotating over more than 512 MiB "
                               "of distinct input batches"},
        "configs": lines,
    }
    print(json.dumps(result), flush=True)


def read_traffic(path):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if any."""
    try:
        data = json.loads(Path(path).read_text())
        return float(data["traffic_bytes_per_launch"]), str(path)
    except Exception:
        return None, None


def _pmc_rows(folder, counter):
    import csv  # noqa: PLC0415
    files = sorted(Path(folder).rglob("*counter_collection.csv"))
    if not files:
        raise SystemExit(f"no counter_collection.csv under {folder}")
    rows = []
    for f in files:
        for r in csv.DictReader(open(f)):
            if r["Counter_Name"] == counter:
                rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"])))
    rows.sort()
    return rows


def _per_launch(rows):
    """KiB per sampler launch: one stream_kernel dispatch plus the tail_kernel after it."""
    out, cur = [], None
    for _, name, v in rows:
        if "oxs::" not in name:
            continue
        if "stream_kernel" in name:
            cur = v
        elif "tail_kernel" in name and cur is not None:
            out.append(cur + v)
            cur = None
    if not out:
        raise SystemExit("no sampler launches in the counter rows")
    return float(np.median(out)), len(out)


def _copy_kib(rows):
    v = [val for _, name, val in rows if "copyBuffer" in name]
    if not v:
        raise SystemExit("no copy dispatches in the calibration rows")
    return float(np.median(v))


def summarize_pmc(fetch_dir, write_dir, copy_fetch_dir, copy_write_dir):
    """HBM bytes per launch from FETCH_SIZE and WRITE_SIZE (KiB per dispatch),
    each scaled by what the same counter reads for a plain 256 MiB device copy."""
    copy_bytes = 256 << 20
    f_kib, n_f = _per_launch(_pmc_rows(fetch_dir, "FETCH_SIZE"))
    w_kib, n_w = _per_launch(_pmc_rows(write_dir, "WRITE_SIZE"))
    cf = copy_bytes / (_copy_kib(_pmc_rows(copy_fetch_dir, "FETCH_SIZE")) * 1024)
    cw = copy_bytes / (_copy_kib(_pmc_rows(copy_write_dir, "WRITE_SIZE")) * 1024)
    fetch_b, write_b = f_kib * 1024 * cf, w_kib * 1024 * cw
    return {
        "traffic_bytes_per_launch": fetch_b + write_b,
        "fetch_bytes_per_launch": fetch_b, "write_bytes_per_launch": write_b,
        "fetch_kib_raw": f_kib, "write_kib_raw": w_kib,
        "copy_scale_fetch": cf, "copy_scale_write": cw,
        "launches_fetch": n_f, "launches_write": n_w,
    }


def summarize_trace(folder):
    """Average duration per launch of this library's kernels from a rocprofv3
    --kernel-trace --stats folder (the *_kernel_stats.csv file)."""
    import csv  # noqa: PLC0415
    stats = next(Path(folder).glob("*kernel_stats.csv"))
    out = {}
    for r in csv.DictReader(open(stats)):
        name = r["Name"]
        for k in ("stream_kernel", "tail_kernel"):
            if f"oxs::{k}<0," in name:  # the f32 kernels (config 2)
                prev = out.get(k)
                if prev is None or int(r["Calls"]) > prev["calls"]:
                    out[k] = {"avg_ns": float(r["AverageNs"]), "calls": int(r["Calls"]), "name": name}
    return out


def read_kernel_trace(path):
    try:
        return json.loads(Path(path).read_text()), str(path)
    except (OSError, ValueError, KeyError):
        return None, None


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=8000)
    ap.add_argument("--warmup", type=int, default=800)
    ap.add_argument("--pool", type=int, default=0,
                    help="distinct input batches; 0 = enough to exceed 2 x 256 MiB (17 x 32.8 MB = 533 MiB)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--eager", action="store_true", help="launch from a Python loop instead of a HIP graph")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only 8 plain 256 MiB device copies (scale for the rocprofv3 byte counters)")
    ap.add_argument("--traffic-summary", default=str(ROOT / "profiles" / "config2_pmc_traffic.json"))
    ap.add_argument("--workload", choices=("sample", "decode", "dfa_mask", "lm_head", "configs", "read_floor", "argmax"),
                    default="sample",
                    help="sample: the headline config-2 line; decode / dfa_mask / lm_head / configs: secondary lines")
    ap.add_argument("--config-ids", default="1,2,3,4,5,2dry",
                    help="--workload configs: which configs (1-5, 2dry = config 2 with DRY on every row)")
    ap.add_argument("--lm-batch", type=int, default=64,
                    help="lm_head: q8_1 columns (64 = config 2's decode batch; 1 = the last prompt token)")
    ap.add_argument("--summarize-pmc", nargs=4, metavar=("FETCH_DIR", "WRITE_DIR", "COPY_FETCH_DIR", "COPY_WRITE_DIR"),
                    help="turn four rocprofv3 --pmc output folders into the traffic summary and exit")
    ap.add_argument("--trace-summary", default=str(ROOT / "profiles" / "config2_kernel_trace.json"))
    ap.add_argument("--summarize-trace", metavar="TRACE_DIR",
                    help="turn a rocprofv3 --kernel-trace --stats folder of this bench into the per-kernel summary and exit")
    args = ap.parse_args()
    if args.summarize_trace:
        summary = summarize_trace(args.summarize_trace)
        Path(args.trace_summary).write_text(json.dumps(summary, indent=1) + "\n")
        print(json.dumps(summary), flush=True)
        return
    if args.summarize_pmc:
        summary = summarize_pmc(*args.summarize_pmc)
        Path(args.traffic_summary).write_text(json.dumps(summary, indent=1) + "\n")
        print(json.dumps(summary), flush=True)
        return

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build samples on one GPU; multi-GPU runs are not part of it "
              "(rows shard across GPUs with no communication)", file=sys.stderr)
        sys.exit(2)

    import torch
    from oxide_sampler import BatchSampler, _abi
    from oxide_sampler import workloads as wl

    if not torch.cuda.is_available():
        print("bench.py: no HIP device", file=sys.stderr)
        sys.exit(1)
    d = torch.device("cuda")
    if args.workload == "decode":
        bench_decode(args, torch)
        return
    if args.workload == "dfa_mask":
        bench_dfa_mask(args, torch)
        return
    if args.workload == "lm_head":
        bench_lm_head(args, torch)
        return
    if args.workload == "read_floor":
        return bench_read_floor(args, torch)
    if args.workload == "argmax":
        return bench_argmax(args, torch)
    if args.workload == "configs":
        bench_configs(args, torch)
        return
    if args.calibrate_copy:
        src = torch.ones(64 << 20, dtype=torch.float32, device=d)  # 256 MiB
        dst = torch.empty_like(src)
        for _ in range(8):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes_read": src.numel() * 4, "copies": 8}), flush=True)
        return
    w = wl.config2()
    B, V = w.batch, w.vocab
    H = int(w.history_len[0])
    pool = make_pool(torch, w, args.pool or pool_batches(B * V * 4))
    cfg, bias_ids, bias_vals, ban_ids = w.packed_configs()
    d_cfg = torch.from_numpy(cfg).to(d)
    d_hist = torch.from_numpy(w.history.view(np.int32).copy()).to(d)
    d_hlen = torch.from_numpy(w.history_len.view(np.int32).copy()).to(d)
    d_u = torch.from_numpy(w.uniforms).to(d)
    kept_ld = 64
    sampler = BatchSampler(B, V, 256)

    # One prepared descriptor per pool entry; outputs are shared.
    outs = {
        "tokens": torch.empty(B, dtype=torch.int32, device=d),
        "status": torch.empty(B, dtype=torch.int32, device=d),
        "kept_count": torch.empty(B, dtype=torch.int32, device=d),
        "kept_ids": torch.empty(B, kept_ld, dtype=torch.int32, device=d),
        "kept_probs": torch.empty(B, kept_ld, dtype=torch.float32, device=d),
    }
    descs = []
    for x in pool:
        b = _abi.OxsBatch()
        b.batch, b.vocab, b.logits_dtype, b.flags = B, V, _abi.OXS_DTYPE_F32, 0
        b.logits_ld, b.logits, b.configs = V, x.data_ptr(), d_cfg.data_ptr()
        b.history, b.history_ld, b.history_len, b.history_cap = d_hist.data_ptr(), d_hist.stride(0), d_hlen.data_ptr(), 0
        b.uniforms = d_u.data_ptr()
        b.out_tokens, b.out_status = outs["tokens"].data_ptr(), outs["status"].data_ptr()
        b.out_kept_count = outs["kept_count"].data_ptr()
        b.out_kept_ids, b.out_kept_probs, b.kept_ld = outs["kept_ids"].data_ptr(), outs["kept_probs"].data_ptr(), kept_ld
        descs.append(b)

    # Eager outputs of the last pool entry (checked against the graph replay)
    # and of entry 0 (checked against the CPU oracle in the baseline leg).
    P = len(descs)
    sampler.launch(descs[P - 1])
    torch.cuda.synchronize()
    tokens_last = outs["tokens"].cpu().numpy().view(np.uint32).copy()
    sampler.launch(descs[0])
    torch.cuda.synchronize()
    tokens0 = outs["tokens"].cpu().numpy().view(np.uint32).copy()
    kept_avg = float(outs["kept_count"].float().mean().item())
    assert (outs["status"] == 0).all().item(), "sampler reported a non-OK row status"

    stream = torch.cuda.Stream()
    mode = "eager"
    graph = None
    if not args.eager:
        try:
            stream.wait_stream(torch.cuda.current_stream())
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                for i in range(P):
                    sampler.launch(descs[i])
            torch.cuda.synchronize()
            mode = "hip_graph"
        except Exception as e:  # fall back to eager launches, and say so
            print(f"bench.py: graph capture failed ({e}); timing eager launches", file=sys.stderr)
            graph = None

    def run_steps(n):
        """n launches (n a multiple of P in graph mode)."""
        with torch.cuda.stream(stream):
            if graph is not None:
                for _ in range(n // P):
                    graph.replay()
            else:
                for i in range(n):
                    sampler.launch(descs[i % P], stream)

    steps = args.steps if graph is None else max(P, (args.steps + P - 1) // P * P)
    warm = args.warmup if graph is None else max(P, (args.warmup + P - 1) // P * P)
    run_steps(warm)
    torch.cuda.synchronize()
    if graph is not None:  # a replay ends with pool entry P-1: same tokens as eager
        with torch.cuda.stream(stream):
            graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(outs["tokens"].cpu().numpy().view(np.uint32), tokens_last), \
            "graph replay differs from the eager launch"

    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ev0.record(stream)
    t0 = time.perf_counter()
    run_steps(steps)
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    elapsed_ms = ev0.elapsed_time(ev1)
    ms_per_step = elapsed_ms / steps
    rows_per_s = B * steps / (elapsed_ms / 1e3)
    # the median per-step time: events between replays of the P-call graph
    # (or between eager groups of P calls), outside the timed region above
    groups = []
    if graph is not None:
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(51)]
        with torch.cuda.stream(stream):
            evs[0].record(stream)
            for i in range(50):
                graph.replay()
                evs[i + 1].record(stream)
        torch.cuda.synchronize()
        groups = [evs[i].elapsed_time(evs[i + 1]) * 1e3 / P for i in range(50)]
    median_us = float(np.median(groups)) if groups else ms_per_step * 1e3

    alg = algorithmic_bytes(B, V, H, kept_avg)
    achieved = alg / (ms_per_step / 1e3) / 1e9
    traffic, traffic_src = read_traffic(args.traffic_summary)
    result = {
        "metric": "sampled rows/sec + achieved HBM GB/s, batch 64 x 128256 vocab full chain",
        "value": rows_per_s,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warm,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": f"synthetic (seeded config-2 batch + {P - 1} GPU-drawn batches of the same distribution)",
        "config": {
            "workload": "config2: B=64 x V=128256 f32 logits, history 512; freq 0.3 + presence 0.2 + repeat 1.05 "
                        "-> temp 0.7 -> top-k 50 -> top-p 0.9 -> min-p 0.05 -> draw with supplied u",
            "batch": B, "vocab": V, "history": H, "pool_batches": P,
            "pool_bytes": P * B * V * 4, "launch": mode,
        },
        "tokens_per_s": rows_per_s,
        "median_us_per_step": median_us,
        "achieved_GBps": achieved,
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic,
            "algorithmic_bytes_per_launch": alg,
            "traffic_source": traffic_src,
            "kernel": "oxs_sample_batch = stream_kernel + tail_kernel (one launch pair, timed together "
                      "with HIP events on their launch stream)",
        },
        "wall_s": wall,
    }
    # The call is two kernels: the HBM-bound stream kernel moves the logits
    # (everything but the tail's candidate lists and outputs); the tail is
    # latency-bound. Their split, from the committed kernel trace of this bench.
    split, split_src = read_kernel_trace(args.trace_summary)
    if split and "stream_kernel" in split:
        stream_bytes = B * (V * 4 + H * 4 + 104)
        sk = split["stream_kernel"]["avg_ns"] * 1e-9
        per = {"stream_kernel": {"avg_us": sk * 1e6, "algorithmic_bytes": stream_bytes,
                                 "achieved": stream_bytes / sk / 1e9, "frac": stream_bytes / sk / 1e9 / HBM_PEAK_GBS,
                                 "bound": "hbm"}}
        if "tail_kernel" in split:
            per["tail_kernel"] = {"avg_us": split["tail_kernel"]["avg_ns"] * 1e-3, "bound": "latency"}
            per["sum_us"] = (split["stream_kernel"]["avg_ns"] + split["tail_kernel"]["avg_ns"]) * 1e-3
        result["roofline"]["per_kernel"] = per
        result["roofline"]["per_kernel_source"] = split_src
    if achieved > 1.05 * HBM_PEAK_GBS:  # roofline.rs:53-style integrity check
        result["roofline"]["warning"] = "achieved exceeds 1.05 x peak: inputs were cached, not streamed"
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(w, tokens0, args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
