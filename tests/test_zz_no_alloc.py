"""oxs_sample_batch_static (the no-allocation entry point) against
oxs_sample_batch on the same inputs: every output identical, over two calls
in a row on one device, the second smaller than the first (the static
workspace keeps the first call's contents)."""
import pytest

import numpy as np

from harness import compare, gpu_sampler, run_gpu, run_oracle, to_device
from oxide_sampler import _abi
from oxide_sampler import workloads as wl
from test_gpu_parity import RTOL_F32, dry_long_workload, dry_many_ids_workload, mixed_workload

pytestmark = pytest.mark.gpu


def banner(msg):
    print(f"\n[case] {msg}", flush=True)


def test_static_matches_sampler_two_calls(torch_gpu):
    big = wl.config2()  # B=64 x V=128256, full chain
    small = mixed_workload(40, 50001, seed=4242)  # every chain shape, DRY rows, ragged histories
    for w, kw in ((big, dict(logits_out=True)), (small, dict(kept_ld=1024, logits_out=True, max_top_k=1024))):
        banner(f"static vs sampler: {w.name} B={w.batch} V={w.vocab}")
        want = run_gpu(w, torch_gpu, **kw)
        got = run_gpu(w, torch_gpu, no_alloc=True, **kw)
        compare(got, want, 0.0, f"static {w.name}")


def dry_penalised_ids(hist: np.ndarray, L: int, allowed: int, V: int) -> int:
    """Distinct ids the DRY pass (sampler.rs:393-415) penalises over a slice: for every match length
    m in [allowed, 32] and every earlier position i whose m ids equal the slice's last m ids, the id
    after them (when it is < V). Brute force over the slice."""
    s = [int(x) for x in hist[-L:]]
    ids = set()
    for m in range(max(allowed, 0), 33):
        if L < m:
            continue
        tail = s[L - m:]
        for i in range(L - m):
            if s[i:i + m] == tail and s[i + m] < V:
                ids.add(s[i + m])
    return len(ids)


def _rows(res, rows):
    pick = lambda a: None if a is None else a[rows]
    return type(res)(*(pick(getattr(res, f)) for f in ("tokens", "status", "kept_count", "kept_ids", "kept_probs",
                                                        "history", "history_len", "mu", "rng_state", "logits_out")))


def test_static_dry_long_slices(torch_gpu):
    # DRY slices of 1500 and 4096 ids: without the sampler's global DRY hash the static workspace
    # counts a long slice's ids in the 2048-slot LDS hash. Rows whose pass penalises more ids than
    # that (an allowed length of 0 penalises the id after every position) report
    # OXS_ROW_UNSUPPORTED; every other row matches the oracle
    w = dry_long_workload(24, 32000, seed=31)
    banner("static: DRY slices of 1500 and 4096 ids B=24 V=32000")
    counts = np.array([dry_penalised_ids(w.history[b, :int(w.history_len[b])],
                                         min(int(w.history_len[b]), w.configs[b].dry_range),
                                         w.configs[b].dry_allowed_length, w.vocab) for b in range(w.batch)])
    over = counts > 2048
    print("distinct penalised ids per row:", counts.tolist(), flush=True)
    assert over.any() and not over.all()  # both kinds of row are exercised
    g = run_gpu(w, torch_gpu, kept_ld=256, no_alloc=True)
    r = run_oracle(w, kept_ld=256)
    assert (g.status[over] == _abi.OXS_ROW_UNSUPPORTED).all() and (g.tokens[over] == 0).all()
    fit = np.nonzero(~over)[0]
    compare(_rows(g, fit), _rows(r, fit), RTOL_F32, "static dry long")


def test_static_dry_ids_past_its_list(torch_gpu):
    # 2100 distinct penalised ids: more than the static workspace's 2048-entry DRY list, so that row
    # reports OXS_ROW_UNSUPPORTED there while the other rows match the oracle; a sampler (default
    # max_dry_ids 8192) runs the whole batch, that row included
    w = dry_many_ids_workload(2100, seed=33)
    banner("static: DRY row with 2100 distinct penalised ids")
    r = run_oracle(w, kept_ld=256)
    g = run_gpu(w, torch_gpu, kept_ld=256, no_alloc=True)
    assert g.status[3] == _abi.OXS_ROW_UNSUPPORTED and g.tokens[3] == 0
    keep = np.arange(w.batch) != 3
    np.testing.assert_array_equal(g.tokens[keep], r.tokens[keep])
    np.testing.assert_array_equal(g.status[keep], r.status[keep])
    compare(run_gpu(w, torch_gpu, kept_ld=256), r, RTOL_F32, "sampler dry 2100 ids")


def test_static_under_graph_capture(torch_gpu):
    # oxs_sample_batch_static captured in a torch CUDA graph, the use it exists for, and replayed
    # three times with eager work and synchronisations between the replays: every replay's outputs
    # equal oxs_sample_batch's on the same inputs. Nothing is recorded and the uniforms are
    # supplied, so the call only reads its inputs and every replay must give the same outputs.
    torch = torch_gpu
    d = torch.device("cuda")
    w = mixed_workload(48, 50001, seed=4243)
    w.mu = None
    w.configs = [c if c.mirostat_mode == 0 else wl.disabled_config(temperature=0.8, top_k=40) for c in w.configs]
    banner(f"static under graph capture: {w.name} B={w.batch} V={w.vocab}")
    want = run_gpu(w, torch, kept_ld=1024, record=False, max_top_k=1024)
    cfg, bias_ids, bias_vals, ban_ids = w.packed_configs()
    logits = to_device(w, torch)
    ins = dict(
        bias_ids=torch.from_numpy(bias_ids.view(np.int32)).to(d) if bias_ids.size else None,
        bias_values=torch.from_numpy(bias_vals).to(d) if bias_vals.size else None,
        ban_ids=torch.from_numpy(ban_ids.view(np.int32)).to(d) if ban_ids.size else None,
        mask=torch.from_numpy(w.mask.view(np.int32)).to(d) if w.mask is not None else None,
        history=torch.from_numpy(w.history.view(np.int32).copy()).to(d),
        history_len=torch.from_numpy(w.history_len.view(np.int32).copy()).to(d),
        history_cap=w.history.shape[1], record=False, uniforms=torch.from_numpy(w.uniforms).to(d), kept_ld=1024)
    d_cfg = torch.from_numpy(cfg).to(d)
    B = w.batch
    out = {k: torch.empty(B, dtype=torch.int32, device=d) for k in ("tokens", "status", "kept_count")}
    out["kept_ids"] = torch.empty(B, 1024, dtype=torch.int32, device=d)
    out["kept_probs"] = torch.empty(B, 1024, dtype=torch.float32, device=d)
    s = gpu_sampler(B, w.vocab, 1024)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    s.sample(logits, d_cfg, stream=st, out=out, no_alloc=True, **ins)  # the device's set-up call, eager
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        s.sample(logits, d_cfg, stream=st, out=out, no_alloc=True, **ins)
    torch.cuda.synchronize()
    for rep in range(3):
        for t in out.values():  # eager work between replays: clear the outputs with fill kernels
            t.fill_(-1)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        kept = out["kept_count"].cpu().numpy().view(np.uint32)
        np.testing.assert_array_equal(out["tokens"].cpu().numpy().view(np.uint32), want.tokens, err_msg=f"replay {rep}")
        np.testing.assert_array_equal(out["status"].cpu().numpy(), want.status, err_msg=f"replay {rep}")
        np.testing.assert_array_equal(kept, want.kept_count, err_msg=f"replay {rep}")
        ids = out["kept_ids"].cpu().numpy().view(np.uint32)
        probs = out["kept_probs"].cpu().numpy()
        for b in range(B):
            n = min(int(kept[b]), 1024)
            np.testing.assert_array_equal(ids[b, :n], want.kept_ids[b, :n], err_msg=f"replay {rep} row {b}")
            np.testing.assert_array_equal(probs[b, :n].view(np.uint32), want.kept_probs[b, :n].view(np.uint32),
                                          err_msg=f"replay {rep} row {b}")


def test_static_rejects_oversize(torch_gpu):
    lib = _abi.load_library()
    b = _abi.OxsBatch()
    b.batch, b.vocab = _abi.OXS_STATIC_MAX_BATCH + 1, 1000
    assert lib.oxs_sample_batch_static(b, None) == _abi.OXS_ERR_LIMITS
    b.batch, b.vocab = 1, _abi.OXS_STATIC_MAX_VOCAB + 1
    assert lib.oxs_sample_batch_static(b, None) == _abi.OXS_ERR_LIMITS
    assert lib.oxs_sample_batch_static(None, None) == _abi.OXS_ERR_INVALID_ARGUMENT
    b.batch, b.vocab = 0, 1000  # nothing to do
    assert lib.oxs_sample_batch_static(b, None) == _abi.OXS_OK
