// oxs_tail.hip — the tail kernel (one block per row: top-M selection and the
// chain) and the wide kernel (rows whose pool exceeds 1024), the second of
// the sampler's launches.
#include <type_traits>

#include "oxs_sampler_dev.h"

namespace oxs {

template <int DT, int PER>
// Leading arguments: what the first loads need, preloaded into SGPRs as in
// stream_kernel.
__global__ __launch_bounds__(kThreads) void tail_kernel(const uint64_t* __restrict__ wave_theta,
                                                        const uint64_t* __restrict__ lists,
                                                        const uint32_t* __restrict__ wave_count,
                                                        const uint64_t* __restrict__ libm, uint32_t S, uint32_t cap_w,
                                                        uint32_t cap_shift, uint32_t rpx, uint32_t B, const Params p) {
  // bucket scatter / sort / exact-path table / chain scratch, and 8 words of
  // padding for the bucket ranking's reads past a bucket
  __shared__ __align__(16) uint64_t s_keys[kTailArea + 8];
  static_assert(kTailArea >= PER * kThreads && kTailArea * 2 >= kMaxChunk, "tail LDS area");
  __shared__ __align__(16) uint64_t s_top[kMaxM];       // sorted top-M keys (sort and exact paths)
  __shared__ __align__(16) uint32_t s_ids[kChainLd];
  __shared__ __align__(16) float s_pr[kChainLd];
  __shared__ __align__(16) float s_hit[16];
  __shared__ __align__(16) uint32_t s_bcount[kBuckets + 64];  // + one dummy slot per lane
  __shared__ __align__(16) uint32_t s_bstart_all[kWavesPerBlock][kBuckets];  // one copy per wavefront
  __shared__ TailShared ts;
  __shared__ LibmTables s_tab;
  static_assert(sizeof(uint32_t) * kChainLd * 3 + sizeof(uint64_t) * kChainLd <= sizeof(s_keys),
                "chain scratch fits the key area");

  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t row = rpx ? grouped_index(blockIdx.x, rpx) : blockIdx.x;
  if (row >= B) return;

  // 1. the row's reads, issued before anything waits: the wavefront
  // thresholds, the candidate slots (two per 16-byte load) with the count of
  // the wavefront that wrote them and the libm tables (vector loads whose
  // addresses need nothing from memory), then the row's record (config,
  // history length, uniform, mu, rng) through the scalar cache, whose wait
  // does not cover the vector loads
  const uint32_t W = S * kWavesPerBlock;
  const uint32_t span = W * cap_w;  // even: cap_w >= 8
  uint64_t wr[kRecPer];  // every wavefront reads all W records (lane + 64 q; clamped repeats change no maximum)
#pragma unroll
  for (int q = 0; q < kRecPer; ++q) {
    const uint32_t w = lane + 64u * q;
    wr[q] = wave_theta[(size_t)row * W + (w < W ? w : W - 1u)];
  }
  uint64_t lk[PER];
  uint32_t lc[PER / 2];
  const ulonglong2* lrow = (const ulonglong2*)(lists + (size_t)row * span);
  const uint32_t* wcrow = wave_count + (size_t)row * W;
#pragma unroll
  for (int q = 0; q < PER / 2; ++q) {  // unconditional loads (clamped index): no branches between them
    const uint32_t pair = tid + q * kThreads;
    const uint32_t at = 2u * pair < span ? pair : 0u;
    const ulonglong2 k2 = lrow[at];
    lk[2 * q] = k2.x;
    lk[2 * q + 1] = k2.y;
    lc[q] = wcrow[(2u * at) >> cap_shift];
  }
  const LibmEntries tabv = fetch_libm_tables(libm);
  __builtin_amdgcn_sched_barrier(0);  // every vector read above is issued before anything waits
  const RowIn rin = load_row_in(p, row);
  const oxs_sampling_config c = rin.cfg;
  const RowXf r = make_row_xf_h(p, c, rin.history_len);
  RowState rs;
  rs.uniform = rin.uniform;
  rs.mu = rin.mu;
  rs.rng = rin.rng;
  rs.history_len = rin.history_len;
  rs.raw = rin.raw;
  rs.dec_pos = 0;
  rs.dec_count = 0;
  rs.dec_steps = 0;
  if constexpr (kind_decode(DT)) {
    if (p.dec_pos) rs.dec_pos = p.dec_pos[row];
    if (p.dec_count) rs.dec_count = p.dec_count[row];
    if (p.host_tokens) rs.dec_steps = p.row_steps[row];
  }
  store_libm_tables(tabv, s_tab);
  for (uint32_t i = tid; i < (uint32_t)kBuckets + 64; i += kThreads) s_bcount[i] = 0;


  // the pool size, at most V (filter_k = min(max(top_k, 256), len), sampler.rs:274)
  const uint32_t M = min(max(c.top_k, 256u), max(p.V, 256u));
  if (M > (uint32_t)kMaxM) {
    if (p.wide_keys && M <= p.wide_cap) return;  // the wide kernel's row
    count_path(p, kPathNone);
    write_row_result<DT>(p, row, 0u, OXS_ROW_UNSUPPORTED, rs);  // sizes this build does not run on the device
    return;
  }
  if (c.mirostat_mode != OXS_MIROSTAT_DISABLED && !p.mu) {
    count_path(p, kPathNone);
    write_row_result<DT>(p, row, 0u, OXS_ROW_MISSING_STATE, rs);
    return;
  }
  // DRY rows: their values, then the exact path (the stream kernel's
  // candidates do not include DRY)
  if (r.dry && !dry_pass<DT>(p, r, row, (uint32_t*)s_keys, s_tab, ts)) {
    count_path(p, kPathNone);
    write_row_result<DT>(p, row, 0u, OXS_ROW_UNSUPPORTED, rs);  // more penalised ids than the DRY hash holds
    return;
  }
  // A DRY row stays on the candidate path when DRY can only lower a value on
  // its way to the key (penalties >= 0: dry_base >= 0; the stages after DRY
  // and the temperature are non-decreasing, as the repetition penalty runs
  // only for repeat_penalty > 0) and its slice fit the LDS hash: a penalised
  // id outside the stream's candidates was below its wavefront's threshold
  // before DRY and stays below it, and a penalised candidate gets its key
  // recomputed here from its DRY value and its count in the repeat window
  // (sampler.rs:203-245).
  const bool dry_cand = r.dry && min(r.hlen, r.dry_range) <= (uint32_t)kDryMax && r.dry_base >= 0.0f;
  if (dry_cand) {
    const uint32_t* hkey = (const uint32_t*)s_keys + kDryKey;
    const float* dval = (const float*)s_keys + kDryVal;
    uint32_t* wcnt = (uint32_t*)s_keys + kDryCnt;  // over the sorted list, now in the row's DRY list
    for (uint32_t h = tid; h < (uint32_t)kDryHash; h += kThreads) wcnt[h] = 0;
    __syncthreads();
    // ids whose bit is clear in the pass's mask were not penalised: no lookup
    const uint64_t bits = ((uint64_t)ts.dry_bits[1] << 32) | ts.dry_bits[0];
    const auto maybe_dry = [bits](uint32_t id) { return ((bits >> ((id * 0x9e3779b1u) >> 26)) & 1u) != 0u; };
    if (r.use_hist) {
      const uint32_t* win = p.history + (size_t)row * p.history_ld + r.wstart;
      for (uint32_t j = tid; j < r.wn; j += kThreads) {
        if (!maybe_dry(win[j])) continue;
        const uint32_t h = dry_lookup(hkey, win[j]);
        if (h < (uint32_t)kDryHash) atomicAdd(&wcnt[h], 1u);
      }
    }
    __syncthreads();
    const float inv_t = r.do_temp ? r.inv_temp : 1.0f;
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const uint32_t slot = 2u * (tid + (q / 2) * kThreads) + (q & 1);
      if (!(slot < span && (slot & (cap_w - 1u)) < lc[q / 2] && lk[q] != 0ull)) continue;
      const uint32_t id = ~(uint32_t)lk[q];
      if (!maybe_dry(id)) continue;
      const uint32_t h = dry_lookup(hkey, id);
      if (h < (uint32_t)kDryHash) lk[q] = comp_key(cand_key(special_post(r, dval[h], wcnt[h]) * inv_t), id);
    }
    if (p.logits_out)  // the stream kernel wrote these ids without DRY
      for (uint32_t h = tid; h < (uint32_t)kDryHash; h += kThreads) {
        const uint32_t id = hkey[h];
        if (id != kEmptySlot)
          p.logits_out[(size_t)row * p.logits_out_ld + id] = special_post(r, dval[h], wcnt[h]) * inv_t;
      }
  }

  // 2. the largest wavefront threshold and the largest key, from the
  // wavefront records, reduced by every wavefront on its own (a record of all
  // ones marks a wavefront whose candidates are incomplete: the exact path);
  // the smallest valid key is needed only when every wavefront kept all of
  // its candidates
  uint32_t valid = 0;
  uint64_t kmn = ~0ull;
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const uint32_t slot = 2u * (tid + (q / 2) * kThreads) + (q & 1);
    const uint64_t k = lk[q];
    // (a key whose value word is 0, -inf or NaN: a candidate that DRY sent
    // there, is not valid)
    if (slot < span && (slot & (cap_w - 1u)) < lc[q / 2] && (k >> 32) != 0ull) {
      valid |= 1u << q;
      kmn = k < kmn ? k : kmn;
    }
  }
  uint32_t th_l = 0, km_l = 0;
#pragma unroll
  for (int q = 0; q < kRecPer; ++q) {
    th_l = max(th_l, (uint32_t)(wr[q] >> 32));
    km_l = max(km_l, (uint32_t)wr[q]);
  }
  const uint32_t th_w = wave_reduce32(th_l, MaxOp{});
  const bool exact = th_w == 0xffffffffu || (r.dry && !dry_cand);
  const uint64_t theta_max = exact ? ~0ull : (uint64_t)th_w << 32;
  uint64_t kmax = (uint64_t)wave_reduce32(km_l, MaxOp{}) << 32;
  const bool all_kept = th_w == kMinValidOrd;  // (the same in every wavefront)
  uint64_t kmin = 0;
  if (all_kept) {
    const uint64_t d = wave_min_u64(kmn);
    if (lane == 0) ts.a_kmin[wave] = d;
  }
  if (dry_cand) {  // the records' largest key predates DRY: the largest of the keys themselves
    uint32_t km = 0;
#pragma unroll
    for (int q = 0; q < PER; ++q)
      if ((valid >> q) & 1u) km = max(km, (uint32_t)(lk[q] >> 32));
    const uint32_t d = wave_reduce32(km, MaxOp{});
    if (lane == 0) ts.a_kmax[wave] = d;
  }
  __syncthreads();  // every bucket count zeroed before any wavefront counts, and a_kmin complete
  if (all_kept) {
    kmin = ts.a_kmin[0];
#pragma unroll
    for (int w = 1; w < kWavesPerBlock; ++w) kmin = ts.a_kmin[w] < kmin ? ts.a_kmin[w] : kmin;
  }
  if (dry_cand) {
    uint32_t km = ts.a_kmax[0];
#pragma unroll
    for (int w = 1; w < kWavesPerBlock; ++w) km = max(km, ts.a_kmax[w]);
    kmax = (uint64_t)km << 32;
  }
  // 3. kept keys: at or above every wavefront threshold (when every
  // wavefront kept all, every valid key)
  uint32_t vm = 0;
  const uint64_t (&yk)[PER] = lk;
#pragma unroll
  for (int q = 0; q < PER; ++q)
    if (((valid >> q) & 1u) && lk[q] >= theta_max) vm |= 1u << q;

  // 4. N >= M kept keys contain the row's top M. Keys are bucketed linearly
  // in value between the largest key and a lower bound of the kept ones (the
  // threshold, or the smallest key when all were kept): rounded subtraction
  // and scaling are monotone, so bucket order agrees with key order, and only
  // the buckets up to the one holding the M-th key are ranked, each key
  // against the members of its bucket.
  const float vmax = key_value(kmax);
  const float vmin = all_kept ? key_value(kmin) : key_value(theta_max);
  const float range = vmax - vmin;
  const float scale = (float)(kBuckets - 1) / range;
  const bool linear = !exact && kmax >= theta_max && range > 0.0f && range <= __FLT_MAX__ &&
                      scale <= __FLT_MAX__ && vmax <= __FLT_MAX__ && vmin >= -__FLT_MAX__;
  uint32_t meff = 0;
  int path = exact ? 2 : 1;  // 0 buckets, 1 sort, 2 exact re-scan
  uint32_t bs[PER];
  uint32_t* s_bstart = s_bstart_all[wave];
  uint32_t last = 0;
  if (linear) {
    // histogram; the returned count is the key's slot inside its bucket. Every
    // slot issues its atomic (unkept ones add 0 to this lane's dummy counter)
    // so that the atomics go out back to back.
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const bool on = (vm >> q) & 1u;
      const uint32_t b = on ? bucket_of(yk[q], vmax, scale) : (uint32_t)kBuckets + lane;
      bs[q] = b | (atomicAdd(&s_bcount[b], on ? 1u : 0u) << 16);  // bucket | slot inside the bucket
    }
    __syncthreads();
    // bucket starts, the count N and the bucket of the M-th key, computed by
    // every wavefront (lane l owns buckets 4l .. 4l+3) into its own copy
    const uint4 c4 = *(const uint4*)&s_bcount[lane * 4];
    const uint32_t loc = c4.x + c4.y + c4.z + c4.w;
    const uint32_t incl = wave_incl_scan(loc);
    const uint32_t N = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
    const uint32_t big = wave_max_u32(max(max(c4.x, c4.y), max(c4.z, c4.w)));
    meff = min(M, N);
    const uint32_t st0 = incl - loc, st1 = st0 + c4.x, st2 = st1 + c4.y, st3 = st2 + c4.z;
    *(uint4*)&s_bstart[lane * 4] = make_uint4(st0, st1, st2, st3);
    uint32_t mine = kBuckets;
    if (st0 < meff && st0 + c4.x >= meff) mine = lane * 4;
    if (st1 < meff && st1 + c4.y >= meff) mine = lane * 4 + 1;
    if (st2 < meff && st2 + c4.z >= meff) mine = lane * 4 + 2;
    if (st3 < meff && st3 + c4.w >= meff) mine = lane * 4 + 3;
    last = wave_reduce32(mine, MinOp{});  // the bucket of the meff-th key
    if (N < M && !all_kept) path = 2;
    else if (big > kBigBucket) path = 1;
    else path = 0;
    wave_sync();
  }
  if (path != 1) count_path(p, path);  // (the sort path counts itself: it may end in the exact path)

  if (path == 0) {
    if (meff == 0) {  // every logit -inf or NaN (:267-270)
      write_row_result<DT>(p, row, 0u, OXS_ROW_EMPTY, rs);
      return;
    }
    const uint32_t span_k = s_bstart[last] + s_bcount[last];  // keys in buckets 0 .. last
    uint32_t start[PER];
#pragma unroll
    for (int q = 0; q < PER; ++q) start[q] = s_bstart[min(bs[q] & 0xffffu, (uint32_t)kBuckets - 1)];
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      if (((vm >> q) & 1u) && (bs[q] & 0xffffu) <= last) s_keys[start[q] + (bs[q] >> 16)] = yk[q];
    }
    __syncthreads();
    // rank inside the bucket; the softmax numerators (:286-290) in the same pass
    for (uint32_t i = tid; i < span_k; i += kThreads) {
      const uint64_t k = s_keys[i];
      const uint32_t b = bucket_of(k, vmax, scale);
      const uint32_t lo = s_bstart[b], hi = lo + s_bcount[b];
      // eight members per step, all read before any is compared (entries past
      // the bucket, up to 7 words into the padding, are masked out)
      uint32_t rank = lo;
      for (uint32_t j = lo; j < hi; j += 8) {
        uint64_t a[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) a[t] = s_keys[j + t];
#pragma unroll
        for (int t = 0; t < 8; ++t) rank += (j + t < hi && a[t] > k) ? 1u : 0u;
      }
      if (rank < meff) {
        s_ids[rank] = ~(uint32_t)k;
        s_pr[rank] = dexpf(key_value(k) - vmax, s_tab);
      }
    }
    __syncthreads();
  } else if (path == 1) {
    const uint32_t N = sort_select(yk, vm, M, s_keys, s_top, ts);
    if (N < M && !all_kept) path = 2;
    count_path(p, path);
    if (path == 1) {
      meff = min(M, N);
      if (meff == 0) {
        write_row_result<DT>(p, row, 0u, OXS_ROW_EMPTY, rs);
        return;
      }
      keys_to_chain(s_top, meff, s_ids, s_pr, s_tab);
    }
  }
  if (path == 2) {
    meff = exact_select_row<DT>(p, r, row, M, (uint32_t*)s_keys, s_bcount, s_top, ts);
    if (meff == 0) {
      write_row_result<DT>(p, row, 0u, OXS_ROW_EMPTY, rs);
      return;
    }
    bitonic_sort<false>(s_top, meff);
    keys_to_chain(s_top, meff, s_ids, s_pr, s_tab);
  }

  // 5. the chain after the top-M selection, in the first wavefront
  if (wave != 0) return;
  uint32_t* scratch = (uint32_t*)s_keys;
  ChainBufs bf;
  bf.ids = s_ids;
  bf.pr = s_pr;
  bf.ids_b = scratch;
  bf.pr_b = (float*)(scratch + kChainLd);
  bf.aux = (float*)(scratch + 2 * kChainLd);
  bf.aux64 = (uint64_t*)(scratch + 3 * kChainLd);
  bf.hit = s_hit;
  bf.big = nullptr;
  wave_chain<DT>(p, c, row, meff, bf, rs, s_tab);
}

// ---------------------------------------------------------------- wide rows

// Rows whose top-M pool exceeds kMaxM (top_k > 1024), one block per row,
// launched after the tail kernel (which leaves these rows alone) when the
// sampler was created with max_top_k > 1024: the exact top-M radix select
// into global memory, a sort there, and the same chain on arrays in global
// memory. sampler.rs:272-279 (filter_k = max(top_k, 256) of the row, sorted).
template <int DT>
__global__ __launch_bounds__(kThreads) void wide_kernel(const Params p) {
  __shared__ __align__(16) uint64_t s_area[kTailArea];  // DRY pass, exact-path chunk table, sort tiles
  __shared__ __align__(16) uint32_t s_hist[kBuckets + 64];
  __shared__ __align__(16) float s_hit[16];
  __shared__ TailShared ts;
  __shared__ LibmTables s_tab;
  const uint32_t row = blockIdx.x;
  const uint32_t tid = threadIdx.x;
  const LibmEntries tabv = fetch_libm_tables(p.libm);
  const RowIn rin = load_row_in(p, row);
  const oxs_sampling_config c = rin.cfg;
  const uint32_t M = min(max(c.top_k, 256u), max(p.V, 256u));
  if (M <= (uint32_t)kMaxM || M > p.wide_cap) return;  // (uniform: the tail kernel's rows)
  const RowXf r = make_row_xf_h(p, c, rin.history_len);
  RowState rs;
  rs.uniform = rin.uniform;
  rs.mu = rin.mu;
  rs.rng = rin.rng;
  rs.history_len = rin.history_len;
  rs.raw = rin.raw;
  rs.dec_pos = 0;
  rs.dec_count = 0;
  rs.dec_steps = 0;
  if constexpr (kind_decode(DT)) {
    if (p.dec_pos) rs.dec_pos = p.dec_pos[row];
    if (p.dec_count) rs.dec_count = p.dec_count[row];
    if (p.host_tokens) rs.dec_steps = p.row_steps[row];
  }
  store_libm_tables(tabv, s_tab);
  __syncthreads();
  if (c.mirostat_mode != OXS_MIROSTAT_DISABLED && !p.mu) {
    count_path(p, kPathNone);
    write_row_result<DT>(p, row, 0u, OXS_ROW_MISSING_STATE, rs);
    return;
  }
  if (r.dry && !dry_pass<DT>(p, r, row, (uint32_t*)s_area, s_tab, ts)) {
    count_path(p, kPathNone);
    write_row_result<DT>(p, row, 0u, OXS_ROW_UNSUPPORTED, rs);
    return;
  }
  count_path(p, kPathExact);
  uint64_t* keys = p.wide_keys + (size_t)row * p.wide_n2;
  const uint32_t meff = exact_select_row<DT>(p, r, row, M, (uint32_t*)s_area, s_hist, keys, ts, p.wide_cap);
  if (meff == 0) {
    write_row_result<DT>(p, row, 0u, OXS_ROW_EMPTY, rs);
    return;
  }
  wide_sort(keys, meff, s_area);
  uint32_t* arr = p.wide_arr + (size_t)row * 7 * p.wide_ld;
  ChainBufs bf;
  bf.ids = arr;
  bf.pr = (float*)(arr + p.wide_ld);
  bf.ids_b = arr + 2 * p.wide_ld;
  bf.pr_b = (float*)(arr + 3 * p.wide_ld);
  bf.aux = (float*)(arr + 4 * p.wide_ld);
  bf.aux64 = (uint64_t*)(arr + 5 * p.wide_ld);  // [5 ld, 7 ld)
  bf.hit = s_hit;
  bf.big = keys;  // free once the chain arrays are written
  keys_to_chain(keys, meff, bf.ids, bf.pr, s_tab);
  if (tid >= 64) return;
  wave_chain<DT>(p, c, row, meff, bf, rs, s_tab);
}

template <int KIND>
static hipError_t launch_tail_k(const Params& p, uint32_t grid_b, hipStream_t st) {
  // the row's candidate union: 2048 keys, or 4096 past 64 wavefront records
  if ((uint64_t)p.S * kWavesPerBlock * p.cap_w > (uint64_t)kUnionMax)
    hipLaunchKernelGGL((tail_kernel<KIND, kUnionBig / kThreads>), dim3(grid_b), dim3(kThreads), 0, st,
                       (const uint64_t*)p.wave_theta, (const uint64_t*)p.lists, (const uint32_t*)p.wave_count, p.libm,
                       p.S, p.cap_w, p.cap_shift, p.rpx, p.B, p);
  else
    hipLaunchKernelGGL((tail_kernel<KIND, kPer>), dim3(grid_b), dim3(kThreads), 0, st, (const uint64_t*)p.wave_theta,
                       (const uint64_t*)p.lists, (const uint32_t*)p.wave_count, p.libm, p.S, p.cap_w, p.cap_shift,
                       p.rpx, p.B, p);
  if (p.wide_keys) hipLaunchKernelGGL((wide_kernel<KIND>), dim3(p.B), dim3(kThreads), 0, st, p);
  return hipGetLastError();
}

hipError_t launch_tail_kind(int kind, const Params& p, uint32_t grid, hipStream_t st) {
  constexpr int F = OXS_DTYPE_F32, H = OXS_DTYPE_BF16, S = kKindSoftcap, D = kKindDecode;
  switch (kind) {
    case F: return launch_tail_k<F>(p, grid, st);
    case H: return launch_tail_k<H>(p, grid, st);
    case F | S: return launch_tail_k<F | S>(p, grid, st);
    case H | S: return launch_tail_k<H | S>(p, grid, st);
    case F | D: return launch_tail_k<F | D>(p, grid, st);
    case H | D: return launch_tail_k<H | D>(p, grid, st);
    case F | S | D: return launch_tail_k<F | S | D>(p, grid, st);
    case H | S | D: return launch_tail_k<H | S | D>(p, grid, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace oxs
