// oxs_sampler.hip — batched token sampler for MI355X (gfx950).
//
// Replaces the per-row CPU chain of crates/oxide-core/src/sampler.rs
// (AcademicSamplerEngine::sample_token, sampler.rs:173-390) with one kernel
// launch per batch. The launch has two roles:
//
// Phase A (every block): block (row, chunk) streams CH logits of one row with
//   coalesced 16-byte loads, applies the grammar mask, bans, biases, newline,
//   repetition/frequency/presence penalties and temperature in registers (in the
//   reference's order, with the reference's IEEE operations), and keeps only a
//   small candidate set: each wavefront finds the c-th largest of its 64 lane
//   maxima (32 ballot steps) and writes every element at or above it as a
//   64-bit key (order-preserving value bits << 32 | ~token id). Keys are unique
//   and order candidates by value descending, then by lower token id.
//
// Tail (the last block of each row, chosen by an atomic ticket): gathers the
//   row's candidate sets, selects the exact top M = max(top_k, 256) by radix
//   select, checks that every wavefront's threshold lies at or below the M-th
//   key (which proves the union holds the row's true top M; otherwise the block
//   re-scans the row exactly), sorts the M keys, and runs softmax, Mirostat or
//   min-p / XTC / top-k / tail-free / typical / top-p, renormalisation and the
//   inverse-CDF draw, using expf/logf/log2f that reproduce glibc bit for bit.
//
// No allocation, no host synchronisation; all workspace comes from the sampler
// handle.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/oxide_sampler.h"
#include "oxs_libm.h"

namespace oxs {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / 64;
constexpr int kUnionMax = 4096;   // candidate keys a row's tail can hold
constexpr int kMaxM = 1024;       // largest max(top_k, 256) run on the device
constexpr int kMaxChunk = 8192;   // logits per block (size of the LDS penalty table)
constexpr int kMaxChunks = 64;    // chunks per row (4 wavefronts each -> <= 256 tail entries)

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kCountMask = 0x0fffffffu;
constexpr uint32_t kBanFlag = 1u << 28;
constexpr uint32_t kBiasFlag = 1u << 29;
constexpr uint32_t kNlFlag = 1u << 30;

struct Params {
  const void* logits;
  int64_t ld;
  uint32_t B, V, flags;
  const oxs_sampling_config* configs;
  const uint32_t* bias_ids;
  const float* bias_values;
  const uint32_t* ban_ids;
  const uint32_t* mask;
  int64_t mask_ld;
  uint32_t* history;
  int64_t history_ld;
  uint32_t* history_len;
  uint32_t history_cap;
  const float* uniforms;
  uint64_t* rng_state;
  float* mu;
  uint32_t* out_tokens;
  int32_t* out_status;
  uint32_t* out_kept_count;
  uint32_t* out_kept_ids;
  float* out_kept_probs;
  int64_t kept_ld;
  float* logits_out;
  int64_t logits_out_ld;
  // geometry
  uint32_t S;          // chunks per row
  uint32_t CH;         // logits per chunk
  uint32_t cap_w;      // key slots per wavefront
  uint32_t c_w;        // lane maxima per wavefront that set its threshold
  uint32_t grid_real;  // B * S
  uint32_t grid_per_xcd;
  // workspace
  uint64_t* lists;       // [B][S*4][cap_w]
  uint64_t* wave_theta;  // [B][S*4]
  uint32_t* wave_count;  // [B][S*4]
  uint32_t* tickets;     // [B]
};

// ---------------------------------------------------------------- keys

__device__ __forceinline__ float neg_inf() { return -__builtin_inff(); }

// Order-preserving map of a float to uint32 (-0.0 and +0.0 map together, as
// f32::partial_cmp treats them as equal).
__device__ __forceinline__ uint32_t f2ord(float x) {
  uint32_t u = __float_as_uint(x);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float ord2f(uint32_t o) {
  uint32_t u = (o & 0x80000000u) ? (o & 0x7fffffffu) : ~o;
  return __uint_as_float(u);
}
// 0 for values that are not candidates (-inf, NaN: sampler.rs:263), else f2ord.
__device__ __forceinline__ uint32_t cand_key(float x) { return (x > neg_inf()) ? f2ord(x) : 0u; }
__device__ __forceinline__ uint64_t comp_key(uint32_t k, uint32_t idx) {
  return ((uint64_t)k << 32) | (uint64_t)(~idx);
}

// ---------------------------------------------------------------- row setup

// Per-row constants of the pre-softmax stages (sampler.rs:184-254).
struct RowXf {
  bool pen_rep, pen_fp, use_hist, nl_active, any_special, do_temp, dry;
  float rp, fp, pp, nl_pen, inv_temp;
  uint32_t hlen, wstart, wn, nl_id;
  uint32_t bias_off, bias_cnt, ban_off, ban_cnt;
};

__device__ __forceinline__ RowXf make_row_xf(const Params& p, const oxs_sampling_config& c,
                                             uint32_t row) {
  RowXf r;
  uint32_t hlen = (p.history && p.history_len) ? p.history_len[row] : 0u;
  if ((int64_t)hlen > p.history_ld) hlen = (uint32_t)p.history_ld;
  r.hlen = hlen;
  r.rp = c.repeat_penalty;
  r.fp = c.frequency_penalty;
  r.pp = c.presence_penalty;
  r.pen_rep = fabsf(c.repeat_penalty - 1.0f) > 1e-5f && c.repeat_penalty > 0.0f;  // :217
  r.pen_fp = fabsf(c.frequency_penalty) > 1e-5f || fabsf(c.presence_penalty) > 1e-5f;  // :232-233
  r.use_hist = hlen > 0 && (r.pen_rep || r.pen_fp);
  uint32_t wlen = c.repeat_last_n > 0 ? c.repeat_last_n : hlen;  // :209-213
  r.wstart = hlen > wlen ? hlen - wlen : 0u;
  r.wn = hlen - r.wstart;
  r.nl_active = c.penalize_nl != 0 && c.newline_token_id < p.V;  // :196-197
  r.nl_id = c.newline_token_id;
  r.nl_pen = c.newline_penalty;
  r.bias_off = c.bias_offset;
  r.bias_cnt = p.bias_ids ? c.bias_count : 0u;
  r.ban_off = c.ban_offset;
  r.ban_cnt = p.ban_ids ? c.ban_count : 0u;
  r.any_special = r.use_hist || r.bias_cnt > 0 || r.ban_cnt > 0 || r.nl_active;
  r.do_temp = c.temperature > 0.0f && c.mirostat_mode == OXS_MIROSTAT_DISABLED;  // :249
  r.inv_temp = 1.0f / c.temperature;                                               // :250
  r.dry = c.dry_multiplier > 0.0f && hlen > 0;                                     // :203
  return r;
}

// The sparse pre-softmax stages for one flagged logit, in reference order:
// ban (:184-188), bias (:189-193), newline (:196-200), repetition (:217-229),
// frequency/presence (:232-245). Temperature is applied by the caller.
__device__ __noinline__ float apply_special(const Params& p, const RowXf& r, float x,
                                            uint32_t entry, uint32_t idx) {
  if (entry & kBanFlag) x = neg_inf();
  if (entry & kBiasFlag) {
    float b = 0.0f;
    for (uint32_t k = 0; k < r.bias_cnt; ++k)  // last entry for an id wins (HashMap::insert)
      if (p.bias_ids[r.bias_off + k] == idx) b = p.bias_values[r.bias_off + k];
    x += b;
  }
  if (entry & kNlFlag) x -= r.nl_pen;
  uint32_t cnt = entry & kCountMask;
  if (cnt) {
    if (r.pen_rep) x = (x > 0.0f) ? x / r.rp : x * r.rp;
    if (r.pen_fp) {
      float t = (float)cnt * r.fp;
      float pen = t + r.pp;
      x = x - pen;
    }
  }
  return x;
}

// Builds the penalty table of logits [c0, c1): window counts in the low bits,
// ban/bias/newline flags in the high bits. Ends with a barrier.
__device__ void build_table(const Params& p, const RowXf& r, uint32_t row, uint32_t c0,
                            uint32_t c1, uint32_t* table) {
  const uint32_t tid = threadIdx.x;
  const uint32_t n = c1 - c0;
  for (uint32_t i = tid * 4; i < n; i += kThreads * 4) {
    *(uint4*)(table + i) = make_uint4(0, 0, 0, 0);
  }
  __syncthreads();
  if (r.use_hist) {
    const uint32_t* h = p.history + (size_t)row * p.history_ld + r.wstart;
    for (uint32_t j = tid; j < r.wn; j += kThreads) {
      uint32_t t = h[j];
      if (t >= c0 && t < c1) atomicAdd(&table[t - c0], 1u);
    }
  }
  for (uint32_t k = tid; k < r.ban_cnt; k += kThreads) {
    uint32_t id = p.ban_ids[r.ban_off + k];
    if (id >= c0 && id < c1) atomicOr(&table[id - c0], kBanFlag);
  }
  for (uint32_t k = tid; k < r.bias_cnt; k += kThreads) {
    uint32_t id = p.bias_ids[r.bias_off + k];
    if (id >= c0 && id < c1) atomicOr(&table[id - c0], kBiasFlag);
  }
  if (tid == 0 && r.nl_active && r.nl_id >= c0 && r.nl_id < c1) atomicOr(&table[r.nl_id - c0], kNlFlag);
  __syncthreads();
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// One logit, scalar path (ragged tails and the exact re-scan).
template <int DT>
__device__ __forceinline__ float load_logit(const Params& p, uint32_t row, uint32_t idx) {
  if (DT == OXS_DTYPE_F32) {
    return ((const float*)p.logits)[(size_t)row * p.ld + idx];
  } else {
    uint16_t b = ((const uint16_t*)p.logits)[(size_t)row * p.ld + idx];
    return __uint_as_float((uint32_t)b << 16);
  }
}

__device__ __forceinline__ bool mask_allows(const Params& p, uint32_t row, uint32_t idx) {
  uint32_t w = p.mask[(size_t)row * p.mask_ld + (idx >> 5)];
  return (w >> (idx & 31)) & 1u;
}

// Full pre-softmax transform of one logit (scalar path).
template <int DT>
__device__ __forceinline__ float transformed_logit(const Params& p, const RowXf& r, uint32_t row,
                                                   uint32_t idx, uint32_t c0,
                                                   const uint32_t* table) {
  float x = load_logit<DT>(p, row, idx);
  if (p.mask && !mask_allows(p, row, idx)) x = neg_inf();
  if (r.any_special) {
    uint32_t e = table[idx - c0];
    if (e) x = apply_special(p, r, x, e, idx);
  }
  if (r.do_temp) x *= r.inv_temp;
  return x;
}

// ---------------------------------------------------------------- block helpers

struct TailShared;  // fwd

__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Exclusive prefix sum over the block; *total gets the block sum.
__device__ uint32_t block_excl_scan(uint32_t v, uint32_t* total, uint32_t* scratch) {
  const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  uint32_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    uint32_t y = __shfl_up(x, o, 64);
    if (lane >= (uint32_t)o) x += y;
  }
  if (lane == 63) scratch[w] = x;
  __syncthreads();
  uint32_t before = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < kWavesPerBlock; ++i) {
    uint32_t s = scratch[i];
    if ((uint32_t)i < w) before += s;
    tot += s;
  }
  __syncthreads();
  *total = tot;
  return x - v + before;
}

__device__ uint64_t block_max_u64(uint64_t v, uint64_t* scratch) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint64_t y = __shfl_xor(v, o, 64);
    v = y > v ? y : v;
  }
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  uint64_t m = scratch[0];
#pragma unroll
  for (int i = 1; i < kWavesPerBlock; ++i) m = scratch[i] > m ? scratch[i] : m;
  __syncthreads();
  return m;
}

__device__ uint64_t block_min_u64(uint64_t v, uint64_t* scratch) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint64_t y = __shfl_xor(v, o, 64);
    v = y < v ? y : v;
  }
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  uint64_t m = scratch[0];
#pragma unroll
  for (int i = 1; i < kWavesPerBlock; ++i) m = scratch[i] < m ? scratch[i] : m;
  __syncthreads();
  return m;
}

struct TailShared {
  uint32_t hist[256];
  uint32_t woff[kMaxChunks * kWavesPerBlock];
  uint32_t wcnt[kMaxChunks * kWavesPerBlock];
  uint32_t scan_scratch[8];
  uint64_t red_scratch[8];
  uint32_t sel_digit, sel_above, sel_count, counter;
  uint32_t n, status, token;
  float inv;
};

// Radix-select step: given a histogram of the next digit among keys matching
// the current prefix, finds the digit holding the kk-th largest key.
__device__ void find_digit(TailShared& ts, uint32_t kk) {
  const uint32_t t = threadIdx.x;
  const uint32_t d = 255u - t;
  uint32_t h = ts.hist[d];
  uint32_t tot;
  uint32_t above = block_excl_scan(h, &tot, ts.scan_scratch);
  if (above < kk && kk <= above + h) {
    ts.sel_digit = d;
    ts.sel_above = above;
    ts.sel_count = h;
  }
  __syncthreads();
}

// The k-th largest of n distinct keys in LDS (1 <= k <= n).
__device__ uint64_t kth_largest(const uint64_t* keys, uint32_t n, uint32_t k, TailShared& ts) {
  const uint32_t tid = threadIdx.x;
  uint64_t prefix = 0, mask = 0;
  uint32_t kk = k;
  for (int d = 0; d < 8; ++d) {
    const int shift = 56 - 8 * d;
    ts.hist[tid] = 0;
    __syncthreads();
    for (uint32_t i = tid; i < n; i += kThreads) {
      uint64_t key = keys[i];
      if ((key & mask) == prefix) atomicAdd(&ts.hist[(uint32_t)(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    find_digit(ts, kk);
    prefix |= (uint64_t)ts.sel_digit << shift;
    mask |= 0xffull << shift;
    kk -= ts.sel_above;
    const uint32_t cnt = ts.sel_count;
    __syncthreads();
    if (cnt == kk) {  // every key of this bucket is in: the k-th is the bucket minimum
      uint64_t mn = ~0ull;
      for (uint32_t i = tid; i < n; i += kThreads) {
        uint64_t key = keys[i];
        if ((key & mask) == prefix && key < mn) mn = key;
      }
      return block_min_u64(mn, ts.red_scratch);
    }
  }
  return prefix;
}

// Sorts n keys in LDS descending (ascending if ASC), padding to a power of two.
template <bool ASC>
__device__ void bitonic_sort(uint64_t* a, uint32_t n) {
  const uint32_t tid = threadIdx.x;
  uint32_t n2 = 1;
  while (n2 < n) n2 <<= 1;
  const uint64_t pad = ASC ? ~0ull : 0ull;
  for (uint32_t i = n + tid; i < n2; i += kThreads) a[i] = pad;
  __syncthreads();
  for (uint32_t k = 2; k <= n2; k <<= 1) {
    for (uint32_t j = k >> 1; j > 0; j >>= 1) {
      for (uint32_t i = tid; i < n2; i += kThreads) {
        uint32_t ixj = i ^ j;
        if (ixj > i) {
          uint64_t x = a[i], y = a[ixj];
          bool second_half = (i & k) != 0;
          bool swap = ASC ? (second_half ? (x < y) : (x > y)) : (second_half ? (x > y) : (x < y));
          if (swap) {
            a[i] = y;
            a[ixj] = x;
          }
        }
      }
      __syncthreads();
    }
  }
}

// Exact top-M of a whole row without the phase-A candidate sets: a radix
// select over all V keys, re-reading the row once per digit. Used only when
// the candidate union cannot be proven to hold the row's top M. Writes the
// top min(M, pool) keys to out (unordered); returns that count.
template <int DT>
__device__ uint32_t exact_select_row(const Params& p, const RowXf& r, uint32_t row, uint32_t M,
                                     uint32_t* table, uint64_t* out, TailShared& ts) {
  const uint32_t tid = threadIdx.x;
  uint64_t prefix = 0, mask = 0;
  uint32_t kk = 0, meff = 0;
  bool done = false;
  for (int d = 0; d < 8 && !done; ++d) {
    const int shift = 56 - 8 * d;
    ts.hist[tid] = 0;
    __syncthreads();
    for (uint32_t c = 0; c < p.S; ++c) {
      const uint32_t c0 = c * p.CH;
      const uint32_t c1 = min(c0 + p.CH, p.V);
      if (r.any_special) build_table(p, r, row, c0, c1, table);
      for (uint32_t i = c0 + tid; i < c1; i += kThreads) {
        uint32_t k = cand_key(transformed_logit<DT>(p, r, row, i, c0, table));
        if (!k) continue;
        uint64_t key = comp_key(k, i);
        if ((key & mask) == prefix) atomicAdd(&ts.hist[(uint32_t)(key >> shift) & 255u], 1u);
      }
      __syncthreads();
    }
    if (d == 0) {
      uint32_t pool;
      block_excl_scan(ts.hist[tid], &pool, ts.scan_scratch);
      meff = min(M, pool);
      kk = meff;
      if (meff == 0) return 0;
    }
    find_digit(ts, kk);
    prefix |= (uint64_t)ts.sel_digit << shift;
    mask |= 0xffull << shift;
    kk -= ts.sel_above;
    if (ts.sel_count == kk) done = true;  // the whole bucket is in
    __syncthreads();
  }
  // Collect every key whose leading digits reach the selected bucket.
  if (tid == 0) ts.counter = 0;
  __syncthreads();
  for (uint32_t c = 0; c < p.S; ++c) {
    const uint32_t c0 = c * p.CH;
    const uint32_t c1 = min(c0 + p.CH, p.V);
    if (r.any_special) build_table(p, r, row, c0, c1, table);
    for (uint32_t i = c0 + tid; i < c1; i += kThreads) {
      uint32_t k = cand_key(transformed_logit<DT>(p, r, row, i, c0, table));
      if (!k) continue;
      uint64_t key = comp_key(k, i);
      if ((key & mask) >= prefix) {
        uint32_t pos = atomicAdd(&ts.counter, 1u);
        if (pos < (uint32_t)kMaxM) out[pos] = key;
      }
    }
    __syncthreads();
  }
  return meff;
}

// ---------------------------------------------------------------- tail math

using oxs_libm::expf_t;
using oxs_libm::log2f_t;
using oxs_libm::logf_t;
__device__ __forceinline__ float dexpf(float x) { return expf_t<true>(x); }
__device__ __forceinline__ float dlogf(float x) { return logf_t<true>(x); }
__device__ __forceinline__ float dlog2f(float x) { return log2f_t<true>(x); }

__device__ __forceinline__ float next_f32(uint64_t* s) {  // sampler.rs:139-153
  uint64_t x = *s;
  x ^= x << 13;
  x ^= x >> 7;
  x ^= x << 17;
  *s = x;
  uint32_t val = (uint32_t)(x >> 40);
  return (float)val / 16777216.0f;
}

// The post-top-M chain of sampler.rs:286-389 for one row. keys[0..n) are
// sorted descending. LDS scratch: ids/pr/aux each kMaxM entries.
__device__ void tail_chain(const Params& p, const oxs_sampling_config& c, uint32_t row,
                           uint64_t* keys, uint32_t n, uint32_t* ids, float* pr, uint64_t* aux,
                           TailShared& ts) {
  const uint32_t tid = threadIdx.x;
  // Softmax over the n kept candidates (:286-295).
  for (uint32_t i = tid; i < n; i += kThreads) {
    uint64_t k = keys[i];
    ids[i] = ~(uint32_t)k;
    pr[i] = ord2f((uint32_t)(k >> 32));
  }
  __syncthreads();
  const float max_logit = pr[0];
  __syncthreads();
  for (uint32_t i = tid; i < n; i += kThreads) pr[i] = dexpf(pr[i] - max_logit);
  __syncthreads();
  if (tid == 0) {
    float sum_exp = 0.0f;
    for (uint32_t i = 0; i < n; ++i) sum_exp += pr[i];
    ts.inv = sum_exp > 0.0f ? 1.0f / sum_exp : 1.0f;
  }
  __syncthreads();
  const float inv_sum = ts.inv;
  for (uint32_t i = tid; i < n; i += kThreads) pr[i] *= inv_sum;
  __syncthreads();

  const bool record = (p.flags & OXS_FLAG_RECORD_HISTORY) != 0;
  uint32_t len = n;  // current candidate count (list lives in ids/pr[0..len))
  uint32_t token = 0;
  uint32_t n_record = 1;

  if (c.mirostat_mode == OXS_MIROSTAT_V1 || c.mirostat_mode == OXS_MIROSTAT_V2) {
    if (tid == 0) {
      float mu = p.mu[row];
      if (c.mirostat_mode == OXS_MIROSTAT_V1) {  // :418-429
        float prob = fmaxf(pr[0], 1e-6f);
        float surprise = -dlog2f(prob);
        float error = surprise - c.mirostat_tau;
        float step = c.mirostat_eta * error;
        mu -= step;
      } else {  // :432-456
        float max_surprise = mu;
        float cum_prob = 0.0f;
        for (uint32_t i = 0; i < n; ++i) {
          float surprise = -dlog2f(fmaxf(pr[i], 1e-8f));
          if (surprise > max_surprise && i > 0) break;
          cum_prob += pr[i];
        }
        float prob = pr[0] / fmaxf(cum_prob, 1e-6f);
        float surprise = -dlog2f(fmaxf(prob, 1e-8f));
        float error = surprise - c.mirostat_tau;
        float step = c.mirostat_eta * error;
        mu -= step;
      }
      p.mu[row] = mu;
      ts.token = ids[0];
      ts.n = n;
    }
    n_record = 2;  // recorded inside the mode function and by the caller (:301, :307)
  } else {
    if (tid == 0) {
      uint32_t start = 0;
      // Min-p (:315-319): keep p >= p_max * min_p, in order.
      if (c.min_p > 0.0f && len > 0) {
        float threshold = pr[0] * c.min_p;
        uint32_t w = 0;
        for (uint32_t i = 0; i < len; ++i) {
          if (pr[i] >= threshold) {
            pr[w] = pr[i];
            ids[w] = ids[i];
            ++w;
          }
        }
        len = w;
      }
      // XTC (:322-328).
      if (c.xtc_probability > 0.0f && len > 1) {
        float p_max = pr[0];
        if (p_max >= c.xtc_threshold && p_max < 0.98f) start = 1;
      }
      uint32_t cnt = len - start;
      // Top-k (:331-333).
      if (c.top_k > 0 && cnt > c.top_k) cnt = c.top_k;
      // Tail-free (:336-338, :459-490).
      if (c.tfs_z < 1.0f && cnt > 2) {
        const float* q = pr + start;
        float sum_d2 = 0.0f;
        for (uint32_t i = 0; i + 2 < cnt; ++i) {
          float d1a = q[i] - q[i + 1];
          float d1b = q[i + 1] - q[i + 2];
          sum_d2 += fabsf(d1a - d1b);
        }
        if (sum_d2 > 0.0f) {
          float inv = 1.0f / sum_d2;
          float cum = 0.0f;
          uint32_t cutoff = cnt;
          for (uint32_t i = 0; i + 2 < cnt; ++i) {
            float d1a = q[i] - q[i + 1];
            float d1b = q[i + 1] - q[i + 2];
            float t = fabsf(d1a - d1b) * inv;
            cum += t;
            if (cum >= c.tfs_z) {
              cutoff = i + 1;
              break;
            }
          }
          cnt = cutoff > 1 ? cutoff : 1;
        }
      }
      // Compact to [0, cnt) for the stages that follow.
      if (start) {
        for (uint32_t i = 0; i < cnt; ++i) {
          pr[i] = pr[i + start];
          ids[i] = ids[i + start];
        }
      }
      ts.n = cnt;
    }
    __syncthreads();
    len = ts.n;
    // Locally typical (:341-343, :493-520): stable sort by |surprisal - H|.
    if (c.typical_p < 1.0f && len > 1) {
      if (tid == 0) {
        float entropy = -0.0f;
        for (uint32_t i = 0; i < len; ++i) {
          float term = pr[i] > 0.0f ? (-pr[i]) * dlogf(pr[i]) : 0.0f;
          entropy += term;
        }
        ts.inv = entropy;
      }
      __syncthreads();
      const float entropy = ts.inv;
      for (uint32_t i = tid; i < len; i += kThreads) {
        float surprisal = pr[i] > 0.0f ? -dlogf(pr[i]) : 0.0f;
        float diff = fabsf(surprisal - entropy);
        aux[i] = ((uint64_t)f2ord(diff) << 32) | i;  // ascending score, then position
      }
      __syncthreads();
      bitonic_sort<true>(aux, len);
      // Gather into keys[] as (id, p) pairs, then back.
      for (uint32_t i = tid; i < len; i += kThreads) {
        uint32_t src = (uint32_t)aux[i];
        keys[i] = ((uint64_t)ids[src] << 32) | __float_as_uint(pr[src]);
      }
      __syncthreads();
      for (uint32_t i = tid; i < len; i += kThreads) {
        ids[i] = (uint32_t)(keys[i] >> 32);
        pr[i] = __uint_as_float((uint32_t)keys[i]);
      }
      __syncthreads();
      if (tid == 0) {
        float cum = 0.0f;
        uint32_t keep = len;
        for (uint32_t i = 0; i < len; ++i) {
          cum += pr[i];
          if (cum >= c.typical_p) {
            keep = i + 1;
            break;
          }
        }
        ts.n = keep;
      }
      __syncthreads();
      len = ts.n;
    }
    if (tid == 0) {
      // Top-p (:346-357).
      if (c.top_p < 1.0f) {
        float cumulative = 0.0f;
        uint32_t cut = len;
        for (uint32_t i = 0; i < len; ++i) {
          cumulative += pr[i];
          if (cumulative >= c.top_p) {
            cut = i + 1;
            break;
          }
        }
        len = cut;
      }
      // Renormalise (:360-368).
      float total = -0.0f;
      for (uint32_t i = 0; i < len; ++i) total += pr[i];
      float inv_total = total > 0.0f ? 1.0f / total : 1.0f;
      for (uint32_t i = 0; i < len; ++i) pr[i] *= inv_total;
      // Draw (:371-385).
      uint32_t picked;
      if (c.temperature <= 1e-6f) {
        picked = len ? ids[0] : 0u;
      } else {
        float r;
        if (p.uniforms) {
          r = p.uniforms[row];
        } else {
          uint64_t s = p.rng_state[row];
          r = next_f32(&s);
          p.rng_state[row] = s;
        }
        float acc = 0.0f;
        uint32_t selected = len ? ids[0] : 0u;
        for (uint32_t i = 0; i < len; ++i) {
          acc += pr[i];
          if (r <= acc) {
            selected = ids[i];
            break;
          }
        }
        picked = selected;
      }
      ts.token = picked;
      ts.n = len;
    }
  }
  __syncthreads();
  token = ts.token;
  len = ts.n;
  // Outputs: token, status, history, candidates_buffer.
  if (tid == 0) {
    int32_t status = OXS_ROW_OK;
    if (record) {
      uint32_t hl = p.history_len[row];
      for (uint32_t k = 0; k < n_record; ++k) {
        if (hl < p.history_cap) {
          p.history[(size_t)row * p.history_ld + hl] = token;
          ++hl;
        } else {
          status = OXS_ROW_HISTORY_FULL;
        }
      }
      p.history_len[row] = hl;
    }
    p.out_tokens[row] = token;
    if (p.out_status) p.out_status[row] = status;
    if (p.out_kept_count) p.out_kept_count[row] = len;
  }
  const uint32_t nk = (uint32_t)min((int64_t)len, p.kept_ld);
  for (uint32_t i = tid; i < nk; i += kThreads) {
    if (p.out_kept_ids) p.out_kept_ids[(size_t)row * p.kept_ld + i] = ids[i];
    if (p.out_kept_probs) p.out_kept_probs[(size_t)row * p.kept_ld + i] = pr[i];
  }
}

__device__ void write_row_result(const Params& p, uint32_t row, uint32_t token, int32_t status) {
  if (threadIdx.x == 0) {
    p.out_tokens[row] = token;
    if (p.out_status) p.out_status[row] = status;
    if (p.out_kept_count) p.out_kept_count[row] = 0;
  }
}

// ---------------------------------------------------------------- kernel

template <int DT, int SLOTS, bool VEC>
__global__ __launch_bounds__(kThreads) void sample_kernel(const Params p) {
  constexpr int EPL = (DT == OXS_DTYPE_F32) ? 4 : 8;  // logits per 16-byte load
  constexpr int TILE = kThreads * EPL;
  constexpr int CH = SLOTS * TILE;
  constexpr size_t ESZ = (DT == OXS_DTYPE_F32) ? 4 : 2;
  static_assert(CH <= kMaxChunk, "chunk exceeds the LDS penalty table");

  __shared__ __align__(16) uint64_t smem_a[kUnionMax];  // penalty table, candidate union, tail arrays
  __shared__ __align__(16) uint64_t smem_keys[kMaxM];   // sorted top-M keys
  __shared__ TailShared ts;
  __shared__ uint32_t s_last;

  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63;
  const uint32_t wave = tid >> 6;
  // XCD-aware numbering: hardware round-robins workgroups over the 8 XCDs, so
  // give each XCD a contiguous range of (row, chunk) ids; a row's chunks then
  // share one L2.
  const uint32_t vid = (blockIdx.x & 7u) * p.grid_per_xcd + (blockIdx.x >> 3);
  if (vid >= p.grid_real) return;
  const uint32_t row = vid / p.S;
  const uint32_t chunk = vid - row * p.S;
  const oxs_sampling_config c = p.configs[(p.flags & OXS_FLAG_SHARED_CONFIG) ? 0 : row];
  const RowXf r = make_row_xf(p, c, row);
  uint32_t* table = (uint32_t*)smem_a;

  const uint32_t c0 = chunk * CH;
  const uint32_t c1 = min(c0 + (uint32_t)CH, p.V);
  const bool full = (c1 - c0) == (uint32_t)CH;

  // ---- issue every load of this block's chunk
  uint32_t raw[SLOTS][EPL];
  uint32_t mw[SLOTS];
#pragma unroll
  for (int s = 0; s < SLOTS; ++s) mw[s] = 0u;
  const char* rowp = (const char*)p.logits + (size_t)row * (size_t)p.ld * ESZ;
  if (VEC && full) {
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
      const uint32_t base = c0 + s * TILE + tid * EPL;
      const u32x4 q = __builtin_nontemporal_load((const u32x4*)(rowp + (size_t)base * ESZ));
      if constexpr (DT == OXS_DTYPE_F32) {
        raw[s][0] = q.x; raw[s][1] = q.y; raw[s][2] = q.z; raw[s][3] = q.w;
      } else {
        raw[s][0] = q.x << 16; raw[s][1] = q.x & 0xffff0000u;
        raw[s][2] = q.y << 16; raw[s][3] = q.y & 0xffff0000u;
        raw[s][4] = q.z << 16; raw[s][5] = q.z & 0xffff0000u;
        raw[s][6] = q.w << 16; raw[s][7] = q.w & 0xffff0000u;
      }
    }
  } else {
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const uint32_t idx = c0 + s * TILE + tid * EPL + e;
        raw[s][e] = idx < c1 ? __float_as_uint(load_logit<DT>(p, row, idx)) : 0xff800000u;
      }
    }
  }
  if (p.mask) {
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
      const uint32_t base = c0 + s * TILE + tid * EPL;
      mw[s] = base < c1 ? p.mask[(size_t)row * p.mask_ld + (base >> 5)] : 0u;
    }
  }
  if (r.any_special) build_table(p, r, row, c0, c1, table);

  // ---- transform in registers, track the lane maximum key
  uint32_t key[SLOTS][EPL];
  uint32_t lane_max = 0;
#pragma unroll
  for (int s = 0; s < SLOTS; ++s) {
    const uint32_t base = c0 + s * TILE + tid * EPL;
    uint32_t ent[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) ent[e] = 0;
    if (r.any_special && base < c1) {
      if (base + EPL <= c1) {
#pragma unroll
        for (int e = 0; e < EPL; e += 4) {
          uint4 t4 = *(const uint4*)(table + (base - c0) + e);
          ent[e] = t4.x; ent[e + 1] = t4.y; ent[e + 2] = t4.z; ent[e + 3] = t4.w;
        }
      } else {
#pragma unroll
        for (int e = 0; e < EPL; ++e)
          if (base + e < c1) ent[e] = table[base - c0 + e];
      }
    }
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const uint32_t idx = base + e;
      float x = __uint_as_float(raw[s][e]);
      if (p.mask && !((mw[s] >> (idx & 31)) & 1u)) x = neg_inf();
      if (ent[e]) x = apply_special(p, r, x, ent[e], idx);
      if (r.do_temp) x *= r.inv_temp;
      if (p.logits_out && idx < c1) p.logits_out[(size_t)row * p.logits_out_ld + idx] = x;
      uint32_t k = (idx < c1) ? cand_key(x) : 0u;
      key[s][e] = k;
      lane_max = k > lane_max ? k : lane_max;
    }
  }

  // ---- wavefront threshold: the c_w-th largest lane maximum
  uint32_t theta = 0;
#pragma unroll 1
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t trial = theta | (1u << bit);
    if ((uint32_t)__popcll(__ballot(lane_max >= trial)) >= p.c_w) theta = trial;
  }
  uint32_t my_cnt = 0;
#pragma unroll
  for (int s = 0; s < SLOTS; ++s)
#pragma unroll
    for (int e = 0; e < EPL; ++e) my_cnt += (key[s][e] != 0u && key[s][e] >= theta) ? 1u : 0u;
  const uint32_t wave_cnt = wave_sum_u32(my_cnt);
  const uint32_t W = p.S * kWavesPerBlock;
  const size_t wslot = (size_t)row * W + (size_t)chunk * kWavesPerBlock + wave;
  uint64_t* out = p.lists + wslot * p.cap_w;
  uint64_t wtheta;
  uint32_t emitted;
  if (wave_cnt <= p.cap_w) {
    uint32_t pos = 0;
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const uint32_t k = key[s][e];
        const bool surv = k != 0u && k >= theta;
        const uint64_t bal = __ballot(surv);
        if (surv) {
          const uint32_t below = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                           __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
          out[pos + below] = comp_key(k, c0 + s * TILE + tid * EPL + e);
        }
        pos += (uint32_t)__popcll(bal);
      }
    }
    wtheta = (uint64_t)theta << 32;  // every key >= (theta, any id) was written
    emitted = wave_cnt;
  } else {
    wtheta = ~0ull;  // overflow: prove nothing, force the exact path
    emitted = 0;
  }
  if (lane == 0) {
    p.wave_theta[wslot] = wtheta;
    p.wave_count[wslot] = emitted;
  }

  // ---- last block of the row runs the tail
  __syncthreads();
  if (tid == 0) {
    __threadfence();
    const uint32_t prev = __hip_atomic_fetch_add(&p.tickets[row], 1u, __ATOMIC_ACQ_REL,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    const bool last = prev == p.S - 1;
    if (last) p.tickets[row] = 0u;  // ready for the next launch
    s_last = last ? 1u : 0u;
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();

  // Rows that ask for stages not run on the device fail loudly.
  const uint32_t M = max(c.top_k, 256u);
  if (r.dry || M > (uint32_t)kMaxM) {
    write_row_result(p, row, 0u, OXS_ROW_UNSUPPORTED);
    return;
  }
  if (c.mirostat_mode != OXS_MIROSTAT_DISABLED && !p.mu) {
    write_row_result(p, row, 0u, OXS_ROW_MISSING_STATE);
    return;
  }

  // 1. wavefront metadata: offsets of each wavefront's keys, largest threshold.
  uint32_t wc = 0;
  uint64_t wt = 0;
  if (tid < W) {
    wc = p.wave_count[(size_t)row * W + tid];
    wt = p.wave_theta[(size_t)row * W + tid];
  }
  uint32_t total;
  const uint32_t woff = block_excl_scan(wc, &total, ts.scan_scratch);
  const uint64_t theta_max = block_max_u64(wt, ts.red_scratch);
  if (tid < W) {
    ts.woff[tid] = woff;
    ts.wcnt[tid] = wc;
  }
  __syncthreads();
  // 2. gather the union into LDS
  uint64_t* U = smem_a;
  const uint32_t span = W * p.cap_w;
  for (uint32_t i = tid; i < span; i += kThreads) {
    const uint32_t w = i / p.cap_w, j = i - w * p.cap_w;
    if (j < ts.wcnt[w]) U[ts.woff[w] + j] = p.lists[((size_t)row * W + w) * p.cap_w + j];
  }
  __syncthreads();

  // 3. the exact top min(M, pool)
  uint32_t meff;
  bool exact = false;
  uint64_t km = 1;
  if (total >= M) {
    km = kth_largest(U, total, M, ts);
    meff = M;
    exact = theta_max > km;
  } else {
    meff = total;
    exact = theta_max != 0;
  }
  if (exact) {
    meff = exact_select_row<DT>(p, r, row, M, (uint32_t*)smem_a, smem_keys, ts);
  } else {
    if (tid == 0) ts.counter = 0;
    __syncthreads();
    for (uint32_t i = tid; i < total; i += kThreads) {
      const uint64_t k = U[i];
      if (k >= km) {
        const uint32_t pos = atomicAdd(&ts.counter, 1u);
        if (pos < (uint32_t)kMaxM) smem_keys[pos] = k;
      }
    }
    __syncthreads();
  }
  if (meff == 0) {  // every logit -inf or NaN (:267-270)
    write_row_result(p, row, 0u, OXS_ROW_EMPTY);
    return;
  }
  bitonic_sort<false>(smem_keys, meff);

  // 4. the chain after the top-M selection
  uint32_t* ids = (uint32_t*)smem_a;
  float* pr = (float*)(ids + kMaxM);
  uint64_t* aux = (uint64_t*)(pr + kMaxM);
  tail_chain(p, c, row, smem_keys, meff, ids, pr, aux, ts);
}

// ---------------------------------------------------------------- host side

struct Geometry {
  int slots;
  uint32_t S, CH, cap_w, c_w;
};

static uint32_t floor_pow2(uint32_t x) {
  uint32_t r = 1;
  while (r * 2 <= x) r *= 2;
  return r;
}

// Chunking: the largest per-block tile count that still gives >= 1024 blocks
// (enough to cover 256 CUs several times), capped by the LDS table and by
// kMaxChunks per row.
static bool choose_geometry(uint32_t B, uint32_t V, int dtype, Geometry* g) {
  const uint32_t epl = dtype == OXS_DTYPE_F32 ? 4 : 8;
  const uint32_t tile = kThreads * epl;
  int best = -1;
  const char* env = getenv("OXS_SLOTS");
  int forced = env ? atoi(env) : 0;
  for (int slots = 8; slots >= 1; slots >>= 1) {
    uint32_t ch = slots * tile;
    if (ch > (uint32_t)kMaxChunk) continue;
    uint32_t S = (V + ch - 1) / ch;
    if (S > (uint32_t)kMaxChunks) continue;
    if (forced) {
      if (slots == forced) best = slots;
      continue;
    }
    best = slots;  // smaller slots keep overwriting while the grid stays small
    if ((uint64_t)B * S >= 1024) break;
  }
  if (best < 0) return false;
  g->slots = best;
  g->CH = best * tile;
  g->S = (V + g->CH - 1) / g->CH;
  const uint32_t W = g->S * kWavesPerBlock;
  g->cap_w = floor_pow2(min(64u, (uint32_t)kUnionMax / W));
  uint32_t c = (3u * 256u + W - 1) / W + 6u;
  g->c_w = max(1u, min(g->cap_w / 2, c));
  return true;
}

template <int DT, int SLOTS, bool VEC>
static hipError_t launch_t(const Params& p, hipStream_t st) {
  const uint32_t grid = 8u * p.grid_per_xcd;
  hipLaunchKernelGGL((sample_kernel<DT, SLOTS, VEC>), dim3(grid), dim3(kThreads), 0, st, p);
  return hipGetLastError();
}

template <int DT, bool VEC>
static hipError_t launch_slots(int slots, const Params& p, hipStream_t st) {
  switch (slots) {
    case 8:
      if constexpr (DT == OXS_DTYPE_F32) return launch_t<DT, 8, VEC>(p, st);
      return hipErrorInvalidValue;  // bf16 chunks stop at 4 slots (8192 logits)
    case 4: return launch_t<DT, 4, VEC>(p, st);
    case 2: return launch_t<DT, 2, VEC>(p, st);
    default: return launch_t<DT, 1, VEC>(p, st);
  }
}

}  // namespace oxs

// ---------------------------------------------------------------- C ABI

struct oxs_sampler {
  int device;
  oxs_limits limits;
  uint64_t* lists;
  uint64_t* wave_theta;
  uint32_t* wave_count;
  uint32_t* tickets;
  size_t bytes;
};

extern "C" {

uint32_t oxs_abi_version(void) { return OXS_ABI_VERSION; }

const char* oxs_status_string(int code) {
  switch (code) {
    case OXS_OK: return "ok";
    case OXS_ERR_INVALID_ARGUMENT: return "invalid argument";
    case OXS_ERR_SHAPE_MISMATCH: return "tensor shape or dimension mismatch";
    case OXS_ERR_LIMITS: return "batch exceeds the sampler's create-time limits";
    case OXS_ERR_HIP: return "HIP runtime error";
    case OXS_ERR_UNSUPPORTED: return "unsupported on this device";
    case OXS_ERR_NO_DEVICE: return "no HIP device";
    default: return "unknown status";
  }
}

void oxs_sampling_config_default(oxs_sampling_config* c) {  // sampler.rs:44-73
  if (!c) return;
  memset(c, 0, sizeof(*c));
  c->temperature = 0.8f;
  c->top_k = 40;
  c->top_p = 0.95f;
  c->min_p = 0.05f;
  c->tfs_z = 1.0f;
  c->typical_p = 1.0f;
  c->xtc_threshold = 0.1f;
  c->xtc_probability = 0.0f;
  c->mirostat_mode = OXS_MIROSTAT_DISABLED;
  c->mirostat_tau = 5.0f;
  c->mirostat_eta = 0.1f;
  c->dry_multiplier = 0.0f;
  c->dry_base = 1.75f;
  c->dry_allowed_length = 2;
  c->dry_range = 1024;
  c->repeat_penalty = 1.1f;
  c->repeat_last_n = 64;
  c->frequency_penalty = 0.0f;
  c->presence_penalty = 0.0f;
  c->penalize_nl = 0;
  c->newline_penalty = 0.5f;
}

uint64_t oxs_rng_state_from_seed(int has_seed, uint64_t seed) {  // sampler.rs:104-128
  const uint64_t kDefault = 0x853c49e6748fea9bull;
  if (!has_seed) return kDefault;
  return seed == 0 ? kDefault : seed;
}

float oxs_mirostat_mu_from_tau(float tau) { return 2.0f * tau; }

int oxs_sampler_create(oxs_sampler** out, const oxs_limits* limits, int device) {
  if (!out || !limits || limits->max_batch == 0 || limits->max_vocab == 0) return OXS_ERR_INVALID_ARGUMENT;
  *out = nullptr;
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0) return OXS_ERR_NO_DEVICE;
  if (device < 0 || device >= ndev) return OXS_ERR_INVALID_ARGUMENT;
  const uint32_t mtk = limits->max_top_k ? limits->max_top_k : 256u;
  if (mtk > (uint32_t)oxs::kMaxM) return OXS_ERR_LIMITS;
  if ((uint64_t)limits->max_vocab > (uint64_t)oxs::kMaxChunks * oxs::kMaxChunk) return OXS_ERR_LIMITS;
  if (hipSetDevice(device) != hipSuccess) return OXS_ERR_HIP;
  oxs_sampler* s = (oxs_sampler*)calloc(1, sizeof(oxs_sampler));
  if (!s) return OXS_ERR_INVALID_ARGUMENT;
  s->device = device;
  s->limits = *limits;
  s->limits.max_top_k = mtk;
  const size_t B = limits->max_batch;
  const size_t W = (size_t)oxs::kMaxChunks * oxs::kWavesPerBlock;
  const size_t b_lists = B * oxs::kUnionMax * sizeof(uint64_t);
  const size_t b_theta = B * W * sizeof(uint64_t);
  const size_t b_count = B * W * sizeof(uint32_t);
  const size_t b_tick = B * sizeof(uint32_t);
  bool ok = hipMalloc((void**)&s->lists, b_lists) == hipSuccess &&
            hipMalloc((void**)&s->wave_theta, b_theta) == hipSuccess &&
            hipMalloc((void**)&s->wave_count, b_count) == hipSuccess &&
            hipMalloc((void**)&s->tickets, b_tick) == hipSuccess &&
            hipMemset(s->tickets, 0, b_tick) == hipSuccess && hipDeviceSynchronize() == hipSuccess;
  s->bytes = b_lists + b_theta + b_count + b_tick;
  if (!ok) {
    oxs_sampler_destroy(s);
    return OXS_ERR_HIP;
  }
  *out = s;
  return OXS_OK;
}

int oxs_sampler_destroy(oxs_sampler* s) {
  if (!s) return OXS_OK;
  if (s->lists) (void)hipFree(s->lists);
  if (s->wave_theta) (void)hipFree(s->wave_theta);
  if (s->wave_count) (void)hipFree(s->wave_count);
  if (s->tickets) (void)hipFree(s->tickets);
  free(s);
  return OXS_OK;
}

size_t oxs_sampler_workspace_bytes(const oxs_sampler* s) { return s ? s->bytes : 0; }

int oxs_sample_batch(oxs_sampler* s, const oxs_batch* b, void* stream) {
  using namespace oxs;
  if (!s || !b) return OXS_ERR_INVALID_ARGUMENT;
  if (b->vocab == 0) return OXS_ERR_SHAPE_MISMATCH;  // sampler.rs:179-181
  if (b->batch == 0) return OXS_OK;
  if (b->batch > s->limits.max_batch || b->vocab > s->limits.max_vocab) return OXS_ERR_LIMITS;
  if (!b->logits || !b->configs || !b->out_tokens) return OXS_ERR_INVALID_ARGUMENT;
  if (b->logits_dtype != OXS_DTYPE_F32 && b->logits_dtype != OXS_DTYPE_BF16) return OXS_ERR_INVALID_ARGUMENT;
  if (b->logits_ld < (int64_t)b->vocab) return OXS_ERR_INVALID_ARGUMENT;
  if (b->allowed_mask && b->mask_ld < (int64_t)((b->vocab + 31) / 32)) return OXS_ERR_INVALID_ARGUMENT;
  if (!b->uniforms && !b->rng_state) return OXS_ERR_INVALID_ARGUMENT;
  if (b->history && (!b->history_len || b->history_ld <= 0)) return OXS_ERR_INVALID_ARGUMENT;
  if (b->flags & OXS_FLAG_RECORD_HISTORY) {
    if (!b->history || !b->history_len || (int64_t)b->history_cap > b->history_ld) return OXS_ERR_INVALID_ARGUMENT;
  }
  if ((b->out_kept_ids || b->out_kept_probs) && b->kept_ld <= 0) return OXS_ERR_INVALID_ARGUMENT;
  if ((b->bias_ids == nullptr) != (b->bias_values == nullptr)) return OXS_ERR_INVALID_ARGUMENT;
  if (b->logits_out) {
    if (b->logits_out_ld < (int64_t)b->vocab) return OXS_ERR_INVALID_ARGUMENT;
    const size_t esz_in = b->logits_dtype == OXS_DTYPE_F32 ? 4 : 2;
    const uintptr_t in_lo = (uintptr_t)b->logits;
    const uintptr_t in_hi = in_lo + ((size_t)(b->batch - 1) * (size_t)b->logits_ld + b->vocab) * esz_in;
    const uintptr_t out_lo = (uintptr_t)b->logits_out;
    const uintptr_t out_hi = out_lo + ((size_t)(b->batch - 1) * (size_t)b->logits_out_ld + b->vocab) * 4;
    if (out_lo < in_hi && in_lo < out_hi) return OXS_ERR_INVALID_ARGUMENT;  // must not overlap
  }

  Geometry g;
  if (!choose_geometry(b->batch, b->vocab, b->logits_dtype, &g)) return OXS_ERR_LIMITS;
  Params p;
  memset(&p, 0, sizeof(p));
  p.logits = b->logits;
  p.ld = b->logits_ld;
  p.B = b->batch;
  p.V = b->vocab;
  p.flags = b->flags;
  p.configs = b->configs;
  p.bias_ids = b->bias_ids;
  p.bias_values = b->bias_values;
  p.ban_ids = b->ban_ids;
  p.mask = b->allowed_mask;
  p.mask_ld = b->mask_ld;
  p.history = b->history;
  p.history_ld = b->history ? b->history_ld : 0;
  p.history_len = b->history ? b->history_len : nullptr;
  p.history_cap = b->history_cap;
  p.uniforms = b->uniforms;
  p.rng_state = b->rng_state;
  p.mu = b->mirostat_mu;
  p.out_tokens = b->out_tokens;
  p.out_status = b->out_status;
  p.out_kept_count = b->out_kept_count;
  p.out_kept_ids = b->out_kept_ids;
  p.out_kept_probs = b->out_kept_probs;
  p.kept_ld = (b->out_kept_ids || b->out_kept_probs) ? b->kept_ld : 0;
  p.logits_out = b->logits_out;
  p.logits_out_ld = b->logits_out_ld;
  p.S = g.S;
  p.CH = g.CH;
  p.cap_w = g.cap_w;
  p.c_w = g.c_w;
  p.grid_real = b->batch * g.S;
  p.grid_per_xcd = (p.grid_real + 7) / 8;
  p.lists = s->lists;
  p.wave_theta = s->wave_theta;
  p.wave_count = s->wave_count;
  p.tickets = s->tickets;

  const size_t esz = b->logits_dtype == OXS_DTYPE_F32 ? 4 : 2;
  const size_t epl = b->logits_dtype == OXS_DTYPE_F32 ? 4 : 8;
  const bool vec = ((uintptr_t)b->logits % 16 == 0) && ((size_t)b->logits_ld % epl == 0) && esz > 0;
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  if (b->logits_dtype == OXS_DTYPE_F32)
    e = vec ? launch_slots<OXS_DTYPE_F32, true>(g.slots, p, st) : launch_slots<OXS_DTYPE_F32, false>(g.slots, p, st);
  else
    e = vec ? launch_slots<OXS_DTYPE_BF16, true>(g.slots, p, st) : launch_slots<OXS_DTYPE_BF16, false>(g.slots, p, st);
  return e == hipSuccess ? OXS_OK : OXS_ERR_HIP;
}

}  // extern "C"
