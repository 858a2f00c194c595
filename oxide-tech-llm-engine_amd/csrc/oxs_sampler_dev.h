// oxs_sampler_dev.h — device code shared by the sampler's kernels: launch
// parameters, order keys, per-row setup, wavefront primitives, the stream
// kernel, and the tail's selection, DRY and chain stages. Included by
// oxs_stream.hip (stream kernel launches), oxs_tail.hip (tail and wide
// kernels) and oxs_sampler.hip (host side), which compile in parallel.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "../../include/oxide_sampler.h"
#include "oxs_libm.h"

namespace oxs {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / 64;
constexpr int kUnionMax = 2048;   // candidate key slots per row
constexpr int kUnionBig = 4096;   // ... for rows of more than 64 wavefront records (V > 16 chunks)
constexpr int kTailArea = 4096;   // 64-bit words of tail LDS shared by the scatter, sort, exact-path table and chain scratch
constexpr int kMaxM = 1024;       // largest max(top_k, 256) run on the device
constexpr int kMaxChunk = 8192;   // logits per stream block (at most) and per exact-path table chunk
constexpr int kMaxChunks = 64;    // chunks per row
constexpr int kBuckets = 256;     // tail counting-sort buckets
constexpr int kRecPer = kMaxChunks * kWavesPerBlock / 64;  // wavefront records per lane a tail wavefront reads
constexpr int kDryMax = 1024;      // longest DRY history slice copied into LDS (longer ones are read in place)
constexpr int kDryHash = 2048;     // DRY id hash slots in LDS (slices of up to kDryMax ids)
constexpr int kDryList = kDryHash;  // entries of a row's DRY list without a global DRY hash (the static workspace)
constexpr int kDryListBig = 8192;   // ... with one, when oxs_limits.max_dry_ids is 0
constexpr int kHistUnroll = 4;    // history-window ids per stream thread read with the logits

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kCountMask = 0x0fffffffu;
constexpr uint32_t kBanFlag = 1u << 28;
constexpr uint32_t kBiasFlag = 1u << 29;
constexpr uint32_t kNlFlag = 1u << 30;
constexpr uint32_t kDryFlag = 1u << 31;  // exact-path table: the id has a DRY value
constexpr uint32_t kFlagDecode = 1u << 31;  // Params.flags: a decode step (oxs_decode_step)

// Kernel kinds (the DT template argument): the logit dtype (OXS_DTYPE_*) plus
// compile-time features, so that launches without a feature carry none of its
// code.
constexpr int kKindSoftcap = 4;  // logits pass through the softcap as they are read
constexpr int kKindDecode = 8;   // tail only: the decode step's bookkeeping
constexpr bool kind_f32(int k) { return (k & 3) == OXS_DTYPE_F32; }
constexpr bool kind_softcap(int k) { return (k & kKindSoftcap) != 0; }
constexpr bool kind_decode(int k) { return (k & kKindDecode) != 0; }

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
  float softcap;  // > 0: logits become softcap * tanh(logit / softcap) as they are read
  // geometry
  uint32_t S;      // chunks per row
  uint32_t CH;     // logits per chunk
  uint32_t cap_w;  // key slots per wavefront (a power of two)
  uint32_t cap_shift;  // log2(cap_w)
  uint32_t c_w;    // lane maxima per wavefront that set its threshold
  uint32_t rpx;    // rows per XCD when rows are grouped by XCD, else 0
  // workspace
  uint64_t* lists;       // [B][S*4][cap_w]
  uint64_t* wave_theta;  // [B][S*4] wavefront records: threshold << 32 | largest key
  uint32_t* wave_count;  // [B][S*4]
  const uint64_t* libm;  // [kLibmWords]: the libm tables (exp2, 1/c, ln c, log2 c) as bit patterns
  uint64_t* dry_list;    // [B][dry_cap]: DRY rows' (id << 32 | value bits), sorted by id
  uint32_t* dry_count;   // [B]
  uint32_t* dry_ghash;   // [B][3][2 * dry_cap] id, count and value slots for slices past kDryMax, or NULL
  uint32_t dry_cap;      // a row's DRY list entries (a power of two)
  // decode step (kFlagDecode): the decode loop's per-row state and host outputs
  uint32_t* dec_token;    // [B] next step's input token
  int32_t* dec_pos;       // [B] position
  uint32_t* dec_count;    // [B] generated count
  uint64_t* host_tokens;  // [B] host memory: (row's step count << 32) | token
  uint32_t* row_steps;    // [B] workspace: decode steps each row has handed to the host
  uint32_t* path_counts;  // [kPathKinds] workspace, or NULL: rows per top-M selection path
  // rows whose M = max(top_k, 256) exceeds kMaxM (the wide kernel), or NULL
  uint64_t* wide_keys;  // [B][wide_n2] a row's top-M keys, then sorted
  uint32_t* wide_arr;   // [B][7 * wide_ld] the chain's arrays of such a row
  uint32_t wide_cap;    // the largest M run (the sampler's max_top_k)
  uint32_t wide_n2;     // a power of two >= wide_cap
  uint32_t wide_ld;     // >= wide_cap + 16, a multiple of 4
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

// Row index of a block under the XCD grouping: the hardware hands workgroups
// to the 8 XCDs round robin, so block i runs on XCD i % 8. With rpx > 0, XCD x
// owns rows [x * rpx, (x + 1) * rpx): the stream blocks and the tail block of a
// row then share one L2.
__device__ __forceinline__ uint32_t grouped_index(uint32_t block, uint32_t per_xcd) {
  return (block & 7u) * per_xcd + (block >> 3);
}

// ---------------------------------------------------------------- row setup

// Per-row constants of the pre-softmax stages (sampler.rs:184-254).
struct RowXf {
  bool pen_rep, pen_fp, use_hist, nl_active, any_special, do_temp, dry;
  float rp, fp, pp, nl_pen, inv_temp, dry_mult, dry_base;
  uint32_t hlen, wstart, wn, nl_id, dry_allowed, dry_range;
  uint32_t bias_off, bias_cnt, ban_off, ban_cnt;
};

// Which optional inputs a launch has (sample_kernel's and stream_kernel's
// `kflags`), so that the row setup needs no kernel-argument load.
constexpr uint32_t kKShared = 1u;   // one config for every row
constexpr uint32_t kKDecode = 2u;   // a decode step (oxs_decode_step)
constexpr uint32_t kKHistory = 4u;  // history and history_len are present
constexpr uint32_t kKBias = 8u;     // bias_ids is present
constexpr uint32_t kKBan = 16u;     // ban_ids is present

// Per-row constants from the config, the history length (clamped to the
// history's row stride) and the launch's presence flags.
__device__ __forceinline__ RowXf make_row_xf(const oxs_sampling_config& c, uint32_t hlen, uint32_t V,
                                             uint32_t history_ld, uint32_t kflags) {
  RowXf r;
  if (!(kflags & kKHistory)) hlen = 0u;
  if (hlen > history_ld) hlen = history_ld;
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
  r.nl_active = c.penalize_nl != 0 && c.newline_token_id < V;  // :196-197
  r.nl_id = c.newline_token_id;
  r.nl_pen = c.newline_penalty;
  r.bias_off = c.bias_offset;
  r.bias_cnt = (kflags & kKBias) ? c.bias_count : 0u;
  r.ban_off = c.ban_offset;
  r.ban_cnt = (kflags & kKBan) ? c.ban_count : 0u;
  r.do_temp = c.temperature > 0.0f && c.mirostat_mode == OXS_MIROSTAT_DISABLED;  // :249
  r.inv_temp = 1.0f / c.temperature;                                               // :250
  r.dry = c.dry_multiplier > 0.0f && hlen > 0;                                     // :203
  r.dry_mult = c.dry_multiplier;
  r.dry_base = c.dry_base;
  r.dry_allowed = c.dry_allowed_length;
  r.dry_range = c.dry_range;
  r.any_special = r.use_hist || r.bias_cnt > 0 || r.ban_cnt > 0 || r.nl_active || r.dry;
  return r;
}

// The launch's presence flags, from its Params.
__device__ __forceinline__ uint32_t launch_kflags(const Params& p) {
  return ((p.flags & OXS_FLAG_SHARED_CONFIG) ? kKShared : 0u) | ((p.flags & kFlagDecode) ? kKDecode : 0u) |
         ((p.history && p.history_len) ? kKHistory : 0u) | (p.bias_ids ? kKBias : 0u) |
         (p.ban_ids ? kKBan : 0u);
}
__device__ __forceinline__ RowXf make_row_xf_h(const Params& p, const oxs_sampling_config& c, uint32_t hlen) {
  return make_row_xf(c, hlen, p.V, (uint32_t)p.history_ld, launch_kflags(p));
}


// The sparse pre-softmax stages for one marked logit, in reference order:
// ban (:184-188), bias (:189-193), newline (:196-200), [DRY (:203-205)],
// repetition (:217-229), frequency/presence (:232-245). Temperature is
// applied by the caller.
__device__ __forceinline__ float special_pre(const uint32_t* bias_ids, const float* bias_values, const RowXf& r,
                                             float x, uint32_t entry, uint32_t idx) {
  if (entry & kBanFlag) x = neg_inf();
  if (entry & kBiasFlag) {
    float b = 0.0f;
    for (uint32_t k = 0; k < r.bias_cnt; ++k)  // the last entry for an id wins (HashMap::insert)
      if (bias_ids[r.bias_off + k] == idx) b = bias_values[r.bias_off + k];
    x += b;
  }
  if (entry & kNlFlag) x -= r.nl_pen;
  return x;
}
__device__ __forceinline__ float special_post(const RowXf& r, float x, uint32_t entry) {
  const uint32_t cnt = entry & kCountMask;
  if (cnt) {
    if (r.pen_rep) x = (x > 0.0f) ? x / r.rp : x * r.rp;
    if (r.pen_fp) {
      const float t = (float)cnt * r.fp;
      const float pen = t + r.pp;
      x = x - pen;
    }
  }
  return x;
}
__device__ __forceinline__ float apply_special(const uint32_t* bias_ids, const float* bias_values,
                                               const RowXf& r, float x, uint32_t entry,
                                               uint32_t idx) {
  return special_post(r, special_pre(bias_ids, bias_values, r, x, entry, idx), entry);
}

// The model's final logit softcap (oxide-backend-cuda/src/lib.rs:3243-3255,
// kernels/vec_ops_activations.cu:131-136), applied to each logit as it is
// read instead of in a pass of its own: cap * tanh(l / cap), with glibc's
// tanhf. Only the softcap kinds of the kernels contain it.
__device__ __forceinline__ float softcap_of(float x, float cap) {
  return cap * oxs_libm::tanhf_fdlibm(x / cap);
}

template <int DT>
__device__ __forceinline__ float load_logit(const Params& p, uint32_t row, uint32_t idx) {
  float x;
  if constexpr (kind_f32(DT)) {
    x = ((const float*)p.logits)[(size_t)row * p.ld + idx];
  } else {
    const uint16_t b = ((const uint16_t*)p.logits)[(size_t)row * p.ld + idx];
    x = __uint_as_float((uint32_t)b << 16);
  }
  if constexpr (kind_softcap(DT)) return softcap_of(x, p.softcap);
  return x;
}

__device__ __forceinline__ bool mask_allows(const Params& p, uint32_t row, uint32_t idx) {
  const uint32_t w = p.mask[(size_t)row * p.mask_ld + (idx >> 5)];
  return (w >> (idx & 31)) & 1u;
}

// ---------------------------------------------------------------- scalar-cache row reads

// The per-row record every lane needs (config, history length, uniform,
// Mirostat mu, xorshift state) is read with scalar loads. Scalar loads count
// on lgkmcnt, so waiting for them never waits for vector loads issued
// earlier, which count on vmcnt in issue order. Loads only: nothing is
// written through the scalar cache.
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x8v __attribute__((ext_vector_type(8)));
typedef uint32_t u32x16v __attribute__((ext_vector_type(16)));
static_assert(sizeof(oxs_sampling_config) == 26 * 4, "SamplingConfig is 26 dwords");

__device__ __forceinline__ uint64_t uniform_addr(const void* ptr) {
  const uint64_t ad = (uint64_t)ptr;
  return ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(ad >> 32)) << 32) |
         (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)ad);
}

struct RowIn {
  oxs_sampling_config cfg;
  uint32_t history_len;
  float uniform;
  float mu;
  uint64_t rng;
  bool raw;  // a decode-step row that takes the argmax of its raw logits
};

// The decode loop's greedy rows (continuous_batching.rs:961-970): a row with
// temperature <= 1e-6 takes the first largest raw logit, with no penalty,
// filter or sampler-state change. That is sample_token with every stage
// disabled and the greedy draw (sampler.rs:371-372): the first candidate of
// the pool sorted by value, then lower index (NaN and -inf are not
// candidates, and a row without candidates gives 0, as the loop's initial
// index does). The caller's state (history, mu, rng, candidates) is left
// untouched.
__device__ __forceinline__ void raw_argmax_config(oxs_sampling_config& c) {
  c.temperature = 0.0f;
  c.top_k = 0;
  c.top_p = 1.0f;
  c.min_p = 0.0f;
  c.tfs_z = 1.0f;
  c.typical_p = 1.0f;
  c.xtc_probability = 0.0f;
  c.mirostat_mode = OXS_MIROSTAT_DISABLED;
  c.dry_multiplier = 0.0f;
  c.repeat_penalty = 1.0f;
  c.frequency_penalty = 0.0f;
  c.presence_penalty = 0.0f;
  c.penalize_nl = 0;
  c.bias_count = 0;
  c.ban_count = 0;
}

// Absent optional inputs read a valid dummy address (the config array) and
// get their defaults.
__device__ __forceinline__ RowIn load_row_in(const Params& p, uint32_t row) {
  const void* dummy = p.configs;
  const uint64_t a_cfg = uniform_addr(p.configs + ((p.flags & OXS_FLAG_SHARED_CONFIG) ? 0 : row));
  const uint64_t a_hl = uniform_addr(p.history_len ? (const void*)(p.history_len + row) : dummy);
  const uint64_t a_u = uniform_addr(p.uniforms ? (const void*)(p.uniforms + row) : dummy);
  const uint64_t a_mu = uniform_addr(p.mu ? (const void*)(p.mu + row) : dummy);
  const uint64_t a_rng = uniform_addr(p.rng_state ? (const void*)(p.rng_state + row) : dummy);
  u32x16v a;
  u32x8v b;
  u32x2v c, rng;
  uint32_t hl, u, mu;
  asm volatile(
      "s_load_dwordx16 %0, %7, 0x0\n\t"
      "s_load_dwordx8 %1, %7, 0x40\n\t"
      "s_load_dwordx2 %2, %7, 0x60\n\t"
      "s_load_dword %3, %8, 0x0\n\t"
      "s_load_dword %4, %9, 0x0\n\t"
      "s_load_dword %5, %10, 0x0\n\t"
      "s_load_dwordx2 %6, %11, 0x0\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&s"(a), "=&s"(b), "=&s"(c), "=&s"(hl), "=&s"(u), "=&s"(mu), "=&s"(rng)
      : "s"(a_cfg), "s"(a_hl), "s"(a_u), "s"(a_mu), "s"(a_rng)
      : "memory");
  uint32_t w[26];
#pragma unroll
  for (int i = 0; i < 16; ++i) w[i] = a[i];
#pragma unroll
  for (int i = 0; i < 8; ++i) w[16 + i] = b[i];
  w[24] = c[0];
  w[25] = c[1];
  RowIn in;
  memcpy(&in.cfg, w, sizeof(in.cfg));
  in.history_len = p.history_len ? hl : 0u;
  in.uniform = p.uniforms ? __uint_as_float(u) : 0.0f;
  in.mu = p.mu ? __uint_as_float(mu) : 0.0f;
  in.rng = p.rng_state ? (((uint64_t)rng[1] << 32) | rng[0]) : 0ull;
  in.raw = (p.flags & kFlagDecode) && in.cfg.temperature <= 1e-6f;  // continuous_batching.rs:961
  if (in.raw) raw_argmax_config(in.cfg);
  return in;
}

// ---------------------------------------------------------------- wavefront and block helpers

// Orders this wavefront's LDS accesses: a wavefront's LDS operations complete in
// issue order, so a fence that stops the compiler from moving memory accesses
// across it is all that one wavefront needs to read what its lanes wrote.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// DPP lane exchanges (gfx9 data-parallel primitives; no LDS traffic).
// CTRL: 0xB1 quad_perm(1,0,3,2) = lane ^ 1, 0x4E quad_perm(2,3,0,1) = lane ^ 2,
// 0x141 row_half_mirror, 0x140 row_mirror, 0x110 + k row_shr:k,
// 0x142 row_bcast:15, 0x143 row_bcast:31.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ uint64_t dpp64(uint64_t v) {
  return ((uint64_t)dpp32<CTRL>((uint32_t)(v >> 32)) << 32) | dpp32<CTRL>((uint32_t)v);
}
__device__ __forceinline__ uint64_t readlane64(uint64_t v, int lane) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), lane);
  return ((uint64_t)hi << 32) | lo;
}
struct MaxOp {
  template <typename T> __device__ T operator()(T a, T b) const { return a > b ? a : b; }
};
struct MinOp {
  template <typename T> __device__ T operator()(T a, T b) const { return a < b ? a : b; }
};
struct AddOp {
  template <typename T> __device__ T operator()(T a, T b) const { return a + b; }
};
// Reduction over the wavefront: lane ^ 1, lane ^ 2, then the mirrors pair each
// quad with its neighbour and each half-row with the other half, so every lane
// holds its 16-lane row's result; the four rows are combined from readlanes.
template <typename Op>
__device__ __forceinline__ uint64_t wave_reduce64(uint64_t v, Op op) {
  v = op(v, dpp64<0xB1>(v));
  v = op(v, dpp64<0x4E>(v));
  v = op(v, dpp64<0x141>(v));
  v = op(v, dpp64<0x140>(v));
  return op(op(readlane64(v, 0), readlane64(v, 16)), op(readlane64(v, 32), readlane64(v, 48)));
}
template <typename Op>
__device__ __forceinline__ uint32_t wave_reduce32(uint32_t v, Op op) {
  v = op(v, dpp32<0xB1>(v));
  v = op(v, dpp32<0x4E>(v));
  v = op(v, dpp32<0x141>(v));
  v = op(v, dpp32<0x140>(v));
  const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 0), r1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 32), r3 = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return op(op(r0, r1), op(r2, r3));
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) { return wave_reduce64(v, MaxOp{}); }
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) { return wave_reduce64(v, MinOp{}); }
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) { return wave_reduce32(v, MaxOp{}); }
// Inclusive prefix sum over the wavefront's lanes: shifts by 1, 2, 4, 8 inside
// each 16-lane row (zeros shifted in), then row totals broadcast forward.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x) {
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xf, 0xf, true);
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xf, 0xf, true);
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xf, 0xf, true);
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xf, 0xf, true);
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xa, 0xf, false);
  x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xc, 0xf, false);
  return x;
}
// Number of set bits of m below this lane.
__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Exclusive prefix sum over the block; *total gets the block sum.
__device__ uint32_t block_excl_scan(uint32_t v, uint32_t* total, uint32_t* scratch) {
  const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint32_t x = wave_incl_scan(v);
  if (lane == 63) scratch[w] = x;
  __syncthreads();
  uint32_t before = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < kWavesPerBlock; ++i) {
    const uint32_t s = scratch[i];
    if ((uint32_t)i < w) before += s;
    tot += s;
  }
  __syncthreads();
  *total = tot;
  return x - v + before;
}

// ---------------------------------------------------------------- marked ids (stream LDS hash)

// A stream block marks the sparse-stage ids of its chunk (history window
// with counts, bans, biases, newline) in an open-addressing LDS hash keyed by
// chunk offset.
constexpr int kHashSlots = 256;
constexpr uint32_t kEmptySlot = 0xffffffffu;
__device__ __forceinline__ uint32_t hash_slot(uint32_t key) { return (key * 0x9e3779b1u) >> 24; }
static_assert(kHashSlots == 256, "hash_slot yields 8 bits");

// Continues an insertion whose home slot held another key; false when full.
__device__ bool hash_insert_from(uint32_t* hkeys, uint32_t* hvals, uint32_t key, uint32_t add, uint32_t orv) {
  uint32_t h = hash_slot(key);
  for (int probe = 0; probe < kHashSlots; ++probe) {
    const uint32_t prev = atomicCAS(&hkeys[h], kEmptySlot, key);
    if (prev == kEmptySlot || prev == key) {
      if (add) atomicAdd(&hvals[h], add);
      if (orv) atomicOr(&hvals[h], orv);
      return true;
    }
    h = (h + 1) & (kHashSlots - 1);
  }
  return false;
}

__device__ __forceinline__ uint32_t hash_lookup(const uint32_t* hkeys, const uint32_t* hvals, uint32_t key) {
  uint32_t h = hash_slot(key);
  for (int probe = 0; probe < kHashSlots; ++probe) {
    const uint32_t k = hkeys[h];
    if (k == key) return hvals[h];
    if (k == kEmptySlot) return 0u;
    h = (h + 1) & (kHashSlots - 1);
  }
  return 0u;
}


// ---------------------------------------------------------------- stream kernel

constexpr uint32_t kMinValidOrd = 0x00800000u;  // f2ord(-FLT_MAX): every candidate key is >= this

// One unit after its logits arrived. The dense stages (grammar mask, end of
// vocabulary) are applied in registers and the values are staged in LDS,
// indexed by chunk offset. When the row has sparse-stage ids (history window,
// bans, biases, newline), one thread per hash slot replaces its id's staged
// value with the exact penalised one and every thread re-reads its values.
// Each wavefront then finds a lower bound of the c_w-th largest of its 64 lane
// maxima and emits every value at or above it as
// (order key of x * inv_temp << 32 | ~token id). Thresholds and comparisons
// use the unscaled values: x -> x * inv_temp is monotone for a finite positive
// scale, and a row with any other scale is sent to the tail's exact path.
template <int DT, int SLOTS, bool VEC, bool MASK, bool WB>
__device__ __forceinline__ void process_unit(const Params& p, uint32_t row, uint32_t chunk, const RowXf& r,
                                             const uint32_t (&raw)[SLOTS][kind_f32(DT) ? 4 : 8],
                                             const uint32_t (&mw)[SLOTS], float* s_x, uint32_t* s_hkeys,
                                             uint32_t* s_hvals, uint32_t* s_full) {
  constexpr int EPL = kind_f32(DT) ? 4 : 8;
  constexpr int TILE = kThreads * EPL;
  constexpr int NE = SLOTS * EPL;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t CH = SLOTS * TILE;
  const uint32_t c0 = chunk * CH;
  const uint32_t c1 = min(c0 + CH, p.V);
  const float inv_t = r.do_temp ? r.inv_temp : 1.0f;
  const bool scale_ok = inv_t > 0.0f && inv_t <= __FLT_MAX__;

  // ---- masked raw logits, staged in LDS at their chunk offsets
  float v[NE];
#pragma unroll
  for (int s = 0; s < SLOTS; ++s) {
    const uint32_t off = s * TILE + tid * EPL;  // chunk-local
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      float x = __uint_as_float(raw[s][e]);
      if (MASK && !((mw[s] >> ((c0 + off + e) & 31)) & 1u)) x = neg_inf();
      if (!VEC && c0 + off + e >= c1) x = neg_inf();
      v[s * EPL + e] = x;
    }
  }
  if (VEC && c1 - c0 < CH) {  // a short last chunk: groups past the end are dropped
#pragma unroll
    for (int s = 0; s < SLOTS; ++s)
      if (c0 + s * TILE + tid * EPL >= c1) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) v[s * EPL + e] = neg_inf();
      }
  }
#pragma unroll
  for (int s = 0; s < SLOTS; ++s)
#pragma unroll
    for (int e = 0; e < EPL; e += 4)
      *(float4*)&s_x[s * TILE + tid * EPL + e] =
          make_float4(v[s * EPL + e], v[s * EPL + e + 1], v[s * EPL + e + 2], v[s * EPL + e + 3]);

  // ---- sparse-stage ids at their exact values (sampler.rs:184-245)
  if (r.any_special) {
    __syncthreads();  // values staged, marks complete
    for (uint32_t h = tid; h < (uint32_t)kHashSlots; h += kThreads) {
      const uint32_t off = s_hkeys[h];
      if (off != kEmptySlot) s_x[off] = apply_special(p.bias_ids, p.bias_values, r, s_x[off], s_hvals[h], c0 + off);
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < SLOTS; ++s)
#pragma unroll
      for (int e = 0; e < EPL; e += 4) {
        const float4 q = *(const float4*)&s_x[s * TILE + tid * EPL + e];
        v[s * EPL + e] = q.x;
        v[s * EPL + e + 1] = q.y;
        v[s * EPL + e + 2] = q.z;
        v[s * EPL + e + 3] = q.w;
      }
  }
  if (WB) {  // what the reference leaves in its logits argument (temperature included)
#pragma unroll
    for (int s = 0; s < SLOTS; ++s)
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const uint32_t idx = c0 + s * TILE + tid * EPL + e;
        if (idx < c1) p.logits_out[(size_t)row * p.logits_out_ld + idx] = v[s * EPL + e] * inv_t;
      }
  }

  // ---- wavefront threshold: a lower bound of the c_w-th largest lane
  // maximum, from the top 16 bits of the order keys
  float lmax = v[0];
#pragma unroll
  for (int i = 1; i < NE; ++i) lmax = fmaxf(lmax, v[i]);  // a NaN only lowers the pruning
  const uint32_t lm = f2ord(lmax);
  uint32_t theta = 0;
#pragma unroll
  for (int bit = 31; bit >= 16; --bit) {
    const uint32_t trial = theta | (1u << bit);
    if ((uint32_t)__popcll(__ballot(lm >= trial)) >= p.c_w) theta = trial;
  }
  float theta_f;
  uint32_t th_ord;  // every candidate of this wavefront whose scaled order key is >= th_ord is emitted
  if (theta < kMinValidOrd) {  // too few candidates: keep every one
    theta = kMinValidOrd;
    theta_f = -__FLT_MAX__;
    th_ord = kMinValidOrd;
  } else {
    theta_f = ord2f(theta);
    // unemitted values are < theta_f, so their scaled values are <= theta_f * inv_t
    th_ord = inv_t == 1.0f ? theta : f2ord(theta_f * inv_t) + 1u;
  }
  uint32_t smask = 0;  // bit i: v[i] >= theta_f (false for -inf; a NaN's bit is dropped at emission)
  if (theta_f < __builtin_inff()) {
    // bit i is the sign of v[i] - tq, inverted: for a finite or -FLT_MAX
    // threshold tq (-0.0 in place of +0.0, so that -0.0 - tq is +0.0) the
    // difference is >= +0.0 exactly when v[i] >= theta_f. v_alignbit shifts
    // each sign bit in, value NE-1 first, so value i lands on bit i.
    const float tq = theta_f == 0.0f ? -0.0f : theta_f;
    uint32_t below = 0;
#pragma unroll
    for (int i = NE - 1; i >= 0; --i) below = __builtin_amdgcn_alignbit(below, __float_as_uint(v[i] - tq), 31);
    smask = ~below & (NE == 32 ? 0xffffffffu : ((1u << (NE & 31)) - 1u));
  } else {  // an infinite or NaN threshold
#pragma unroll
    for (int i = 0; i < NE; ++i) smask |= (v[i] >= theta_f ? 1u : 0u) << i;
  }

  // ---- survivors into this wavefront's list; slots from the wavefront's
  // ballot of the lanes that emit, in lane order
  const size_t wslot = ((size_t)row * p.S + chunk) * kWavesPerBlock + wave;
  uint64_t* out = p.lists + wslot * p.cap_w;
  uint32_t base = 0;
  while (true) {
    if (__ballot(smask != 0u) == 0) break;
    bool want = false;
    uint64_t key = 0;
    if (smask) {
      const uint32_t b = __builtin_ctz(smask);
      smask &= smask - 1u;
      const uint32_t sl = b / EPL, e = b % EPL;
      const uint32_t off = sl * TILE + tid * EPL + e;
      const uint32_t k = cand_key(s_x[off] * inv_t);
      want = k != 0u;
      key = comp_key(k, c0 + off);
    }
    const uint64_t m = __ballot(want);
    if (want) {
      const uint32_t q = base + lanes_below(m);
      if (q < p.cap_w) out[q] = key;
    }
    base += (uint32_t)__popcll(m);
  }
  const uint32_t kmax32 = cand_key(ord2f(wave_max_u32(lm)) * inv_t);  // the wavefront's largest key
  if (lane == 0) {
    const bool bad = base > p.cap_w || (r.any_special && *s_full != 0u) || !scale_ok;
    p.wave_theta[wslot] = bad ? ~0ull : (((uint64_t)th_ord << 32) | kmax32);
    p.wave_count[wslot] = bad ? 0u : base;
  }
}

// The chunk's sparse-stage ids into the LDS hash: a count per
// history window occurrence, a flag per ban, bias and newline. The first claim
// of every window id's home slot goes out at once, collisions after. Ends
// with no barrier: the next block barrier completes the marks.
__device__ __forceinline__ void build_marks(const Params& p, const RowXf& r, uint32_t row, uint32_t c0,
                                            uint32_t c1, const uint32_t (&hv)[kHistUnroll],
                                            uint32_t* s_hkeys, uint32_t* s_hvals, uint32_t* s_full) {
  const uint32_t tid = threadIdx.x;
  bool ok = true;
  uint32_t prev[kHistUnroll];
#pragma unroll
  for (int q = 0; q < kHistUnroll; ++q) {
    const uint32_t t = r.use_hist && tid + q * kThreads < r.wn ? hv[q] : 0xffffffffu;
    const bool in = t >= c0 && t < c1;
    prev[q] = in ? atomicCAS(&s_hkeys[hash_slot(t - c0)], kEmptySlot, t - c0) : 0u;
  }
#pragma unroll
  for (int q = 0; q < kHistUnroll; ++q) {
    const uint32_t t = r.use_hist && tid + q * kThreads < r.wn ? hv[q] : 0xffffffffu;
    if (!(t >= c0 && t < c1)) continue;
    if (prev[q] == kEmptySlot || prev[q] == t - c0) atomicAdd(&s_hvals[hash_slot(t - c0)], 1u);
    else ok &= hash_insert_from(s_hkeys, s_hvals, t - c0, 1u, 0u);
  }
  if (r.use_hist) {
    const uint32_t* hrow = p.history + (size_t)row * p.history_ld + r.wstart;
    for (uint32_t j = tid + kHistUnroll * kThreads; j < r.wn; j += kThreads) {  // long windows
      const uint32_t t = hrow[j];
      if (t >= c0 && t < c1) ok &= hash_insert_from(s_hkeys, s_hvals, t - c0, 1u, 0u);
    }
  }
  for (uint32_t k = tid; k < r.ban_cnt; k += kThreads) {
    const uint32_t id = p.ban_ids[r.ban_off + k];
    if (id >= c0 && id < c1) ok &= hash_insert_from(s_hkeys, s_hvals, id - c0, 0u, kBanFlag);
  }
  for (uint32_t k = tid; k < r.bias_cnt; k += kThreads) {
    const uint32_t id = p.bias_ids[r.bias_off + k];
    if (id >= c0 && id < c1) ok &= hash_insert_from(s_hkeys, s_hvals, id - c0, 0u, kBiasFlag);
  }
  if (tid == 0 && r.nl_active && r.nl_id >= c0 && r.nl_id < c1)
    ok &= hash_insert_from(s_hkeys, s_hvals, r.nl_id - c0, 0u, kNlFlag);
  if (!ok) *s_full = 1;
}

// One (row, chunk) per block. The first half of the chunk's logits is issued
// at once (its addresses need nothing from memory); the row's record comes
// through the scalar cache meanwhile; then the history window ids and the
// second half. The marks are built when the window ids arrive, which waits
// for the first half only (vector loads complete in issue order), while the
// second half is still in flight.
// The arguments before the Params copy are what the first loads need; they
// arrive in SGPRs at wave launch (kernel-argument preloading), so those loads
// issue without waiting for a kernel-argument fetch.
template <int DT, int SLOTS, bool VEC, bool MASK, bool WB>
__global__ __launch_bounds__(kThreads) void stream_kernel(const void* __restrict__ logits,
                                                          const oxs_sampling_config* __restrict__ configs,
                                                          const uint32_t* __restrict__ history_len,
                                                          const uint32_t* __restrict__ history, uint32_t ld,
                                                          uint32_t S, uint32_t rpx, uint32_t V, uint32_t kflags,
                                                          uint32_t history_ld, const Params p) {
  constexpr int EPL = kind_f32(DT) ? 4 : 8;  // logits per 16-byte load
  constexpr int TILE = kThreads * EPL;
  constexpr int CH = SLOTS * TILE;
  constexpr int NE = SLOTS * EPL;  // logits per lane
  constexpr int H1 = (SLOTS + 1) / 2;  // loads issued before the row's record is read
  constexpr size_t ESZ = kind_f32(DT) ? 4 : 2;
  static_assert(CH <= kMaxChunk, "chunk too large");
  static_assert(NE <= 32, "one survivor bit per logit of a lane");

  __shared__ __align__(16) float s_x[NE * kThreads];  // each thread's masked raw logits (private slots)
  __shared__ uint32_t s_hkeys[kHashSlots];
  __shared__ uint32_t s_hvals[kHashSlots];
  __shared__ uint32_t s_full;

  const uint32_t tid = threadIdx.x;
  // the block's (row, chunk). With rpx > 0 the hardware's round-robin
  // placement of blocks on the 8 XCDs (block i on XCD i % 8) gives XCD x the
  // chunks of rows [x * rpx, (x + 1) * rpx), so that a row's stream blocks and
  // its tail block share one L2.
  const uint32_t k = rpx ? grouped_index(blockIdx.x, rpx * S) : blockIdx.x;
  const uint32_t row = k / S, chunk = k - row * S;  // (the grid is exactly batch x S blocks)
  const uint32_t c0 = chunk * CH;
  const uint32_t c1 = min(c0 + (uint32_t)CH, V);

  // The row's record (config dwords in lanes 0-25, history length in lane
  // 26), one vector load per lane issued before any logit: vector loads
  // complete in issue order, so waiting for it waits for nothing else.
  const uint32_t lane = tid & 63;
  const uint32_t* cfgw = (const uint32_t*)(configs + ((kflags & kKShared) ? 0u : row));
  const uint32_t rec = lane < 26u ? cfgw[lane] : (lane == 26u && (kflags & kKHistory) ? history_len[row] : 0u);
  __builtin_amdgcn_sched_barrier(0);

  uint32_t raw[SLOTS][EPL];
  const char* rowp = (const char*)logits + (size_t)row * (size_t)ld * ESZ;
  auto load_slot = [&](int s) {
    const uint32_t base = c0 + s * TILE + tid * EPL;
    if constexpr (VEC) {
      // V is a multiple of EPL here: past-the-end groups re-read the row's
      // last group (in bounds) and their values are dropped later.
      const uint32_t at = base < c1 ? base : V - EPL;
      const u32x4 q = __builtin_nontemporal_load((const u32x4*)(rowp + (size_t)at * ESZ));
      if constexpr (kind_f32(DT)) {
        raw[s][0] = q.x; raw[s][1] = q.y; raw[s][2] = q.z; raw[s][3] = q.w;
      } else {
        raw[s][0] = q.x << 16; raw[s][1] = q.x & 0xffff0000u;
        raw[s][2] = q.y << 16; raw[s][3] = q.y & 0xffff0000u;
        raw[s][4] = q.z << 16; raw[s][5] = q.z & 0xffff0000u;
        raw[s][6] = q.w << 16; raw[s][7] = q.w & 0xffff0000u;
      }
    } else {
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const uint32_t idx = base + e;
        raw[s][e] = __float_as_uint(load_logit<DT>(p, row, idx < c1 ? idx : p.V - 1));
      }
    }
  };
  uint32_t mw[SLOTS];
#pragma unroll
  for (int s = 0; s < H1; ++s) load_slot(s);
#pragma unroll
  for (int s = 0; s < SLOTS; ++s) {
    mw[s] = 0xffffffffu;
    if constexpr (MASK) {
      const uint32_t b2 = c0 + s * TILE + tid * EPL;
      mw[s] = p.mask[(size_t)row * p.mask_ld + ((b2 < c1 ? b2 : p.V - 1) >> 5)];
    }
  }
  for (uint32_t i = tid; i < (uint32_t)kHashSlots; i += kThreads) {
    s_hkeys[i] = kEmptySlot;
    s_hvals[i] = 0;
  }
  if (tid == 0) s_full = 0;
  __builtin_amdgcn_sched_barrier(0);
  oxs_sampling_config cfg;
  {
    uint32_t w[26];
#pragma unroll
    for (int i = 0; i < 26; ++i) w[i] = (uint32_t)__builtin_amdgcn_readlane((int)rec, i);
    memcpy(&cfg, w, sizeof(cfg));
  }
  const uint32_t hlen = (uint32_t)__builtin_amdgcn_readlane((int)rec, 26);
  if ((kflags & kKDecode) && cfg.temperature <= 1e-6f) raw_argmax_config(cfg);  // continuous_batching.rs:961
  const RowXf r = make_row_xf(cfg, hlen, V, history_ld, kflags);
  // history window ids, read without a branch (an in-bounds dummy address
  // where the row has none)
  uint32_t hv[kHistUnroll];
  const uint32_t* hsrc = r.use_hist ? history + (size_t)row * history_ld + r.wstart : (const uint32_t*)configs;
  const uint32_t hn = r.use_hist ? r.wn : 0u;
#pragma unroll
  for (int q = 0; q < kHistUnroll; ++q) {
    const uint32_t j = tid + q * kThreads;
    // (a relaxed atomic load: the compiler keeps it here, ahead of the second
    // half, instead of sinking it into the branch that reads it)
    hv[q] = __hip_atomic_load(hsrc + (j < hn ? j : 0u), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
  }
  __builtin_amdgcn_sched_barrier(0);  // the history window ahead of the second half
#pragma unroll
  for (int s = H1; s < SLOTS; ++s) load_slot(s);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (kind_softcap(DT) && VEC) {  // (the scalar loads above went through load_logit)
#pragma unroll
    for (int s = 0; s < SLOTS; ++s)
#pragma unroll
      for (int e = 0; e < EPL; ++e) raw[s][e] = __float_as_uint(softcap_of(__uint_as_float(raw[s][e]), p.softcap));
  }
  if (r.any_special) {
    __syncthreads();  // tables cleared
    build_marks(p, r, row, c0, c1, hv, s_hkeys, s_hvals, &s_full);
  }

  process_unit<DT, SLOTS, VEC, MASK, WB>(p, row, chunk, r, raw, mw, s_x, s_hkeys, s_hvals, &s_full);
}

// ---------------------------------------------------------------- tail helpers

struct TailShared {
  uint64_t a_kmin[kWavesPerBlock];  // per-wavefront smallest valid keys
  uint32_t scan_scratch[8];
  uint32_t sel_digit, sel_above, sel_count, counter;
  uint32_t dry_full;  // the DRY pass found more distinct ids than its hash holds
  float dry_pen[33];  // DRY penalty per match length (dry_pass_lds)
  uint32_t dry_hist[kWavesPerBlock][64];  // per wavefront: occurrences per match length (dry_pass_lds)
  uint32_t dry_bits[2];  // bit (id * 0x9e3779b1) >> 26 of every penalised id (dry_pass_lds)
  uint32_t a_kmax[kWavesPerBlock];  // per-wavefront largest keys (DRY candidate rows)
};

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
        const uint32_t ixj = i ^ j;
        if (ixj > i) {
          const uint64_t x = a[i], y = a[ixj];
          const bool second_half = (i & k) != 0;
          const bool swap = ASC ? (second_half ? (x < y) : (x > y)) : (second_half ? (x > y) : (x < y));
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

// One compare-exchange of the bitonic network that sorts descending: entry i
// against i ^ j (> i) at merge size k (as bitonic_sort<false>).
__device__ __forceinline__ void bitonic_cx(uint64_t* a, uint32_t la, uint32_t i, uint32_t j, uint32_t k) {
  const uint32_t lb = la ^ j;
  const uint64_t x = a[la], y = a[lb];
  const bool swap = (i & k) ? (x > y) : (x < y);
  if (swap) {
    a[la] = y;
    a[lb] = x;
  }
}

// The steps j = j0, j0 / 2, ..., 1 of merge size k on the tile of `tile_n`
// entries of g starting at tb, in LDS (tile_n <= kTailArea).
__device__ void bitonic_tile(uint64_t* g, uint32_t tb, uint32_t tile_n, uint32_t k, uint32_t j0, uint64_t* tile) {
  const uint32_t tid = threadIdx.x;
  for (uint32_t i = tid; i < tile_n; i += kThreads) tile[i] = g[tb + i];
  __syncthreads();
  for (uint32_t kk = (k ? k : 2); kk <= (k ? k : tile_n); kk <<= 1) {
    for (uint32_t j = (k ? j0 : kk >> 1); j > 0; j >>= 1) {
      for (uint32_t li = tid; li < tile_n; li += kThreads)
        if ((li ^ j) > li) bitonic_cx(tile, li, tb + li, j, kk);
      __syncthreads();
    }
  }
  for (uint32_t i = tid; i < tile_n; i += kThreads) g[tb + i] = tile[i];
  __syncthreads();
}

// Sorts g[0 .. n) descending in global memory (g has room for the next power
// of two of n, padded with zeros, which no key equals): the bitonic network,
// with every step whose partner distance is below the LDS tile done on tiles
// in LDS and only the longer ones as passes over global memory.
__device__ void wide_sort(uint64_t* g, uint32_t n, uint64_t* tile) {
  const uint32_t tid = threadIdx.x;
  uint32_t n2 = 1;
  while (n2 < n) n2 <<= 1;
  for (uint32_t i = n + tid; i < n2; i += kThreads) g[i] = 0ull;
  __syncthreads();
  const uint32_t T = min(n2, (uint32_t)kTailArea);
  for (uint32_t tb = 0; tb < n2; tb += T) bitonic_tile(g, tb, T, 0u, 0u, tile);  // merge sizes 2 .. T
  for (uint32_t k = 2 * T; k <= n2; k <<= 1) {
    for (uint32_t j = k >> 1; j >= T; j >>= 1) {
      for (uint32_t i = tid; i < n2; i += kThreads)
        if ((i ^ j) > i) bitonic_cx(g, i, i, j, k);
      __syncthreads();
    }
    for (uint32_t tb = 0; tb < n2; tb += T) bitonic_tile(g, tb, T, k, T >> 1, tile);
  }
}

// Radix-select step: given a histogram of the next digit among keys matching
// the current prefix, finds the digit holding the kk-th largest key.
__device__ void find_digit(const uint32_t* hist, TailShared& ts, uint32_t kk) {
  const uint32_t t = threadIdx.x;
  const uint32_t d = 255u - t;
  const uint32_t h = hist[d];
  uint32_t tot;
  const uint32_t above = block_excl_scan(h, &tot, ts.scan_scratch);
  if (above < kk && kk <= above + h) {
    ts.sel_digit = d;
    ts.sel_above = above;
    ts.sel_count = h;
  }
  __syncthreads();
}

// Dense penalty table of logits [c0, c1) for the exact path: window counts in
// the low bits, ban/bias/newline flags in the high bits. Ends with a barrier.
__device__ __forceinline__ void build_table(const Params& p, const RowXf& r, uint32_t row, uint32_t c0,
                            uint32_t c1, uint32_t* table) {
  const uint32_t tid = threadIdx.x;
  for (uint32_t i = tid; i < c1 - c0; i += kThreads) table[i] = 0;
  __syncthreads();
  if (r.use_hist) {
    const uint32_t* h = p.history + (size_t)row * p.history_ld + r.wstart;
    for (uint32_t j = tid; j < r.wn; j += kThreads) {
      const uint32_t t = h[j];
      if (t >= c0 && t < c1) atomicAdd(&table[t - c0], 1u);
    }
  }
  for (uint32_t k = tid; k < r.ban_cnt; k += kThreads) {
    const uint32_t id = p.ban_ids[r.ban_off + k];
    if (id >= c0 && id < c1) atomicOr(&table[id - c0], kBanFlag);
  }
  for (uint32_t k = tid; k < r.bias_cnt; k += kThreads) {
    const uint32_t id = p.bias_ids[r.bias_off + k];
    if (id >= c0 && id < c1) atomicOr(&table[id - c0], kBiasFlag);
  }
  if (tid == 0 && r.nl_active && r.nl_id >= c0 && r.nl_id < c1) atomicOr(&table[r.nl_id - c0], kNlFlag);
  if (r.dry) {
    const uint64_t* dl = p.dry_list + (size_t)row * p.dry_cap;
    const uint32_t nd = p.dry_count[row];
    for (uint32_t k = tid; k < nd; k += kThreads) {
      const uint32_t id = (uint32_t)(dl[k] >> 32);
      if (id >= c0 && id < c1) atomicOr(&table[id - c0], kDryFlag);
    }
  }
  __syncthreads();
}

// The DRY-stage value of id (the row's sorted DRY list holds it).
__device__ __forceinline__ float dry_value(const Params& p, uint32_t row, uint32_t id) {
  const uint64_t* dl = p.dry_list + (size_t)row * p.dry_cap;
  uint32_t lo = 0, hi = p.dry_count[row];
  while (hi - lo > 1) {
    const uint32_t mid = (lo + hi) >> 1;
    if ((uint32_t)(dl[mid] >> 32) <= id) lo = mid;
    else hi = mid;
  }
  return __uint_as_float((uint32_t)dl[lo]);
}

template <int DT>
__device__ __forceinline__ float transformed_logit(const Params& p, const RowXf& r, uint32_t row,
                                                   uint32_t idx, uint32_t c0,
                                                   const uint32_t* table) {
  float x = load_logit<DT>(p, row, idx);
  if (p.mask && !mask_allows(p, row, idx)) x = neg_inf();
  if (r.any_special) {
    const uint32_t e = table[idx - c0];
    if (e & kDryFlag) x = special_post(r, dry_value(p, row, idx), e);  // mask, ban, bias, newline, DRY included
    else if (e) x = apply_special(p.bias_ids, p.bias_values, r, x, e, idx);
  }
  if (r.do_temp) x *= r.inv_temp;
  return x;
}

// Exact top-M of a whole row without the candidate sets: a radix select over
// all V keys, re-reading the row once per digit. Used only when the candidate
// keys cannot be proven to hold the row's top M. Writes the top min(M, pool)
// keys to out (unordered, at most `cap`: M <= cap); returns that count.
template <int DT>
__device__ __forceinline__ uint32_t exact_select_row(const Params& p, const RowXf& r, uint32_t row, uint32_t M,
                                     uint32_t* table, uint32_t* hist, uint64_t* out,
                                     TailShared& ts, uint32_t cap = kMaxM) {
  const uint32_t tid = threadIdx.x;
  uint64_t prefix = 0, mask = 0;
  uint32_t kk = 0, meff = 0;
  bool done = false;
  for (int d = 0; d < 8 && !done; ++d) {
    const int shift = 56 - 8 * d;
    hist[tid] = 0;
    __syncthreads();
    for (uint32_t c0 = 0; c0 < p.V; c0 += (uint32_t)kMaxChunk) {  // table chunks (the LDS table's size)
      const uint32_t c1 = min(c0 + (uint32_t)kMaxChunk, p.V);
      if (r.any_special) build_table(p, r, row, c0, c1, table);
      for (uint32_t i = c0 + tid; i < c1; i += kThreads) {
        const float y = transformed_logit<DT>(p, r, row, i, c0, table);
        // the row's whole write-back again: the stream kernel's has no DRY, and
        // a chunk whose sparse-stage ids overflowed its LDS hash (a record
        // marked bad, which is what sends the row here) wrote values without
        // some of its penalties
        if (d == 0 && p.logits_out) p.logits_out[(size_t)row * p.logits_out_ld + i] = y;
        const uint32_t k = cand_key(y);
        if (!k) continue;
        const uint64_t key = comp_key(k, i);
        if ((key & mask) == prefix) atomicAdd(&hist[(uint32_t)(key >> shift) & 255u], 1u);
      }
      __syncthreads();
    }
    if (d == 0) {
      uint32_t pool;
      block_excl_scan(hist[tid], &pool, ts.scan_scratch);
      meff = min(M, pool);
      kk = meff;
      if (meff == 0) return 0;
    }
    find_digit(hist, ts, kk);
    prefix |= (uint64_t)ts.sel_digit << shift;
    mask |= 0xffull << shift;
    kk -= ts.sel_above;
    if (ts.sel_count == kk) done = true;  // the whole bucket is in
    __syncthreads();
  }
  if (tid == 0) ts.counter = 0;
  __syncthreads();
  for (uint32_t c0 = 0; c0 < p.V; c0 += (uint32_t)kMaxChunk) {
    const uint32_t c1 = min(c0 + (uint32_t)kMaxChunk, p.V);
    if (r.any_special) build_table(p, r, row, c0, c1, table);
    for (uint32_t i = c0 + tid; i < c1; i += kThreads) {
      const uint32_t k = cand_key(transformed_logit<DT>(p, r, row, i, c0, table));
      if (!k) continue;
      const uint64_t key = comp_key(k, i);
      if ((key & mask) >= prefix) {
        const uint32_t pos = atomicAdd(&ts.counter, 1u);
        if (pos < cap) out[pos] = key;
      }
    }
    __syncthreads();
  }
  return meff;
}

__device__ __forceinline__ float key_value(uint64_t k) { return ord2f((uint32_t)(k >> 32)); }

// ---------------------------------------------------------------- tail math

// The glibc-exact exp/ln/log2 tables, copied into LDS at tail start so the
// chain's lookups are LDS reads rather than global-memory round trips.
struct LibmTables {
  uint64_t exp2[32];
  double invc[16];
  double lnc[16];
  double log2c[16];
};

// The tables come from a workspace copy (made when the sampler is created):
// ordinary reads issued with the row's first loads; stored into LDS later.
constexpr int kLibmWords = 32 + 16 * 3;
struct LibmEntries {
  uint64_t e, i, l, g;
};
__device__ __forceinline__ LibmEntries fetch_libm_tables(const uint64_t* w) {
  const uint32_t tid = threadIdx.x;
  return LibmEntries{w[tid & 31u], w[32 + (tid & 15u)], w[48 + (tid & 15u)], w[64 + (tid & 15u)]};
}
__device__ __forceinline__ void store_libm_tables(const LibmEntries& v, LibmTables& t) {
  const uint32_t tid = threadIdx.x;
  if (tid < 32) t.exp2[tid] = v.e;
  if (tid < 16) {
    t.invc[tid] = __longlong_as_double((long long)v.i);
    t.lnc[tid] = __longlong_as_double((long long)v.l);
    t.log2c[tid] = __longlong_as_double((long long)v.g);
  }
}

__device__ __forceinline__ float dexpf(float x, const LibmTables& t) {
  return oxs_libm::expf_t<true>(x, t.exp2);
}
__device__ __forceinline__ float dlogf(float x, const LibmTables& t) {
  return oxs_libm::logf_t<true>(x, t.invc, t.lnc);
}
__device__ __forceinline__ float dlog2f(float x, const LibmTables& t) {
  return oxs_libm::log2f_t<true>(x, t.invc, t.log2c);
}

__device__ __forceinline__ float next_f32(uint64_t* s) {  // sampler.rs:139-153
  uint64_t x = *s;
  x ^= x << 13;
  x ^= x >> 7;
  x ^= x << 17;
  *s = x;
  const uint32_t val = (uint32_t)(x >> 40);
  return (float)val / 16777216.0f;
}

struct Ident {
  __device__ float operator()(float v) const { return v; }
};
struct Scaled {
  float k;
  __device__ float operator()(float v) const { return v * k; }
};
// (v * k1) * k2 with both products rounded, as two successive scalings.
struct Scaled2 {
  float k1, k2;
  __device__ float operator()(float v) const { return (v * k1) * k2; }
};

__device__ __forceinline__ float4 ld4(const float* a) { return *(const float4*)a; }

struct Chain {
  uint32_t stop;  // index + 1 of the element that reached the stop value, else n
  float sum;      // running sum there, else the total
  bool hit;
};

// 16 ordered adds of one group; t[j] is the running sum after element j.
template <typename F>
__device__ __forceinline__ float add16(float x, float4 q0, float4 q1, float4 q2, float4 q3, F f,
                                       float (&t)[16]) {
  const float v[16] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w,
                       q2.x, q2.y, q2.z, q2.w, q3.x, q3.y, q3.z, q3.w};
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    x = x + f(v[j]);
    t[j] = x;
  }
  return x;
}

// First j < lim with t[j] >= stop (16 when none): one lane stores the group's
// running sums, sixteen lanes test one each.
__device__ __forceinline__ uint32_t first_hit16(const float (&t)[16], uint32_t lim, float stop, float* hit,
                                                float* at) {
  const uint32_t l = threadIdx.x & 63;
  if (l == 0) {
#pragma unroll
    for (int q = 0; q < 4; ++q) *(float4*)(hit + 4 * q) = make_float4(t[4 * q], t[4 * q + 1], t[4 * q + 2], t[4 * q + 3]);
  }
  wave_sync();
  const float mine = hit[l & 15u];
  const uint64_t m = __ballot(l < lim && mine >= stop);
  uint32_t j = 16;
  if (m) {
    j = (uint32_t)__builtin_ctzll(m);
    *at = hit[j];
  }
  wave_sync();
  return j;
}

// The reference's ordered f32 running sum init + f(a[0]) + f(a[1]) + ...,
// computed by every lane of one wavefront from broadcast LDS reads, 16 values
// per group with the next group read ahead. With STOP it ends at the first
// index whose running sum is >= stop. A group is searched only when its last
// running sum is not below stop: the addends are >= 0, so the running sum never
// decreases and a group without a hit ends below stop (a NaN sum sends the
// group to the search, which finds no hit, as the reference's comparisons find
// none). The final partial group adds -0.0 in place of the missing elements,
// which leaves every float unchanged. `a` is 16-byte aligned and readable 16
// entries past n; `hit` is 16 floats of LDS.
template <bool STOP, typename F>
__device__ __forceinline__ Chain seq_chain(const float* a, uint32_t n, float init, float stop, F f, float* hit) {
  float s = init;
  if (n == 0) return Chain{0u, s, false};
  const uint32_t full = n & ~15u;
  float4 p0 = ld4(a), p1 = ld4(a + 4), p2 = ld4(a + 8), p3 = ld4(a + 12);
  uint32_t base = 0;
  float t[16];
  float at = 0.0f;
  for (; base + 32 <= full; base += 32) {
    const float4 r0 = ld4(a + base + 16), r1 = ld4(a + base + 20), r2 = ld4(a + base + 24), r3 = ld4(a + base + 28);
    __builtin_amdgcn_sched_barrier(0);
    s = add16(s, p0, p1, p2, p3, f, t);
    if (STOP && !(s < stop)) {
      const uint32_t j = first_hit16(t, 16u, stop, hit, &at);
      if (j < 16) return Chain{base + j + 1, at, true};
    }
    __builtin_amdgcn_sched_barrier(0);
    p0 = ld4(a + base + 32);
    p1 = ld4(a + base + 36);
    p2 = ld4(a + base + 40);
    p3 = ld4(a + base + 44);
    __builtin_amdgcn_sched_barrier(0);
    s = add16(s, r0, r1, r2, r3, f, t);
    if (STOP && !(s < stop)) {
      const uint32_t j = first_hit16(t, 16u, stop, hit, &at);
      if (j < 16) return Chain{base + 16 + j + 1, at, true};
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  if (base < full) {
    s = add16(s, p0, p1, p2, p3, f, t);
    if (STOP && !(s < stop)) {
      const uint32_t j = first_hit16(t, 16u, stop, hit, &at);
      if (j < 16) return Chain{base + j + 1, at, true};
    }
    base += 16;
    p0 = ld4(a + base);
    p1 = ld4(a + base + 4);
    p2 = ld4(a + base + 8);
    p3 = ld4(a + base + 12);
  }
  if (base < n) {
    const uint32_t rem = n - base;
    const float v[16] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w,
                         p2.x, p2.y, p2.z, p2.w, p3.x, p3.y, p3.z, p3.w};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float add = (uint32_t)j < rem ? f(v[j]) : -0.0f;
      s = s + add;
      t[j] = s;
    }
    if (STOP && !(s < stop)) {
      const uint32_t j = first_hit16(t, rem, stop, hit, &at);
      if (j < 16) return Chain{base + j + 1, at, true};
    }
  }
  return Chain{n, s, false};
}

// Per-row values the chain and the decode step need from global memory, read
// at tail start.
struct RowState {
  float uniform;
  float mu;
  uint64_t rng;
  uint32_t history_len;
  bool raw;            // a raw decode row: no history, no candidates buffer
  int32_t dec_pos;     // decode step: the row's position and generated count,
  uint32_t dec_count;  // and the steps it has handed to the host
  uint32_t dec_steps;
};

// The decode loop's bookkeeping once a row's token is known, by the thread
// that wrote it (continuous_batching.rs:974-976; the device-side advance and
// host hand-off of megakernel_ops.cu:331-347): the next step's input token,
// position and generated count, and the token in host memory. The host slot
// is one 8-byte system-scope store of (the row's step count << 32 | token),
// written through to host memory: the host polls each slot for its expected
// count, so no row waits for another or for the store's acknowledgement.
template <int DT>
__device__ __forceinline__ void decode_advance(const Params& p, uint32_t row, uint32_t token, const RowState& rs) {
  if constexpr (!kind_decode(DT)) return;
  if (p.dec_token) p.dec_token[row] = token;
  if (p.dec_pos) p.dec_pos[row] = rs.dec_pos + 1;
  if (p.dec_count) p.dec_count[row] = rs.dec_count + 1u;
  if (p.host_tokens) {
    const uint32_t n = rs.dec_steps + 1u;
    p.row_steps[row] = n;
    __hip_atomic_store(p.host_tokens + row, ((uint64_t)n << 32) | token, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

// A row that ends before the chain. A raw decode row leaves the caller's
// candidates buffer as it was.
template <int DT>
__device__ __forceinline__ void write_row_result(const Params& p, uint32_t row, uint32_t token, int32_t status,
                                                 const RowState& rs) {
  if (threadIdx.x == 0) {
    p.out_tokens[row] = token;
    if (p.out_status) p.out_status[row] = status;
    if (p.out_kept_count && !rs.raw) p.out_kept_count[row] = 0;
    decode_advance<DT>(p, row, token, rs);
  }
}

// Which way a row's top M was found, counted per row when the sampler's path
// counters are on (oxs_sampler_count_paths).
constexpr int kPathBuckets = 0;  // bucketed counting sort of the candidate keys
constexpr int kPathSort = 1;     // bitonic sort of the candidate keys
constexpr int kPathExact = 2;    // radix select over the whole row
constexpr int kPathNone = 3;     // the row ended before the selection (unsupported, missing state)
constexpr int kPathKinds = 4;
__device__ __forceinline__ void count_path(const Params& p, int path) {
  if (p.path_counts && threadIdx.x == 0) atomicAdd(&p.path_counts[path], 1u);
}

// LDS arrays of the chain; each is readable 16 entries past kMaxM.
constexpr int kChainLd = kMaxM + 16;
struct ChainBufs {
  uint32_t* ids;  // the candidates, sorted, and their exps on entry
  float* pr;
  uint32_t* ids_b;
  float* pr_b;
  float* aux;
  uint64_t* aux64;
  float* hit;  // 16 floats
  uint64_t* big;  // global scratch of a power of two >= n entries (wide rows), or NULL
};


// Stable in-place compaction of (ids, pr)[0..len) by one wavefront: a step
// reads 4 x 64 entries, keeps those with keep(v), and writes them below the
// step, after all of its reads. v = xf(pr[i]) is what is kept.
template <typename X, typename K>
__device__ __forceinline__ uint32_t wave_compact(uint32_t* ids, float* pr, uint32_t len, X xf, K keep) {
  const uint32_t l = threadIdx.x;
  uint32_t kept = 0;
  for (uint32_t r0 = 0; r0 < len; r0 += 256) {
    uint32_t id[4];
    float v[4];
    uint64_t m[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {  // unconditional reads (clamped index)
      const uint32_t i = r0 + 64u * t + l;
      const uint32_t at = i < len ? i : 0u;
      id[t] = ids[at];
      v[t] = xf(pr[at]);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) m[t] = __ballot(r0 + 64u * t + l < len && keep(v[t]));
    wave_sync();
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if ((m[t] >> l) & 1u) {
        const uint32_t at = kept + lanes_below(m[t]);
        ids[at] = id[t];
        pr[at] = v[t];
      }
      kept += (uint32_t)__popcll(m[t]);
    }
    wave_sync();
  }
  return kept;
}

// Number of leading entries of d[lo .. lo + n) for which `holds` is false,
// when it is false up to some point and true after it (binary lifting with
// steps top, top / 2, ..., 1; top is the largest power of two not above n).
template <typename P>
__device__ __forceinline__ uint32_t count_false(const uint32_t* d, uint32_t lo, uint32_t n, uint32_t top, P holds) {
  uint32_t cnt = 0;
  for (uint32_t step = top; step; step >>= 1) {
    const uint32_t at = cnt + step;
    if (at <= n && !holds(d[lo + at - 1])) cnt = at;
  }
  return cnt;
}

// Typical's stable sort (sampler.rs:508) when its scores are V-shaped:
// d (ordered score bits) non-increasing on [0, m) and non-decreasing on
// [m, len), as |surprisal - H| is over candidates sorted by probability. The
// rank of key (d[i] << 32 | i) then needs no comparison with every other key:
//   i >= m: the keys of [m, i) and those of [0, m) with d <= d[i] are below it;
//   i <  m: those of [0, m) with d < d[i], those of [first with d == d[i], i)
//           and those of [m, len) with d < d[i],
// each a count over one monotone run. Writes the sorted (ids, pr) to
// (ids_b, pr_b). One wavefront.
__device__ __forceinline__ void typical_rank_v(const uint32_t* ids, const float* pr, const uint32_t* d, uint32_t len,
                                               uint32_t m, uint32_t* ids_b, float* pr_b) {
  const uint32_t l = threadIdx.x & 63;
  const uint32_t nl = m, nr = len - m;
  const uint32_t tl = nl > 1 ? 1u << (31 - __builtin_clz(nl)) : nl;
  const uint32_t tr = nr > 1 ? 1u << (31 - __builtin_clz(nr)) : nr;
  for (uint32_t i = l; i < len; i += 64) {
    const uint32_t v = d[i];
    const uint32_t le = count_false(d, 0, nl, tl, [=](uint32_t x) { return x <= v; });  // [0, le): d > v
    uint32_t rank;
    if (i >= m) {
      rank = (i - m) + (nl - le);
    } else {
      const uint32_t lt = count_false(d, 0, nl, tl, [=](uint32_t x) { return x < v; });  // [0, lt): d >= v
      const uint32_t rlt = count_false(d, m, nr, tr, [=](uint32_t x) { return x >= v; });  // [m, m + rlt): d < v
      rank = (nl - lt) + (i - le) + rlt;
    }
    ids_b[rank] = ids[i];
    pr_b[rank] = pr[i];
  }
}

// Typical's stable sort of a long list (wide rows) by one wavefront: keys
// (d[i] << 32 | i) sorted ascending by a bitonic network in global memory
// (sk: a power of two >= len entries), then (ids, pr) gathered in that order.
__device__ void wave_sort_by_score(const uint32_t* ids, const float* pr, const uint32_t* d, uint32_t len,
                                   uint64_t* sk, uint32_t* ids_b, float* pr_b) {
  const uint32_t l = threadIdx.x & 63;
  uint32_t n2 = 1;
  while (n2 < len) n2 <<= 1;
  for (uint32_t i = l; i < n2; i += 64) sk[i] = i < len ? ((uint64_t)d[i] << 32) | i : ~0ull;
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");  // this wavefront's stores complete
  for (uint32_t k = 2; k <= n2; k <<= 1) {
    for (uint32_t j = k >> 1; j > 0; j >>= 1) {
      for (uint32_t i = l; i < n2; i += 64) {
        const uint32_t ixj = i ^ j;
        if (ixj > i) {
          const uint64_t x = sk[i], y = sk[ixj];
          if ((i & k) ? (x < y) : (x > y)) {
            sk[i] = y;
            sk[ixj] = x;
          }
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
    }
  }
  for (uint32_t r = l; r < len; r += 64) {
    const uint32_t i = (uint32_t)sk[r];
    ids_b[r] = ids[i];
    pr_b[r] = pr[i];
  }
}

// The chain after the top-M selection (sampler.rs:286-389) on the n
// candidates in bf.ids, sorted, with bf.pr = exp(logit - max logit) (the
// softmax numerators, :286-290), run by one wavefront (threads 0..63) with no
// block barriers: parallel stages split the candidates over the lanes; the
// reference's ordered sums run in every lane at once (seq_chain), so each lane
// holds each result.
template <int DT>
__device__ __forceinline__ void wave_chain(const Params& p, const oxs_sampling_config& c, uint32_t row, uint32_t n,
                           ChainBufs bf, const RowState& rs, const LibmTables& tab) {
  const uint32_t l = threadIdx.x;
  uint32_t* ids = bf.ids;
  float* pr = bf.pr;
  // Softmax normalisation (:291-295): the scaling by 1 / sum is applied by the
  // next pass that reads the numerators.
  const float sum_exp = seq_chain<false>(pr, n, 0.0f, 0.0f, Ident{}, bf.hit).sum;
  const float inv_sum = sum_exp > 0.0f ? 1.0f / sum_exp : 1.0f;
  const Scaled to_prob{inv_sum};

  uint32_t len = n, n_record = 1, token;
  float inv_total = 1.0f;
  const bool mirostat = c.mirostat_mode == OXS_MIROSTAT_V1 || c.mirostat_mode == OXS_MIROSTAT_V2;
  // While every stage keeps a prefix of the sorted list (min-p, top-k, top-p)
  // the probabilities p_i = exp_i * inv_sum stay implicit: each reader scales
  // by k_in. p is non-increasing, so min-p's retain (:315-319) keeps a prefix,
  // found by counting. XTC, tail-free, typical and Mirostat get the
  // probabilities written out first (k_in = 1, and v * 1 is v).
  const bool lazy = !mirostat && !(c.xtc_probability > 0.0f) && !(c.tfs_z < 1.0f) && !(c.typical_p < 1.0f) &&
                    sum_exp > 0.0f && sum_exp <= __FLT_MAX__;
  const float k_in = lazy ? inv_sum : 1.0f;
  if (lazy) {
    if (c.min_p > 0.0f && len > 0) {
      const float threshold = to_prob(pr[0]) * c.min_p;
      uint32_t cnt = 0;
      for (uint32_t r0 = 0; r0 < n; r0 += 64) {
        const uint32_t i = r0 + l;
        const uint64_t m = __ballot(i < n && to_prob(pr[i < n ? i : 0u]) >= threshold);
        cnt += (uint32_t)__popcll(m);
        if (m != ~0ull) break;  // the prefix ended
      }
      len = cnt;
    }
  } else if (!mirostat && c.min_p > 0.0f && len > 0) {
    // Min-p (:315-319): keep p >= p_max * min_p, in order; the pass also turns
    // the exps into probabilities.
    const float threshold = to_prob(pr[0]) * c.min_p;
    len = wave_compact(ids, pr, len, to_prob, [=](float v) { return v >= threshold; });
  } else {
    for (uint32_t r0 = 0; r0 < n; r0 += 256) {
      float v[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint32_t i = r0 + 64u * t + l;
        v[t] = pr[i < n ? i : 0u];
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint32_t i = r0 + 64u * t + l;
        if (i < n) pr[i] = to_prob(v[t]);
      }
    }
    wave_sync();
  }

  if (mirostat) {
    const float mu0 = rs.mu;
    float mu = mu0;
    if (c.mirostat_mode == OXS_MIROSTAT_V1) {  // :418-429
      const float prob = fmaxf(pr[0], 1e-6f);
      const float surprise = -dlog2f(prob, tab);
      const float error = surprise - c.mirostat_tau;
      const float step = c.mirostat_eta * error;
      mu -= step;
    } else {  // :432-456: the prefix ends before the first i > 0 whose surprise exceeds mu
      uint32_t first = n;
      for (uint32_t r0 = 0; r0 < n; r0 += 64) {
        const uint32_t i = r0 + l;
        const bool over = i < n && i > 0 && -dlog2f(fmaxf(pr[i], 1e-8f), tab) > mu0;
        const uint64_t m = __ballot(over);
        if (m) {
          first = r0 + (uint32_t)__builtin_ctzll(m);
          break;
        }
      }
      const float cum_prob = seq_chain<false>(pr, first, 0.0f, 0.0f, Ident{}, bf.hit).sum;
      const float prob = pr[0] / fmaxf(cum_prob, 1e-6f);
      const float surprise = -dlog2f(fmaxf(prob, 1e-8f), tab);
      const float error = surprise - c.mirostat_tau;
      const float step = c.mirostat_eta * error;
      mu -= step;
    }
    if (l == 0) p.mu[row] = mu;
    token = ids[0];
    n_record = 2;  // recorded inside the mode function and by the caller (:301, :307)
  } else {
    // XTC (:322-328): drop the top choice.
    if (c.xtc_probability > 0.0f && len > 1) {
      const float p_max = pr[0];
      if (p_max >= c.xtc_threshold && p_max < 0.98f) {
        for (uint32_t r0 = 0; r0 + 1 < len; r0 += 64) {
          const uint32_t i = r0 + 1 + l;
          uint32_t id = 0;
          float v = 0.0f;
          if (i < len) {
            id = ids[i];
            v = pr[i];
          }
          wave_sync();
          if (i < len) {
            ids[i - 1] = id;
            pr[i - 1] = v;
          }
          wave_sync();
        }
        len -= 1;
      }
    }
    // Top-k (:331-333).
    if (c.top_k > 0 && len > c.top_k) len = c.top_k;
    // Tail-free (:336-338, :459-490).
    if (c.tfs_z < 1.0f && len > 2) {
      float* d2 = bf.aux;
      const uint32_t m = len - 2;
      for (uint32_t i = l; i < m; i += 64) {
        const float d1a = pr[i] - pr[i + 1];
        const float d1b = pr[i + 1] - pr[i + 2];
        d2[i] = fabsf(d1a - d1b);
      }
      wave_sync();
      const float sum_d2 = seq_chain<false>(d2, m, 0.0f, 0.0f, Ident{}, bf.hit).sum;
      uint32_t keep = len;
      if (sum_d2 > 0.0f) {
        const float inv = 1.0f / sum_d2;
        const Chain ch = seq_chain<true>(d2, m, 0.0f, c.tfs_z, Scaled{inv}, bf.hit);
        const uint32_t cutoff = ch.hit ? ch.stop : len;
        keep = cutoff > 1 ? cutoff : 1;
      }
      len = keep;
    }
    // Locally typical (:341-343, :493-520): stable sort by |surprisal - H|,
    // by rank counting over (score, position) keys.
    if (c.typical_p < 1.0f && len > 1) {
      float* terms = bf.aux;
      float* lg = (float*)bf.ids_b;  // ln p, until the sorted ids are written there
      for (uint32_t i = l; i < len; i += 64) {
        const float x = pr[i] > 0.0f ? dlogf(pr[i], tab) : 0.0f;
        lg[i] = x;
        terms[i] = pr[i] > 0.0f ? (-pr[i]) * x : 0.0f;
      }
      wave_sync();
      const float entropy = seq_chain<false>(terms, len, -0.0f, 0.0f, Ident{}, bf.hit).sum;
      wave_sync();
      // scores (ascending score, then position), over the entropy terms
      uint32_t* d = (uint32_t*)bf.aux;
      uint64_t mn = ~0ull;
      for (uint32_t i = l; i < len; i += 64) {
        const float surprisal = pr[i] > 0.0f ? -lg[i] : 0.0f;
        const uint32_t sc = f2ord(fabsf(surprisal - entropy));
        d[i] = sc;
        const uint64_t k = ((uint64_t)sc << 32) | i;
        mn = k < mn ? k : mn;
      }
      wave_sync();
      const uint32_t m = (uint32_t)wave_min_u64(mn);  // the first smallest score
      bool v_shaped = true;
      for (uint32_t i = l; i + 1 < len; i += 64) {
        const uint32_t a = d[i], b = d[i + 1];
        if (i + 1 < m ? a < b : (i >= m && a > b)) v_shaped = false;
      }
      if (__ballot(!v_shaped) == 0) {
        typical_rank_v(ids, pr, d, len, m, bf.ids_b, bf.pr_b);
      } else if (len > (uint32_t)kMaxM && bf.big) {  // any other shape, a long list: sorted
        wave_sort_by_score(ids, pr, d, len, bf.big, bf.ids_b, bf.pr_b);
      } else {  // any other shape: each key ranked against every key
        uint64_t* sk = bf.aux64;
        for (uint32_t i = l; i < len; i += 64) sk[i] = ((uint64_t)d[i] << 32) | i;
        if (l == 0) sk[len] = ~0ull;  // pad for the pairwise reads below
        wave_sync();
        for (uint32_t g = 0; g < len; g += 256) {
          uint64_t mine[4];
          uint32_t rank[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const uint32_t i = g + l + 64u * t;
            mine[t] = i < len ? sk[i] : 0ull;
            rank[t] = 0;
          }
          for (uint32_t j = 0; j < len; j += 2) {
            const uint64_t a0 = sk[j], a1 = sk[j + 1];
#pragma unroll
            for (int t = 0; t < 4; ++t) rank[t] += (a0 < mine[t] ? 1u : 0u) + (a1 < mine[t] ? 1u : 0u);
          }
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const uint32_t i = g + l + 64u * t;
            if (i < len) {
              bf.ids_b[rank[t]] = ids[i];
              bf.pr_b[rank[t]] = pr[i];
            }
          }
        }
      }
      wave_sync();
      ids = bf.ids_b;
      pr = bf.pr_b;
      len = seq_chain<true>(pr, len, 0.0f, c.typical_p, Ident{}, bf.hit).stop;
    }
    // Top-p (:346-357) cuts at the first running sum >= top_p; the
    // renormalisation total (:360-368) is the running sum at that cut.
    {
      const Chain ch = c.top_p < 1.0f ? seq_chain<true>(pr, len, 0.0f, c.top_p, Scaled{k_in}, bf.hit)
                                      : seq_chain<false>(pr, len, 0.0f, 0.0f, Scaled{k_in}, bf.hit);
      len = ch.stop;
      inv_total = ch.sum > 0.0f ? 1.0f / ch.sum : 1.0f;
    }
    // Draw (:371-385) over the renormalised p: greedy below 1e-6, else the
    // first running sum >= r; the fallback is the first candidate.
    if (c.temperature <= 1e-6f) {
      token = len ? ids[0] : 0u;
    } else {
      float rnd;
      if (p.uniforms) {
        rnd = rs.uniform;
      } else {
        uint64_t st = rs.rng;
        rnd = next_f32(&st);
        if (l == 0) p.rng_state[row] = st;
      }
      const Chain ch = seq_chain<true>(pr, len, 0.0f, rnd, Scaled2{k_in, inv_total}, bf.hit);
      token = ch.hit ? ids[ch.stop - 1] : (len ? ids[0] : 0u);
    }
  }
  // Outputs: token, status, history, candidates_buffer.
  if (l == 0) {
    int32_t status = OXS_ROW_OK;
    if ((p.flags & OXS_FLAG_RECORD_HISTORY) && !rs.raw) {
      uint32_t hl = rs.history_len;
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
    if (p.out_kept_count && !rs.raw) p.out_kept_count[row] = len;
    decode_advance<DT>(p, row, token, rs);
  }
  const uint32_t nk = rs.raw ? 0u : (uint32_t)min((int64_t)len, p.kept_ld);
  for (uint32_t i = l; i < nk; i += 64) {
    if (p.out_kept_ids) p.out_kept_ids[(size_t)row * p.kept_ld + i] = ids[i];
    if (p.out_kept_probs) p.out_kept_probs[(size_t)row * p.kept_ld + i] = (pr[i] * k_in) * inv_total;
  }
}

// ---------------------------------------------------------------- top-M selection

constexpr int kPer = kUnionMax / kThreads;  // candidate key slots per tail thread (kUnionBig: twice as many)
constexpr uint32_t kBigBucket = 64;         // largest bucket ranked by direct comparison
static_assert(kBuckets == 4 * 64, "4 buckets per lane of a scanning wavefront");

__device__ __forceinline__ uint32_t bucket_of(uint64_t k, float vmax, float scale) {
  return min((uint32_t)((vmax - key_value(k)) * scale), (uint32_t)kBuckets - 1);
}

// Fallback selection: all kept register keys (bit q of vm) into tmp, a bitonic
// sort, the first meff into out. Returns the number of kept keys.
template <int PER>
__device__ __forceinline__ uint32_t sort_select(const uint64_t (&lk)[PER], uint32_t vm, uint32_t M, uint64_t* tmp,
                                uint64_t* out, TailShared& ts) {
  const uint32_t cnt = (uint32_t)__popc(vm);
  uint32_t n;
  uint32_t pos = block_excl_scan(cnt, &n, ts.scan_scratch);
#pragma unroll
  for (int q = 0; q < PER; ++q)
    if ((vm >> q) & 1u) tmp[pos++] = lk[q];
  __syncthreads();
  const uint32_t meff = min(M, n);
  if (meff == 0) return 0;
  bitonic_sort<false>(tmp, n);
  for (uint32_t i = threadIdx.x; i < meff; i += kThreads) out[i] = tmp[i];
  __syncthreads();
  return n;
}

// ---------------------------------------------------------------- DRY

__device__ __forceinline__ float dpowf(float x, float y, const LibmTables& t) {
  return oxs_libm::powf_t<true>(x, y, t.exp2, t.invc, t.log2c);
}

// Ban (:184-188), bias (:189-193) and newline (:196-200) for one id, found in
// the row's lists.
__device__ __forceinline__ float pre_stages_of(const Params& p, const RowXf& r, uint32_t id, float x) {
  uint32_t e = 0;
  for (uint32_t k = 0; k < r.ban_cnt; ++k)
    if (p.ban_ids[r.ban_off + k] == id) e |= kBanFlag;
  for (uint32_t k = 0; k < r.bias_cnt; ++k)
    if (p.bias_ids[r.bias_off + k] == id) e |= kBiasFlag;
  if (r.nl_active && id == r.nl_id) e |= kNlFlag;
  return special_pre(p.bias_ids, p.bias_values, r, x, e, id);
}

// LDS layout of the DRY pass over a slice of up to kDryMax ids (u32 offsets
// into the tail's 32 KB area); the tail's DRY candidate step reads the hash.
constexpr int kDrySlice = 0;                 // [kDryMax] the slice; then the occurrences sorted by slot
constexpr int kDryKey = kDrySlice + kDryMax;  // [kDryHash] penalised ids (kEmptySlot: free)
constexpr int kDryVal = kDryKey + kDryHash;   // [kDryHash] their values
constexpr int kDryCnt = kDryVal + kDryHash;   // [kDryHash] occurrences per slot, then cursors; then the list
constexpr int kDryOcc = kDryCnt + kDryHash;   // [kDryMax] (slot << 6 | match length) per penalising occurrence
static_assert(kDryOcc + kDryMax <= 2 * kTailArea, "DRY LDS layout fits the tail area");

// DRY (sampler.rs:393-415) over a slice of L <= kDryMax ids, in one pass
// over the slice instead of one per match length. The occurrence at position
// q (q < L) matches at length ml exactly when ml <= lambda(q), the length of
// the longest common suffix of slice[..q) and the whole slice (at most 32 and
// q): slice[q - ml .. q) == slice[L - ml .. L) holds for every shorter length
// once it holds for one. So slice[q] takes one penalty per length in
// [allowed, lambda(q)], and an id's value is its pre-stage value minus, for
// ml = 32 down to allowed, pen(ml) once per occurrence with lambda >= ml, one
// rounded subtraction at a time (the reference's order; the penalties of one
// length are equal). The ids go into an LDS hash, each occurrence into a list
// sorted by slot with a counting sort, and each slot's thread runs its id's
// subtractions. Leaves the hash (ids, values) in LDS for dry_lookup.
template <int DT>
__device__ __forceinline__ void dry_pass_lds(const Params& p, const RowXf& r, uint32_t row, uint32_t L,
                                             uint32_t* lds, const LibmTables& tab, TailShared& ts, uint64_t* dl) {
  const uint32_t tid = threadIdx.x;
  uint32_t* slice = lds + kDrySlice;
  uint32_t* hkey = lds + kDryKey;
  float* val = (float*)(lds + kDryVal);
  uint32_t* cnt = lds + kDryCnt;
  uint32_t* occ = lds + kDryOcc;
  const uint32_t* hs = p.history + (size_t)row * p.history_ld + (r.hlen - L);
  static_assert(kDryMax <= 4 * kThreads, "four slice positions per thread");
  for (uint32_t i = tid; i < L; i += kThreads) slice[i] = hs[i];
  for (uint32_t h = tid; h < (uint32_t)kDryHash; h += kThreads) {
    hkey[h] = kEmptySlot;
    cnt[h] = 0;
  }
  const uint32_t allowed = min(r.dry_allowed, 33u);
  if (tid == 0) {
    ts.counter = 0;    // occurrences
    ts.sel_above = 0;  // penalised ids with at most 8 occurrences
    ts.sel_count = 0;  // ... with more
    ts.sel_digit = 0;  // distinct penalised ids
    ts.dry_bits[0] = 0;
    ts.dry_bits[1] = 0;
  }
  __syncthreads();  // (also orders the caller's libm tables in LDS before the dpowf below)
  if (tid <= 32u && tid >= allowed)  // pen(ml), :408-409, read after the next barrier
    ts.dry_pen[tid] = r.dry_mult * dpowf(r.dry_base, (float)(tid - allowed), tab);
  // lambda(q) for this thread's (at most four) positions q = tid + 256 i, eight
  // comparisons per step, all of a step's LDS reads issued before any compare.
  // An id seen for the first time has its logit (and mask word) loaded at once
  // and used after the loop, so those global reads overlap the rest of it.
  const uint32_t last = L ? slice[L - 1] : 0u;  // the slice's last id
  uint32_t first_h[4];
  float first_x[4];
  bool first_m[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    first_h[i] = kEmptySlot;
    first_x[i] = 0.0f;
    first_m[i] = true;
    const uint32_t q = tid + (uint32_t)i * kThreads;
    if (q >= L) continue;
    const uint32_t lim = min(q, 32u);
    uint32_t k = 0;
    if (lim > 0 && slice[q - 1] == last) k = 1;  // most positions end here
    while (k > 0 && k < lim) {
      uint32_t a[8], b[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const uint32_t kk = k + (uint32_t)t;
        a[t] = slice[kk < lim ? q - 1 - kk : 0u];
        b[t] = slice[kk < lim ? L - 1 - kk : 0u];
      }
      uint32_t run = 0;
      bool go = true;
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        go = go && k + (uint32_t)t < lim && a[t] == b[t];
        run += go ? 1u : 0u;
      }
      k += run;
      if (run < 8u) break;
    }
    const uint32_t next = slice[q];
    if (k < allowed || next >= p.V) continue;  // no length in [allowed, k]; logits.get_mut(next) is None
    uint32_t h = (next * 0x9e3779b1u) >> 21;
    for (int probe = 0; probe < kDryHash; ++probe) {  // at most L <= kDryHash / 2 distinct ids
      const uint32_t prev = atomicCAS(&hkey[h], kEmptySlot, next);
      if (prev == kEmptySlot) {  // first sight: the value before DRY, loaded now and used below
        atomicAdd(&ts.sel_digit, 1u);
        const uint32_t bit = (next * 0x9e3779b1u) >> 26;
        atomicOr(&ts.dry_bits[bit >> 5], 1u << (bit & 31u));
        first_h[i] = h;
        first_x[i] = load_logit<DT>(p, row, next);
        first_m[i] = !p.mask || mask_allows(p, row, next);
      }
      if (prev == kEmptySlot || prev == next) break;
      h = (h + 1) & (kDryHash - 1);
    }
    atomicAdd(&cnt[h], 1u);
    occ[atomicAdd(&ts.counter, 1u)] = (h << 6) | k;
  }
  __syncthreads();
  // counting sort of the occurrences by slot: each thread owns slots tid + 256 j
  constexpr int kPerT = kDryHash / kThreads;
  uint32_t mine[kPerT], sum = 0;
#pragma unroll
  for (int j = 0; j < kPerT; ++j) {
    mine[j] = cnt[tid + j * kThreads];
    sum += mine[j];
  }
  uint32_t total;
  const uint32_t start0 = block_excl_scan(sum, &total, ts.scan_scratch);
  uint32_t start = start0;
  // the slots of thread tid are not contiguous: a second pass gives each its start
  // (slots in order tid, tid + 256, ...; their ranges in the sorted list follow that order)
#pragma unroll
  for (int j = 0; j < kPerT; ++j) {
    cnt[tid + j * kThreads] = start;  // cursor
    start += mine[j];
  }
  __syncthreads();
  const uint32_t n_occ = ts.counter;
  for (uint32_t o = tid; o < n_occ; o += kThreads) {
    const uint32_t e = occ[o];
    slice[atomicAdd(&cnt[e >> 6], 1u)] = e & 63u;  // the match lengths, grouped by slot
  }
  __syncthreads();
  // the values before DRY of the ids this thread saw first (their loads were
  // issued in the lambda loop)
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (first_h[i] != kEmptySlot) {
      const uint32_t id = hkey[first_h[i]];
      val[first_h[i]] = pre_stages_of(p, r, id, first_m[i] ? first_x[i] : neg_inf());
    }
  // the penalised ids as lists of (slot << 11 | occurrences) over the free
  // occurrence area, ids of at most 8 occurrences from its start, the others
  // from its end (all of them there when there are at most four ids); each
  // slot's start in cnt (a slot's occurrences end at its cursor and start at
  // the previous slot's of this thread)
  const bool few = ts.sel_digit <= (uint32_t)kWavesPerBlock;
  {
    uint32_t prev_end = start0;
#pragma unroll
    for (int j = 0; j < kPerT; ++j) {
      const uint32_t h = tid + j * kThreads;
      const uint32_t end = cnt[h];
      const uint32_t n = end - prev_end;
      prev_end = end;
      if (n) {
        const uint32_t at = n <= 8u && !few ? atomicAdd(&ts.sel_above, 1u)
                                            : (uint32_t)kDryMax - 1u - atomicAdd(&ts.sel_count, 1u);
        occ[at] = (h << 11) | n;  // h < 2048, n <= kDryMax
        cnt[h] = end - n;
      }
    }
  }
  __syncthreads();
  // Each id's subtractions, longest match length first (:405-413): pen(ml)
  // once per occurrence with lambda >= ml, for ml = 32 down to allowed, each a
  // rounded subtraction. (Kept as rolled loops: unrolling them over the 33
  // lengths raised the whole tail kernel's register spills and slowed rows
  // without DRY.)
  const uint32_t n_light = ts.sel_above, n_heavy = ts.sel_count;
  // ids of up to 8 occurrences, one per thread, their lengths in registers and
  // the next length's penalty read ahead
#pragma unroll 1
  for (uint32_t c = tid; c < n_light; c += kThreads) {
    const uint32_t h = occ[c] >> 11, n = occ[c] & 2047u;
    const uint32_t* lam = slice + cnt[h];
    float v = val[h];
    uint32_t lr[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) lr[i] = (uint32_t)i < n ? lam[i] : 0u;
    uint32_t top = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) top = max(top, lr[i]);
    float pen = top >= allowed ? ts.dry_pen[top] : 0.0f;
    for (uint32_t ml = top + 1; ml-- > allowed;) {
      uint32_t act = 0;  // occurrences matching at this length
#pragma unroll
      for (int i = 0; i < 8; ++i) act += ((uint32_t)i < n && lr[i] >= ml) ? 1u : 0u;
      const float pen_next = ml > allowed ? ts.dry_pen[ml - 1] : 0.0f;  // (read ahead)
      uint32_t a = act;  // act subtractions of pen, four per loop step (:411)
      for (; a >= 4u; a -= 4u) v = (((v - pen) - pen) - pen) - pen;
      const float v2 = (v - pen) - pen;
      v = (a & 2u) ? v2 : v;
      const float v1 = v - pen;
      v = (a & 1u) ? v1 : v;
      pen = pen_next;
    }
    val[h] = v;
  }
  // ids of more occurrences (or every id when there are at most four), one per
  // wavefront: a histogram of the match lengths in LDS, then lane l holds the
  // occurrences matching at length l (a suffix sum) and the penalty pen(l), and
  // the subtractions run with wavefront-uniform counts read from those lanes
  const uint32_t lane = tid & 63u, wave = tid >> 6;
  uint32_t* hist = ts.dry_hist[wave];
  const float pen_l = lane <= 32u && lane >= allowed ? ts.dry_pen[lane] : 0.0f;
#pragma unroll 1
  for (uint32_t c = wave; c < n_heavy; c += kWavesPerBlock) {
    const uint32_t e = occ[(uint32_t)kDryMax - 1u - c];
    const uint32_t h = e >> 11, n = e & 2047u;
    const uint32_t* lam = slice + cnt[h];
    hist[lane] = 0;
    wave_sync();
    for (uint32_t b0 = lane; b0 < n; b0 += 64) atomicAdd(&hist[lam[b0]], 1u);
    wave_sync();
    const uint32_t x = hist[lane];  // (lanes above 32 hold 0)
    const uint32_t incl = wave_incl_scan(x);
    const uint32_t act_l = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63) - incl + x;  // lambda >= lane
    float v = val[h];
#pragma unroll 1
    for (int ml = 32; ml >= (int)allowed; --ml) {
      const uint32_t na = (uint32_t)__builtin_amdgcn_readlane((int)act_l, ml);
      const float pen = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(pen_l), ml));
      uint32_t a = 0;
      for (; a + 4u <= na; a += 4u) v = (((v - pen) - pen) - pen) - pen;  // :411
      for (; a < na; ++a) v = v - pen;
    }
    if (lane == 0) val[h] = v;
    wave_sync();
  }
  __syncthreads();
  // the list: (id << 32 | value bits), sorted by id, built over the cursors
  uint64_t* keys = (uint64_t*)cnt;  // [kDryMax]
  if (tid == 0) ts.counter = 0;
  __syncthreads();
  for (uint32_t h = tid; h < (uint32_t)kDryHash; h += kThreads) {
    const uint32_t id = hkey[h];
    if (id != kEmptySlot) keys[atomicAdd(&ts.counter, 1u)] = ((uint64_t)id << 32) | __float_as_uint(val[h]);
  }
  __syncthreads();
  const uint32_t nd = ts.counter;
  bitonic_sort<true>(keys, nd);
  for (uint32_t i = tid; i < nd; i += kThreads) dl[i] = keys[i];
  if (tid == 0) p.dry_count[row] = nd;
  __syncthreads();
}

// DRY (sampler.rs:393-415) for one row, by its tail block. Over the last
// dry_range history ids, for match lengths 32 down to allowed_length, every
// earlier position whose n-gram equals the slice's suffix penalises the id
// after it by multiplier * base^(length - allowed_length). An id's value starts
// at its logit after the mask, bans, biases and newline, and takes its
// penalties one rounded subtraction at a time in the reference's order
// (longer matches first; the penalties of one length are equal, so their order
// inside a length does not matter). The ids and values go to the row's list,
// sorted by id. A slice of up to kDryMax ids is copied into LDS and its ids
// counted in an LDS hash (kDryHash slots: room for every id of the slice); a
// longer one is read where it lies and counted in the row's global hash
// (2 * dry_cap slots) when the workspace has one, else in the LDS hash.
// Returns false (the row cannot be run) when the penalised ids outnumber what
// the hash or the list holds. Uses the first 32 KB of `lds`; after a slice of
// up to kDryMax ids, the LDS hash (ids and values) is left for dry_lookup.
template <int DT>
__device__ __forceinline__ bool dry_pass(const Params& p, const RowXf& r, uint32_t row, uint32_t* lds,
                                         const LibmTables& tab, TailShared& ts) {
  const uint32_t tid = threadIdx.x;
  const uint32_t L = min(r.hlen, r.dry_range);  // :394-396
  if (L <= (uint32_t)kDryMax) {
    dry_pass_lds<DT>(p, r, row, L, lds, tab, ts, p.dry_list + (size_t)row * p.dry_cap);
    return true;  // (at most L <= kDryHash / 2 distinct ids)
  }
  const uint32_t* sl = p.history + (size_t)row * p.history_ld + (r.hlen - L);  // read in place
  const bool global = p.dry_ghash != nullptr;
  const uint32_t slots = global ? 2u * p.dry_cap : (uint32_t)kDryHash;  // a power of two
  const uint32_t shift = 32u - (31u - __builtin_clz(slots));
  uint32_t* hkey = global ? p.dry_ghash + (size_t)row * 3 * slots : lds + kDryMax;  // ids (kEmptySlot: free)
  uint32_t* cnt = hkey + slots;                // matches at the current length
  float* val = (float*)(cnt + slots);          // values
  for (uint32_t h = tid; h < slots; h += kThreads) {
    hkey[h] = kEmptySlot;
    cnt[h] = 0;
  }
  if (tid == 0) {
    ts.dry_full = 0;
    ts.counter = 0;
  }
  __syncthreads();
  const int allowed = (int)min(r.dry_allowed, 33u);
  for (int ml = 32; ml >= allowed; --ml) {  // (allowed..=32).rev()
    if (L < (uint32_t)ml) continue;         // :399-401
    const uint32_t n = L - (uint32_t)ml;
    for (uint32_t i = tid; i < n; i += kThreads) {
      bool m = true;
      for (int t = 0; t < ml && m; ++t) m = sl[i + t] == sl[L - ml + t];
      if (!m) continue;
      const uint32_t next = sl[i + ml];
      if (next >= p.V) continue;  // logits.get_mut(next) is None
      uint32_t h = (next * 0x9e3779b1u) >> shift;
      bool placed = false;
      for (uint32_t probe = 0; probe < slots; ++probe) {
        const uint32_t prev = atomicCAS(&hkey[h], kEmptySlot, next);
        if (prev == kEmptySlot) {  // first sight: the value before DRY
          float x = load_logit<DT>(p, row, next);
          if (p.mask && !mask_allows(p, row, next)) x = neg_inf();
          val[h] = pre_stages_of(p, r, next, x);
          if (atomicAdd(&ts.counter, 1u) >= p.dry_cap) ts.dry_full = 1;  // more ids than the list holds
        }
        if (prev == kEmptySlot || prev == next) {
          atomicAdd(&cnt[h], 1u);
          placed = true;
          break;
        }
        h = (h + 1) & (slots - 1);
      }
      if (!placed) ts.dry_full = 1;  // every slot holds another id
    }
    __syncthreads();
    const float exponent = (float)(ml - allowed);
    const float pen = r.dry_mult * dpowf(r.dry_base, exponent, tab);  // :408-409
    for (uint32_t h = tid; h < slots; h += kThreads) {
      const uint32_t k = cnt[h];
      if (k) {
        float v = val[h];
        for (uint32_t j = 0; j < k; ++j) v = v - pen;  // :411
        val[h] = v;
        cnt[h] = 0;
      }
    }
    __syncthreads();
  }
  if (ts.dry_full) return false;  // (read after the barrier that ends the last length)
  uint64_t* dl = p.dry_list + (size_t)row * p.dry_cap;
  if (tid == 0) ts.counter = 0;
  __syncthreads();
  uint32_t nd;
  if (global) {  // the list in place, sorted in global memory
    for (uint32_t h = tid; h < slots; h += kThreads) {
      const uint32_t id = hkey[h];
      if (id != kEmptySlot) dl[atomicAdd(&ts.counter, 1u)] = ((uint64_t)id << 32) | __float_as_uint(val[h]);
    }
    __syncthreads();
    nd = ts.counter;
    // ascending by id: sorted descending on the complemented ids, then complemented back
    for (uint32_t i = tid; i < nd; i += kThreads) dl[i] = ~dl[i];
    wide_sort(dl, nd, (uint64_t*)lds);
    for (uint32_t i = tid; i < nd; i += kThreads) dl[i] = ~dl[i];
  } else {  // (id << 32 | value bits) from the LDS table into registers, then into LDS over the
            // start of the area, the table included (its entries are in registers by then)
    constexpr int kPerT = kDryHash / kThreads;
    uint64_t mine[kPerT];
    uint32_t held = 0;  // bit q: slot tid + q * kThreads holds an id
#pragma unroll
    for (int q = 0; q < kPerT; ++q) {
      const uint32_t h = tid + q * kThreads;
      const uint32_t id = hkey[h];
      mine[q] = ((uint64_t)id << 32) | __float_as_uint(val[h]);
      if (id != kEmptySlot) held |= 1u << q;
    }
    __syncthreads();
    uint64_t* keys = (uint64_t*)lds;  // [kDryHash]
#pragma unroll
    for (int q = 0; q < kPerT; ++q)
      if ((held >> q) & 1u) keys[atomicAdd(&ts.counter, 1u)] = mine[q];
    __syncthreads();
    nd = ts.counter;
    bitonic_sort<true>(keys, nd);
    for (uint32_t i = tid; i < nd; i += kThreads) dl[i] = keys[i];
  }
  if (tid == 0) p.dry_count[row] = nd;
  __syncthreads();
  return true;
}

// The LDS DRY hash dry_pass leaves after a slice of up to kDryMax ids: the
// slot holding `id`, or kDryHash when the row's DRY pass did not penalise it.
__device__ __forceinline__ uint32_t dry_lookup(const uint32_t* hkey, uint32_t id) {
  uint32_t h = (id * 0x9e3779b1u) >> 21;
  for (int probe = 0; probe < kDryHash; ++probe) {
    const uint32_t k = hkey[h];
    if (k == id) return h;
    if (k == kEmptySlot) break;
    h = (h + 1) & (kDryHash - 1);
  }
  return kDryHash;
}

// ---------------------------------------------------------------- tail kernel

// ids / exps of sorted keys[0..n) (n >= 1) into the chain arrays; ends with a barrier.
__device__ void keys_to_chain(const uint64_t* keys, uint32_t n, uint32_t* ids, float* pr, const LibmTables& tab) {
  const float max_logit = key_value(keys[0]);
  for (uint32_t i = threadIdx.x; i < n; i += kThreads) {
    const uint64_t k = keys[i];
    ids[i] = ~(uint32_t)k;
    pr[i] = dexpf(key_value(k) - max_logit, tab);
  }
  __syncthreads();
}

// Launchers of the kernels of oxs_stream.hip and oxs_tail.hip (kind: the
// logit dtype plus kKindSoftcap / kKindDecode bits).
hipError_t launch_stream_kind(int kind, int slots, bool vec, bool mask, const Params& p, uint32_t grid,
                              hipStream_t st);
hipError_t launch_tail_kind(int kind, const Params& p, uint32_t grid, hipStream_t st);

}  // namespace oxs
