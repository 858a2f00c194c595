// oxs_sampler.hip — batched token sampler for MI355X (gfx950).
//
// Replaces the per-row CPU chain of crates/oxide-core/src/sampler.rs
// (AcademicSamplerEngine::sample_token, sampler.rs:173-390) with two kernels
// per batch, launched back to back on the caller's stream:
//
// stream_kernel (grid: rows x chunks). Each block streams CH logits of one row
//   with coalesced 16-byte loads and keeps only a small candidate set per
//   wavefront. The dense stage (grammar mask) is applied in registers. The
//   sparse stages (bans, biases, newline, repetition/frequency/presence over
//   the history window) touch few ids: while the second half of the chunk is
//   still in flight, the block hashes those ids in LDS; once the values are
//   staged in LDS, one thread per hash entry writes its id's exact value. Each
//   wavefront finds a lower bound of the c-th largest of its 64 lane maxima
//   (16 ballot steps) and writes every value at or above it as a 64-bit key
//   (order-preserving bits of value * inv_temp << 32 | ~token id): keys are
//   unique and order candidates by value descending, then lower token id.
//
// tail_kernel (one block per row). Reads the row's candidate keys and the
//   wavefront thresholds into registers; if at least M = max(top_k, 256) keys
//   lie at or above the largest threshold, those keys provably contain the
//   row's top M (otherwise the block re-scans the row exactly). A bucketed
//   counting sort yields the sorted top M. One wavefront then runs softmax,
//   Mirostat or min-p / XTC / top-k / tail-free / typical / top-p,
//   renormalisation and the inverse-CDF draw without block barriers, with
//   expf/logf/log2f that reproduce glibc bit for bit and with every float sum
//   in the reference's order.
//
// The kernel boundary makes the candidate keys visible to the tail on every
// XCD without per-block cache write-backs. Nothing is allocated and nothing
// waits on the host; all workspace comes from the sampler handle.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>
#include <stdlib.h>
#include <string.h>

#include "../../include/oxide_sampler.h"
#include "oxs_libm.h"
#include "oxs_sampler_dev.h"

namespace oxs {

// ---------------------------------------------------------------- read floor

// The stream kernel's access pattern with nothing else: one block per
// (row, 8192-float chunk), eight 16-byte non-temporal loads per thread, the
// chunk's largest value (bits) written to sink[block]. Its time per launch is
// the floor one pass over the logits can reach.
__global__ __launch_bounds__(kThreads) void read_floor_kernel(const float* __restrict__ x, int64_t ld, uint32_t V,
                                                              uint32_t S, uint32_t* __restrict__ sink) {
  const uint32_t row = blockIdx.x / S, chunk = blockIdx.x - row * S;
  const uint32_t c0 = chunk * (uint32_t)kMaxChunk, c1 = min(c0 + (uint32_t)kMaxChunk, V);
  const char* rp = (const char*)(x + (size_t)row * ld);
  u32x4 q[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const uint32_t base = c0 + s * kThreads * 4 + threadIdx.x * 4;
    const uint32_t at = base < c1 ? base : V - 4;
    q[s] = __builtin_nontemporal_load((const u32x4*)(rp + (size_t)at * 4));
  }
  uint32_t m = 0;
#pragma unroll
  for (int s = 0; s < 8; ++s) m = max(max(max(m, q[s].x), max(q[s].y, q[s].z)), q[s].w);
  m = wave_reduce32(m, MaxOp{});
  __shared__ uint32_t sm[kWavesPerBlock];
  if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) sink[blockIdx.x] = max(max(sm[0], sm[1]), max(sm[2], sm[3]));
}

// ---------------------------------------------------------------- argmax

// launch_cuda_argmax (oxide-backend-cuda/src/kernels/sampling_dfa.cu:161-178):
// per row, the largest logit above -1e30 (its running maxima start at -1e30
// and only a strictly larger value replaces one, so NaN and values <= -1e30
// are never taken); a row without one gives token 0 and value -1e30.
//
// Which of several equal maxima the reference returns follows from its thread
// layout. With more than one row (one 1024-thread block per row, :2-68),
// thread t keeps the first maximum among ids i = t (mod 1024), and the two
// __shfl_down_sync trees (offsets 16 .. 1, the lower lane kept unless the
// other value is strictly larger) keep, among tied lanes, the one whose 5-bit
// index reversed bit for bit is smallest: first over the warps, then over the
// lanes of the winning warp. With one row (24 blocks of 256 threads striding
// the row by 6144, :70-159) the same holds for the block, then the warp (of
// 8), then the lane. -0.0 equals +0.0 there, and the value returned is the
// winning logit's own bits.
//
// Here every logit becomes a 64-bit key ordered exactly as that rule orders
// candidates: (order-preserving value bits << 32) | (priority << 1) | (1 for
// -0.0), the priority being the reversed warp and lane (and block) indices
// and the thread's visiting order, complemented so that larger is preferred.
// A total order reduces in any grouping, so a row is split over as many
// blocks as fill the GPU; each block folds its best key into the row's slot
// with a device-scope atomic maximum, and the row's last block (a ticket)
// writes the result and clears the slot for the next launch. The slots are
// file-scope device memory, as the reference's g_argmax_scratch_* are: calls
// that overlap on one device race on them.
constexpr uint32_t kArgRows = 16384;  // rows per launch (the host splits larger batches)
static __device__ uint64_t g_arg_best[kArgRows];
static __device__ uint32_t g_arg_ticket[kArgRows];

__device__ __forceinline__ uint32_t rev5(uint32_t x) { return __builtin_bitreverse32(x) >> 27; }
__device__ __forceinline__ uint32_t rev3(uint32_t x) { return __builtin_bitreverse32(x) >> 29; }

// The priority of logit i (31 bits, larger preferred) and its inverse. ONE:
// the batch-1 layout (q = i / 6144 < 2^18), else the 1024-thread layout
// (q = i >> 10 < 2^21); both hold for i < 2^30.
template <bool ONE>
__device__ __forceinline__ uint32_t arg_priority(uint32_t i) {
  if constexpr (ONE) {
    const uint32_t q = i / 6144u, g = i - q * 6144u;
    return ((31u - rev5(g >> 8)) << 26) | ((7u - rev3((g >> 5) & 7u)) << 23) | ((31u - rev5(g & 31u)) << 18) |
           (0x3ffffu - q);
  } else {
    const uint32_t q = i >> 10, t = i & 1023u;
    return ((31u - rev5(t >> 5)) << 26) | ((31u - rev5(t & 31u)) << 21) | (0x1fffffu - q);
  }
}
template <bool ONE>
__device__ __forceinline__ uint32_t arg_index(uint32_t pr) {
  if constexpr (ONE) {
    const uint32_t blk = rev5(31u - (pr >> 26)), w = rev3(7u - ((pr >> 23) & 7u)), l = rev5(31u - ((pr >> 18) & 31u));
    return (0x3ffffu - (pr & 0x3ffffu)) * 6144u + blk * 256u + w * 32u + l;
  } else {
    const uint32_t w = rev5(31u - (pr >> 26)), l = rev5(31u - ((pr >> 21) & 31u));
    return (0x1fffffu - (pr & 0x1fffffu)) * 1024u + w * 32u + l;
  }
}
template <bool ONE>
__device__ __forceinline__ void arg_write(uint64_t k, uint32_t row, uint32_t* out_token, float* out_val) {
  uint32_t tok = 0;
  float val = -1e30f;
  if (k) {
    const uint32_t o = (uint32_t)(k >> 32);
    tok = arg_index<ONE>((uint32_t)k >> 1);
    // bit 0 is the winner's sign bit: it tells -0.0 from +0.0
    val = o == 0x80000000u ? ((k & 1u) ? -0.0f : 0.0f) : ord2f(o);
  }
  out_token[row] = tok;
  if (out_val) out_val[row] = val;
}

// One block of TH threads per (row, chunk of NS * 4 * TH logits); NS 16-byte
// loads per thread in flight (VEC: 16-byte aligned rows, V % 4 == 0), or
// scalar loads. Each
// lane first takes the largest of its values (from -1e30, so that only larger
// values count; fmaxf drops NaN), then, among its values equal to it, the
// largest (priority << 1 | sign bit): its key. Keys reduce by maximum.
template <bool ONE, int NS, bool VEC, int TH>
__global__ __launch_bounds__(TH) void argmax_kernel(const float* __restrict__ logits, uint32_t V, int64_t ld,
                                                          uint32_t S, uint32_t* __restrict__ out_token,
                                                          float* __restrict__ out_val) {
  constexpr uint32_t CH = NS * TH * 4;
  __shared__ uint64_t s_best[TH / 64];
  const uint32_t tid = threadIdx.x;
  const uint32_t row = blockIdx.x / S, chunk = blockIdx.x - row * S;
  const uint32_t c0 = chunk * CH;
  const float* x = logits + (size_t)row * (size_t)ld;
  float f[NS][4];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const uint32_t base = c0 + s * TH * 4 + tid * 4;
    if constexpr (VEC) {
      const uint32_t at = base < V ? base : V - 4;  // in bounds; dropped below
      const u32x4 q = __builtin_nontemporal_load((const u32x4*)(x + at));
      f[s][0] = __uint_as_float(q.x);
      f[s][1] = __uint_as_float(q.y);
      f[s][2] = __uint_as_float(q.z);
      f[s][3] = __uint_as_float(q.w);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) f[s][e] = x[base + e < V ? base + e : V - 1];
    }
  }
  if (c0 + CH > V) {  // the row's last chunk: ids past V drop out
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (c0 + s * TH * 4 + tid * 4 + e >= V) f[s][e] = neg_inf();
  }
  float m = -1e30f;
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int e = 0; e < 4; ++e) m = fmaxf(m, f[s][e]);
  uint32_t lo = 0;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const uint32_t base = c0 + s * TH * 4 + tid * 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t c = __builtin_amdgcn_alignbit(arg_priority<ONE>(base + e), __float_as_uint(f[s][e]), 31);
      lo = max(lo, f[s][e] == m ? c : 0u);
    }
  }
  uint64_t best = m > -1e30f ? ((uint64_t)f2ord(m) << 32) | lo : 0ull;
  best = wave_max_u64(best);
  if ((tid & 63) == 0) s_best[tid >> 6] = best;
  __syncthreads();
  if (tid != 0) return;
  uint64_t b = s_best[0];
#pragma unroll
  for (int w = 1; w < TH / 64; ++w) b = s_best[w] > b ? s_best[w] : b;
  if (S == 1) {
    arg_write<ONE>(b, row, out_token, out_val);
    return;
  }
  // The row's blocks meet in its slot. The ticket is issued only once this
  // block's maximum has returned, i.e. has been performed where device-scope
  // atomics on the slot are serialised; the row's last ticket therefore
  // follows every block's maximum, and its exchange reads (and clears) the
  // final one. Atomics only: no other memory is handed between blocks, so no
  // cache write-back or invalidation is needed.
  const uint64_t old = __hip_atomic_fetch_max(&g_arg_best[row], b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  uint32_t one = 1u;
  asm volatile("" : "+v"(one) : "v"(old));  // `one` now depends on the returned maximum
  const uint32_t t = __hip_atomic_fetch_add(&g_arg_ticket[row], one, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (t + 1u != S) return;
  const uint64_t k = __hip_atomic_exchange(&g_arg_best[row], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_exchange(&g_arg_ticket[row], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // (an RMW, as the tickets)
  arg_write<ONE>(k, row, out_token, out_val);
}

template <bool ONE, int NS, int TH>
static void launch_argmax_ns(bool vec, uint32_t grid, hipStream_t st, const float* x, uint32_t V, int64_t ld,
                             uint32_t S, uint32_t* tok, float* val) {
  if (vec)
    hipLaunchKernelGGL((argmax_kernel<ONE, NS, true, TH>), dim3(grid), dim3(TH), 0, st, x, V, ld, S, tok, val);
  else
    hipLaunchKernelGGL((argmax_kernel<ONE, NS, false, TH>), dim3(grid), dim3(TH), 0, st, x, V, ld, S, tok, val);
}

// Rows [0, rows) of one launch (rows <= kArgRows); one: the batch-1 rule.
// Chunks of 32768, 16384, 8192 or 4096 logits (1024-thread blocks), else
// 1024 (256 threads): the largest that still gives a block per CU. Larger
// chunks mean fewer blocks meeting in a row's slot, whose atomics queue on
// one address: 16 blocks per row cost 1.3 us more than 4 at 64 x 128256.
static hipError_t launch_argmax(bool one, const float* x, uint32_t V, int64_t ld, uint32_t rows, uint32_t* tok,
                                float* val, hipStream_t st) {
  const bool vec = ((uintptr_t)x % 16u) == 0 && ld % 4 == 0 && V % 4 == 0;
  constexpr uint32_t chunks[5] = {32768, 16384, 8192, 4096, 1024};
  int pick = 4;
  for (int c = 0; c < 4; ++c)
    if ((V + (uint64_t)chunks[c] - 1) / chunks[c] * rows >= 256u) {
      pick = c;
      break;
    }
  const uint32_t S = (uint32_t)((V + (uint64_t)chunks[pick] - 1) / chunks[pick]);
  const uint32_t grid = rows * S;
  switch (pick) {
    case 0: one ? launch_argmax_ns<true, 8, 1024>(vec, grid, st, x, V, ld, S, tok, val)
                : launch_argmax_ns<false, 8, 1024>(vec, grid, st, x, V, ld, S, tok, val); break;
    case 1: one ? launch_argmax_ns<true, 4, 1024>(vec, grid, st, x, V, ld, S, tok, val)
                : launch_argmax_ns<false, 4, 1024>(vec, grid, st, x, V, ld, S, tok, val); break;
    case 2: one ? launch_argmax_ns<true, 2, 1024>(vec, grid, st, x, V, ld, S, tok, val)
                : launch_argmax_ns<false, 2, 1024>(vec, grid, st, x, V, ld, S, tok, val); break;
    case 3: one ? launch_argmax_ns<true, 1, 1024>(vec, grid, st, x, V, ld, S, tok, val)
                : launch_argmax_ns<false, 1, 1024>(vec, grid, st, x, V, ld, S, tok, val); break;
    default: one ? launch_argmax_ns<true, 1, 256>(vec, grid, st, x, V, ld, S, tok, val)
                 : launch_argmax_ns<false, 1, 256>(vec, grid, st, x, V, ld, S, tok, val); break;
  }
  return hipGetLastError();
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
// (several per CU on 256 CUs), within kMaxChunk and kMaxChunks, but no
// smaller chunks than needed to keep a row at 64 wavefront records: past
// that, each wavefront's share of the 2048-key union drops to 16 keys or
// fewer and its threshold to the 8th lane maximum, and most rows of a small
// batch would fail the top-M proof and take the exact re-scan.
static bool choose_geometry(uint32_t B, uint32_t V, int dtype, Geometry* g) {
  const uint32_t epl = dtype == OXS_DTYPE_F32 ? 4 : 8;
  const uint32_t tile = kThreads * epl;
  int best = -1;
  for (int slots = 8; slots >= 1; slots >>= 1) {
    const uint32_t ch = slots * tile;
    if (ch > (uint32_t)kMaxChunk) continue;
    const uint32_t S = (V + ch - 1) / ch;
    if (S > (uint32_t)kMaxChunks) continue;
    if (best >= 0 && S * (uint32_t)kWavesPerBlock > 64u) break;
    best = slots;  // smaller slots keep overwriting while the grid stays small
    if ((uint64_t)B * S >= 1024) break;
  }
  if (best < 0) return false;
  g->slots = best;
  g->CH = best * tile;
  g->S = (V + g->CH - 1) / g->CH;
  const uint32_t W = g->S * kWavesPerBlock;
  g->cap_w = floor_pow2(min(32u, (uint32_t)(W > 64u ? kUnionBig : kUnionMax) / W));
  const uint32_t cw = (3u * 256u + W - 1) / W + 6u;
  g->c_w = max(1u, min(g->cap_w / 2, cw));
  return true;
}

static hipError_t launch_kind(int kind, int slots, bool vec, bool mask, const Params& p, uint32_t grid_a,
                              uint32_t grid_b, hipStream_t st) {
  const hipError_t e = launch_stream_kind(kind, slots, vec, mask, p, grid_a, st);
  if (e != hipSuccess) return e;
  return launch_tail_kind(kind, p, grid_b, st);
}

}  // namespace oxs

// ---------------------------------------------------------------- C ABI

struct oxs_sampler {
  int device;
  oxs_limits limits;
  uint64_t* lists;
  uint64_t* wave_theta;
  uint32_t* wave_count;
  uint64_t* libm;
  uint64_t* dry_list;
  uint32_t* dry_count;
  uint32_t* dry_ghash;  // [max_batch][3][2 * dry_cap]
  uint32_t dry_cap;     // a row's DRY list entries: max_dry_ids kept to max_vocab, a power of two
  uint32_t* row_steps;  // [max_batch] decode steps each row has handed to the host
  uint32_t* path_counts;  // [kPathKinds] rows per top-M selection path
  uint64_t* wide_keys;    // rows with top_k > 1024 (max_top_k > 1024 only), else NULL
  uint32_t* wide_arr;
  uint32_t wide_n2, wide_ld;
  bool count_paths;
  size_t bytes;
};

namespace oxs {

// The device memory one sampling call uses besides its inputs and outputs,
// and the batch it is sized for: a sampler's allocations, or the static
// array of the no-allocation entry point.
struct Workspace {
  uint32_t max_batch, max_vocab;
  uint64_t* lists;        // [max_batch][union slots]
  uint64_t* wave_theta;   // [max_batch][kMaxChunks * kWavesPerBlock]
  uint32_t* wave_count;   // [max_batch][kMaxChunks * kWavesPerBlock]
  uint64_t* libm;         // [kLibmWords]
  uint64_t* dry_list;     // [max_batch][dry_cap]
  uint32_t* dry_count;    // [max_batch]
  uint32_t* dry_ghash;    // [max_batch][3][2 * dry_cap], or null: DRY slices past kDryMax use the LDS hash
  uint32_t dry_cap;
  uint32_t* row_steps;    // [max_batch] (decode steps only; may be null otherwise)
  uint32_t* path_counts;  // [kPathKinds] or null (counting off)
  uint64_t* wide_keys;    // [max_batch][wide_n2] or null: rows with max(top_k, 256) > kMaxM are then unsupported
  uint32_t* wide_arr;     // [max_batch][7 * wide_ld]
  uint32_t wide_cap, wide_n2, wide_ld;
};

__device__ __forceinline__ uint64_t libm_word(uint32_t i) {  // the workspace's libm layout
  if (i < 32u) return oxs_libm::kExp2Tab[i];
  if (i < 48u) return (uint64_t)__double_as_longlong(oxs_libm::kLogInvc[i - 32u]);
  if (i < 64u) return (uint64_t)__double_as_longlong(oxs_libm::kLnLogc[i - 48u]);
  return (uint64_t)__double_as_longlong(oxs_libm::kLog2Logc[i - 64u]);
}

// Copies the libm tables into a workspace (one block; threads past
// kLibmWords do nothing).
__global__ void libm_fill_kernel(uint64_t* __restrict__ dst) {
  if (threadIdx.x < (uint32_t)kLibmWords) dst[threadIdx.x] = libm_word(threadIdx.x);
}

// ------------------------------------------------ no-allocation workspace
// The workspace of oxs_sample_batch_static: one file-scope device array per
// GPU, laid out as below for OXS_STATIC_MAX_BATCH rows of up to
// OXS_STATIC_MAX_VOCAB logits. Host code never uses `scratch` itself (on the
// host the name stands for no device address): each device's address comes
// from hipGetSymbolAddress, once, and is kept in g_static_ws.
constexpr size_t kStaticB = OXS_STATIC_MAX_BATCH;
constexpr size_t kStaticW = (size_t)kMaxChunks * kWavesPerBlock;  // wavefront records per row
constexpr size_t kStOffLists = 0;                                         // u64 [B][kUnionBig]
constexpr size_t kStOffTheta = kStOffLists + kStaticB * kUnionBig;        // u64 [B][W]
constexpr size_t kStOffDry = kStOffTheta + kStaticB * kStaticW;           // u64 [B][kDryList]
constexpr size_t kStOffLibm = kStOffDry + kStaticB * kDryList;            // u64 [kLibmWords]
constexpr size_t kStOffCount = kStOffLibm + (size_t)kLibmWords;           // u32 [B][W]
constexpr size_t kStOffDryCount = kStOffCount + kStaticB * kStaticW / 2;  // u32 [B]
constexpr size_t kStaticWords = kStOffDryCount + kStaticB / 2;
static_assert(OXS_STATIC_MAX_VOCAB <= (uint64_t)kMaxChunks * kMaxChunk, "static vocabulary beyond the row limit");
static_assert(kStaticB % 2 == 0 && kStaticW % 2 == 0, "u32 regions start on 8-byte boundaries");

static __device__ __align__(256) uint64_t scratch[kStaticWords];

constexpr int kStaticMaxDevices = 64;
struct StaticWs {
  uint64_t* base;  // this device's copy of `scratch` (device address), null until set up
};
static StaticWs g_static_ws[kStaticMaxDevices];
static std::mutex g_static_mu;

// The workspace view of a device's static array.
static Workspace static_workspace(uint64_t* base) {
  Workspace w;
  w.max_batch = OXS_STATIC_MAX_BATCH;
  w.max_vocab = OXS_STATIC_MAX_VOCAB;
  w.lists = base + kStOffLists;
  w.wave_theta = base + kStOffTheta;
  w.wave_count = (uint32_t*)(base + kStOffCount);
  w.libm = base + kStOffLibm;
  w.dry_list = base + kStOffDry;
  w.dry_count = (uint32_t*)(base + kStOffDryCount);
  w.dry_ghash = nullptr;
  w.dry_cap = kDryList;
  w.row_steps = nullptr;
  w.path_counts = nullptr;
  w.wide_keys = nullptr;
  w.wide_arr = nullptr;
  w.wide_cap = w.wide_n2 = w.wide_ld = 0;
  return w;
}

}  // namespace oxs

static oxs::Workspace sampler_workspace(const oxs_sampler* s) {
  oxs::Workspace w;
  w.max_batch = s->limits.max_batch;
  w.max_vocab = s->limits.max_vocab;
  w.lists = s->lists;
  w.wave_theta = s->wave_theta;
  w.wave_count = s->wave_count;
  w.libm = s->libm;
  w.dry_list = s->dry_list;
  w.dry_count = s->dry_count;
  w.dry_ghash = s->dry_ghash;
  w.dry_cap = s->dry_cap;
  w.row_steps = s->row_steps;
  w.path_counts = s->count_paths ? s->path_counts : nullptr;
  w.wide_keys = s->wide_keys;
  w.wide_arr = s->wide_arr;
  w.wide_cap = s->limits.max_top_k;
  w.wide_n2 = s->wide_n2;
  w.wide_ld = s->wide_ld;
  return w;
}

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
    case OXS_ERR_TIMEOUT: return "timed out waiting for the device";
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
  // a pool never holds more than V keys (filter_k = min(max(top_k, 256), len), sampler.rs:274)
  const uint32_t mtk = min(limits->max_top_k ? limits->max_top_k : 256u, max(limits->max_vocab, 256u));
  if ((uint64_t)limits->max_vocab > (uint64_t)oxs::kMaxChunks * oxs::kMaxChunk) return OXS_ERR_LIMITS;
  if (hipSetDevice(device) != hipSuccess) return OXS_ERR_HIP;
  oxs_sampler* s = (oxs_sampler*)calloc(1, sizeof(oxs_sampler));
  if (!s) return OXS_ERR_INVALID_ARGUMENT;
  s->device = device;
  s->limits = *limits;
  s->limits.max_top_k = mtk;
  const size_t B = limits->max_batch;
  const size_t W = (size_t)oxs::kMaxChunks * oxs::kWavesPerBlock;
  {  // a slice penalises at most V distinct ids; slices of up to kDryMax ids (the LDS pass) always fit
    const uint32_t asked = limits->max_dry_ids ? limits->max_dry_ids : (uint32_t)oxs::kDryListBig;
    const uint32_t want = min(max(asked, (uint32_t)oxs::kDryMax), limits->max_vocab);
    uint32_t cap = 2;
    while (cap < want) cap <<= 1;
    s->dry_cap = cap;
  }
  const size_t dcap = s->dry_cap;
  // rows over 16 chunks (more than 64 wavefront records) use the 4096-key union
  const size_t b_lists =
      B * (size_t)(limits->max_vocab > 16u * (uint32_t)oxs::kMaxChunk ? oxs::kUnionBig : oxs::kUnionMax) *
      sizeof(uint64_t);
  const size_t b_theta = B * W * sizeof(uint64_t);
  const size_t b_count = B * W * sizeof(uint32_t);
  bool ok = hipMalloc((void**)&s->lists, b_lists) == hipSuccess &&
                  hipMalloc((void**)&s->wave_theta, b_theta) == hipSuccess &&
                  hipMalloc((void**)&s->wave_count, b_count) == hipSuccess &&
                  hipMalloc((void**)&s->libm, oxs::kLibmWords * sizeof(uint64_t)) == hipSuccess &&
                  hipMalloc((void**)&s->dry_list, B * dcap * sizeof(uint64_t)) == hipSuccess &&
                  hipMalloc((void**)&s->dry_ghash, B * 6 * dcap * sizeof(uint32_t)) == hipSuccess &&
                  hipMalloc((void**)&s->dry_count, B * sizeof(uint32_t)) == hipSuccess &&
                  hipMalloc((void**)&s->row_steps, B * sizeof(uint32_t)) == hipSuccess &&
                  hipMemset(s->row_steps, 0, B * sizeof(uint32_t)) == hipSuccess &&
                  hipMalloc((void**)&s->path_counts, oxs::kPathKinds * sizeof(uint32_t)) == hipSuccess &&
                  hipMemset(s->path_counts, 0, oxs::kPathKinds * sizeof(uint32_t)) == hipSuccess;
  size_t b_wide = 0;
  if (ok && mtk > (uint32_t)oxs::kMaxM) {  // rows with top_k > 1024: the wide kernel's workspace
    uint32_t n2 = 1;
    while (n2 < mtk) n2 <<= 1;
    s->wide_n2 = n2;
    s->wide_ld = (mtk + 16u + 3u) & ~3u;
    const size_t b_wk = B * (size_t)n2 * sizeof(uint64_t), b_wa = B * 7 * (size_t)s->wide_ld * sizeof(uint32_t);
    ok = hipMalloc((void**)&s->wide_keys, b_wk) == hipSuccess && hipMalloc((void**)&s->wide_arr, b_wa) == hipSuccess;
    b_wide = b_wk + b_wa;
  }
  s->bytes = b_lists + b_theta + b_count + oxs::kLibmWords * sizeof(uint64_t) +
             B * (dcap * (sizeof(uint64_t) + 6 * sizeof(uint32_t)) + 2 * sizeof(uint32_t)) +
             oxs::kPathKinds * sizeof(uint32_t) +
             b_wide;
  if (ok) {  // the libm tables, as bit patterns, in the workspace
    uint64_t host[oxs::kLibmWords];
    ok = hipMemcpyFromSymbol(host, HIP_SYMBOL(oxs_libm::kExp2Tab), 32 * sizeof(uint64_t)) == hipSuccess &&
         hipMemcpyFromSymbol(host + 32, HIP_SYMBOL(oxs_libm::kLogInvc), 16 * sizeof(double)) == hipSuccess &&
         hipMemcpyFromSymbol(host + 48, HIP_SYMBOL(oxs_libm::kLnLogc), 16 * sizeof(double)) == hipSuccess &&
         hipMemcpyFromSymbol(host + 64, HIP_SYMBOL(oxs_libm::kLog2Logc), 16 * sizeof(double)) == hipSuccess &&
         hipMemcpy(s->libm, host, sizeof(host), hipMemcpyHostToDevice) == hipSuccess;
  }
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
  if (s->libm) (void)hipFree(s->libm);
  if (s->dry_list) (void)hipFree(s->dry_list);
  if (s->dry_count) (void)hipFree(s->dry_count);
  if (s->dry_ghash) (void)hipFree(s->dry_ghash);
  if (s->row_steps) (void)hipFree(s->row_steps);
  if (s->path_counts) (void)hipFree(s->path_counts);
  if (s->wide_keys) (void)hipFree(s->wide_keys);
  if (s->wide_arr) (void)hipFree(s->wide_arr);
  free(s);
  return OXS_OK;
}

size_t oxs_sampler_workspace_bytes(const oxs_sampler* s) { return s ? s->bytes : 0; }

int oxs_sampler_count_paths(oxs_sampler* s, int enable) {
  if (!s) return OXS_ERR_INVALID_ARGUMENT;
  if (hipSetDevice(s->device) != hipSuccess) return OXS_ERR_HIP;
  if (hipDeviceSynchronize() != hipSuccess ||
      hipMemset(s->path_counts, 0, oxs::kPathKinds * sizeof(uint32_t)) != hipSuccess ||
      hipDeviceSynchronize() != hipSuccess)
    return OXS_ERR_HIP;
  s->count_paths = enable != 0;
  return OXS_OK;
}

int oxs_sampler_path_counts(const oxs_sampler* s, uint32_t* counts) {
  if (!s || !counts) return OXS_ERR_INVALID_ARGUMENT;
  if (hipSetDevice(s->device) != hipSuccess) return OXS_ERR_HIP;
  if (hipDeviceSynchronize() != hipSuccess ||
      hipMemcpy(counts, s->path_counts, oxs::kPathKinds * sizeof(uint32_t), hipMemcpyDeviceToHost) != hipSuccess)
    return OXS_ERR_HIP;
  return OXS_OK;
}

}  // extern "C"

// One sampling launch pair over workspace `ws`; `io` (a decode step) may be NULL.
static int sample_impl(const oxs::Workspace& ws, const oxs_batch* b, const oxs_decode_io* io, void* stream) {
  using namespace oxs;
  if (!b) return OXS_ERR_INVALID_ARGUMENT;
  if (b->vocab == 0) return OXS_ERR_SHAPE_MISMATCH;  // sampler.rs:179-181
  if (b->batch == 0) return OXS_OK;
  if (b->batch > ws.max_batch || b->vocab > ws.max_vocab) return OXS_ERR_LIMITS;
  if (!b->logits || !b->configs || !b->out_tokens) return OXS_ERR_INVALID_ARGUMENT;
  if (b->logits_dtype != OXS_DTYPE_F32 && b->logits_dtype != OXS_DTYPE_BF16) return OXS_ERR_INVALID_ARGUMENT;
  if (b->logits_ld < (int64_t)b->vocab || b->logits_ld > (int64_t)UINT32_MAX) return OXS_ERR_INVALID_ARGUMENT;
  if (b->allowed_mask && b->mask_ld != 0 && b->mask_ld < (int64_t)((b->vocab + 31) / 32))
    return OXS_ERR_INVALID_ARGUMENT;  // 0: one mask for every row
  if (!b->uniforms && !b->rng_state) return OXS_ERR_INVALID_ARGUMENT;
  if (b->history && (!b->history_len || b->history_ld <= 0 || b->history_ld > (int64_t)UINT32_MAX))
    return OXS_ERR_INVALID_ARGUMENT;
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
  p.softcap = b->logit_softcap > 0.0f ? b->logit_softcap : 0.0f;  // NaN and <= 0: off (lib.rs:3244)
  p.S = g.S;
  p.CH = g.CH;
  p.cap_w = g.cap_w;
  p.cap_shift = (uint32_t)__builtin_ctz(g.cap_w);
  p.c_w = g.c_w;
  p.lists = ws.lists;
  p.wave_theta = ws.wave_theta;
  p.wave_count = ws.wave_count;
  p.libm = ws.libm;
  p.dry_list = ws.dry_list;
  p.dry_count = ws.dry_count;
  p.dry_ghash = ws.dry_ghash;
  p.dry_cap = ws.dry_cap;
  p.path_counts = ws.path_counts;
  p.wide_keys = ws.wide_keys;
  p.wide_arr = ws.wide_arr;
  p.wide_cap = ws.wide_cap;
  p.wide_n2 = ws.wide_n2;
  p.wide_ld = ws.wide_ld;
  if (io) {
    if (!ws.row_steps) return OXS_ERR_INVALID_ARGUMENT;
    p.flags |= kFlagDecode;
    p.dec_token = io->current_token;
    p.dec_pos = io->current_position;
    p.dec_count = io->generated_count;
    p.host_tokens = io->host_tokens;
    p.row_steps = ws.row_steps;
  }
  // Group rows by XCD when the batch divides evenly over the 8 XCDs.
  p.rpx = (b->batch % 8 == 0) ? b->batch / 8 : 0;
  const uint32_t epl = b->logits_dtype == OXS_DTYPE_F32 ? 4 : 8;
  const bool vec = ((uintptr_t)b->logits % 16 == 0) && ((size_t)b->logits_ld % epl == 0) &&
                   (b->vocab % epl == 0);
  const bool mask = b->allowed_mask != nullptr;
  const uint32_t grid_a = b->batch * g.S;
  const uint32_t grid_b = b->batch;
  hipStream_t st = (hipStream_t)stream;
  const int kind = b->logits_dtype | (p.softcap > 0.0f ? kKindSoftcap : 0) | (io ? kKindDecode : 0);
  const hipError_t e = launch_kind(kind, g.slots, vec, mask, p, grid_a, grid_b, st);
  return e == hipSuccess ? OXS_OK : OXS_ERR_HIP;
}

extern "C" {

int oxs_sample_batch(oxs_sampler* s, const oxs_batch* b, void* stream) {
  if (!s || (b && (b->flags & oxs::kFlagDecode))) return OXS_ERR_INVALID_ARGUMENT;  // not a public flag
  return sample_impl(sampler_workspace(s), b, nullptr, stream);
}

int oxs_decode_step(oxs_sampler* s, const oxs_batch* b, const oxs_decode_io* io, void* stream) {
  if (!s || !io || (b && (b->flags & oxs::kFlagDecode))) return OXS_ERR_INVALID_ARGUMENT;
  return sample_impl(sampler_workspace(s), b, io, stream);
}

int oxs_sample_batch_static(const oxs_batch* b, void* stream) {
  using namespace oxs;
  if (!b || (b->flags & kFlagDecode)) return OXS_ERR_INVALID_ARGUMENT;
  if (b->batch > OXS_STATIC_MAX_BATCH || b->vocab > OXS_STATIC_MAX_VOCAB) return OXS_ERR_LIMITS;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return OXS_ERR_NO_DEVICE;
  if (dev < 0 || dev >= kStaticMaxDevices) return OXS_ERR_UNSUPPORTED;
  uint64_t* base = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_static_mu);
    base = g_static_ws[dev].base;
    if (!base) {  // this device's first call: find its copy of the array, fill the libm tables
      hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
      if (hipStreamIsCapturing((hipStream_t)stream, &cs) != hipSuccess) return OXS_ERR_HIP;
      if (cs != hipStreamCaptureStatusNone) return OXS_ERR_INVALID_ARGUMENT;  // set-up waits: not under capture
      uint64_t* ptr = nullptr;
      if (hipGetSymbolAddress((void**)&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return OXS_ERR_HIP;
      hipLaunchKernelGGL(libm_fill_kernel, dim3(1), dim3(kThreads), 0, (hipStream_t)stream, ptr + kStOffLibm);
      if (hipGetLastError() != hipSuccess || hipStreamSynchronize((hipStream_t)stream) != hipSuccess)
        return OXS_ERR_HIP;
      g_static_ws[dev].base = ptr;
      base = ptr;
    }
  }
  return sample_impl(static_workspace(base), b, nullptr, stream);
}

int oxs_host_alloc(size_t bytes, void** out) {
  if (!out || bytes == 0) return OXS_ERR_INVALID_ARGUMENT;
  *out = nullptr;
  // mapped and coherent: the GPU's stores reach the host without a copy
  void* h = nullptr;
  if (hipHostMalloc(&h, bytes, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess) return OXS_ERR_HIP;
  void* d = nullptr;
  if (hipHostGetDevicePointer(&d, h, 0) != hipSuccess || d != h) {  // one address on both sides
    (void)hipHostFree(h);
    return OXS_ERR_UNSUPPORTED;
  }
  memset(h, 0, bytes);
  *out = h;
  return OXS_OK;
}

int oxs_argmax(const float* logits, uint32_t vocab, int64_t logits_ld, uint32_t batch, uint32_t* out_token,
               float* out_max_val, void* stream) {
  if (batch == 0) return OXS_OK;
  if (vocab == 0) return OXS_ERR_SHAPE_MISMATCH;
  if (!logits || !out_token || logits_ld < (int64_t)vocab || vocab > (1u << 30)) return OXS_ERR_INVALID_ARGUMENT;
  for (uint32_t r0 = 0; r0 < batch; r0 += oxs::kArgRows) {  // groups of rows that share the slots in turn
    const uint32_t rows = batch - r0 < oxs::kArgRows ? batch - r0 : oxs::kArgRows;
    const hipError_t e = oxs::launch_argmax(batch == 1, logits + (size_t)r0 * (size_t)logits_ld, vocab, logits_ld,
                                            rows, out_token + r0, out_max_val ? out_max_val + r0 : nullptr,
                                            (hipStream_t)stream);
    if (e != hipSuccess) return OXS_ERR_HIP;
  }
  return OXS_OK;
}

int oxs_read_floor(const float* logits, uint32_t vocab, int64_t logits_ld, uint32_t batch, uint32_t* sink,
                   void* stream) {
  if (batch == 0) return OXS_OK;
  if (!logits || !sink || vocab < 4 || vocab % 4 != 0 || logits_ld < (int64_t)vocab || logits_ld % 4 != 0 ||
      ((uintptr_t)logits & 15u) != 0)
    return OXS_ERR_INVALID_ARGUMENT;
  const uint32_t S = (vocab + oxs::kMaxChunk - 1) / oxs::kMaxChunk;
  hipLaunchKernelGGL(oxs::read_floor_kernel, dim3(batch * S), dim3(oxs::kThreads), 0, (hipStream_t)stream, logits,
                     logits_ld, vocab, S, sink);
  return hipGetLastError() == hipSuccess ? OXS_OK : OXS_ERR_HIP;
}

int oxs_host_free(void* ptr) {
  if (!ptr) return OXS_OK;
  return hipHostFree(ptr) == hipSuccess ? OXS_OK : OXS_ERR_HIP;
}

int oxs_host_wait(const uint64_t* slots, uint32_t count, uint32_t step, uint32_t* tokens, uint64_t spin_limit) {
  if (!slots || (count && !tokens)) return OXS_ERR_INVALID_ARGUMENT;
  const volatile uint64_t* v = slots;
  for (uint64_t spins = 0;; ++spins) {
    uint32_t i = 0;
    for (; i < count; ++i) {
      const uint64_t x = v[i];  // one 8-byte load: the tag and its token together
      if ((int32_t)((uint32_t)(x >> 32) - step) < 0) break;
      tokens[i] = (uint32_t)x;
    }
    if (i == count) return OXS_OK;
    if (spin_limit && spins >= spin_limit) return OXS_ERR_TIMEOUT;
  }
}

}  // extern "C"
