// oxs_dfa.hip — grammar masks from a DFA for MI355X (gfx950).
//
// For a batch of rows, each in its own DFA state, walks every vocabulary
// token's bytes through the transition table (crates/oxide-core/src/dfa.rs:110-148,
// crates/oxide-server/src/grammar_engine.rs:42-65) and writes the packed
// allowed-token bitmask that oxs_sample_batch reads (oxs_batch.allowed_mask).
//
// One thread per token: its bytes are read kMaxBytes at a time into registers,
// once, and each piece is walked from every row of the block's row group, whose
// states stay in registers, four rows interleaved so that four independent
// table reads are in flight per step. The table sits in LDS when it fits. A walk is a chain of dependent table reads, so the table
// lookups bound this kernel, not HBM (the token bytes and offsets are read once
// per row group). A wavefront's 64 consecutive tokens give two mask words per
// row from one ballot.
//
// A walk depends only on the state it starts from, so a decode loop computes
// the masks of every state once per grammar and vocabulary (this kernel over
// the states themselves) and gathers one row per sequence each step
// (mask_gather_kernel): a copy of ceil(V / 32) words per row.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/oxide_sampler.h"

namespace oxs_grammar {

constexpr int kThreads = 256;
constexpr int kTokPerThread = 4;      // tokens per thread (amortises the table's load into LDS)
constexpr int kRowsPerBlock = 16;     // rows walked per block
constexpr int kRowIlp = 4;            // rows walked together
constexpr int kMaxBytes = 16;         // token bytes read and walked per piece
constexpr uint32_t kLdsStates = 48;   // tables of up to 48 states (48 KB) are copied into LDS
constexpr uint32_t kErr = OXS_DFA_ERROR_STATE;
static_assert(kRowsPerBlock % kRowIlp == 0, "rows are walked kRowIlp at a time");

struct Params {
  const uint32_t* trans;
  uint32_t num_states;
  const uint32_t* offsets;
  const uint8_t* bytes;
  uint32_t num_bytes;
  uint32_t V;
  const uint32_t* states;
  uint32_t B;
  uint32_t* mask;
  int64_t mask_ld;
};

// One transition (DfaSchemaGrammar::transition, dfa.rs:110-126): a current
// state outside the table or an error entry ends the walk as invalid.
__device__ __forceinline__ void step(const uint32_t* T, uint32_t ns, uint32_t byte, uint32_t& s, bool& ok) {
  if (!ok) return;
  if (s >= ns) {
    ok = false;
    return;
  }
  s = T[s * 256u + byte];
  ok = s != kErr;
}

template <bool LDS>
__global__ __launch_bounds__(kThreads) void dfa_mask_kernel(const Params p) {
  extern __shared__ __align__(16) uint32_t s_trans[];  // [num_states * 256] with LDS
  const uint32_t tid = threadIdx.x, lane = tid & 63;
  if (LDS) {
    const uint32_t n4 = p.num_states * 64u;  // 16-byte groups
    for (uint32_t i = tid; i < n4; i += kThreads) ((uint4*)s_trans)[i] = ((const uint4*)p.trans)[i];
    __syncthreads();
  }
  const uint32_t* T = LDS ? s_trans : p.trans;
  const uint32_t ns = p.num_states;
  const uint32_t r0 = blockIdx.y * kRowsPerBlock;
  const uint32_t nr = min((uint32_t)kRowsPerBlock, p.B - r0);
  const uint32_t words = (p.V + 31u) / 32u;
  uint32_t st0[kRowsPerBlock];  // the row group's start states
#pragma unroll
  for (int q = 0; q < kRowsPerBlock; ++q) st0[q] = p.states[r0 + ((uint32_t)q < nr ? q : 0u)];
  for (int k = 0; k < kTokPerThread; ++k) {
    // consecutive tokens per wavefront, the wavefront's first one 64-aligned
    const uint32_t t = (blockIdx.x * kTokPerThread + k) * kThreads + tid;
    bool in = t < p.V;
    uint32_t b0 = 0, len = 0;
    if (in) {
      b0 = p.offsets[t];
      const uint32_t e = p.offsets[t + 1];
      if (e >= b0 && e <= p.num_bytes) len = e - b0;
      else in = false;  // a range outside the byte array: not allowed, nothing read
    }
    uint32_t s[kRowsPerBlock];
    bool ok[kRowsPerBlock];
#pragma unroll
    for (int q = 0; q < kRowsPerBlock; ++q) {
      s[q] = st0[q];
      ok[q] = in && (uint32_t)q < nr;
    }
    // the token's bytes kMaxBytes at a time, each piece read once and walked
    // from every row's state (kRowIlp rows interleaved); a lane stops when no
    // row can still allow its token
    for (uint32_t j0 = 0; j0 < len; j0 += kMaxBytes) {
      uint32_t by[kMaxBytes];
#pragma unroll
      for (int j = 0; j < kMaxBytes; ++j) by[j] = j0 + j < len ? p.bytes[b0 + j0 + j] : 0u;
      const uint32_t n = min(len - j0, (uint32_t)kMaxBytes);
#pragma unroll
      for (int q0 = 0; q0 < kRowsPerBlock; q0 += kRowIlp) {
#pragma unroll
        for (int j = 0; j < kMaxBytes; ++j) {
          if ((uint32_t)j < n) {
#pragma unroll
            for (int q = q0; q < q0 + kRowIlp; ++q) step(T, ns, by[j], s[q], ok[q]);
          }
        }
      }
      bool any = false;
#pragma unroll
      for (int q = 0; q < kRowsPerBlock; ++q) any |= ok[q];
      if (!any) break;
    }
    const uint32_t wbase = (t - lane) / 32u;  // the wavefront's first mask word
#pragma unroll
    for (int q = 0; q < kRowsPerBlock; ++q) {
      const uint64_t m = __ballot(ok[q]);
      if ((uint32_t)q < nr) {
        uint32_t* row = p.mask + (size_t)(r0 + q) * p.mask_ld;
        if (lane == 0 && wbase < words) row[wbase] = (uint32_t)m;
        if (lane == 32 && wbase + 1 < words) row[wbase + 1] = (uint32_t)(m >> 32);
      }
    }
  }
}

// Tables of at most 64 states: each token is walked once from every start
// state at the same time (independent lookups), leaving a 64-bit word whose
// bit s says whether the token walks from state s; each row's mask bit is then
// one test of its own state's bit. That is num_states x length lookups per
// token instead of rows x length. A state outside the table allows only tokens
// with no bytes. A block covers kStTok * 256 tokens and kStRows rows; the mask
// words of kStBatch rows at a time are gathered in LDS from the wavefronts'
// ballots and written as one contiguous run per row.
constexpr uint32_t kSetStates = 64;
constexpr int kStTok = 2;     // tokens per thread
constexpr int kStRows = 32;   // rows per block
constexpr int kStBatch = 8;   // rows staged in LDS per round
constexpr int kStWords = kStTok * kThreads / 32;  // mask words per row and block
template <int NS, bool LDS>  // NS: a bound on num_states (8, 16 or 64)
__global__ __launch_bounds__(kThreads) void dfa_mask_states_kernel(const Params p) {
  extern __shared__ __align__(16) uint32_t s_trans[];  // [num_states * 256] with LDS
  __shared__ uint32_t s_words[kStBatch][kStWords];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (LDS) {
    const uint32_t n4 = p.num_states * 64u;
    for (uint32_t i = tid; i < n4; i += kThreads) ((uint4*)s_trans)[i] = ((const uint4*)p.trans)[i];
    __syncthreads();
  }
  const uint32_t* T = LDS ? s_trans : p.trans;
  const uint32_t ns = p.num_states;  // <= NS
  const uint32_t words = (p.V + 31u) / 32u;
  const uint32_t tbase = blockIdx.x * (kStTok * kThreads);
  const uint32_t r0 = blockIdx.y * kStRows;
  const uint32_t nr = min((uint32_t)kStRows, p.B - r0);
  const uint32_t my_state = p.states[r0 + (lane < nr ? lane : 0u)];  // lane q holds row r0 + q's state
  uint64_t alive[kStTok];
  bool empty[kStTok];
#pragma unroll
  for (int k = 0; k < kStTok; ++k) {
    const uint32_t t = tbase + k * kThreads + tid;
    bool in = t < p.V;
    uint32_t b0 = 0, len = 0;
    if (in) {
      b0 = p.offsets[t];
      const uint32_t e = p.offsets[t + 1];
      if (e >= b0 && e <= p.num_bytes) len = e - b0;
      else in = false;  // a range outside the byte array: not allowed, nothing read
    }
    uint32_t cur[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) cur[s] = (uint32_t)s;
    uint64_t a = ns >= 64u ? ~0ull : ((1ull << ns) - 1ull);
    if (!in) a = 0;
    // the bytes kMaxBytes at a time, all loads of a piece issued together
    for (uint32_t j0 = 0; j0 < len && a; j0 += kMaxBytes) {
      uint32_t by[kMaxBytes];
#pragma unroll
      for (int j = 0; j < kMaxBytes; ++j) by[j] = j0 + j < len ? p.bytes[b0 + j0 + j] : 0u;
      const uint32_t n = min(len - j0, (uint32_t)kMaxBytes);
#pragma unroll
      for (int j = 0; j < kMaxBytes; ++j) {
        if ((uint32_t)j < n) {
#pragma unroll
          for (int s = 0; s < NS; ++s) {
            if ((a >> s) & 1ull) {  // (DfaSchemaGrammar::transition, dfa.rs:110-126)
              const uint32_t c = cur[s];
              const uint32_t nxt = c < ns ? T[c * 256u + by[j]] : kErr;
              if (nxt == kErr) a &= ~(1ull << s);
              cur[s] = nxt;
            }
          }
        }
      }
    }
    alive[k] = a;
    empty[k] = in && len == 0;  // allowed from every state, even outside the table
  }
  static_assert(kStRows <= 64, "one row state per lane");
  for (uint32_t rb = 0; rb < nr; rb += kStBatch) {
#pragma unroll
    for (int q = 0; q < kStBatch; ++q) {
      if (rb + q < nr) {
        const uint32_t st = (uint32_t)__builtin_amdgcn_readlane((int)my_state, (int)(rb + q));
#pragma unroll
        for (int k = 0; k < kStTok; ++k) {
          const bool ok = st < ns ? ((alive[k] >> st) & 1ull) != 0 : empty[k];
          const uint64_t m = __ballot(ok);
          const uint32_t w = (k * kThreads + 64u * wave) / 32u;  // block-local word of this ballot
          if (lane == 0) {
            s_words[q][w] = (uint32_t)m;
            s_words[q][w + 1] = (uint32_t)(m >> 32);
          }
        }
      }
    }
    __syncthreads();
    if (tid < (uint32_t)(kStBatch * kStWords)) {
      const uint32_t q = tid / kStWords, w = tid % kStWords;
      const uint32_t gw = blockIdx.x * kStWords + w;
      if (rb + q < nr && gw < words) p.mask[(size_t)(r0 + rb + q) * p.mask_ld + gw] = s_words[q][w];
    }
    __syncthreads();
  }
}

template <int NS>
static void launch_states(const Params& p, dim3 grid, bool lds, size_t lds_bytes, hipStream_t st) {
  if (lds) hipLaunchKernelGGL((dfa_mask_states_kernel<NS, true>), grid, dim3(kThreads), lds_bytes, st, p);
  else hipLaunchKernelGGL((dfa_mask_states_kernel<NS, false>), grid, dim3(kThreads), 0, st, p);
}

// Row b of the output is row min(states[b], num_states) of the per-state
// masks (row num_states holds the masks of every state outside the table).
constexpr int kGatherWords = 4 * kThreads;  // words per gather block
__global__ __launch_bounds__(kThreads) void mask_gather_kernel(const uint32_t* __restrict__ table, uint32_t num_states,
                                                              int64_t table_ld, uint32_t words,
                                                              const uint32_t* __restrict__ states,
                                                              uint32_t* __restrict__ mask, int64_t mask_ld) {
  const uint32_t row = blockIdx.y;
  const uint32_t s = min(states[row], num_states);
  const uint32_t* src = table + (size_t)s * table_ld;
  uint32_t* dst = mask + (size_t)row * mask_ld;
  const uint32_t w0 = blockIdx.x * kGatherWords;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t w = w0 + k * kThreads + threadIdx.x;
    if (w < words) dst[w] = src[w];
  }
}

// ---------------------------------------------------------------- static masks

// The first character of a token's text, decoded from UTF-8 (Rust's
// text.chars().next()); a malformed sequence (bad continuation, truncation,
// overlong form, surrogate, beyond U+10FFFF) gives U+FFFD, as a lossy decode
// would (the reference's vocabulary is always valid UTF-8).
__device__ __forceinline__ uint32_t first_char(const uint8_t* b, uint32_t len) {
  const uint32_t c0 = b[0];
  if (c0 < 0x80u) return c0;
  uint32_t n, c;
  if ((c0 & 0xe0u) == 0xc0u) { n = 1; c = c0 & 0x1fu; }
  else if ((c0 & 0xf0u) == 0xe0u) { n = 2; c = c0 & 0x0fu; }
  else if ((c0 & 0xf8u) == 0xf0u) { n = 3; c = c0 & 0x07u; }
  else return 0xfffdu;
  if (len < n + 1) return 0xfffdu;
  for (uint32_t i = 1; i <= n; ++i) {
    const uint32_t ci = b[i];
    if ((ci & 0xc0u) != 0x80u) return 0xfffdu;
    c = (c << 6) | (ci & 0x3fu);
  }
  const uint32_t least = n == 1 ? 0x80u : n == 2 ? 0x800u : 0x10000u;
  if (c < least || (c >= 0xd800u && c <= 0xdfffu) || c > 0x10ffffu) return 0xfffdu;
  return c;
}

__device__ __forceinline__ void write_mask_bits(bool ok, uint32_t t, uint32_t words, uint32_t* mask) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint64_t m = __ballot(ok);
  const uint32_t wbase = (t - lane) / 32u;
  if (lane == 0 && wbase < words) mask[wbase] = (uint32_t)m;
  if (lane == 32 && wbase + 1 < words) mask[wbase + 1] = (uint32_t)(m >> 32);
}

struct GbnfParams {
  const uint32_t* ranges;  // [n_ranges][2]
  uint32_t n_ranges;
  const uint32_t* lit_off;  // [n_lits + 1]
  const uint8_t* lit_bytes;
  uint32_t n_lits;
  const uint32_t* offsets;
  const uint8_t* bytes;
  uint32_t num_bytes;
  uint32_t V;
  uint32_t* mask;
};

// GbnfGrammarEngine::apply_grammar_mask (crates/oxide-core/src/sampler.rs:555-583):
// a token with no characters is left alone; otherwise it is allowed when its
// first character lies in one of the rule's ranges, or when a literal starts
// with its text or its text starts with a literal. One thread per token.
__global__ __launch_bounds__(kThreads) void gbnf_mask_kernel(const GbnfParams p) {
  const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
  bool ok = false;
  if (t < p.V) {
    const uint32_t b0 = p.offsets[t], e = p.offsets[t + 1];
    if (e >= b0 && e <= p.num_bytes) {
      const uint32_t len = e - b0;
      const uint8_t* tb = p.bytes + b0;
      if (len == 0) {
        ok = true;  // text.chars().next() is None: not masked
      } else {
        const uint32_t c = first_char(tb, len);
        for (uint32_t i = 0; i < p.n_ranges && !ok; ++i) ok = c >= p.ranges[2 * i] && c <= p.ranges[2 * i + 1];
        for (uint32_t i = 0; i < p.n_lits && !ok; ++i) {
          const uint32_t lb = p.lit_off[i], ll = p.lit_off[i + 1] - lb;
          const uint32_t n = min(ll, len);  // lit.starts_with(text) || text.starts_with(lit): equal first n bytes
          bool same = true;
          for (uint32_t j = 0; j < n && same; ++j) same = p.lit_bytes[lb + j] == tb[j];
          ok = same;
        }
      }
    }
  }
  write_mask_bits(ok, t, (p.V + 31u) / 32u, p.mask);
}

// GrammarLogitMasker::mask_logits (crates/oxide-core/src/grammar_mask.rs:55-65):
// a token whose byte b is given (token_ascii[t] < 256) is masked unless
// allowed[b]; a token without one (Rust's None) is left alone.
__global__ __launch_bounds__(kThreads) void ascii_mask_kernel(const uint8_t* __restrict__ allowed,
                                                             const uint16_t* __restrict__ token_ascii, uint32_t V,
                                                             uint32_t* __restrict__ mask) {
  const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
  bool ok = false;
  if (t < V) {
    const uint32_t b = token_ascii[t];
    ok = b >= 256u || allowed[b] != 0;
  }
  write_mask_bits(ok, t, (V + 31u) / 32u, mask);
}

}  // namespace oxs_grammar

extern "C" int oxs_dfa_mask(const oxs_dfa* dfa, const oxs_token_bytes* tokens, const uint32_t* states,
                            uint32_t batch, uint32_t* mask, int64_t mask_ld, void* stream) {
  using namespace oxs_grammar;
  if (!dfa || !tokens) return OXS_ERR_INVALID_ARGUMENT;
  if (batch == 0 || tokens->vocab == 0) return OXS_OK;
  if ((dfa->num_states && !dfa->transitions) || !tokens->offsets || !tokens->bytes || !states || !mask)
    return OXS_ERR_INVALID_ARGUMENT;
  if (mask_ld < (int64_t)((tokens->vocab + 31u) / 32u)) return OXS_ERR_INVALID_ARGUMENT;
  // token indices stay below 2^31 and row groups within the grid's y extent
  if (tokens->vocab > (1u << 31) || batch > 65535u * (uint32_t)min(kRowsPerBlock, kStRows))
    return OXS_ERR_INVALID_ARGUMENT;
  Params p;
  p.trans = dfa->transitions;
  p.num_states = dfa->num_states;
  p.offsets = tokens->offsets;
  p.bytes = tokens->bytes;
  p.num_bytes = tokens->num_bytes;
  p.V = tokens->vocab;
  p.states = states;
  p.B = batch;
  p.mask = mask;
  p.mask_ld = mask_ld;
  hipStream_t st = (hipStream_t)stream;
  // the table is copied into LDS in 16-byte pieces: small and 16-byte aligned tables only
  const bool lds = p.num_states <= kLdsStates && ((uintptr_t)p.trans & 15u) == 0;
  const size_t lds_bytes = lds ? p.num_states * 256u * sizeof(uint32_t) : 0;
  if (p.num_states <= kSetStates) {
    const uint32_t per_block = (uint32_t)(kStTok * kThreads);
    const dim3 grid((p.V + per_block - 1) / per_block, (batch + kStRows - 1) / kStRows);
    if (p.num_states <= 8) launch_states<8>(p, grid, lds, lds_bytes, st);
    else if (p.num_states <= 16) launch_states<16>(p, grid, lds, lds_bytes, st);
    else launch_states<64>(p, grid, lds, lds_bytes, st);
  } else {
    const uint32_t per_block = (uint32_t)(kThreads * kTokPerThread);
    const dim3 grid((p.V + per_block - 1) / per_block, (batch + kRowsPerBlock - 1) / kRowsPerBlock);
    hipLaunchKernelGGL(dfa_mask_kernel<false>, grid, dim3(kThreads), 0, st, p);
  }
  return hipGetLastError() == hipSuccess ? OXS_OK : OXS_ERR_HIP;
}

extern "C" int oxs_dfa_mask_gather(const uint32_t* state_masks, uint32_t num_states, int64_t state_masks_ld,
                                   uint32_t vocab, const uint32_t* states, uint32_t batch, uint32_t* mask,
                                   int64_t mask_ld, void* stream) {
  using namespace oxs_grammar;
  if (batch == 0 || vocab == 0) return OXS_OK;
  const uint32_t words = (vocab + 31u) / 32u;
  if (!state_masks || !states || !mask || state_masks_ld < (int64_t)words || mask_ld < (int64_t)words)
    return OXS_ERR_INVALID_ARGUMENT;
  if (batch > 65535u) return OXS_ERR_INVALID_ARGUMENT;  // one grid row per batch row
  const dim3 grid((words + kGatherWords - 1) / kGatherWords, batch);
  hipLaunchKernelGGL(mask_gather_kernel, grid, dim3(kThreads), 0, (hipStream_t)stream, state_masks, num_states,
                     state_masks_ld, words, states, mask, mask_ld);
  return hipGetLastError() == hipSuccess ? OXS_OK : OXS_ERR_HIP;
}

extern "C" int oxs_gbnf_mask(const oxs_gbnf_rule* rule, const oxs_token_bytes* tokens, uint32_t* mask,
                             void* stream) {
  using namespace oxs_grammar;
  if (!rule || !tokens) return OXS_ERR_INVALID_ARGUMENT;
  if (tokens->vocab == 0) return OXS_OK;
  if (!tokens->offsets || !tokens->bytes || !mask || (rule->num_ranges && !rule->ranges) ||
      (rule->num_literals && (!rule->literal_offsets || !rule->literal_bytes)))
    return OXS_ERR_INVALID_ARGUMENT;
  if (tokens->vocab > (1u << 31)) return OXS_ERR_INVALID_ARGUMENT;
  GbnfParams p;
  p.ranges = rule->ranges;
  p.n_ranges = rule->num_ranges;
  p.lit_off = rule->literal_offsets;
  p.lit_bytes = rule->literal_bytes;
  p.n_lits = rule->num_literals;
  p.offsets = tokens->offsets;
  p.bytes = tokens->bytes;
  p.num_bytes = tokens->num_bytes;
  p.V = tokens->vocab;
  p.mask = mask;
  hipLaunchKernelGGL(gbnf_mask_kernel, dim3((p.V + kThreads - 1) / kThreads), dim3(kThreads), 0,
                     (hipStream_t)stream, p);
  return hipGetLastError() == hipSuccess ? OXS_OK : OXS_ERR_HIP;
}

extern "C" int oxs_ascii_mask(const uint8_t* allowed_ascii, const uint16_t* token_ascii, uint32_t vocab,
                              uint32_t* mask, void* stream) {
  using namespace oxs_grammar;
  if (vocab == 0) return OXS_OK;
  if (!allowed_ascii || !token_ascii || !mask || vocab > (1u << 31)) return OXS_ERR_INVALID_ARGUMENT;
  hipLaunchKernelGGL(ascii_mask_kernel, dim3((vocab + kThreads - 1) / kThreads), dim3(kThreads), 0,
                     (hipStream_t)stream, allowed_ascii, token_ascii, vocab, mask);
  return hipGetLastError() == hipSuccess ? OXS_OK : OXS_ERR_HIP;
}
