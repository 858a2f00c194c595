// oxs_oracle.cpp — CPU restatement of crates/oxide-core/src/sampler.rs.
//
// TEST INFRASTRUCTURE ONLY (see oxs_oracle.h): the checker for the GPU
// sampler and the CPU baseline of bench.py. Build: oracle/Makefile
// (g++ -O2 -ffp-contract=off, no fast-math, glibc libm).
#include "oxs_oracle.h"

#include <math.h>
#include <string.h>

#include <algorithm>
#include <thread>
#include <unordered_map>
#include <unordered_set>
#include <vector>

namespace {

struct Cand {
  uint32_t id;
  float p;
};

// Descending by value, ties by lower token index. Candidates never hold NaN
// (they are filtered by `l > -inf`, sampler.rs:263), and -0.0 == +0.0 here as
// under f32::partial_cmp (sampler.rs:277, :283).
inline bool cand_desc(const Cand& a, const Cand& b) {
  if (a.p > b.p) return true;
  if (a.p < b.p) return false;
  return a.id < b.id;
}

// Rust's f32 Iterator::sum folds from -0.0 (sampler.rs:360, :494-497).
inline float rust_sum_init() { return -0.0f; }

// sampler.rs:393-415: DRY. For match_len from 32 down to allowed_len, every
// earlier occurrence of the history suffix of that length penalises the token
// that followed it; penalties accumulate in loop order.
void apply_dry_penalty(const oxs_sampling_config& c, float* logits, uint32_t vocab,
                       const uint32_t* history, uint32_t history_len) {
  uint32_t scan_start = history_len > c.dry_range ? history_len - c.dry_range : 0;
  const uint32_t* h = history + scan_start;
  uint32_t n = history_len - scan_start;
  if (c.dry_allowed_length > 32) return;  // (allowed..=32).rev() is empty
  for (int64_t match_len = 32; match_len >= (int64_t)c.dry_allowed_length; --match_len) {
    if ((int64_t)n < match_len) continue;
    const uint32_t* suffix = h + (n - match_len);
    int64_t upto = (int64_t)n - match_len;  // saturating_sub: n >= match_len here
    for (int64_t i = 0; i < upto; ++i) {
      bool eq = true;
      for (int64_t j = 0; j < match_len; ++j) {
        if (h[i + j] != suffix[j]) { eq = false; break; }
      }
      if (!eq) continue;
      uint32_t next_token = h[i + match_len];  // i + match_len < n always
      float exponent = (float)(uint64_t)(match_len - c.dry_allowed_length);
      float pw = powf(c.dry_base, exponent);
      float penalty = c.dry_multiplier * pw;
      if (next_token < vocab) logits[next_token] -= penalty;
    }
  }
}

// sampler.rs:459-490: tail-free sampling on the (un-renormalised) sorted list.
void apply_tail_free_sampling(const oxs_sampling_config& c, std::vector<Cand>& cand) {
  size_t n = cand.size();
  if (n < 3) return;
  std::vector<float> d1(n - 1), d2(n - 2);
  for (size_t i = 0; i + 1 < n; ++i) d1[i] = cand[i].p - cand[i + 1].p;
  float sum_d2 = 0.0f;
  for (size_t i = 0; i + 1 < d1.size(); ++i) {
    float diff = fabsf(d1[i] - d1[i + 1]);
    d2[i] = diff;
    sum_d2 += diff;
  }
  if (sum_d2 <= 0.0f) return;
  float inv_sum = 1.0f / sum_d2;
  float cum = 0.0f;
  size_t cutoff = n;
  for (size_t i = 0; i < d2.size(); ++i) {
    float t = d2[i] * inv_sum;
    cum += t;
    if (cum >= c.tfs_z) { cutoff = i + 1; break; }
  }
  cand.resize(std::max<size_t>(cutoff, 1));
}

// sampler.rs:493-520: locally typical sampling. Re-orders the candidates by
// |surprisal - entropy| (stable sort) and keeps the prefix reaching typical_p.
void apply_locally_typical_sampling(const oxs_sampling_config& c, std::vector<Cand>& cand) {
  float entropy = rust_sum_init();
  for (const Cand& x : cand) {
    float term = x.p > 0.0f ? (-x.p) * logf(x.p) : 0.0f;
    entropy += term;
  }
  struct Scored { uint32_t id; float p; float diff; };
  std::vector<Scored> scored(cand.size());
  for (size_t i = 0; i < cand.size(); ++i) {
    float surprisal = cand[i].p > 0.0f ? -logf(cand[i].p) : 0.0f;
    scored[i] = {cand[i].id, cand[i].p, fabsf(surprisal - entropy)};
  }
  std::stable_sort(scored.begin(), scored.end(),
                   [](const Scored& a, const Scored& b) { return a.diff < b.diff; });
  float cum = 0.0f;
  std::vector<Cand> keep;
  for (const Scored& s : scored) {
    cum += s.p;
    keep.push_back({s.id, s.p});
    if (cum >= c.typical_p) break;
  }
  cand.swap(keep);
}

struct RowIo {
  uint32_t* history;
  uint32_t* history_len;
  uint32_t history_cap;
  bool record;
  float* mu;
  uint64_t* rng_state;
  const float* uniform;
  uint32_t* token;
  uint32_t* kept_ids;
  float* kept_probs;
  uint32_t* kept_count;
  uint32_t kept_cap;
};

// Appends to generated_tokens (SamplerState::record_token, sampler.rs:155-157).
bool record(RowIo& io, uint32_t tok) {
  if (!io.record) return true;
  if (*io.history_len >= io.history_cap) return false;
  io.history[(*io.history_len)++] = tok;
  return true;
}

void write_kept(RowIo& io, const std::vector<Cand>& cand) {
  if (io.kept_count) *io.kept_count = (uint32_t)cand.size();
  size_t n = std::min<size_t>(cand.size(), io.kept_cap);
  for (size_t i = 0; i < n; ++i) {
    if (io.kept_ids) io.kept_ids[i] = cand[i].id;
    if (io.kept_probs) io.kept_probs[i] = cand[i].p;
  }
}

// AcademicSamplerEngine::sample_token, sampler.rs:173-390.
int sample_row(const oxs_sampling_config& c, const uint32_t* bias_ids, const float* bias_values,
               const uint32_t* ban_ids, float* logits, uint32_t vocab, RowIo& io) {
  const float NEG_INF = -INFINITY;
  if (vocab == 0) return OXO_SHAPE_MISMATCH;  // :179-181

  // 1. Bans, then biases (:184-193). A HashMap holds each id once; a repeated
  // id in the CSR list behaves like repeated insert (last wins).
  for (uint32_t k = 0; k < c.ban_count; ++k) {
    uint32_t id = ban_ids[c.ban_offset + k];
    if (id < vocab) logits[id] = NEG_INF;
  }
  for (uint32_t k = 0; k < c.bias_count; ++k) {
    uint32_t id = bias_ids[c.bias_offset + k];
    bool later = false;
    for (uint32_t j = k + 1; j < c.bias_count; ++j)
      if (bias_ids[c.bias_offset + j] == id) { later = true; break; }
    if (later) continue;
    if (id < vocab) logits[id] += bias_values[c.bias_offset + k];
  }

  // 2. Newline penalty (:196-200).
  if (c.penalize_nl && c.newline_token_id < vocab) logits[c.newline_token_id] -= c.newline_penalty;

  const uint32_t hist_len = *io.history_len;
  // 3. DRY (:203-205).
  if (c.dry_multiplier > 0.0f && hist_len > 0) apply_dry_penalty(c, logits, vocab, io.history, hist_len);

  // 3b. Sliding-window repetition, frequency and presence penalties (:208-246).
  if (hist_len > 0) {
    uint32_t window_len = c.repeat_last_n > 0 ? c.repeat_last_n : hist_len;
    uint32_t start = hist_len > window_len ? hist_len - window_len : 0;
    const uint32_t* w = io.history + start;
    uint32_t wn = hist_len - start;
    if (fabsf(c.repeat_penalty - 1.0f) > 1e-5f && c.repeat_penalty > 0.0f) {
      std::unordered_set<uint32_t> seen;
      for (uint32_t j = 0; j < wn; ++j) {
        uint32_t tok = w[j];
        if (seen.insert(tok).second && tok < vocab) {
          float& l = logits[tok];
          if (l > 0.0f) l /= c.repeat_penalty;
          else l *= c.repeat_penalty;
        }
      }
    }
    if (fabsf(c.frequency_penalty) > 1e-5f || fabsf(c.presence_penalty) > 1e-5f) {
      std::unordered_map<uint32_t, uint64_t> counts;
      for (uint32_t j = 0; j < wn; ++j) counts[w[j]] += 1;
      for (const auto& kv : counts) {
        if (kv.first < vocab) {
          float t = (float)kv.second * c.frequency_penalty;
          float pen = t + c.presence_penalty;
          logits[kv.first] -= pen;
        }
      }
    }
  }

  // 4. Temperature, skipped under Mirostat (:249-254).
  if (c.temperature > 0.0f && c.mirostat_mode == OXS_MIROSTAT_DISABLED) {
    float inv_temp = 1.0f / c.temperature;
    for (uint32_t i = 0; i < vocab; ++i) logits[i] *= inv_temp;
  }

  // 5. Candidate pool: every id with l > -inf (drops -inf and NaN) (:257-265).
  std::vector<Cand> cand;
  cand.reserve(1024);
  for (uint32_t i = 0; i < vocab; ++i)
    if (logits[i] > NEG_INF) cand.push_back({i, logits[i]});
  if (cand.empty()) {  // :267-270
    *io.token = 0;
    write_kept(io, cand);
    return OXO_EMPTY;
  }

  // Keep the top max(top_k, 256) and sort them descending (:274-283).
  size_t filter_k = std::min<size_t>(std::max<size_t>(c.top_k, 256), cand.size());
  if (filter_k < cand.size()) {
    std::nth_element(cand.begin(), cand.begin() + (filter_k - 1), cand.end(), cand_desc);
    cand.resize(filter_k);
  }
  std::sort(cand.begin(), cand.end(), cand_desc);

  // Softmax over the kept candidates only (:286-295).
  float max_logit = cand[0].p;
  float sum_exp = 0.0f;
  for (Cand& x : cand) {
    x.p = expf(x.p - max_logit);
    sum_exp += x.p;
  }
  float inv_sum = sum_exp > 0.0f ? 1.0f / sum_exp : 1.0f;
  for (Cand& x : cand) x.p *= inv_sum;

  bool ok = true;
  // 6. Mirostat (:298-312; v1 :418-429; v2 :432-456). The token is recorded
  // twice: inside the mode function and again by the caller.
  if (c.mirostat_mode == OXS_MIROSTAT_V1) {
    uint32_t selected = cand[0].id;
    float prob = fmaxf(cand[0].p, 1e-6f);
    float surprise = -log2f(prob);
    float error = surprise - c.mirostat_tau;
    float step = c.mirostat_eta * error;
    *io.mu -= step;
    ok &= record(io, selected);
    ok &= record(io, selected);
    *io.token = selected;
    write_kept(io, cand);
    return ok ? OXO_OK : OXO_HISTORY_FULL;
  }
  if (c.mirostat_mode == OXS_MIROSTAT_V2) {
    float max_surprise = *io.mu;
    size_t cutoff = 1;
    float cum_prob = 0.0f;
    for (size_t i = 0; i < cand.size(); ++i) {
      float surprise = -log2f(fmaxf(cand[i].p, 1e-8f));
      if (surprise > max_surprise && i > 0) break;
      cum_prob += cand[i].p;
      cutoff = i + 1;
    }
    (void)cutoff;
    uint32_t selected = cand[0].id;
    float prob = cand[0].p / fmaxf(cum_prob, 1e-6f);
    float surprise = -log2f(fmaxf(prob, 1e-8f));
    float error = surprise - c.mirostat_tau;
    float step = c.mirostat_eta * error;
    *io.mu -= step;
    ok &= record(io, selected);
    ok &= record(io, selected);
    *io.token = selected;
    write_kept(io, cand);
    return ok ? OXO_OK : OXO_HISTORY_FULL;
  }

  // 7. Min-p (:315-319): retain p >= p_max * min_p (a filter, not a prefix cut).
  if (c.min_p > 0.0f && !cand.empty()) {
    float threshold = cand[0].p * c.min_p;
    std::vector<Cand> kept;
    for (const Cand& x : cand)
      if (x.p >= threshold) kept.push_back(x);
    cand.swap(kept);
  }
  // 8. XTC (:322-328): deterministically drop the top choice.
  if (c.xtc_probability > 0.0f && cand.size() > 1) {
    float p_max = cand[0].p;
    if (p_max >= c.xtc_threshold && p_max < 0.98f) cand.erase(cand.begin());
  }
  // 9. Top-k (:331-333).
  if (c.top_k > 0 && cand.size() > c.top_k) cand.resize(c.top_k);
  // 10. Tail-free (:336-338).
  if (c.tfs_z < 1.0f && cand.size() > 2) apply_tail_free_sampling(c, cand);
  // 11. Locally typical (:341-343).
  if (c.typical_p < 1.0f && cand.size() > 1) apply_locally_typical_sampling(c, cand);
  // 12. Top-p (:346-357).
  if (c.top_p < 1.0f) {
    float cumulative = 0.0f;
    size_t cut = cand.size();
    for (size_t i = 0; i < cand.size(); ++i) {
      cumulative += cand[i].p;
      if (cumulative >= c.top_p) { cut = std::min(i + 1, cand.size()); break; }
    }
    cand.resize(cut);
  }
  // Renormalise (:360-368).
  float total = rust_sum_init();
  for (const Cand& x : cand) total += x.p;
  float inv_total = total > 0.0f ? 1.0f / total : 1.0f;
  for (Cand& x : cand) x.p *= inv_total;

  // Draw (:371-385): greedy below 1e-6, else the first candidate whose
  // running sum reaches r; the fallback is the first candidate.
  uint32_t picked;
  if (c.temperature <= 1e-6f) {
    picked = cand.empty() ? 0 : cand[0].id;
  } else {
    uint64_t fallback_state = 0x853c49e6748fea9bull;  // SamplerState::default() (:98)
    float r = io.uniform ? *io.uniform : oxo_next_f32(io.rng_state ? io.rng_state : &fallback_state);
    float acc = 0.0f;
    uint32_t selected = cand.empty() ? 0 : cand[0].id;
    for (const Cand& x : cand) {
      acc += x.p;
      if (r <= acc) { selected = x.id; break; }
    }
    picked = selected;
  }
  ok &= record(io, picked);  // :387
  *io.token = picked;
  write_kept(io, cand);
  return ok ? OXO_OK : OXO_HISTORY_FULL;
}

inline float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

}  // namespace

extern "C" {

uint64_t oxo_next_u64(uint64_t* state) {
  uint64_t x = *state;
  x ^= x << 13;
  x ^= x >> 7;
  x ^= x << 17;
  *state = x;
  return x;
}

float oxo_next_f32(uint64_t* state) {
  uint32_t val = (uint32_t)(oxo_next_u64(state) >> 40);
  return (float)val / 16777216.0f;
}

int oxo_sample_token(const oxs_sampling_config* cfg, const uint32_t* bias_ids,
                     const float* bias_values, const uint32_t* ban_ids, float* logits,
                     uint32_t vocab, uint32_t* history, uint32_t* history_len,
                     uint32_t history_cap, float* mu, uint64_t* rng_state,
                     const float* uniform, uint32_t* token, uint32_t* kept_ids,
                     float* kept_probs, uint32_t* kept_count, uint32_t kept_cap) {
  RowIo io{history, history_len, history_cap, true, mu, rng_state, uniform,
           token, kept_ids, kept_probs, kept_count, kept_cap};
  return sample_row(*cfg, bias_ids, bias_values, ban_ids, logits, vocab, io);
}

// continuous_batching.rs:961-970: the first index whose logit is larger than
// every earlier one, starting from -inf at index 0 (so NaN never wins and a row
// of -inf and NaN gives 0).
static uint32_t raw_argmax(const float* row, uint32_t vocab) {
  uint32_t best = 0;
  float max_val = -INFINITY;
  for (uint32_t i = 0; i < vocab; ++i) {
    if (row[i] > max_val) {
      max_val = row[i];
      best = i;
    }
  }
  return best;
}

// Rows of a batch (oxo_sample_batch), or of a decode step when `dec` is set:
// then a row with temperature <= 1e-6 is the loop's raw argmax and touches no
// sampler state, and every row advances the loop's per-sequence fields
// (continuous_batching.rs:957-977).
static int batch_rows(const oxs_batch* b, const oxs_decode_io* dec, int n_threads) {
  if (b->vocab == 0) return OXO_SHAPE_MISMATCH;
  auto work = [b, dec](uint32_t lo, uint32_t hi) {
    std::vector<float> row(b->vocab);
    for (uint32_t r = lo; r < hi; ++r) {
      const oxs_sampling_config& c = b->configs[(b->flags & OXS_FLAG_SHARED_CONFIG) ? 0 : r];
      if (b->logits_dtype == OXS_DTYPE_BF16) {
        const uint16_t* src = (const uint16_t*)b->logits + (size_t)r * b->logits_ld;
        for (uint32_t i = 0; i < b->vocab; ++i) row[i] = bf16_to_f32(src[i]);
      } else {
        const float* src = (const float*)b->logits + (size_t)r * b->logits_ld;
        memcpy(row.data(), src, sizeof(float) * b->vocab);
      }
      if (b->logit_softcap > 0.0f) {  // lib.rs:3243-3255 / vec_ops_activations.cu:131-136, before sampling
        const float cap = b->logit_softcap;
        for (uint32_t i = 0; i < b->vocab; ++i) row[i] = cap * tanhf(row[i] / cap);
      }
      if (b->allowed_mask) {
        const uint32_t* m = b->allowed_mask + (size_t)r * b->mask_ld;
        for (uint32_t i = 0; i < b->vocab; ++i)
          if (!((m[i >> 5] >> (i & 31)) & 1u)) row[i] = -INFINITY;
      }
      if (dec && c.temperature <= 1e-6f) {  // :961-970
        const uint32_t tok = raw_argmax(row.data(), b->vocab);
        bool any = false;
        for (uint32_t i = 0; i < b->vocab && !any; ++i) any = row[i] > -INFINITY;
        b->out_tokens[r] = tok;
        if (b->out_status) b->out_status[r] = any ? OXO_OK : OXO_EMPTY;
        if (dec->current_token) dec->current_token[r] = tok;
        if (dec->current_position) dec->current_position[r] += 1;
        if (dec->generated_count) dec->generated_count[r] += 1;
        continue;
      }
      uint32_t zero_len = 0;
      uint32_t* hist = b->history ? b->history + (size_t)r * b->history_ld : nullptr;
      uint32_t* hlen = b->history_len ? &b->history_len[r] : &zero_len;
      uint32_t local_len = *hlen;
      bool rec = (b->flags & OXS_FLAG_RECORD_HISTORY) != 0;
      float mu_dummy = 0.0f;
      uint32_t tok = 0;
      RowIo io{hist, rec ? hlen : &local_len, b->history_cap, rec,
               b->mirostat_mu ? &b->mirostat_mu[r] : &mu_dummy,
               b->rng_state ? &b->rng_state[r] : nullptr,
               b->uniforms ? &b->uniforms[r] : nullptr, &tok,
               b->out_kept_ids ? b->out_kept_ids + (size_t)r * b->kept_ld : nullptr,
               b->out_kept_probs ? b->out_kept_probs + (size_t)r * b->kept_ld : nullptr,
               b->out_kept_count ? &b->out_kept_count[r] : nullptr,
               (uint32_t)b->kept_ld};
      int st = sample_row(c, b->bias_ids, b->bias_values, b->ban_ids, row.data(), b->vocab, io);
      if (b->logits_out) memcpy(b->logits_out + (size_t)r * b->logits_out_ld, row.data(), sizeof(float) * b->vocab);
      b->out_tokens[r] = tok;
      if (b->out_status) b->out_status[r] = st;
      if (dec) {  // :973-976 (every status here carries its token; errors give 0)
        if (dec->current_token) dec->current_token[r] = tok;
        if (dec->current_position) dec->current_position[r] += 1;
        if (dec->generated_count) dec->generated_count[r] += 1;
      }
    }
  };
  if (n_threads <= 1 || b->batch <= 1) {
    work(0, b->batch);
  } else {
    uint32_t nt = std::min<uint32_t>((uint32_t)n_threads, b->batch);
    std::vector<std::thread> ts;
    for (uint32_t t = 0; t < nt; ++t) {
      uint32_t lo = (uint32_t)((uint64_t)b->batch * t / nt);
      uint32_t hi = (uint32_t)((uint64_t)b->batch * (t + 1) / nt);
      ts.emplace_back(work, lo, hi);
    }
    for (auto& t : ts) t.join();
  }
  return 0;
}

int oxo_sample_batch(const oxs_batch* b, int n_threads) { return batch_rows(b, nullptr, n_threads); }

int oxo_decode_step(const oxs_batch* b, const oxs_decode_io* io, int n_threads) {
  return batch_rows(b, io, n_threads);
}

uint32_t oxo_raw_argmax(const float* row, uint32_t vocab) { return raw_argmax(row, vocab); }

float oxo_expf(float x) { return expf(x); }
float oxo_logf(float x) { return logf(x); }
float oxo_log2f(float x) { return log2f(x); }
float oxo_powf(float x, float y) { return powf(x, y); }

}  // extern "C"

// grammar_engine.rs:42-65 / dfa.rs:110-148: walk each token's bytes from the
// row's state; DfaSchemaGrammar::transition fails for a current state outside
// the table (:111-116) or an error entry (:119-124).
void oxo_dfa_mask(const uint32_t* transitions, uint32_t num_states, const uint32_t* offsets,
                  const uint8_t* bytes, uint32_t num_bytes, uint32_t vocab, const uint32_t* states,
                  uint32_t batch, uint32_t* mask, int64_t mask_ld) {
  const uint32_t words = (vocab + 31) / 32;
  for (uint32_t b = 0; b < batch; ++b) {
    uint32_t* row = mask + (size_t)b * mask_ld;
    for (uint32_t w = 0; w < words; ++w) row[w] = 0;
    for (uint32_t t = 0; t < vocab; ++t) {
      const uint32_t lo = offsets[t], hi = offsets[t + 1];
      if (hi < lo || hi > num_bytes) continue;
      uint32_t state = states[b];
      bool valid = true;
      for (uint32_t i = lo; i < hi; ++i) {
        if (state >= num_states) { valid = false; break; }
        const uint32_t next = transitions[(size_t)state * 256 + bytes[i]];
        if (next == 0xffffffffu) { valid = false; break; }
        state = next;
      }
      if (valid) row[t / 32] |= 1u << (t % 32);
    }
  }
}

// The first character of UTF-8 text (text.chars().next()); U+FFFD for a
// malformed sequence (bad or missing continuation, overlong form, surrogate,
// beyond U+10FFFF), as String::from_utf8_lossy would give.
static uint32_t utf8_first(const uint8_t* b, uint32_t len) {
  const uint32_t c0 = b[0];
  if (c0 < 0x80) return c0;
  uint32_t need, c;
  if (c0 >= 0xc0 && c0 < 0xe0) { need = 1; c = c0 & 0x1f; }
  else if (c0 >= 0xe0 && c0 < 0xf0) { need = 2; c = c0 & 0x0f; }
  else if (c0 >= 0xf0 && c0 < 0xf8) { need = 3; c = c0 & 0x07; }
  else return 0xfffd;
  if (len <= need) return 0xfffd;
  for (uint32_t i = 1; i <= need; ++i) {
    if ((b[i] & 0xc0) != 0x80) return 0xfffd;
    c = (c << 6) | (b[i] & 0x3f);
  }
  static const uint32_t kLeast[4] = {0, 0x80, 0x800, 0x10000};  // shortest form of each length
  if (c < kLeast[need] || (c >= 0xd800 && c <= 0xdfff) || c > 0x10ffff) return 0xfffd;
  return c;
}

// GbnfGrammarEngine::apply_grammar_mask (sampler.rs:555-583), one row.
void oxo_gbnf_mask(const uint32_t* ranges, uint32_t num_ranges, const uint32_t* lit_off, const uint8_t* lit_bytes,
                   uint32_t num_lits, const uint32_t* offsets, const uint8_t* bytes, uint32_t num_bytes,
                   uint32_t vocab, uint32_t* mask) {
  for (uint32_t w = 0; w < (vocab + 31) / 32; ++w) mask[w] = 0;
  for (uint32_t t = 0; t < vocab; ++t) {
    const uint32_t lo = offsets[t], hi = offsets[t + 1];
    if (hi < lo || hi > num_bytes) continue;
    const uint32_t len = hi - lo;
    bool allowed;
    if (len == 0) {
      allowed = true;  // no first character: :560 skips the token
    } else {
      const uint32_t c = utf8_first(bytes + lo, len);
      allowed = false;
      for (uint32_t i = 0; i < num_ranges && !allowed; ++i)  // :561-567
        if (c >= ranges[2 * i] && c <= ranges[2 * i + 1]) allowed = true;
      for (uint32_t i = 0; i < num_lits && !allowed; ++i) {  // :568-575
        const uint32_t ll = lit_off[i + 1] - lit_off[i];
        const bool lit_starts_with_text = len <= ll && memcmp(lit_bytes + lit_off[i], bytes + lo, len) == 0;
        const bool text_starts_with_lit = ll <= len && memcmp(bytes + lo, lit_bytes + lit_off[i], ll) == 0;
        allowed = lit_starts_with_text || text_starts_with_lit;
      }
    }
    if (allowed) mask[t / 32] |= 1u << (t % 32);
  }
}

// GrammarLogitMasker::mask_logits (grammar_mask.rs:55-65), one row.
void oxo_ascii_mask(const uint8_t* allowed_ascii, const uint16_t* token_ascii, uint32_t vocab, uint32_t* mask) {
  for (uint32_t w = 0; w < (vocab + 31) / 32; ++w) mask[w] = 0;
  for (uint32_t t = 0; t < vocab; ++t) {
    const bool masked = token_ascii[t] < 256 && !allowed_ascii[token_ascii[t]];  // is_some_and(!allowed)
    if (!masked) mask[t / 32] |= 1u << (t % 32);
  }
}

// launch_cuda_argmax (sampling_dfa.cu:161-178), simulated thread by thread.
// Which of several equal maxima wins depends on the kernels' thread layout,
// so the oracle runs that layout literally:
//  - each thread scans ids start, start + stride, ... with a running maximum
//    that starts at (-1e30, id 0) and is replaced only by a strictly larger
//    value (:13-23, :81-91);
//  - a warp of 32 lanes reduces with __shfl_down_sync at offsets 16, 8, 4, 2,
//    1: lane l takes lane l + off's pair only when that value is strictly
//    larger; a source lane past 31 is the lane itself (:26-33);
//  - lane 0 of each warp stores its pair, and the first warp reduces the
//    stored pairs the same way, lanes past the warp count holding
//    (-1e30, 0) (:44-58).
// batch > 1: one 1024-thread block per row (:2-68, :173-175).
// batch == 1: 24 blocks of 256 threads stride the row by 6144, each block
// reduces to one pair, and one warp reduces the 24 pairs (:70-159, :165-171).
namespace {
struct ArgPair {
  float v;
  uint32_t i;
};
ArgPair arg_thread_scan(const float* row, uint32_t vocab, uint32_t start, uint32_t stride) {
  ArgPair p{-1e30f, 0u};
  for (uint64_t i = start; i < vocab; i += stride)
    if (row[i] > p.v) p = ArgPair{row[i], (uint32_t)i};
  return p;
}
ArgPair arg_warp_tree(const ArgPair (&in)[32]) {
  ArgPair lane[32];
  for (int l = 0; l < 32; ++l) lane[l] = in[l];
  for (int off = 16; off > 0; off >>= 1) {
    ArgPair before[32];
    for (int l = 0; l < 32; ++l) before[l] = lane[l];  // every lane reads before any lane updates
    for (int l = 0; l < 32; ++l) {
      const ArgPair other = l + off < 32 ? before[l + off] : before[l];
      if (other.v > before[l].v) lane[l] = other;
    }
  }
  return lane[0];
}
// One block of `threads` threads (a multiple of 32) whose thread t scans from
// first + t with the given stride.
ArgPair arg_block(const float* row, uint32_t vocab, uint32_t threads, uint32_t first, uint32_t stride) {
  ArgPair warps[32];
  const uint32_t nw = threads / 32;
  for (uint32_t w = 0; w < nw; ++w) {
    ArgPair lanes[32];
    for (uint32_t l = 0; l < 32; ++l) lanes[l] = arg_thread_scan(row, vocab, first + w * 32 + l, stride);
    warps[w] = arg_warp_tree(lanes);
  }
  for (uint32_t w = nw; w < 32; ++w) warps[w] = ArgPair{-1e30f, 0u};
  return arg_warp_tree(warps);
}
}  // namespace

void oxo_argmax_floor(const float* row, uint32_t vocab, uint32_t batch, uint32_t* token, float* value) {
  ArgPair r;
  if (batch == 1) {
    constexpr uint32_t kBlocks = 24, kThreadsPer = 256;
    ArgPair blocks[32];
    for (uint32_t b = 0; b < kBlocks; ++b)
      blocks[b] = arg_block(row, vocab, kThreadsPer, b * kThreadsPer, kBlocks * kThreadsPer);
    for (uint32_t b = kBlocks; b < 32; ++b) blocks[b] = ArgPair{-1e30f, 0u};
    r = arg_warp_tree(blocks);
  } else {
    r = arg_block(row, vocab, 1024, 0, 1024);
  }
  *token = r.i;
  *value = r.v;
}

// ---------------------------------------------------------------- LM head (Q8_0 x q8_1)

// IEEE binary16 <-> binary32: the conversions behind __half2float and
// __float2half (round to nearest, ties to even), written from the formats.
float oxo_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
  uint32_t bits;
  if (e == 0) {
    const float v = (float)mant * (1.0f / 16777216.0f);  // mant * 2^-24, exact
    memcpy(&bits, &v, 4);
    bits |= sign;
  } else if (e == 31) {
    bits = sign | 0x7f800000u | (mant << 13);
  } else {
    bits = sign | ((e - 15u + 127u) << 23) | (mant << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t oxo_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));  // NaN stays NaN
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);                         // >= 65520: infinity
  if (ax < 0x38800000u) {  // below 2^-14: a subnormal half, round(|f| * 2^24)
    float a;
    memcpy(&a, &ax, 4);
    return (uint16_t)(sign | (uint32_t)nearbyintf(a * 16777216.0f));
  }
  uint32_t h = ((((ax >> 23) - 127u + 15u)) << 10) | ((ax >> 13) & 0x3ffu);
  const uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;  // a carry moves into the exponent
  return (uint16_t)(sign | h);
}

// quantize_f32_to_q8_1_cuda_kernel (norms_rope.cu:2-29): one 32-lane group per
// block; amax and sum by an xor butterfly over offsets 16, 8, 4, 2, 1 (lane 0's
// sum is stored); d = amax / 127, id = 1 / d (0 when d == 0),
// q = (int8) roundf(x * id); ds = (half d, half sum).
void oxo_quantize_q8_1(const float* x, uint32_t n, uint8_t* y) {
  for (uint32_t blk = 0; blk < n / 32; ++blk) {
    const float* v = x + (size_t)blk * 32;
    float a[32], s[32];
    for (int i = 0; i < 32; ++i) {
      a[i] = fabsf(v[i]);
      s[i] = v[i];
    }
    for (int o = 16; o > 0; o >>= 1) {
      float a2[32], s2[32];
      for (int i = 0; i < 32; ++i) {
        a2[i] = fmaxf(a[i], a[i ^ o]);
        s2[i] = s[i] + s[i ^ o];
      }
      memcpy(a, a2, sizeof a);
      memcpy(s, s2, sizeof s);
    }
    const float d = a[0] / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    uint8_t* out = y + (size_t)blk * 36;
    const uint16_t hd = oxo_f32_to_f16(d), hs = oxo_f32_to_f16(s[0]);
    memcpy(out, &hd, 2);
    memcpy(out + 2, &hs, 2);
    for (int i = 0; i < 32; ++i) out[4 + i] = (uint8_t)(int8_t)roundf(v[i] * id);
  }
}

// mmvq_q8_0_cuda_kernel (quant_gemv_standard.cu:425-513), per (column c,
// token t): the lanes with sub_idx 0 of block_in_warp j = 0..3 accumulate the
// blocks b = j, j + 4, ... in increasing b as
// thread_dot += (d * d8) * (float)dot_int, which nvcc's default contraction
// (-fmad=true; build.rs passes only -O3) makes fmaf(d * d8, dot, thread_dot);
// dot_int is the exact integer dot of the 32 quants (dp4a and an integer
// butterfly). Then two shuffles down add lane 16 into lane 0 and lane 24 into
// lane 8, then lane 8 into lane 0: (A0 + A2) + (A1 + A3).
void oxo_mmvq_q8_0(float* y, const uint8_t* w, const uint8_t* x, uint32_t m, uint32_t k, uint32_t batch) {
  const uint32_t nb = k / 32;
  for (uint32_t c = 0; c < batch; ++c) {
    for (uint32_t t = 0; t < m; ++t) {
      float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      for (uint32_t b = 0; b < nb; ++b) {
        const uint8_t* wb = w + ((size_t)t * nb + b) * 34;
        const uint8_t* xb = x + ((size_t)c * nb + b) * 36;
        int dot = 0;
        for (int e = 0; e < 32; ++e) dot += (int)(int8_t)wb[2 + e] * (int)(int8_t)xb[4 + e];
        uint16_t hw, hx;
        memcpy(&hw, wb, 2);
        memcpy(&hx, xb, 2);
        const float dd = oxo_f16_to_f32(hw) * oxo_f16_to_f32(hx);
        acc[b % 4] = fmaf(dd, (float)dot, acc[b % 4]);
      }
      y[(size_t)c * m + t] = (acc[0] + acc[2]) + (acc[1] + acc[3]);
    }
  }
}
