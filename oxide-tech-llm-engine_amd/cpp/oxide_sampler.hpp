// oxide_sampler.hpp — the reference sampler's API in C++17 over the C ABI.
//
// SamplingConfig, MirostatMode, SamplerState and AcademicSamplerEngine keep
// the names, defaults, argument meaning and error behaviour of
// crates/oxide-core/src/sampler.rs:15-390, so code written against the
// reference reads the same. sample_token runs its row through
// oxs_sample_batch on the GPU (include/oxide_sampler.h) and brings every side
// effect of the reference back to the caller's objects: the penalised,
// temperature-scaled logits (the reference mutates its `&mut [f32]`), the
// recorded tokens, mirostat_mu, rng_state and candidates_buffer.
//
// Header-only; link liboxide_sampler.so and the HIP runtime (amdhip64). There
// is no CPU fallback: without a HIP device every call throws EngineError.
#pragma once

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <limits>
#include <mutex>
#include <optional>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <utility>
#include <vector>

#include "../../include/oxide_sampler.h"

namespace oxide {

// EngineError (crates/oxide-core/src/error.rs): ShapeMismatch for an empty
// row (sampler.rs:179-181); Device for anything the GPU path reports.
class EngineError : public std::runtime_error {
 public:
  enum class Kind { ShapeMismatch, Device };
  EngineError(Kind kind, const std::string& what) : std::runtime_error(what), kind_(kind) {}
  Kind kind() const { return kind_; }

 private:
  Kind kind_;
};

// sampler.rs:76-83.
enum class MirostatMode : int32_t {
  Disabled = OXS_MIROSTAT_DISABLED,
  V1 = OXS_MIROSTAT_V1,
  V2 = OXS_MIROSTAT_V2,
};

// sampler.rs:16-42 with the defaults of sampler.rs:44-73.
struct SamplingConfig {
  float temperature = 0.8f;
  uint32_t top_k = 40;
  float top_p = 0.95f;
  float min_p = 0.05f;
  float tfs_z = 1.0f;
  float typical_p = 1.0f;
  float xtc_threshold = 0.1f;
  float xtc_probability = 0.0f;
  MirostatMode mirostat_mode = MirostatMode::Disabled;
  float mirostat_tau = 5.0f;
  float mirostat_eta = 0.1f;
  float dry_multiplier = 0.0f;
  float dry_base = 1.75f;
  uint32_t dry_allowed_length = 2;
  uint32_t dry_range = 1024;
  float repeat_penalty = 1.1f;
  uint32_t repeat_last_n = 64;
  float frequency_penalty = 0.0f;
  float presence_penalty = 0.0f;
  bool penalize_nl = false;
  float newline_penalty = 0.5f;
  std::unordered_map<uint32_t, float> logit_biases;
  std::unordered_set<uint32_t> banned_tokens;
  std::optional<uint64_t> seed;
};

// sampler.rs:85-158 (Default at :93-102).
struct SamplerState {
  static constexpr uint64_t kDefaultRng = 0x853c49e6748fea9bull;  // sampler.rs:98, :110, :118

  float mirostat_mu = 10.0f;
  std::vector<uint32_t> generated_tokens;
  uint64_t rng_state = kDefaultRng;
  std::vector<std::pair<uint32_t, float>> candidates_buffer;

  // SamplerState::new(target_tau): mu = 2 tau (sampler.rs:105-113).
  static SamplerState create(float target_tau) {
    SamplerState s;
    s.mirostat_mu = 2.0f * target_tau;
    return s;
  }
  // SamplerState::new_with_seed (sampler.rs:115-128): seed 0 keeps the default state.
  static SamplerState new_with_seed(float target_tau, uint64_t seed) {
    SamplerState s = create(target_tau);
    s.rng_state = seed == 0 ? kDefaultRng : seed;
    return s;
  }
  // SamplerState::from_config (sampler.rs:130-135).
  static SamplerState from_config(const SamplingConfig& c) {
    return c.seed ? new_with_seed(c.mirostat_tau, *c.seed) : create(c.mirostat_tau);
  }
  // xorshift64 (sampler.rs:138-145).
  uint64_t next_u64() {
    uint64_t x = rng_state;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    rng_state = x;
    return x;
  }
  // The top 24 bits as a float in [0, 1) (sampler.rs:147-153).
  float next_f32() { return static_cast<float>(static_cast<uint32_t>(next_u64() >> 40)) / 16777216.0f; }
  void record_token(uint32_t token) { generated_tokens.push_back(token); }
};

namespace detail {

inline void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw EngineError(EngineError::Kind::Device, std::string(what) + ": " + hipGetErrorString(e));
}

inline void oxs_check(int rc, const char* what) {
  if (rc == OXS_OK) return;
  if (rc == OXS_ERR_SHAPE_MISMATCH)
    throw EngineError(EngineError::Kind::ShapeMismatch, "Tensor shape or dimension mismatch");
  throw EngineError(EngineError::Kind::Device, std::string(what) + ": " + oxs_status_string(rc));
}

// A device allocation that only grows.
class DeviceBuffer {
 public:
  DeviceBuffer() = default;
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  ~DeviceBuffer() {
    if (ptr_) (void)hipFree(ptr_);
  }
  void* ensure(size_t bytes) {
    bytes = std::max<size_t>(bytes, 16);
    if (bytes > size_) {
      if (ptr_) hip_check(hipFree(ptr_), "hipFree");
      ptr_ = nullptr;
      hip_check(hipMalloc(&ptr_, bytes), "hipMalloc");
      size_ = bytes;
    }
    return ptr_;
  }
  template <typename T>
  T* put(const T* host, size_t n) {
    void* p = ensure(n * sizeof(T));
    if (n) hip_check(hipMemcpy(p, host, n * sizeof(T), hipMemcpyHostToDevice), "hipMemcpy");
    return static_cast<T*>(p);
  }
  template <typename T>
  void get(T* host, size_t n) const {
    if (n) hip_check(hipMemcpy(host, ptr_, n * sizeof(T), hipMemcpyDeviceToHost), "hipMemcpy");
  }

 private:
  void* ptr_ = nullptr;
  size_t size_ = 0;
};

// SamplingConfig as the C record, with its bias and ban lists appended to CSR arrays.
inline oxs_sampling_config to_c(const SamplingConfig& c, uint32_t newline_token_id, std::vector<uint32_t>& bias_ids,
                                std::vector<float>& bias_values, std::vector<uint32_t>& ban_ids) {
  oxs_sampling_config r;
  std::memset(&r, 0, sizeof(r));
  r.temperature = c.temperature;
  r.top_k = c.top_k;
  r.top_p = c.top_p;
  r.min_p = c.min_p;
  r.tfs_z = c.tfs_z;
  r.typical_p = c.typical_p;
  r.xtc_threshold = c.xtc_threshold;
  r.xtc_probability = c.xtc_probability;
  r.mirostat_mode = static_cast<int32_t>(c.mirostat_mode);
  r.mirostat_tau = c.mirostat_tau;
  r.mirostat_eta = c.mirostat_eta;
  r.dry_multiplier = c.dry_multiplier;
  r.dry_base = c.dry_base;
  r.dry_allowed_length = c.dry_allowed_length;
  r.dry_range = c.dry_range;
  r.repeat_penalty = c.repeat_penalty;
  r.repeat_last_n = c.repeat_last_n;
  r.frequency_penalty = c.frequency_penalty;
  r.presence_penalty = c.presence_penalty;
  r.penalize_nl = c.penalize_nl ? 1u : 0u;
  r.newline_penalty = c.newline_penalty;
  r.newline_token_id = newline_token_id;
  r.bias_offset = static_cast<uint32_t>(bias_ids.size());
  r.bias_count = static_cast<uint32_t>(c.logit_biases.size());
  for (const auto& kv : c.logit_biases) {
    bias_ids.push_back(kv.first);
    bias_values.push_back(kv.second);
  }
  r.ban_offset = static_cast<uint32_t>(ban_ids.size());
  r.ban_count = static_cast<uint32_t>(c.banned_tokens.size());
  std::vector<uint32_t> bans(c.banned_tokens.begin(), c.banned_tokens.end());
  std::sort(bans.begin(), bans.end());
  ban_ids.insert(ban_ids.end(), bans.begin(), bans.end());
  return r;
}

}  // namespace detail

// sampler.rs:160-390: one row per sample_token call, run on the GPU.
class AcademicSamplerEngine {
 public:
  explicit AcademicSamplerEngine(SamplingConfig config) : config(std::move(config)) {}
  // AcademicSamplerEngine::new (sampler.rs:168).
  static AcademicSamplerEngine create(SamplingConfig config) { return AcademicSamplerEngine(std::move(config)); }
  AcademicSamplerEngine(const AcademicSamplerEngine& o) : config(o.config) {}
  ~AcademicSamplerEngine() {
    if (handle_) (void)oxs_sampler_destroy(handle_);
  }

  // sample_token(&self, logits: &mut [f32], state: &mut SamplerState,
  // newline_token_id: u32) -> Result<u32> (sampler.rs:173-390). Throws
  // EngineError::ShapeMismatch for an empty row; an all -inf row returns 0
  // and records nothing (:267-270).
  uint32_t sample_token(std::vector<float>& logits, SamplerState& state, uint32_t newline_token_id) const {
    const uint32_t V = static_cast<uint32_t>(logits.size());
    if (V == 0) throw EngineError(EngineError::Kind::ShapeMismatch, "Tensor shape or dimension mismatch");
    std::lock_guard<std::mutex> lock(mu_);
    const uint32_t kept_ld = std::max<uint32_t>(256, config.top_k);
    if (!handle_ || V > vocab_ || kept_ld > top_k_) {
      if (handle_) detail::oxs_check(oxs_sampler_destroy(handle_), "oxs_sampler_destroy");
      handle_ = nullptr;
      oxs_limits lim{1, std::max(V, vocab_), std::max(kept_ld, top_k_), 0u};
      int dev = 0;
      detail::hip_check(hipGetDevice(&dev), "hipGetDevice");
      detail::oxs_check(oxs_sampler_create(&handle_, &lim, dev), "oxs_sampler_create");
      vocab_ = lim.max_vocab;
      top_k_ = lim.max_top_k;
    }
    std::vector<uint32_t> bias_ids, ban_ids;
    std::vector<float> bias_values;
    const oxs_sampling_config cfg = detail::to_c(config, newline_token_id, bias_ids, bias_values, ban_ids);
    const uint32_t hlen = static_cast<uint32_t>(state.generated_tokens.size());
    const uint32_t cap = hlen + 2;  // room for Mirostat's two records
    std::vector<uint32_t> hist(cap, 0u);
    std::copy(state.generated_tokens.begin(), state.generated_tokens.end(), hist.begin());

    oxs_batch b;
    std::memset(&b, 0, sizeof(b));
    b.batch = 1;
    b.vocab = V;
    b.logits_dtype = OXS_DTYPE_F32;
    b.flags = OXS_FLAG_RECORD_HISTORY;
    b.logits_ld = V;
    b.logits = d_logits_.put(logits.data(), V);
    b.configs = d_cfg_.put(&cfg, 1);
    if (!bias_ids.empty()) {
      b.bias_ids = d_bias_ids_.put(bias_ids.data(), bias_ids.size());
      b.bias_values = d_bias_values_.put(bias_values.data(), bias_values.size());
    }
    if (!ban_ids.empty()) b.ban_ids = d_ban_ids_.put(ban_ids.data(), ban_ids.size());
    b.history = d_hist_.put(hist.data(), cap);
    b.history_ld = cap;
    b.history_len = d_hlen_.put(&hlen, 1);
    b.history_cap = cap;
    b.rng_state = d_rng_.put(&state.rng_state, 1);
    b.mirostat_mu = d_mu_.put(&state.mirostat_mu, 1);
    b.out_tokens = static_cast<uint32_t*>(d_token_.ensure(4));
    b.out_status = static_cast<int32_t*>(d_status_.ensure(4));
    b.out_kept_count = static_cast<uint32_t*>(d_kept_count_.ensure(4));
    b.out_kept_ids = static_cast<uint32_t*>(d_kept_ids_.ensure(kept_ld * 4u));
    b.out_kept_probs = static_cast<float*>(d_kept_probs_.ensure(kept_ld * 4u));
    b.kept_ld = kept_ld;
    b.logits_out = static_cast<float*>(d_logits_out_.ensure(V * 4u));
    b.logits_out_ld = V;
    detail::oxs_check(oxs_sample_batch(handle_, &b, nullptr), "oxs_sample_batch");
    detail::hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");

    uint32_t token = 0, kept = 0, new_len = 0;
    int32_t status = 0;
    d_token_.get(&token, 1);
    d_status_.get(&status, 1);
    if (status == OXS_ROW_UNSUPPORTED || status == OXS_ROW_MISSING_STATE)
      throw EngineError(EngineError::Kind::Device, "the row asks for a stage this build does not run on the GPU");
    d_logits_out_.get(logits.data(), V);
    d_hlen_.get(&new_len, 1);
    d_hist_.get(hist.data(), new_len);
    state.generated_tokens.assign(hist.begin(), hist.begin() + new_len);
    d_mu_.get(&state.mirostat_mu, 1);
    d_rng_.get(&state.rng_state, 1);
    d_kept_count_.get(&kept, 1);
    kept = std::min(kept, kept_ld);
    std::vector<uint32_t> ids(kept);
    std::vector<float> probs(kept);
    d_kept_ids_.get(ids.data(), kept);
    d_kept_probs_.get(probs.data(), kept);
    state.candidates_buffer.clear();
    for (uint32_t i = 0; i < kept; ++i) state.candidates_buffer.emplace_back(ids[i], probs[i]);
    return token;
  }

  SamplingConfig config;

 private:
  // The device side of one engine, made on first use (the reference engine
  // owns no device state); sample_token takes &self, so it is guarded.
  mutable std::mutex mu_;
  mutable oxs_sampler* handle_ = nullptr;
  mutable uint32_t vocab_ = 0, top_k_ = 0;
  mutable detail::DeviceBuffer d_logits_, d_cfg_, d_bias_ids_, d_bias_values_, d_ban_ids_, d_hist_, d_hlen_, d_rng_,
      d_mu_, d_token_, d_status_, d_kept_count_, d_kept_ids_, d_kept_probs_, d_logits_out_;
};

// GbnfRule (sampler.rs:523-529); ranges are inclusive code-point pairs.
struct GbnfRule {
  std::string rule_name;
  std::vector<std::pair<char32_t, char32_t>> allowed_char_ranges;
  std::vector<std::string> literal_strings;
};

// GbnfGrammarEngine (sampler.rs:531-585). The mask of the start rule is
// computed on the GPU by oxs_gbnf_mask, one bit per token.
struct GbnfGrammarEngine {
  std::unordered_map<std::string, GbnfRule> rules;
  std::string start_rule;

  // sampler.rs:539-553.
  static GbnfGrammarEngine new_json_grammar() {
    GbnfGrammarEngine g;
    g.rules["root"] = GbnfRule{"root", {{U'{', U'{'}, {U'[', U'['}, {U'"', U'"'}}, {"true", "false", "null"}};
    g.start_rule = "root";
    return g;
  }

  // Packed allowed-token words (bit t % 32 of word t / 32) for vocab_tokens
  // (UTF-8 texts); empty when the start rule is missing (nothing is masked).
  std::vector<uint32_t> token_mask(const std::vector<std::string>& vocab_tokens) const {
    const auto it = rules.find(start_rule);
    if (it == rules.end()) return {};
    const GbnfRule& rule = it->second;
    const uint32_t V = static_cast<uint32_t>(vocab_tokens.size());
    std::vector<uint32_t> offsets(V + 1, 0u);
    uint64_t total = 0;
    for (uint32_t t = 0; t < V; ++t) {
      total += vocab_tokens[t].size();
      if (total > 0xFFFFFFFFull) throw EngineError(EngineError::Kind::Device, "token texts exceed 2^32 bytes");
      offsets[t + 1] = static_cast<uint32_t>(total);
    }
    std::string bytes;
    bytes.reserve(total);
    for (const auto& s : vocab_tokens) bytes += s;
    std::vector<uint32_t> ranges;
    for (const auto& r : rule.allowed_char_ranges) {
      ranges.push_back(static_cast<uint32_t>(r.first));
      ranges.push_back(static_cast<uint32_t>(r.second));
    }
    std::vector<uint32_t> lit_off(rule.literal_strings.size() + 1, 0u);
    std::string lit_bytes;
    for (size_t i = 0; i < rule.literal_strings.size(); ++i) {
      lit_bytes += rule.literal_strings[i];
      lit_off[i + 1] = static_cast<uint32_t>(lit_bytes.size());
    }
    const uint32_t words = (V + 31) / 32;
    detail::DeviceBuffer d_off, d_bytes, d_ranges, d_loff, d_lbytes, d_mask;
    oxs_token_bytes tb{V, static_cast<uint32_t>(total), d_off.put(offsets.data(), offsets.size()),
                       reinterpret_cast<const uint8_t*>(d_bytes.put(bytes.data(), bytes.size()))};
    oxs_gbnf_rule cr{static_cast<uint32_t>(ranges.size() / 2), d_ranges.put(ranges.data(), ranges.size()),
                     static_cast<uint32_t>(rule.literal_strings.size()), d_loff.put(lit_off.data(), lit_off.size()),
                     reinterpret_cast<const uint8_t*>(d_lbytes.put(lit_bytes.data(), lit_bytes.size()))};
    auto* mask = static_cast<uint32_t*>(d_mask.ensure(std::max<uint32_t>(words, 1) * 4u));
    detail::oxs_check(oxs_gbnf_mask(&cr, &tb, mask, nullptr), "oxs_gbnf_mask");
    detail::hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    std::vector<uint32_t> out(words);
    d_mask.get(out.data(), words);
    return out;
  }

  // apply_grammar_mask(&self, logits: &mut [f32], vocab_tokens: &[String])
  // (sampler.rs:556-584): disallowed tokens below logits.size() become -inf.
  void apply_grammar_mask(std::vector<float>& logits, const std::vector<std::string>& vocab_tokens) const {
    const std::vector<uint32_t> m = token_mask(vocab_tokens);
    if (m.empty()) return;
    const size_t n = std::min(logits.size(), vocab_tokens.size());
    for (size_t t = 0; t < n; ++t)
      if (!((m[t / 32] >> (t % 32)) & 1u)) logits[t] = -std::numeric_limits<float>::infinity();
  }
};

}  // namespace oxide
