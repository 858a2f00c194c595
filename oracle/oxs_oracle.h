/*
 * oxs_oracle.h — CPU restatement of the reference sampler, for tests only.
 *
 * TEST INFRASTRUCTURE. Nothing in the product links, loads or calls this
 * code: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * use it, as the checker and the CPU baseline.
 *
 * It restates crates/oxide-core/src/sampler.rs stage by stage (each function
 * cites the lines it follows) in C++ built with -O2 -ffp-contract=off and no
 * fast-math, calling the platform libm's expf/logf/log2f/powf exactly where
 * Rust's f32::{exp, ln, log2, powf} do, so on the same host it produces the
 * same floats as the Rust code.
 *
 * Two deliberate differences from the reference, both part of the parity
 * contract:
 *   - the draw may use an injected uniform instead of state.next_f32();
 *   - ties between equal logits are ordered by the lower token index (the
 *     reference leaves the order after select_nth_unstable_by unspecified,
 *     sampler.rs:276).
 */
#ifndef OXS_ORACLE_H
#define OXS_ORACLE_H

#include <stdint.h>
#include "../include/oxide_sampler.h"

#ifdef __cplusplus
extern "C" {
#endif

#define OXO_OK 0
#define OXO_EMPTY 1            /* Ok(0) without record_token (sampler.rs:267-270) */
#define OXO_HISTORY_FULL 2     /* sampled, but history_cap reached */
#define OXO_SHAPE_MISMATCH (-2)

/* SamplerState::next_u64 / next_f32 (sampler.rs:139-153). */
uint64_t oxo_next_u64(uint64_t* state);
float oxo_next_f32(uint64_t* state);

/*
 * AcademicSamplerEngine::sample_token (sampler.rs:173-390) on one row.
 *   cfg, bias_ids/bias_values/ban_ids: the row's SamplingConfig (CSR ranges
 *       of cfg index these arrays);
 *   logits[vocab]: mutated in place exactly as the reference does;
 *   history[*history_len] (capacity history_cap): generated_tokens, appended;
 *   mu: mirostat_mu; rng_state: used only when uniform is NULL;
 *   kept_ids/kept_probs (capacity kept_cap, may be NULL): candidates_buffer.
 * Returns OXO_OK / OXO_EMPTY / OXO_HISTORY_FULL / OXO_SHAPE_MISMATCH and the
 * token in *token (0 when empty).
 */
int oxo_sample_token(const oxs_sampling_config* cfg, const uint32_t* bias_ids,
                     const float* bias_values, const uint32_t* ban_ids, float* logits,
                     uint32_t vocab, uint32_t* history, uint32_t* history_len,
                     uint32_t history_cap, float* mu, uint64_t* rng_state,
                     const float* uniform, uint32_t* token, uint32_t* kept_ids,
                     float* kept_probs, uint32_t* kept_count, uint32_t kept_cap);

/*
 * The same descriptor as oxs_sample_batch, with HOST pointers, sampled row by
 * row (a logit softcap first, cap * tanhf(l / cap) with the platform tanhf as
 * the backend's softcap pass does before sampling; then the packed mask by
 * writing -inf, as the reference's grammar maskers do). Logits are copied per row, so the input is not
 * modified. n_threads > 1 splits rows statically over that many threads.
 * Returns 0 or OXO_SHAPE_MISMATCH.
 */
int oxo_sample_batch(const oxs_batch* batch, int n_threads);

/*
 * The decode stage of ContinuousBatchingEngine::step
 * (crates/oxide-engine/src/continuous_batching.rs:957-977) over the same
 * descriptor: a row with temperature <= 1e-6 takes oxo_raw_argmax of its
 * (masked) logits and leaves history, mu, rng and the kept arrays alone; other
 * rows are sampled as by oxo_sample_batch. Then io's current_token,
 * current_position and generated_count advance (host pointers; the host_*
 * fields are ignored).
 */
int oxo_decode_step(const oxs_batch* batch, const oxs_decode_io* io, int n_threads);

/* continuous_batching.rs:961-970: first index of the largest logit, NaN never
 * larger, 0 for a row with no value above -inf. */
uint32_t oxo_raw_argmax(const float* row, uint32_t vocab);

/*
 * StructuredOutputEngine::compute_token_mask (oxide-server/src/grammar_engine.rs:42-65),
 * equivalently the -inf pattern of DfaSchemaGrammar::apply_dfa_mask
 * (oxide-core/src/dfa.rs:130-148), for `batch` rows in states[b], as the packed
 * mask oxs_dfa_mask writes (bit t % 32 of word t / 32 set = token t allowed;
 * bits past vocab cleared). Host pointers. Token t is bytes[offsets[t] ..
 * offsets[t + 1]); a range outside [0, num_bytes) is not allowed.
 */
void oxo_dfa_mask(const uint32_t* transitions, uint32_t num_states, const uint32_t* offsets,
                  const uint8_t* bytes, uint32_t num_bytes, uint32_t vocab, const uint32_t* states,
                  uint32_t batch, uint32_t* mask, int64_t mask_ld);

/* The static masks of oxs_gbnf_mask (sampler.rs:555-583) and oxs_ascii_mask
 * (grammar_mask.rs:55-65), host pointers, one row of ceil(vocab / 32) words. */
void oxo_gbnf_mask(const uint32_t* ranges, uint32_t num_ranges, const uint32_t* lit_off, const uint8_t* lit_bytes,
                   uint32_t num_lits, const uint32_t* offsets, const uint8_t* bytes, uint32_t num_bytes,
                   uint32_t vocab, uint32_t* mask);
void oxo_ascii_mask(const uint8_t* allowed_ascii, const uint16_t* token_ascii, uint32_t vocab, uint32_t* mask);

/* oxs_argmax on one row of a launch over `batch` rows (launch_cuda_argmax,
 * sampling_dfa.cu:161-178): batch 1 takes the 24-block path, any other batch
 * the one-block-per-row path; each is simulated thread by thread. */
void oxo_argmax_floor(const float* row, uint32_t vocab, uint32_t batch, uint32_t* token, float* value);

/* glibc's expf etc., exported so tests can compare the device emulation. */
float oxo_expf(float x);
float oxo_logf(float x);
float oxo_log2f(float x);
float oxo_powf(float x, float y);

/* LM head (Q8_0 weights x q8_1 activations), the reference CUDA backend's
 * formats: IEEE half conversions, launch_cuda_quantize_q8_1
 * (norms_rope.cu:2-29) and launch_cuda_mmvq_q8_0 (quant_gemv_standard.cu:425-513)
 * on the GGUF layout ([m][k / 32] 34-byte blocks; y is [batch][m]). */
float oxo_f16_to_f32(uint16_t h);
uint16_t oxo_f32_to_f16(float f);
void oxo_quantize_q8_1(const float* x, uint32_t n, uint8_t* y);
void oxo_mmvq_q8_0(float* y, const uint8_t* w, const uint8_t* x, uint32_t m, uint32_t k, uint32_t batch);

#ifdef __cplusplus
}
#endif

#endif
