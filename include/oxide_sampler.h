/*
 * oxide_sampler.h — C ABI of the MI355X (gfx950) batched token sampler.
 *
 * This is the drop-in boundary for the hot path of the reference engine's CPU
 * sampler, crates/oxide-core/src/sampler.rs (AcademicSamplerEngine::sample_token,
 * sampler.rs:173-390). One call samples a whole batch of rows on the GPU, on the
 * caller's HIP stream, with the reference's chain and per-row configuration:
 *
 *   mask -> bans -> biases -> newline penalty -> repetition / frequency /
 *   presence penalties -> temperature -> top-M (M = max(top_k, 256)) -> softmax
 *   -> Mirostat v1/v2 | (min-p -> XTC -> top-k -> tail-free -> locally typical
 *   -> top-p -> renormalise -> inverse-CDF draw)
 *
 * Conventions (mirroring the reference's FFI precedent,
 * crates/oxide-hardware/oxide-backend-cuda/src/driver.rs:671-690):
 *   - int return, 0 = success, negative = error (OXS_ERR_*);
 *   - device pointers are plain typed pointers (DevicePtr<T>,
 *     crates/oxide-core/src/memory.rs:9), never dereferenced on the host;
 *   - the stream argument is last and is a hipStream_t passed as void*;
 *   - all device workspace is allocated once by oxs_sampler_create (the
 *     preallocated-arena pattern of crates/oxide-alloc/src/device_arena.rs:7-80),
 *     so oxs_sample_batch allocates nothing, never synchronises and makes no
 *     host round trip.
 *
 * Ties between equal logits are broken by the lower token index.
 */
#ifndef OXIDE_SAMPLER_H
#define OXIDE_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OXS_ABI_VERSION 4u

/* Return codes. EngineError (crates/oxide-core/src/error.rs:6) has one variant
 * on this path, ShapeMismatch (error.rs:52; sampler.rs:179-181). */
#define OXS_OK 0
#define OXS_ERR_INVALID_ARGUMENT (-1)
#define OXS_ERR_SHAPE_MISMATCH (-2) /* vocab == 0, as sampler.rs:179-181 */
#define OXS_ERR_LIMITS (-3)         /* batch/vocab/top_k beyond oxs_limits */
#define OXS_ERR_HIP (-4)            /* a HIP runtime call failed */
#define OXS_ERR_UNSUPPORTED (-5)    /* a feature this build does not run on the GPU */
#define OXS_ERR_NO_DEVICE (-6)
#define OXS_ERR_TIMEOUT (-7)        /* oxs_host_wait gave up */

/* Per-row outcome written to out_status[b]. */
#define OXS_ROW_OK 0            /* Ok(token); token recorded (sampler.rs:387) */
#define OXS_ROW_EMPTY 1         /* every logit -inf or NaN: Ok(0), nothing recorded (sampler.rs:267-270) */
#define OXS_ROW_HISTORY_FULL 2  /* Ok(token), but the device history had no room to record it */
#define OXS_ROW_UNSUPPORTED 3   /* the row needs more than the sampler was sized for: a pool max(top_k, 256)
                                   (at most V) above oxs_limits.max_top_k, or a DRY pass penalising more
                                   distinct ids than oxs_limits.max_dry_ids (2048 through
                                   oxs_sample_batch_static, which also refuses pools above 1024);
                                   token 0 */
#define OXS_ROW_MISSING_STATE 4 /* a Mirostat row but oxs_batch.mirostat_mu is NULL; token 0 */

/* MirostatMode, sampler.rs:77-82. */
#define OXS_MIROSTAT_DISABLED 0
#define OXS_MIROSTAT_V1 1
#define OXS_MIROSTAT_V2 2

/* Logits element type. The reference is f32 only (sampler.rs:175); bf16 rows
 * are widened exactly (bits << 16) before the chain. */
#define OXS_DTYPE_F32 0
#define OXS_DTYPE_BF16 1

/* oxs_batch.flags */
#define OXS_FLAG_RECORD_HISTORY 1u  /* append the sampled token(s) to history (record_token, sampler.rs:155-157) */
#define OXS_FLAG_SHARED_CONFIG 2u   /* configs points at ONE config used by every row */

/*
 * SamplingConfig (sampler.rs:17-42) for one row, as plain scalars. The Rust
 * usize fields are narrowed to uint32. logit_biases (a HashMap<u32,f32>) and
 * banned_tokens (a HashSet<u32>) become ranges into the batch's CSR arrays
 * (oxs_batch.bias_ids/bias_values and oxs_batch.ban_ids). A bias list that
 * repeats an id behaves like repeated HashMap::insert: the last entry wins.
 * newline_token_id is sample_token's third argument (sampler.rs:177).
 * The seed field of SamplingConfig maps to the row's rng_state
 * (see oxs_rng_state_from_seed).
 */
typedef struct oxs_sampling_config {
  float temperature;
  uint32_t top_k;
  float top_p;
  float min_p;
  float tfs_z;
  float typical_p;
  float xtc_threshold;
  float xtc_probability;
  int32_t mirostat_mode;
  float mirostat_tau;
  float mirostat_eta;
  float dry_multiplier;
  float dry_base;
  uint32_t dry_allowed_length;
  uint32_t dry_range;
  float repeat_penalty;
  uint32_t repeat_last_n;
  float frequency_penalty;
  float presence_penalty;
  uint32_t penalize_nl;
  float newline_penalty;
  uint32_t newline_token_id;
  uint32_t bias_offset;
  uint32_t bias_count;
  uint32_t ban_offset;
  uint32_t ban_count;
} oxs_sampling_config;

/* Sizes fixed at create time; every workspace buffer is sized from these. */
typedef struct oxs_limits {
  uint32_t max_batch;  /* rows per call */
  uint32_t max_vocab;  /* V per row */
  uint32_t max_top_k;  /* largest top_k any row may use; 0 means 256. Above 1024 the sampler also
                          holds [max_batch] x ~36 bytes x max_top_k of workspace for those rows */
  uint32_t max_dry_ids; /* most distinct ids one row's DRY pass may penalise over a slice
                           (min(history_len, dry_range), sampler.rs:394-396) longer than 1024 ids;
                           0 means 8192 (at least 1024 is kept). The sampler holds [max_batch] x
                           32 bytes x (max_dry_ids, kept to max_vocab, rounded up to a power of two)
                           for these rows: 256 KiB per row at 8192. A slice of n ids penalises at most min(n, V) ids, so
                           max_dry_ids >= min(longest slice, max_vocab) runs every DRY row; a row
                           that penalises more returns OXS_ROW_UNSUPPORTED */
} oxs_limits;

/*
 * One batched sampling call. Every pointer is a device pointer unless noted.
 * Row b's state (the reference's SamplerState, sampler.rs:86-91) is:
 *   history[b*history_ld .. + history_len[b]]  generated_tokens
 *   mirostat_mu[b]                              mirostat_mu
 *   rng_state[b]                                rng_state (xorshift64, sampler.rs:139-153)
 * and its candidates_buffer after the call is out_kept_ids/out_kept_probs.
 */
typedef struct oxs_batch {
  uint32_t batch;         /* rows B */
  uint32_t vocab;         /* V */
  int32_t logits_dtype;   /* OXS_DTYPE_* */
  uint32_t flags;         /* OXS_FLAG_* */
  int64_t logits_ld;      /* elements between consecutive rows (>= vocab) */
  const void* logits;     /* [B][logits_ld], read only */

  const oxs_sampling_config* configs; /* [B], or [1] with OXS_FLAG_SHARED_CONFIG */
  const uint32_t* bias_ids;           /* CSR arrays indexed by the config ranges (may be NULL if unused) */
  const float* bias_values;
  const uint32_t* ban_ids;

  const uint32_t* allowed_mask; /* optional [B][mask_ld] words: bit (i%32) of word i/32 set = token i allowed */
  int64_t mask_ld;              /* >= ceil(vocab / 32), or 0: one mask shared by every row */

  uint32_t* history;      /* [B][history_ld] token ids (may be NULL when every history_len is 0 and nothing is recorded) */
  int64_t history_ld;
  uint32_t* history_len;  /* [B]; updated when OXS_FLAG_RECORD_HISTORY is set */
  uint32_t history_cap;   /* room per row for recording (<= history_ld) */

  const float* uniforms;  /* optional [B] u in [0,1): replaces state.next_f32() (sampler.rs:374) */
  uint64_t* rng_state;    /* optional [B]; advanced by one draw when uniforms is NULL */
  float* mirostat_mu;     /* [B] in/out; required when any row uses Mirostat */

  uint32_t* out_tokens;   /* [B] sampled token ids */
  int32_t* out_status;    /* optional [B] OXS_ROW_* */
  uint32_t* out_kept_count; /* optional [B] size of candidates_buffer after the call */
  uint32_t* out_kept_ids;   /* optional [B][kept_ld] */
  float* out_kept_probs;    /* optional [B][kept_ld] */
  int64_t kept_ld;

  /* Optional [B][logits_out_ld] f32: receives each row's logits after the
   * softcap (if any), bans, biases, newline, DRY and window penalties and
   * temperature, i.e. what the reference leaves in its `logits: &mut [f32]`
   * argument (sampler.rs:184-254; checked by academic_samplers_test.rs:75),
   * with masked ids at -inf. Must not overlap `logits`. */
  float* logits_out;
  int64_t logits_out_ld;

  /* The model's final logit softcap (final_logit_softcapping), done by the
   * reference as a pass of its own over the logits before sampling
   * (oxide-backend-cuda/src/lib.rs:3243-3255, launch_cuda_logit_softcap,
   * kernels/vec_ops_activations.cu:131-136). When > 0, every logit becomes
   * cap * tanhf(logit / cap) as it is read, before the mask and every
   * sampler stage; tanhf is glibc's (Rust's f32::tanh). 0 (or NaN) = off. */
  float logit_softcap;
} oxs_batch;

typedef struct oxs_sampler oxs_sampler;

/* ABI version of the loaded library (OXS_ABI_VERSION at build time). */
uint32_t oxs_abi_version(void);

/* Human-readable text for an OXS_* return code. */
const char* oxs_status_string(int code);

/* SamplingConfig::default() (sampler.rs:44-73), with newline_token_id = 0 and
 * empty bias/ban ranges. */
void oxs_sampling_config_default(oxs_sampling_config* cfg);

/* Initial rng_state of SamplerState::new (has_seed = 0) or
 * SamplerState::new_with_seed (sampler.rs:104-128; seed 0 maps to the default). */
uint64_t oxs_rng_state_from_seed(int has_seed, uint64_t seed);

/* Initial mirostat_mu of SamplerState::new(tau) = 2 * tau (sampler.rs:108). */
float oxs_mirostat_mu_from_tau(float tau);

/*
 * Creates a sampler on HIP device `device`, allocating every device buffer it
 * will ever need. Replaces AcademicSamplerEngine::new (sampler.rs:168), which
 * owned no device state. Not thread-safe; one sampler per stream.
 */
int oxs_sampler_create(oxs_sampler** out, const oxs_limits* limits, int device);

/* Frees the sampler's device workspace. Waits for nothing: the caller must
 * have synchronised the streams it used. */
int oxs_sampler_destroy(oxs_sampler* sampler);

/* Bytes of device workspace the sampler holds. */
size_t oxs_sampler_workspace_bytes(const oxs_sampler* sampler);

/*
 * Diagnostics, no counterpart in the reference: per-row counts of how each
 * row's top M = max(top_k, 256) candidates were found, for tests and tuning.
 * counts[OXS_PATH_BUCKETS]: a bucketed counting sort of the stream phase's
 * candidate keys (the fast path); [OXS_PATH_SORT]: a bitonic sort of those
 * keys (a bucket held too many); [OXS_PATH_EXACT]: a radix select over the
 * whole row (the candidates could not be proven to hold the top M, or the
 * row uses DRY); [OXS_PATH_NONE]: the row ended before the selection
 * (OXS_ROW_UNSUPPORTED, OXS_ROW_MISSING_STATE).
 * oxs_sampler_count_paths turns the counting on (enable != 0) or off for later
 * calls and zeroes the counts; oxs_sampler_path_counts copies them out. Both
 * synchronise the device: not for the decode loop.
 */
#define OXS_PATH_BUCKETS 0
#define OXS_PATH_SORT 1
#define OXS_PATH_EXACT 2
#define OXS_PATH_NONE 3
int oxs_sampler_count_paths(oxs_sampler* sampler, int enable);
int oxs_sampler_path_counts(const oxs_sampler* sampler, uint32_t counts[4]);

/*
 * Diagnostics: the read floor of the sampler's stream phase. Reads `batch`
 * rows of `vocab` f32 logits (16-byte aligned, vocab and logits_ld multiples
 * of 4) in the stream kernel's grid and load pattern and nothing else; each
 * (row, 8192-logit chunk) block writes one word to sink (batch * ceil(vocab /
 * 8192) words). No counterpart in the reference: it measures how fast one
 * pass over the logits can go.
 */
int oxs_read_floor(const float* logits, uint32_t vocab, int64_t logits_ld, uint32_t batch, uint32_t* sink,
                   void* stream);

/*
 * Samples every row of `batch` on `stream` (a hipStream_t; NULL = default
 * stream). Replaces B serial calls of
 *   AcademicSamplerEngine::sample_token(&self, logits: &mut [f32],
 *       state: &mut SamplerState, newline_token_id: u32) -> Result<u32>
 * (sampler.rs:173-178) at continuous_batching.rs:970-973 and
 * oxide-backend-cuda/src/lib.rs:3302/:6057. Asynchronous and stream ordered:
 * results are valid once the stream reaches this point. `logits` is read
 * only; the reference's in-place side effect is available through
 * oxs_batch.logits_out.
 * Returns OXS_ERR_SHAPE_MISMATCH for vocab == 0, OXS_ERR_LIMITS when the batch
 * exceeds the create-time limits, OXS_ERR_INVALID_ARGUMENT for missing
 * required pointers, OXS_ERR_HIP if the launch fails.
 */
int oxs_sample_batch(oxs_sampler* sampler, const oxs_batch* batch, void* stream);

/*
 * oxs_sample_batch without a sampler and without any allocation: the same
 * kernels and results, with the workspace in a fixed device array of this
 * library (one per GPU, about 13 MiB, held until the process ends) instead
 * of a sampler's. It has no counterpart in the reference; it is for callers
 * that cannot allocate device memory: code under HIP graph capture, serving
 * loops and harnesses that forbid hipMalloc.
 *   - batches up to OXS_STATIC_MAX_BATCH rows of up to OXS_STATIC_MAX_VOCAB
 *     logits; larger: OXS_ERR_LIMITS;
 *   - sized as a sampler with max_top_k = 1024 and a DRY list of 2048 ids:
 *     a row whose pool max(top_k, 256) (at most V) exceeds 1024, or whose DRY
 *     pass penalises more than 2048 distinct ids, returns OXS_ROW_UNSUPPORTED
 *     (token 0) while the other rows run;
 *   - runs on the calling thread's current device; the first call on a device
 *     sets the array up (finds its address and fills its constant tables,
 *     waiting for that on `stream`), so it must not be under stream capture
 *     (OXS_ERR_INVALID_ARGUMENT there); later calls only launch;
 *   - every call on one device shares that device's array: calls that overlap
 *     on one GPU (other streams, other threads) race and give wrong results;
 *   - per-path counting (oxs_sampler_count_paths) does not apply.
 * Other errors as oxs_sample_batch.
 */
#define OXS_STATIC_MAX_BATCH 256u
#define OXS_STATIC_MAX_VOCAB 524288u
int oxs_sample_batch_static(const oxs_batch* batch, void* stream);

/*
 * Decode-loop state beside the sampler state (ActiveSequence,
 * crates/oxide-engine/src/continuous_batching.rs:453-470), device arrays
 * unless noted; every pointer is optional.
 */
typedef struct oxs_decode_io {
  uint32_t* current_token;    /* [B] set to the sampled token: the next step's input (:974) */
  int32_t* current_position;  /* [B] += 1 (:975) */
  uint32_t* generated_count;  /* [B] += 1 (:976) */
  /* Host memory from oxs_host_alloc (megakernel_ops.cu:331-347's
   * h_sampled_token and its step counter): host_tokens[b] receives
   * (n << 32) | token in one 8-byte store, where n counts the decode steps on
   * this sampler that passed host_tokens and included row b (the first one
   * writes n = 1). The host polls each row's slot for its expected n instead
   * of synchronising the stream. */
  uint64_t* host_tokens;
} oxs_decode_io;

/*
 * One decode step of the scheduler's decode stage for B sequences at once
 * (continuous_batching.rs:957-977), replacing its per-sequence loop:
 *   - a row whose config has temperature <= 1e-6 takes the first largest of
 *     its raw logits (:961-970): no penalties, filters or history, and its
 *     rng_state, mirostat_mu and candidates buffer (out_kept_*) are left as
 *     they were; the allowed mask, if any, still applies;
 *   - every other row is sample_token(logits, state, newline_token_id)
 *     exactly as in oxs_sample_batch (:971-972); a failing row gives token 0
 *     (unwrap_or(0), :973);
 *   - then io's arrays are advanced (:974-976) and the tokens handed to the
 *     host. Calls that overlap on one sampler race on its per-row step counts.
 * Same arguments and errors as oxs_sample_batch, plus `io`; asynchronous;
 * allocates nothing and issues only kernels, so it can be captured in a HIP
 * graph. newline_token_id is the config's (the loop passes 10, :972).
 */
int oxs_decode_step(oxs_sampler* sampler, const oxs_batch* batch, const oxs_decode_io* io, void* stream);

/*
 * Batched argmax, replacing launch_cuda_argmax(const float*, int vocab_size,
 * uint32_t* out_token, float* out_max_val, int batch_size, cudaStream_t)
 * (oxide-backend-cuda/src/kernels/sampling_dfa.cu:161-178; driver.rs:671-679),
 * the CUDA backend's greedy path (oxide-backend-cuda/src/lib.rs:2479, :3266,
 * :4063). For each row of logits [batch][logits_ld] (f32, device): the largest
 * value above -1e30 and its token id, NaN and values <= -1e30 never taken (the
 * reference's running maximum starts at -1e30 and only a strictly larger value
 * replaces it); a row without one gives token 0 and -1e30. Among equal maxima
 * the winner is the reference's, which follows its thread layout (not the
 * lowest id): with batch > 1 (one 1024-thread block per row, :2-68) the id
 * whose thread t = id % 1024 has the smallest bit-reversed 5-bit warp index
 * (t / 32), then lane index (t % 32), and that thread's first such id; with
 * batch 1 (24 blocks of 256 threads striding by 6144, :70-159) the same over
 * block, warp and lane of id % 6144. -0.0 and +0.0 are equal, and out_max_val
 * receives the winning logit's own bits. out_max_val may be NULL.
 * Asynchronous; allocates nothing. Rows are split over several blocks, which
 * meet in file-scope device slots (as the reference's batch-1 path does):
 * calls that overlap on one device race on them. OXS_ERR_SHAPE_MISMATCH for
 * vocab 0; OXS_ERR_INVALID_ARGUMENT for vocab > 2^30.
 */
int oxs_argmax(const float* logits, uint32_t vocab, int64_t logits_ld, uint32_t batch, uint32_t* out_token,
               float* out_max_val, void* stream);

/* Page-locked host memory that the GPU writes directly (mapped, coherent; the
 * same address on host and device), zeroed. For oxs_decode_io's host fields.
 * OXS_ERR_UNSUPPORTED when the device address would differ from the host's. */
int oxs_host_alloc(size_t bytes, void** out);
int oxs_host_free(void* ptr);

/* Host side of the hand-off: spins until every one of `count` slots of
 * oxs_decode_io.host_tokens carries a step count of at least `step` (modulo
 * 2^32), copying each slot's token into tokens[i] as it reads it; no HIP call.
 * A spin_limit of 0 waits without limit; otherwise OXS_ERR_TIMEOUT after that
 * many passes. Replaces the host's wait on h_sampled_token's counter
 * (megakernel_ops.cu:331-347). */
int oxs_host_wait(const uint64_t* slots, uint32_t count, uint32_t step, uint32_t* tokens, uint64_t spin_limit);

/*
 * Grammar masks from a DFA (the producer of oxs_batch.allowed_mask).
 *
 * DfaSchemaGrammar (crates/oxide-core/src/dfa.rs:4-148): a transition table of
 * num_states x 256 next states, OXS_DFA_ERROR_STATE meaning "no transition".
 * For every row b and token t < vocab, bit (t % 32) of word t / 32 of row b's
 * mask is set when the token's bytes walk the table from states[b] without an
 * error: every step needs a current state < num_states and a next state other
 * than OXS_DFA_ERROR_STATE (DfaSchemaGrammar::transition, dfa.rs:110-126). A
 * token with no bytes is allowed. This is compute_token_mask
 * (crates/oxide-server/src/grammar_engine.rs:42-65) and the -inf pattern of
 * apply_dfa_mask (dfa.rs:130-148) for a batch of rows, as a packed bitmask:
 * bits past vocab in the last word are cleared; words past ceil(vocab / 32)
 * are not written.
 */
#define OXS_DFA_ERROR_STATE 0xffffffffu

typedef struct oxs_dfa {
  uint32_t num_states;
  const uint32_t* transitions; /* [num_states][256], device */
} oxs_dfa;

typedef struct oxs_token_bytes {
  uint32_t vocab;
  uint32_t num_bytes;      /* bytes in `bytes`; a token whose range is not inside it is not allowed */
  const uint32_t* offsets; /* [vocab + 1]: token t is bytes[offsets[t] .. offsets[t + 1]), device */
  const uint8_t* bytes;    /* device */
} oxs_token_bytes;

/*
 * Writes mask[b * mask_ld + w] for b < batch, w < ceil(vocab / 32), from
 * states[b] (device [batch]). Asynchronous on `stream`; allocates nothing.
 * Returns OXS_ERR_INVALID_ARGUMENT for missing pointers, mask_ld too small,
 * vocab above 2^31 or batch above 1048560, OXS_ERR_HIP if the launch fails.
 */
int oxs_dfa_mask(const oxs_dfa* dfa, const oxs_token_bytes* tokens, const uint32_t* states, uint32_t batch,
                 uint32_t* mask, int64_t mask_ld, void* stream);

/*
 * Grammar masks by state. A token's walk depends only on the state it starts
 * from, so the masks of a grammar over a vocabulary can be computed once, with
 * oxs_dfa_mask over the states 0 .. num_states (the last one stands for every
 * state outside the table, from which only tokens with no bytes are allowed),
 * into state_masks[(num_states + 1) * state_masks_ld] words, and each step's
 * masks then gathered: row b of `mask` is row min(states[b], num_states) of
 * state_masks. The result equals oxs_dfa_mask on the same states.
 * Asynchronous on `stream`; allocates nothing. Returns
 * OXS_ERR_INVALID_ARGUMENT for missing pointers, a leading dimension below
 * ceil(vocab / 32) or batch above 65535.
 */
int oxs_dfa_mask_gather(const uint32_t* state_masks, uint32_t num_states, int64_t state_masks_ld, uint32_t vocab,
                        const uint32_t* states, uint32_t batch, uint32_t* mask, int64_t mask_ld, void* stream);

/*
 * Static grammar masks (one row, the same for every step), written as
 * mask[ceil(vocab / 32)] words; pass them to oxs_batch with mask_ld = 0 to
 * share them across rows.
 *
 * GbnfGrammarEngine::apply_grammar_mask (crates/oxide-core/src/sampler.rs:555-583)
 * for the start rule: token t's text (tokens, UTF-8) is allowed when it is
 * empty (no first character: the reference leaves it alone), when its first
 * character, decoded from UTF-8 (a malformed sequence decodes to U+FFFD), lies
 * in one of `ranges` ([lo, hi] code points, inclusive), or when a literal
 * starts with its text or its text starts with a literal. All pointers device.
 */
typedef struct oxs_gbnf_rule {
  uint32_t num_ranges;
  const uint32_t* ranges;          /* [num_ranges][2] */
  uint32_t num_literals;
  const uint32_t* literal_offsets; /* [num_literals + 1] into literal_bytes */
  const uint8_t* literal_bytes;
} oxs_gbnf_rule;

int oxs_gbnf_mask(const oxs_gbnf_rule* rule, const oxs_token_bytes* tokens, uint32_t* mask, void* stream);

/*
 * GrammarLogitMasker::mask_logits (crates/oxide-core/src/grammar_mask.rs:55-65):
 * token t with an ASCII byte (token_ascii[t] < 256) is masked unless
 * allowed_ascii[that byte] != 0; token_ascii[t] >= 256 stands for Rust's None
 * (left alone). allowed_ascii is [256], token_ascii [vocab]; device pointers.
 * The reference masks only min(vocab_ascii_bytes.len(), logits.len()) tokens:
 * pass that count as vocab.
 */
int oxs_ascii_mask(const uint8_t* allowed_ascii, const uint16_t* token_ascii, uint32_t vocab, uint32_t* mask,
                   void* stream);

/*
 * LM head: the projection that produces the logits the sampler reads, in the
 * reference's GGUF Q8_0 format (oxide-backend-cuda/src/lib.rs:4013-4035, the
 * batched decode; :3229-3243 for the last prompt token).
 *
 * q8_1 activations: n / 32 blocks of 36 bytes, {f16 d, f16 sum, int8 qs[32]}
 * (common_types.cuh:8-11). Q8_0 weights: m rows (tokens) of k / 32 blocks of
 * 34 bytes, {f16 d, int8 qs[32]} (common_types.cuh:13-16).
 */

/* launch_cuda_quantize_q8_1 (kernels/launch_wrappers.cu:143-154,
 * quantize_f32_to_q8_1_cuda_kernel norms_rope.cu:2-29): each 32-value block of
 * x becomes d = amax / 127, qs = roundf(x / d) (x * (1 / d), 0 when d == 0),
 * sum = the 32 values summed in the kernel's butterfly order. n / 32 blocks
 * are written (a remainder is ignored, as there); n == 0 does nothing. */
int oxs_quantize_q8_1(const float* x, uint32_t n, void* y_q8_1, void* stream);

/* Bytes of the packed weight layout oxs_mmvq_q8_0 reads for an m x k Q8_0
 * matrix: per 32 tokens and per 32-wide block of k, 1024 bytes of quants in
 * the order the matrix cores take them and 64 bytes of scales (1088 bytes;
 * tokens past m are zero). 0 when k is not a multiple of 128. */
size_t oxs_q8_0_packed_bytes(uint32_t m, uint32_t k);

/* Repacks GGUF Q8_0 rows (w, [m][k / 32] 34-byte blocks) into the packed
 * layout, once at model load. k must be a multiple of 128
 * (OXS_ERR_UNSUPPORTED otherwise). No counterpart in the reference, whose
 * kernel reads the GGUF blocks directly. w_packed must be 16-byte aligned. */
int oxs_pack_q8_0(const void* w, uint32_t m, uint32_t k, void* w_packed, void* stream);

/* launch_cuda_mmvq_q8_0 (kernels/launch_wrappers.cu:156-200,
 * mmvq_q8_0_cuda_kernel quant_gemv_standard.cu:418-513): y[c][t] for batch
 * column c < batch and token t < m, from the packed weights and the q8_1
 * activations x ([batch][k / 32] blocks). Each value is the reference's, bit
 * for bit: per block b the exact integer dot of the 32 quants, accumulated as
 * A[b % 4] = fmaf(d_w * d_x, (float)dot, A[b % 4]) in increasing b, then
 * (A0 + A2) + (A1 + A3). m == 0 or batch == 0 does nothing; k must be a
 * multiple of 128. w_packed must be 16-byte aligned, x_q8_1 and y 4-byte
 * aligned (OXS_ERR_INVALID_ARGUMENT otherwise). */
int oxs_mmvq_q8_0(float* y, const void* w_packed, const void* x_q8_1, uint32_t m, uint32_t k, uint32_t batch,
                  void* stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* OXIDE_SAMPLER_H */
