// zero_alloc_test.cpp — the C ABI's promise that a sampling call allocates
// nothing, checked the way the reference checks its decode loop
// (crates/oxide-engine/tests/test_zero_alloc_forward_decode.rs:9-85 with the
// counting allocator of crates/oxide-core/src/zero_alloc_guard.rs:9-41): count
// allocations across many steady-state calls and require none.
//
// Host: malloc, calloc, realloc, memalign, posix_memalign, aligned_alloc and
// operator new are defined in this executable, so every library in the process
// resolves to them. Each one counts a call whose caller lies inside
// liboxide_sampler.so's mapped range (the library's own allocations) and,
// separately, every call made while the window is open (the HIP runtime's
// included, reported for information). Device: hipMemGetInfo before and after.
//
// The window covers 1000 oxs_sample_batch calls, 1000 oxs_decode_step calls
// and 1000 oxs_sample_batch_static calls on a config-2 shaped batch
// (64 x 128256 f32), after a warm-up (for the static entry point, its set-up
// call on the device). Prints one
// JSON line; exits 0 when the library made no host allocation and the device's
// free memory did not change.
#include <hip/hip_runtime.h>
#include <link.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <cerrno>
#include <new>
#include <vector>

#include "../../include/oxide_sampler.h"

extern "C" void* __libc_malloc(size_t);
extern "C" void* __libc_calloc(size_t, size_t);
extern "C" void* __libc_realloc(void*, size_t);
extern "C" void* __libc_memalign(size_t, size_t);
extern "C" void __libc_free(void*);

static uintptr_t g_lo = 0, g_hi = 0;  // liboxide_sampler.so's mapped range
static std::atomic<bool> g_on{false};
static std::atomic<uint64_t> g_lib_allocs{0}, g_all_allocs{0};

static inline void note(void* caller) {
  if (!g_on.load(std::memory_order_relaxed)) return;
  g_all_allocs.fetch_add(1, std::memory_order_relaxed);
  const uintptr_t a = (uintptr_t)caller;
  if (a >= g_lo && a < g_hi) g_lib_allocs.fetch_add(1, std::memory_order_relaxed);
}

extern "C" {
void* malloc(size_t n) {
  note(__builtin_return_address(0));
  return __libc_malloc(n);
}
void* calloc(size_t a, size_t b) {
  note(__builtin_return_address(0));
  return __libc_calloc(a, b);
}
void* realloc(void* p, size_t n) {
  note(__builtin_return_address(0));
  return __libc_realloc(p, n);
}
void* memalign(size_t al, size_t n) {
  note(__builtin_return_address(0));
  return __libc_memalign(al, n);
}
void* aligned_alloc(size_t al, size_t n) {
  note(__builtin_return_address(0));
  return __libc_memalign(al, n);
}
int posix_memalign(void** out, size_t al, size_t n) {
  note(__builtin_return_address(0));
  void* p = __libc_memalign(al, n);
  if (!p) return ENOMEM;
  *out = p;
  return 0;
}
void free(void* p) { __libc_free(p); }
}

void* operator new(size_t n) {
  note(__builtin_return_address(0));
  void* p = __libc_malloc(n ? n : 1);
  if (!p) throw std::bad_alloc();
  return p;
}
void* operator new[](size_t n) {
  note(__builtin_return_address(0));
  void* p = __libc_malloc(n ? n : 1);
  if (!p) throw std::bad_alloc();
  return p;
}
void operator delete(void* p) noexcept { __libc_free(p); }
void operator delete[](void* p) noexcept { __libc_free(p); }
void operator delete(void* p, size_t) noexcept { __libc_free(p); }
void operator delete[](void* p, size_t) noexcept { __libc_free(p); }

static int find_library(struct dl_phdr_info* info, size_t, void*) {
  const char* name = info->dlpi_name;
  if (!name || !strstr(name, "liboxide_sampler.so")) return 0;
  uintptr_t lo = UINTPTR_MAX, hi = 0;
  for (int i = 0; i < info->dlpi_phnum; ++i) {
    const ElfW(Phdr)& ph = info->dlpi_phdr[i];
    if (ph.p_type != PT_LOAD) continue;
    const uintptr_t a = info->dlpi_addr + ph.p_vaddr;
    if (a < lo) lo = a;
    if (a + ph.p_memsz > hi) hi = a + ph.p_memsz;
  }
  g_lo = lo;
  g_hi = hi;
  return 1;
}

#define HIP_OK(x)                                                    \
  do {                                                               \
    if ((x) != hipSuccess) {                                         \
      fprintf(stderr, "%s failed at line %d\n", #x, __LINE__);       \
      return 2;                                                      \
    }                                                                \
  } while (0)
#define OXS_OK_(x)                                                   \
  do {                                                               \
    const int rc_ = (x);                                             \
    if (rc_ != OXS_OK) {                                             \
      fprintf(stderr, "%s -> %d at line %d\n", #x, rc_, __LINE__);   \
      return 2;                                                      \
    }                                                                \
  } while (0)

int main() {
  const uint32_t B = 64, V = 128256, H = 512, CAP = 4096;
  const int kCalls = 1000;
  dl_iterate_phdr(find_library, nullptr);
  if (g_hi == 0) {
    fprintf(stderr, "liboxide_sampler.so is not mapped\n");
    return 2;
  }
  HIP_OK(hipSetDevice(0));
  hipStream_t st;
  HIP_OK(hipStreamCreate(&st));

  oxs_limits lim = {B, V, 256, 0};
  oxs_sampler* s = nullptr;
  OXS_OK_(oxs_sampler_create(&s, &lim, 0));

  // a config-2 shaped batch (values need only be finite and varied)
  std::vector<float> logits((size_t)B * V);
  uint64_t x = 0x5EED0002ull;
  for (auto& v : logits) {
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    v = (float)((int64_t)(x >> 40) - (1 << 23)) * (6.0f / (1 << 23));
  }
  std::vector<oxs_sampling_config> cfg(B);
  for (auto& c : cfg) {
    oxs_sampling_config_default(&c);
    c.frequency_penalty = 0.3f;
    c.presence_penalty = 0.2f;
    c.repeat_penalty = 1.05f;
    c.repeat_last_n = H;
    c.temperature = 0.7f;
    c.top_k = 50;
    c.top_p = 0.9f;
    c.min_p = 0.05f;
    c.newline_token_id = 10;
  }
  std::vector<uint32_t> hist((size_t)B * CAP), hlen(B, H);
  for (auto& t : hist) {
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    t = (uint32_t)(x % V);
  }
  std::vector<float> u(B, 0.37f);
  std::vector<uint64_t> rng(B, 0x853c49e6748fea9bull);

  float *d_logits, *d_u;
  oxs_sampling_config* d_cfg;
  uint32_t *d_hist, *d_hlen, *d_tok, *d_kc, *d_kid, *d_cur, *d_cnt;
  int32_t *d_status, *d_pos;
  float* d_kp;
  uint64_t* d_rng;
  HIP_OK(hipMalloc(&d_logits, logits.size() * 4));
  HIP_OK(hipMalloc(&d_cfg, B * sizeof(oxs_sampling_config)));
  HIP_OK(hipMalloc(&d_hist, hist.size() * 4));
  HIP_OK(hipMalloc(&d_hlen, B * 4));
  HIP_OK(hipMalloc(&d_u, B * 4));
  HIP_OK(hipMalloc(&d_rng, B * 8));
  HIP_OK(hipMalloc(&d_tok, B * 4));
  HIP_OK(hipMalloc(&d_status, B * 4));
  HIP_OK(hipMalloc(&d_kc, B * 4));
  HIP_OK(hipMalloc(&d_kid, B * 64 * 4));
  HIP_OK(hipMalloc(&d_kp, B * 64 * 4));
  HIP_OK(hipMalloc(&d_cur, B * 4));
  HIP_OK(hipMalloc(&d_pos, B * 4));
  HIP_OK(hipMalloc(&d_cnt, B * 4));
  HIP_OK(hipMemcpy(d_logits, logits.data(), logits.size() * 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(d_cfg, cfg.data(), B * sizeof(oxs_sampling_config), hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(d_hist, hist.data(), hist.size() * 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(d_hlen, hlen.data(), B * 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(d_u, u.data(), B * 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(d_rng, rng.data(), B * 8, hipMemcpyHostToDevice));
  HIP_OK(hipMemset(d_cur, 0, B * 4));
  HIP_OK(hipMemset(d_pos, 0, B * 4));
  HIP_OK(hipMemset(d_cnt, 0, B * 4));
  void* host_tokens = nullptr;
  OXS_OK_(oxs_host_alloc(B * 8, &host_tokens));

  oxs_batch b;
  memset(&b, 0, sizeof(b));
  b.batch = B;
  b.vocab = V;
  b.logits_dtype = OXS_DTYPE_F32;
  b.logits_ld = V;
  b.logits = d_logits;
  b.configs = d_cfg;
  b.history = d_hist;
  b.history_ld = CAP;
  b.history_len = d_hlen;
  b.uniforms = d_u;
  b.out_tokens = d_tok;
  b.out_status = d_status;
  b.out_kept_count = d_kc;
  b.out_kept_ids = d_kid;
  b.out_kept_probs = d_kp;
  b.kept_ld = 64;
  // the decode step: device xorshift draws, history recorded (room for every step)
  oxs_batch bd = b;
  bd.uniforms = nullptr;
  bd.rng_state = d_rng;
  bd.flags = OXS_FLAG_RECORD_HISTORY;
  bd.history_cap = CAP;
  oxs_decode_io io = {d_cur, d_pos, d_cnt, (uint64_t*)host_tokens};

  for (int i = 0; i < 10; ++i) {  // warm-up: code objects loaded, queues created
    OXS_OK_(oxs_sample_batch(s, &b, st));
    OXS_OK_(oxs_decode_step(s, &bd, &io, st));
  }
  OXS_OK_(oxs_sample_batch_static(&b, st));  // the no-allocation entry point's set-up call on this device
  HIP_OK(hipStreamSynchronize(st));
  HIP_OK(hipMemcpy(d_hlen, hlen.data(), B * 4, hipMemcpyHostToDevice));
  HIP_OK(hipDeviceSynchronize());
  size_t free0 = 0, free1 = 0, total = 0;
  HIP_OK(hipMemGetInfo(&free0, &total));

  g_on.store(true);
  int rc_sample = OXS_OK, rc_decode = OXS_OK, rc_static = OXS_OK;
  for (int i = 0; i < kCalls && rc_sample == OXS_OK; ++i) rc_sample = oxs_sample_batch(s, &b, st);
  for (int i = 0; i < kCalls && rc_decode == OXS_OK; ++i) rc_decode = oxs_decode_step(s, &bd, &io, st);
  for (int i = 0; i < kCalls && rc_static == OXS_OK; ++i) rc_static = oxs_sample_batch_static(&b, st);
  g_on.store(false);

  HIP_OK(hipStreamSynchronize(st));
  HIP_OK(hipMemGetInfo(&free1, &total));
  const uint64_t lib_allocs = g_lib_allocs.load(), all_allocs = g_all_allocs.load();
  printf("{\"sample_batch_calls\": %d, \"decode_step_calls\": %d, \"sample_batch_static_calls\": %d, "
         "\"rc_sample\": %d, \"rc_decode\": %d, \"rc_static\": %d, "
         "\"library_host_allocations\": %llu, \"process_host_allocations\": %llu, "
         "\"device_free_bytes_before\": %zu, \"device_free_bytes_after\": %zu}\n",
         kCalls, kCalls, kCalls, rc_sample, rc_decode, rc_static, (unsigned long long)lib_allocs,
         (unsigned long long)all_allocs, free0, free1);
  fflush(stdout);
  oxs_host_free(host_tokens);
  oxs_sampler_destroy(s);
  const bool ok = rc_sample == OXS_OK && rc_decode == OXS_OK && rc_static == OXS_OK && lib_allocs == 0 &&
                  free0 == free1;
  return ok ? 0 : 1;
}
