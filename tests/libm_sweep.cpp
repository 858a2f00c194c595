// Sweeps the device libm emulation (oxs_libm.h, compiled here as host C++)
// against the host's glibc expf/logf/log2f/powf/tanhf, bit for bit.
//
// usage: libm_sweep FUSED STRIDE
//   FUSED  1 compares the fused-multiply-add form (what glibc's ifunc picks on
//          a CPU with FMA), 0 the generic form;
//   STRIDE visits every STRIDE-th 32-bit pattern, plus a dense pass over the
//          softmax range [-104, 0] of expf and over [2^-27, 1] of the logs.
// Prints "<fn> <checked> <mismatches> <first mismatching input bits>" per
// function; exits 1 if any mismatch.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include "../oxide-tech-llm-engine_amd/csrc/oxs_libm.h"

using namespace oxs_libm;

namespace {

bool same(float a, float b) { return (isnan(a) && isnan(b)) || f2u(a) == f2u(b); }

struct Tally {
  unsigned long long checked = 0, bad = 0;
  uint32_t first = 0;
  void add(uint32_t bits, bool ok) {
    ++checked;
    if (!ok && bad++ == 0) first = bits;
  }
};

template <bool FUSED>
int run(uint64_t stride) {
  Tally te, tl, t2;
  auto check_all = [&](uint32_t bits) {
    float x = u2f(bits);
    te.add(bits, same(expf_t<FUSED>(x), expf(x)));
    tl.add(bits, same(logf_t<FUSED>(x), logf(x)));
    t2.add(bits, same(log2f_t<FUSED>(x), log2f(x)));
  };
  for (uint64_t b = 0; b <= 0xffffffffull; b += stride) check_all((uint32_t)b);
  // Dense passes over the ranges the sampler evaluates most: expf of
  // (logit - max) <= 0 and the logs of probabilities in (0, 1].
  for (uint32_t b = f2u(-104.0f); b >= 0x80000000u; b -= 13) {
    float x = u2f(b);
    te.add(b, same(expf_t<FUSED>(x), expf(x)));
  }
  for (uint32_t b = f2u(7.450580596923828e-09f); b <= f2u(1.0f); b += 11) {
    float x = u2f(b);
    tl.add(b, same(logf_t<FUSED>(x), logf(x)));
    t2.add(b, same(log2f_t<FUSED>(x), log2f(x)));
  }
  // powf: every stride-th base with the integer exponents DRY uses (0..40),
  // plus bases and exponents from the same sweep
  Tally tp;
  for (uint64_t b = 0; b <= 0xffffffffull; b += stride * 64) {
    const float x = u2f((uint32_t)b);
    for (int e = 0; e <= 40; ++e) {
      const float y = (float)e;
      tp.add((uint32_t)b, same(powf_t<FUSED>(x, y), powf(x, y)));
    }
    const float y2 = u2f((uint32_t)(b * 2654435761ull));
    tp.add((uint32_t)b, same(powf_t<FUSED>(x, y2), powf(x, y2)));
  }
  // tanhf (one form: plain float steps): the stride sweep, plus every float
  // in [-40, 40], the arguments l / cap of logit softcaps
  Tally tt;
  for (uint64_t b = 0; b <= 0xffffffffull; b += stride) {
    const float x = u2f((uint32_t)b);
    tt.add((uint32_t)b, same(tanhf_fdlibm(x), tanhf(x)));
  }
  for (uint32_t b = 0; b <= f2u(40.0f); b += 3) {
    const float x = u2f(b);
    tt.add(b, same(tanhf_fdlibm(x), tanhf(x)) && same(tanhf_fdlibm(-x), tanhf(-x)));
  }
  printf("expf %llu %llu %08x\n", te.checked, te.bad, te.first);
  printf("tanhf %llu %llu %08x\n", tt.checked, tt.bad, tt.first);
  printf("powf %llu %llu %08x\n", tp.checked, tp.bad, tp.first);
  printf("logf %llu %llu %08x\n", tl.checked, tl.bad, tl.first);
  printf("log2f %llu %llu %08x\n", t2.checked, t2.bad, t2.first);
  return (te.bad | tl.bad | t2.bad | tp.bad | tt.bad) ? 1 : 0;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 3) {
    fprintf(stderr, "usage: %s FUSED STRIDE\n", argv[0]);
    return 2;
  }
  int fused = atoi(argv[1]);
  uint64_t stride = strtoull(argv[2], nullptr, 10);
  if (stride == 0) stride = 1;
  return fused ? run<true>(stride) : run<false>(stride);
}
