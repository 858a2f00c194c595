// Single-precision exp/ln/log2/pow (and tanh, at the end) that reproduce, bit
// for bit, the glibc >= 2.27 implementations that Rust's f32::{exp, ln, log2,
// powf, tanh} lower to on x86_64-linux-gnu.
//
// The reference sampler (crates/oxide-core/src/sampler.rs:289 exp, :424 and
// :440/:451 log2, :496/:502 ln, :409 powf) calls the platform libm. glibc's single
// precision routines are the published ARM optimized-routines algorithms
// (Szabolcs Nagy, 2017; MIT licence): evaluate in double precision with a
// 32-entry 2^(i/32) table (exp) or a 16-entry (1/c, log c) table (ln, log2) and
// a short polynomial, then round once to float. Because every step is plain
// IEEE double arithmetic, the same sequence of operations on the GPU's IEEE
// f64 units yields the same float.
//
// glibc builds these routines twice on x86_64 and picks one at load time
// (ifunc): a generic build and an FMA build in which the compiler fuses each
// multiply feeding an add. The two builds differ in the last bit for a small
// fraction of inputs, so both are provided here (template argument FUSED).
// The device uses the fused form: glibc selects it on every x86_64 CPU with
// FMA, which includes every host CPU an MI355X is paired with.
//
// Each routine takes its table as an argument (defaulting to the constant
// tables below) so that device code can pass copies held in LDS.
//
// This header compiles as HIP device code and as plain host C++ (for the
// tests that sweep it against the host libm). Build with -ffp-contract=off.
#pragma once
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define OXS_HD __host__ __device__ __forceinline__
#define OXS_CONST_TABLE __device__ __constant__
#else
#define OXS_HD static inline
#define OXS_CONST_TABLE static const
#include <math.h>
#endif

namespace oxs_libm {

OXS_HD uint32_t f2u(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
OXS_HD float u2f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }
OXS_HD uint64_t d2u(double x) { uint64_t u; memcpy(&u, &x, 8); return u; }
OXS_HD double u2d(uint64_t u) { double x; memcpy(&x, &u, 8); return x; }

OXS_HD double fma_d(double a, double b, double c) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_fma(a, b, c);
#else
  return fma(a, b, c);
#endif
}

// a*b + c, either fused (one rounding) or as two rounded operations.
template <bool FUSED>
OXS_HD double mad(double a, double b, double c) {
  if (FUSED) return fma_d(a, b, c);
  double p = a * b;
  return p + c;
}

// 2^(i/32) as double bits, minus i<<47 so that adding k<<47 scales by 2^(k/32).
// Each entry is the correctly rounded double of 2^(i/32) (derivable from the
// definition; the table-generation check lives in the tests).
OXS_CONST_TABLE uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// (1/c, ln c) and (1/c, log2 c) for the 16 subintervals of [0x3f330000, 2*0x3f330000).
OXS_CONST_TABLE double kLogInvc[16] = {
    0x1.661ec79f8f3bep+0, 0x1.571ed4aaf883dp+0, 0x1.49539f0f010bp+0,  0x1.3c995b0b80385p+0,
    0x1.30d190c8864a5p+0, 0x1.25e227b0b8eap+0,  0x1.1bb4a4a1a343fp+0, 0x1.12358f08ae5bap+0,
    0x1.0953f419900a7p+0, 0x1p+0,               0x1.e608cfd9a47acp-1, 0x1.ca4b31f026aap-1,
    0x1.b2036576afce6p-1, 0x1.9c2d163a1aa2dp-1, 0x1.886e6037841edp-1, 0x1.767dcf5534862p-1,
};
OXS_CONST_TABLE double kLnLogc[16] = {
    -0x1.57bf7808caadep-2, -0x1.2bef0a7c06ddbp-2, -0x1.01eae7f513a67p-2, -0x1.b31d8a68224e9p-3,
    -0x1.6574f0ac07758p-3, -0x1.1aa2bc79c81p-3,   -0x1.a4e76ce8c0e5ep-4, -0x1.1973c5a611cccp-4,
    -0x1.252f438e10c1ep-5, 0x0p+0,                0x1.aa5aa5df25984p-5,  0x1.c5e53aa362eb4p-4,
    0x1.526e57720db08p-3,  0x1.bc2860d22477p-3,   0x1.1058bc8a07ee1p-2,  0x1.4043057b6ee09p-2,
};
OXS_CONST_TABLE double kLog2Logc[16] = {
    -0x1.efec65b963019p-2, -0x1.b0b6832d4fca4p-2, -0x1.7418b0a1fb77bp-2, -0x1.39de91a6dcf7bp-2,
    -0x1.01d9bf3f2b631p-2, -0x1.97c1d1b3b7afp-3,  -0x1.2f9e393af3c9fp-3, -0x1.960cbbf788d5cp-4,
    -0x1.a6f9db6475fcep-5, 0x0p+0,                0x1.338ca9f24f53dp-4,  0x1.476a9543891bap-3,
    0x1.e840b4ac4e4d2p-3,  0x1.40645f0c6651cp-2,  0x1.88e9c2c1b9ff8p-2,  0x1.ce0a44eb17bccp-2,
};

// expf: x*32/ln2 = k + r, exp(x) = 2^(k/32) * 2^(r/32), 2^(r/32) by a cubic.
template <bool FUSED>
OXS_HD float expf_t(float x, const uint64_t* exp2tab = kExp2Tab) {
  const double kInvLn2N = 0x1.71547652b82fep+0 * 32;
  const double kShift = 0x1.8p+52;
  const double C0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
  const double C1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
  const double C2 = 0x1.62e42ff0c52d6p-1 / 32;
  uint32_t ux = f2u(x);
  uint32_t abstop = (ux >> 20) & 0x7ff;
  if (abstop >= (f2u(88.0f) >> 20)) {
    if (ux == 0xff800000u) return 0.0f;            // exp(-inf) = 0
    if (abstop >= 0x7f8) return x + x;             // nan, +inf
    if (x > 0x1.62e42ep6f) return u2f(0x7f800000u); // overflow -> +inf
    if (x < -0x1.9fe368p6f) return 0.0f;           // underflow -> +0
  }
  double xd = (double)x;
  double kd, r;
  if (FUSED) {
    // The fused build computes z = InvLn2N*x once per use, fused into both
    // the rounding shift and the reduction.
    kd = fma_d(kInvLn2N, xd, kShift);
  } else {
    double z = kInvLn2N * xd;
    kd = z + kShift;
  }
  uint64_t ki = d2u(kd);
  kd -= kShift;
  if (FUSED) {
    r = fma_d(kInvLn2N, xd, -kd);
  } else {
    double z = kInvLn2N * xd;
    r = z - kd;
  }
  uint64_t t = exp2tab[ki % 32];
  t += ki << 47;
  double s = u2d(t);
  double zz = mad<FUSED>(C0, r, C1);
  double r2 = r * r;
  double y = mad<FUSED>(C2, r, 1.0);
  y = mad<FUSED>(zz, r2, y);
  y = y * s;
  return (float)y;
}

// Shared argument reduction of logf/log2f: x = 2^k z, z in [OFF, 2 OFF).
// Returns false (and sets *special) for zero, negative, inf, nan inputs.
template <bool LOG2>
OXS_HD bool log_special(float x, uint32_t* ix_io, float* special) {
  uint32_t ix = *ix_io;
  if (ix == 0x3f800000u) { *special = 0.0f; return true; }
  if (ix - 0x00800000u >= 0x7f800000u - 0x00800000u) {
    if (ix * 2 == 0) { *special = u2f(0xff800000u); return true; }         // -inf
    if (ix == 0x7f800000u) { *special = x; return true; }                   // +inf
    if ((ix & 0x80000000u) || ix * 2 >= 0xff000000u) {                      // nan
      *special = u2f(0x7fc00000u);
      if (ix * 2 > 0xff000000u) *special = x;
      return true;
    }
    // subnormal: normalise
    ix = f2u(x * 0x1p23f);
    ix -= 23u << 23;
  }
  *ix_io = ix;
  return false;
}

template <bool FUSED>
OXS_HD float logf_t(float x, const double* invc_tab = kLogInvc, const double* logc_tab = kLnLogc) {
  const double kLn2 = 0x1.62e42fefa39efp-1;
  const double A0 = -0x1.00ea348b88334p-2, A1 = 0x1.5575b0be00b6ap-2, A2 = -0x1.ffffef20a4123p-2;
  uint32_t ix = f2u(x);
  float sp;
  if (log_special<false>(x, &ix, &sp)) return sp;
  uint32_t tmp = ix - 0x3f330000u;
  int i = (int)((tmp >> (23 - 4)) % 16);
  int k = (int32_t)tmp >> 23;
  uint32_t iz = ix - (tmp & 0xff800000u);
  double invc = invc_tab[i], logc = logc_tab[i];
  double z = (double)u2f(iz);
  double r = mad<FUSED>(z, invc, -1.0);
  double y0 = mad<FUSED>((double)k, kLn2, logc);
  double r2 = r * r;
  double y = mad<FUSED>(A1, r, A2);
  y = mad<FUSED>(A0, r2, y);
  y = mad<FUSED>(y, r2, y0 + r);
  return (float)y;
}

template <bool FUSED>
OXS_HD float log2f_t(float x, const double* invc_tab = kLogInvc, const double* logc_tab = kLog2Logc) {
  const double A0 = -0x1.712b6f70a7e4dp-2, A1 = 0x1.ecabf496832ep-2, A2 = -0x1.715479ffae3dep-1,
               A3 = 0x1.715475f35c8b8p0;
  uint32_t ix = f2u(x);
  float sp;
  if (log_special<true>(x, &ix, &sp)) return sp;
  uint32_t tmp = ix - 0x3f330000u;
  int i = (int)((tmp >> (23 - 4)) % 16);
  uint32_t top = tmp & 0xff800000u;
  uint32_t iz = ix - top;
  int k = (int32_t)tmp >> 23;
  double invc = invc_tab[i], logc = logc_tab[i];
  double z = (double)u2f(iz);
  double r = mad<FUSED>(z, invc, -1.0);
  double y0 = logc + (double)k;
  double r2 = r * r;
  double y = mad<FUSED>(A1, r, A2);
  y = mad<FUSED>(A0, r2, y);
  double p = mad<FUSED>(A3, r, y0);
  y = mad<FUSED>(y, r2, p);
  return (float)y;
}

// powf (the same published algorithm family): log2(x) in double from the
// 16-entry (1/c, log2 c) table and a degree-5 polynomial, times y, then
// exp2 of that from the 32-entry 2^(i/32) table and a cubic, rounded once.
// Covers every input; the sampler calls it with finite exponents only.
template <bool FUSED>
OXS_HD double powf_log2(uint32_t ix, const double* invc_tab, const double* logc_tab) {
  const double A0 = 0x1.27616c9496e0bp-2, A1 = -0x1.71969a075c67ap-2, A2 = 0x1.ec70a6ca7baddp-2,
               A3 = -0x1.7154748bef6c8p-1, A4 = 0x1.71547652ab82bp0;
  uint32_t tmp = ix - 0x3f330000u;
  int i = (int)((tmp >> (23 - 4)) % 16);
  uint32_t top = tmp & 0xff800000u;
  uint32_t iz = ix - top;
  int k = (int32_t)top >> 23;
  double invc = invc_tab[i], logc = logc_tab[i];
  double z = (double)u2f(iz);
  double r = mad<FUSED>(z, invc, -1.0);
  double y0 = logc + (double)k;
  double r2 = r * r;
  double y = mad<FUSED>(A0, r, A1);
  double p = mad<FUSED>(A2, r, A3);
  double r4 = r2 * r2;
  double q = mad<FUSED>(A4, r, y0);
  q = mad<FUSED>(p, r2, q);
  y = mad<FUSED>(y, r4, q);
  return y;
}

template <bool FUSED>
OXS_HD double powf_exp2(double xd, uint64_t sign_bias, const uint64_t* exp2tab) {
  const double kShift = 0x1.8p+52 / 32;
  const double C0 = 0x1.c6af84b912394p-5, C1 = 0x1.ebfce50fac4f3p-3, C2 = 0x1.62e42ff0c52d6p-1;
  double kd = xd + kShift;
  uint64_t ki = d2u(kd);
  kd -= kShift;
  double r = xd - kd;
  uint64_t t = exp2tab[ki % 32];
  uint64_t ski = ki + sign_bias;
  t += ski << (52 - 5);
  double s = u2d(t);
  double z = mad<FUSED>(C0, r, C1);
  double r2 = r * r;
  double y = mad<FUSED>(C2, r, 1.0);
  y = mad<FUSED>(z, r2, y);
  return y * s;
}

// 0 when y is not an integer, 1 when odd, 2 when even (y's bits iy).
OXS_HD int powf_checkint(uint32_t iy) {
  int e = (int)(iy >> 23 & 0xff);
  if (e < 0x7f) return 0;
  if (e > 0x7f + 23) return 2;
  if (iy & ((1u << (0x7f + 23 - e)) - 1)) return 0;
  if (iy & (1u << (0x7f + 23 - e))) return 1;
  return 2;
}

OXS_HD bool powf_zeroinfnan(uint32_t ix) { return 2 * ix - 1 >= 2u * 0x7f800000u - 1; }
OXS_HD bool powf_issignaling(uint32_t ix) { return 2 * (ix ^ 0x00400000u) > 2u * 0x7fc00000u; }

template <bool FUSED>
OXS_HD float powf_t(float x, float y, const uint64_t* exp2tab = kExp2Tab, const double* invc_tab = kLogInvc,
                    const double* logc_tab = kLog2Logc) {
  uint64_t sign_bias = 0;
  uint32_t ix = f2u(x), iy = f2u(y);
  if (ix - 0x00800000u >= 0x7f800000u - 0x00800000u || powf_zeroinfnan(iy)) {
    // x is subnormal, negative, zero, inf or nan, or y is zero, inf or nan
    if (powf_zeroinfnan(iy)) {
      // a signalling nan operand still yields a nan where pow would give 1
      if (2 * iy == 0) return powf_issignaling(ix) ? x + y : 1.0f;
      if (ix == 0x3f800000u) return powf_issignaling(iy) ? x + y : 1.0f;
      if (2 * ix > 2u * 0x7f800000u || 2 * iy > 2u * 0x7f800000u) return x + y;
      if (2 * ix == 2 * 0x3f800000u) return 1.0f;
      if ((2 * ix < 2 * 0x3f800000u) == !(iy & 0x80000000u)) return 0.0f;  // |x| < 1 && y == inf, or |x| > 1 && y == -inf
      return y * y;
    }
    if (powf_zeroinfnan(ix)) {
      float x2 = x * x;
      if ((ix & 0x80000000u) && powf_checkint(iy) == 1) x2 = -x2;
      return (iy & 0x80000000u) ? 1.0f / x2 : x2;
    }
    // x and y are non-zero finite
    if (ix & 0x80000000u) {
      int yint = powf_checkint(iy);
      if (yint == 0) return u2f(0x7fc00000u);  // negative base, non-integer exponent
      if (yint == 1) sign_bias = 1ull << (5 + 11);
      ix &= 0x7fffffffu;
    }
    if (ix < 0x00800000u) {  // subnormal: normalise
      ix = f2u(u2f(ix) * 0x1p23f);
      ix &= 0x7fffffffu;
      ix -= 23u << 23;
    }
  }
  double logx = powf_log2<FUSED>(ix, invc_tab, logc_tab);
  double ylogx = (double)y * logx;
  if (((d2u(ylogx) >> 47) & 0xffff) >= (d2u(126.0) >> 47)) {
    // |y * log2(x)| >= 126
    if (ylogx > 0x1.fffffffd1d571p+6) return sign_bias ? -u2f(0x7f800000u) : u2f(0x7f800000u);  // overflow
    if (ylogx <= -150.0) return sign_bias ? -0.0f : 0.0f;                                         // underflow
  }
  return (float)powf_exp2<FUSED>(ylogx, sign_bias, exp2tab);
}

// ---------------------------------------------------------------- tanhf

// glibc's single-precision tanh and expm1 (sysdeps/ieee754/flt-32/s_tanhf.c
// and s_expm1f.c, the Sun fdlibm algorithms in float arithmetic): Rust's
// f32::tanh on x86_64-linux-gnu, used for the logit softcap cap * tanh(l / cap)
// (oxide-backend-cuda/src/kernels/vec_ops_activations.cu:131-136). The
// operations are plain IEEE float steps, so no fused form exists; the host
// glibc agrees with this restatement on every one of the 2^32 inputs.
//
// expm1f: x = k ln2 + r with |r| <= ln2 / 2 (ln2 split into a high part exact
// in products with k and a low part), expm1(r) from a degree-5 rational
// correction in r^2 / 2, then rescaled by 2^k.
OXS_HD float expm1f_fdlibm(float x) {
  const float one = 1.0f, huge = 1.0e+30f, tiny = 1.0e-30f;
  const float o_threshold = u2f(0x42b17180u), ln2_hi = u2f(0x3f317180u), ln2_lo = u2f(0x3717f7d1u),
              invln2 = u2f(0x3fb8aa3bu);
  const float Q1 = u2f(0xbd088889u), Q2 = u2f(0x3ad00d01u), Q3 = u2f(0xb8a670cdu), Q4 = u2f(0x36867e54u),
              Q5 = u2f(0xb457edbbu);
  float y, hi, lo, c = 0.0f, t, e, hxs, hfx, r1;
  int32_t k;
  uint32_t hx = f2u(x);
  const uint32_t xsb = hx & 0x80000000u;
  hx &= 0x7fffffffu;
  if (hx >= 0x4195b844u) {    // |x| >= 27 ln2
    if (hx >= 0x42b17218u) {  // |x| >= 88.72...
      if (hx > 0x7f800000u) return x + x;                 // NaN
      if (hx == 0x7f800000u) return xsb == 0 ? x : -1.0f;  // exp(+-inf) - 1
      if (x > o_threshold) return huge * huge;            // overflow
    }
    if (xsb != 0) return tiny - one;  // x < -27 ln2: -1
  }
  if (hx > 0x3eb17218u) {    // |x| > ln2 / 2: reduce
    if (hx < 0x3f851592u) {  // and |x| < 3 ln2 / 2
      if (xsb == 0) {
        hi = x - ln2_hi;
        lo = ln2_lo;
        k = 1;
      } else {
        hi = x + ln2_hi;
        lo = -ln2_lo;
        k = -1;
      }
    } else {
      k = (int32_t)(invln2 * x + (xsb == 0 ? 0.5f : -0.5f));
      t = (float)k;
      hi = x - t * ln2_hi;  // exact
      lo = t * ln2_lo;
    }
    x = hi - lo;
    c = (hi - x) - lo;
  } else if (hx < 0x33000000u) {  // |x| < 2^-25: x
    t = huge + x;
    return x - (t - (huge + x));
  } else {
    k = 0;
  }
  hfx = 0.5f * x;
  hxs = x * hfx;
  r1 = one + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
  t = 3.0f - r1 * hfx;
  e = hxs * ((r1 - t) / (6.0f - x * t));
  if (k == 0) return x - (x * e - hxs);
  e = (x * (e - c) - c);
  e -= hxs;
  if (k == -1) return 0.5f * (x - e) - 0.5f;
  if (k == 1) {
    if (x < -0.25f) return -2.0f * (e - (x + 0.5f));
    return one + 2.0f * (x - e);
  }
  if (k <= -2 || k > 56) {  // exp(x) - 1 from exp(x)
    y = one - (e - x);
    if (k == 128) y = y * 2.0f * 0x1p127f;
    else y = u2f(f2u(y) + ((uint32_t)k << 23));
    return y - one;
  }
  if (k < 23) {
    t = u2f(0x3f800000u - (0x1000000u >> k));  // 1 - 2^-k
    y = t - (e - x);
  } else {
    t = u2f((uint32_t)(0x7f - k) << 23);  // 2^-k
    y = x - (e + t);
    y += one;
  }
  return u2f(f2u(y) + ((uint32_t)k << 23));
}

// tanh(x) = 1 - 2 / (expm1(2|x|) + 2) for |x| >= 1, -t / (t + 2) with
// t = expm1(-2|x|) below, x(1 + x) for |x| < 2^-55, +-1 from |x| >= 22.
OXS_HD float tanhf_fdlibm(float x) {
  const float one = 1.0f, two = 2.0f, tiny = 1.0e-30f;
  float t, z;
  const uint32_t jx = f2u(x), ix = jx & 0x7fffffffu;
  if (ix >= 0x7f800000u) return (jx >> 31) == 0 ? one / x + one : one / x - one;  // +-inf: +-1; NaN
  if (ix < 0x41b00000u) {  // |x| < 22
    if (ix == 0) return x;
    if (ix < 0x24000000u) return x * (one + x);
    if (ix >= 0x3f800000u) {
      t = expm1f_fdlibm(two * (jx >> 31 ? -x : x));
      z = one - two / (t + two);
    } else {
      t = expm1f_fdlibm(-two * (jx >> 31 ? -x : x));
      z = -t / (t + two);
    }
  } else {
    z = one - tiny;
  }
  return (jx >> 31) == 0 ? z : -z;
}

}  // namespace oxs_libm
