/*
 * bl_math.h — scalar arithmetic of the token-selection path that must match the reference bit for bit.
 *
 * The reference lowers Boring float32 to Rust f32, whose exp/tanh call the host glibc (2.35) expf and
 * tanhf. These device functions reimplement those published algorithms:
 *   bl_expf  — the table-driven exp of ARM optimized-routines as shipped in glibc (32-entry 2^(i/32)
 *              table, cubic polynomial in double, result rounded once). The glibc x86-64 build selected
 *              on FMA-capable hosts fuses the range reduction z = x*N/ln2 into the rounding and remainder
 *              steps; the fma() calls below reproduce that. Exhaustively equal to host glibc expf on
 *              every float in [-104, 89] (2.24e9 inputs) and at the special values.
 *   bl_tanhf — fdlibm's float tanh built on fdlibm's float expm1 (glibc sysdeps/ieee754/flt-32),
 *              evaluated in float arithmetic. Exhaustively equal to host glibc tanhf on all 2^32 inputs.
 *   bl_logf  — the table-driven log of ARM optimized-routines as shipped in glibc (below).
 * The table below is 2^(i/32) rounded to double minus (i << 47); it is derived, not copied: the test
 * suite recomputes it from high-precision arithmetic.
 *
 * Compile with -ffp-contract=off: every float/double operation here is a single IEEE operation.
 */
#ifndef BL_MATH_H
#define BL_MATH_H

#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define BL_FN __host__ __device__ inline
#else
#include <math.h>
#define BL_FN static inline
#endif

BL_FN uint32_t bl_f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
BL_FN float bl_u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
BL_FN uint64_t bl_d2u(double d) {
  uint64_t u;
  memcpy(&u, &d, 8);
  return u;
}
BL_FN double bl_u2d(uint64_t u) {
  double d;
  memcpy(&d, &u, 8);
  return d;
}

#if defined(__HIP_DEVICE_COMPILE__)
#define BL_FMA(a, b, c) __builtin_fma((a), (b), (c))
#else
#define BL_FMA(a, b, c) fma((a), (b), (c))
#endif

/* ---------------- expf ---------------- */
#define BL_EXP2_BITS 5
#define BL_EXP2_N 32

#if defined(__HIP_DEVICE_COMPILE__)
__constant__
#else
static
#endif
const uint64_t bl_exp2_tab[BL_EXP2_N] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

/* expf with the 2^(i/32) table read through tab(i) (a kernel may stage the table in LDS) */
template <class Tab>
BL_FN float bl_expf_tab(float x, Tab tab) {
  /* polynomial for 2^(r/N) - 1 on |r| <= 1/2 (coefficients of the published algorithm, scaled by N) */
  const double N = (double)BL_EXP2_N;
  const double C0 = 0x1.c6af84b912394p-5 / N / N / N, C1 = 0x1.ebfce50fac4f3p-3 / N / N,
               C2 = 0x1.62e42ff0c52d6p-1 / N;
  const double INVLN2N = 0x1.71547652b82fep+0 * N, SHIFT = 0x1.8p+52;
  uint32_t ux = bl_f2u(x);
  uint32_t abstop = (ux >> 20) & 0x7ff;
  if (abstop >= (0x42b00000u >> 20)) { /* |x| >= 88 or NaN */
    if (ux == 0xff800000u) return 0.0f;
    if (abstop >= (0x7f800000u >> 20)) return x + x;
    if (x > 0x1.62e42ep6f) return bl_u2f(0x7f800000u);
    if (x < -0x1.9fe368p6f) return 0.0f;
  }
  double xd = (double)x;
  double kd = BL_FMA(INVLN2N, xd, SHIFT);
  uint64_t ki = bl_d2u(kd);
  kd -= SHIFT;
  double r = BL_FMA(INVLN2N, xd, -kd);
  uint64_t t = tab((uint32_t)(ki % BL_EXP2_N));
  t += ki << (52 - BL_EXP2_BITS);
  double s = bl_u2d(t);
  double z = BL_FMA(C0, r, C1);
  double r2 = r * r;
  double y = BL_FMA(C2, r, 1.0);
  y = BL_FMA(z, r2, y);
  y = y * s;
  return (float)y;
}

BL_FN float bl_expf(float x) {
  return bl_expf_tab(x, [](uint32_t i) { return bl_exp2_tab[i]; });
}

/* ---------------- logf ---------------- */
/* ARM optimized-routines logf (as in glibc >= 2.28): x = 2^k z with z in [0x1.66p-1, 0x1.66p0) split
 * by the top 4 mantissa bits into 16 subintervals; log(x) = log1p(z/c - 1) + log(c) + k ln2 with
 * (1/c, log c) from the table, log1p by a cubic in double, one rounding to float at the end.
 * Equal to host glibc logf on every positive float (CPU, tests/cpu/check_exact.cpp samples it) and on
 * all 2^32 bit patterns on the device (tests/golden/math_digest.bin). */
/* (1/c, log c) of the 16 subintervals, interleaved */
#if defined(__HIP_DEVICE_COMPILE__)
__constant__
#else
static
#endif
const double bl_log_tab[32] = {
    0x1.661ec79f8f3bep+0, -0x1.57bf7808caadep-2, 0x1.571ed4aaf883dp+0, -0x1.2bef0a7c06ddbp-2,
    0x1.49539f0f010bp+0, -0x1.01eae7f513a67p-2, 0x1.3c995b0b80385p+0, -0x1.b31d8a68224e9p-3,
    0x1.30d190c8864a5p+0, -0x1.6574f0ac07758p-3, 0x1.25e227b0b8eap+0, -0x1.1aa2bc79c81p-3,
    0x1.1bb4a4a1a343fp+0, -0x1.a4e76ce8c0e5ep-4, 0x1.12358f08ae5bap+0, -0x1.1973c5a611cccp-4,
    0x1.0953f419900a7p+0, -0x1.252f438e10c1ep-5, 0x1p+0, 0x0p+0,
    0x1.e608cfd9a47acp-1, 0x1.aa5aa5df25984p-5, 0x1.ca4b31f026aap-1, 0x1.c5e53aa362eb4p-4,
    0x1.b2036576afce6p-1, 0x1.526e57720db08p-3, 0x1.9c2d163a1aa2dp-1, 0x1.bc2860d22477p-3,
    0x1.886e6037841edp-1, 0x1.1058bc8a07ee1p-2, 0x1.767dcf5534862p-1, 0x1.4043057b6ee09p-2};

/* logf with the (1/c, log c) table read through tab(j), j = 2 i and 2 i + 1 (a kernel may stage the table
 * in LDS) */
template <class Tab>
BL_FN float bl_logf_tab(float x, Tab tab) {
  const double LN2 = 0x1.62e42fefa39efp-1, A0 = -0x1.00ea348b88334p-2, A1 = 0x1.5575b0be00b6ap-2,
               A2 = -0x1.ffffef20a4123p-2;
  uint32_t ix = bl_f2u(x);
  if (ix == 0x3f800000u) return 0.0f;
  if (ix - 0x00800000u >= 0x7f800000u - 0x00800000u) {
    if (ix * 2u == 0u) return bl_u2f(0xff800000u); /* -inf */
    if (ix == 0x7f800000u) return x;
    if ((ix & 0x80000000u) || ix * 2u >= 0xff000000u) return bl_u2f(0x7fc00000u); /* NaN */
    ix = bl_f2u(x * 0x1p23f); /* subnormal: normalise */
    ix -= 23u << 23;
  }
  const uint32_t tmp = ix - 0x3f330000u;
  const int i = (int)((tmp >> 19) % 16u);
  const int k = (int32_t)tmp >> 23;
  const uint32_t iz = ix - (tmp & 0xff800000u);
  const double z = (double)bl_u2f(iz);
  const double r = z * tab(2 * i) - 1.0;
  const double y0 = tab(2 * i + 1) + (double)k * LN2;
  const double r2 = r * r;
  double y = A1 * r + A2;
  y = A0 * r2 + y;
  y = y * r2 + (y0 + r);
  return (float)y;
}

BL_FN float bl_logf(float x) {
  return bl_logf_tab(x, [](int j) { return bl_log_tab[j]; });
}

/* ---------------- powf ---------------- */
/* ARM optimized-routines powf (as in glibc >= 2.28): log2(x) in double from the (1/c, log2 c) table of the
 * same 16 subintervals as logf's (log2 c = log c / ln 2 rounded) and a degree-5 polynomial, y log2(x) in
 * double, then 2^(y log2 x) by expf's 2^(i/32) table and cubic; special cases (zero, infinity, NaN and
 * signalling NaN, negative x with integer y, subnormal x, overflow and underflow in round-to-nearest) as
 * the published code handles them. As for expf, the multiply-adds are fused the way the glibc x86-64
 * build for FMA-capable hosts fuses them. Equal to host glibc powf on all 2^32 inputs of powf(x, 0.7),
 * powf(2, x) and powf(x, y(x)) with y a multiple of 1/512 in [-8, 8] (tests/golden/math_digest.bin, on
 * the device) and on 4 million random and structured pairs (tests/cpu/check_exact.cpp). */
#if defined(__HIP_DEVICE_COMPILE__)
__constant__
#else
static
#endif
const double bl_log2_tab[32] = {
    0x1.661ec79f8f3bep+0, -0x1.efec65b963019p-2, 0x1.571ed4aaf883dp+0, -0x1.b0b6832d4fca4p-2,
    0x1.49539f0f010bp+0, -0x1.7418b0a1fb77bp-2, 0x1.3c995b0b80385p+0, -0x1.39de91a6dcf7cp-2,
    0x1.30d190c8864a5p+0, -0x1.01d9bf3f2b631p-2, 0x1.25e227b0b8eap+0, -0x1.97c1d1b3b7af1p-3,
    0x1.1bb4a4a1a343fp+0, -0x1.2f9e393af3c9fp-3, 0x1.12358f08ae5bap+0, -0x1.960cbbf788d5bp-4,
    0x1.0953f419900a7p+0, -0x1.a6f9db6475fcep-5, 0x1p+0, 0x0p+0,
    0x1.e608cfd9a47acp-1, 0x1.338ca9f24f53ep-4, 0x1.ca4b31f026aap-1, 0x1.476a9543891bbp-3,
    0x1.b2036576afce6p-1, 0x1.e840b4ac4e4d2p-3, 0x1.9c2d163a1aa2dp-1, 0x1.40645f0c6651cp-2,
    0x1.886e6037841edp-1, 0x1.88e9c2c1b9ff8p-2, 0x1.767dcf5534862p-1, 0x1.ce0a44eb17bcdp-2};

/* y is an integer: 0 no, 1 odd, 2 even */
BL_FN int bl_pow_checkint(uint32_t iy) {
  const int e = (int)(iy >> 23 & 0xff);
  if (e < 0x7f) return 0;
  if (e > 0x7f + 23) return 2;
  if (iy & ((1u << (0x7f + 23 - e)) - 1u)) return 0;
  if (iy & (1u << (0x7f + 23 - e))) return 1;
  return 2;
}
BL_FN bool bl_pow_zeroinfnan(uint32_t ix) { return 2u * ix - 1u >= 2u * 0x7f800000u - 1u; }
BL_FN bool bl_pow_snan(uint32_t ix) { return 2u * (ix ^ 0x00400000u) > 2u * 0x7fc00000u; }

BL_FN float bl_powf(float x, float y) {
  const double A0 = 0x1.27616c9496e0bp-2, A1 = -0x1.71969a075c67ap-2, A2 = 0x1.ec70a6ca7baddp-2,
               A3 = -0x1.7154748bef6c8p-1, A4 = 0x1.71547652ab82bp0;
  const double C0 = 0x1.c6af84b912394p-5, C1 = 0x1.ebfce50fac4f3p-3, C2 = 0x1.62e42ff0c52d6p-1;
  const double SHIFT = 0x1.8p+52 / BL_EXP2_N;
  uint64_t sign_bias = 0;
  uint32_t ix = bl_f2u(x);
  const uint32_t iy = bl_f2u(y);
  if (ix - 0x00800000u >= 0x7f800000u - 0x00800000u || bl_pow_zeroinfnan(iy)) {
    if (bl_pow_zeroinfnan(iy)) {
      if (2u * iy == 0u) return bl_pow_snan(ix) ? x + y : 1.0f;
      if (ix == 0x3f800000u) return bl_pow_snan(iy) ? x + y : 1.0f;
      if (2u * ix > 2u * 0x7f800000u || 2u * iy > 2u * 0x7f800000u) return x + y;
      if (2u * ix == 2u * 0x3f800000u) return 1.0f;
      if ((2u * ix < 2u * 0x3f800000u) == !(iy & 0x80000000u)) return 0.0f;
      return y * y;
    }
    if (bl_pow_zeroinfnan(ix)) {
      float x2 = x * x;
      if ((ix & 0x80000000u) && bl_pow_checkint(iy) == 1) x2 = -x2;
      return (iy & 0x80000000u) ? 1.0f / x2 : x2;
    }
    if (ix & 0x80000000u) { /* negative x: y must be an integer */
      const int yint = bl_pow_checkint(iy);
      if (yint == 0) return bl_u2f(0x7fc00000u);
      if (yint == 1) sign_bias = 1ull << (BL_EXP2_BITS + 11);
      ix &= 0x7fffffffu;
    }
    if (ix < 0x00800000u) { /* subnormal x: normalise */
      ix = bl_f2u(bl_u2f(ix) * 0x1p23f);
      ix &= 0x7fffffffu;
      ix -= 23u << 23;
    }
  }
  /* log2(x) */
  const uint32_t tmp = ix - 0x3f330000u;
  const int i = (int)((tmp >> 19) % 16u);
  const uint32_t top = tmp & 0xff800000u;
  const uint32_t iz = ix - top;
  const int k = (int32_t)top >> 23;
  const double z = (double)bl_u2f(iz);
  const double r = BL_FMA(z, bl_log2_tab[2 * i], -1.0);
  const double y0 = bl_log2_tab[2 * i + 1] + (double)k;
  const double r2 = r * r;
  double p = BL_FMA(A0, r, A1);
  const double q0 = BL_FMA(A2, r, A3);
  const double r4 = r2 * r2;
  double q = BL_FMA(A4, r, y0);
  q = BL_FMA(q0, r2, q);
  p = BL_FMA(p, r4, q);
  const double ylogx = (double)y * p;
  if ((bl_d2u(ylogx) >> 47 & 0xffff) >= bl_d2u(126.0) >> 47) {
    if (ylogx > 0x1.fffffffd1d571p+6) return sign_bias ? bl_u2f(0xff800000u) : bl_u2f(0x7f800000u);
    if (ylogx <= -150.0) return sign_bias ? -0.0f : 0.0f;
  }
  /* 2^ylogx */
  double kd = ylogx + SHIFT;
  const uint64_t ki = bl_d2u(kd);
  kd -= SHIFT;
  const double rr = ylogx - kd;
  uint64_t t = bl_exp2_tab[ki % BL_EXP2_N];
  t += (ki + sign_bias) << (52 - BL_EXP2_BITS);
  const double s = bl_u2d(t);
  const double zz = BL_FMA(C0, rr, C1);
  const double rr2 = rr * rr;
  double yy = BL_FMA(C2, rr, 1.0);
  yy = BL_FMA(zz, rr2, yy);
  yy = yy * s;
  return (float)yy;
}

/* ---------------- expm1f / tanhf (float arithmetic) ---------------- */
BL_FN float bl_expm1f(float x) {
  const float huge = 1.0e+30f, tiny = 1.0e-30f, one = 1.0f, o_threshold = 8.8721679688e+01f,
              ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f, invln2 = 1.4426950216e+00f,
              Q1 = -3.3333335072e-02f, Q2 = 1.5873016091e-03f, Q3 = -7.9365076090e-05f, Q4 = 4.0082177293e-06f,
              Q5 = -2.0109921195e-07f;
  float y, hi, lo, c = 0.0f, t, e, hxs, hfx, r1;
  int32_t k;
  uint32_t hx = bl_f2u(x);
  uint32_t xsb = hx & 0x80000000u;
  hx &= 0x7fffffffu;
  if (hx >= 0x4195b844u) {
    if (hx >= 0x42b17218u) {
      if (hx > 0x7f800000u) return x + x;
      if (hx == 0x7f800000u) return (xsb == 0) ? x : -1.0f;
      if (x > o_threshold) return huge * huge;
    }
    if (xsb != 0) return tiny - one;
  }
  if (hx > 0x3eb17218u) {
    if (hx < 0x3F851592u) {
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
      float kf = invln2 * x;
      kf = kf + ((xsb == 0) ? 0.5f : -0.5f);
      k = (int32_t)kf;
      t = (float)k;
      float th = t * ln2_hi;
      hi = x - th;
      lo = t * ln2_lo;
    }
    x = hi - lo;
    c = (hi - x) - lo;
  } else if (hx < 0x33000000u) {
    t = huge + x;
    return x - (t - (huge + x));
  } else {
    k = 0;
  }
  hfx = 0.5f * x;
  hxs = x * hfx;
  float p = hxs * Q5;
  p = Q4 + p;
  p = hxs * p;
  p = Q3 + p;
  p = hxs * p;
  p = Q2 + p;
  p = hxs * p;
  p = Q1 + p;
  p = hxs * p;
  r1 = one + p;
  float rh = r1 * hfx;
  t = 3.0f - rh;
  float xt = x * t;
  float den = 6.0f - xt;
  float num = r1 - t;
  e = num / den;
  e = hxs * e;
  if (k == 0) {
    float xe = x * e;
    xe = xe - hxs;
    return x - xe;
  }
  float ec = e - c;
  ec = x * ec;
  e = ec - c;
  e -= hxs;
  if (k == -1) {
    float d = x - e;
    d = 0.5f * d;
    return d - 0.5f;
  }
  if (k == 1) {
    if (x < -0.25f) {
      float d = x + 0.5f;
      d = e - d;
      return -2.0f * d;
    }
    float d = x - e;
    d = 2.0f * d;
    return one + d;
  }
  if (k <= -2 || k > 56) {
    float d = e - x;
    y = one - d;
    y = bl_u2f(bl_f2u(y) + ((uint32_t)k << 23));
    return y - one;
  }
  if (k < 23) {
    t = bl_u2f(0x3f800000u - (0x1000000u >> k));
    float d = e - x;
    y = t - d;
    y = bl_u2f(bl_f2u(y) + ((uint32_t)k << 23));
  } else {
    t = bl_u2f((uint32_t)(0x7f - k) << 23);
    float d = e + t;
    y = x - d;
    y += one;
    y = bl_u2f(bl_f2u(y) + ((uint32_t)k << 23));
  }
  return y;
}

BL_FN float bl_tanhf(float x) {
  const float one = 1.0f, tiny = 1.0e-30f;
  float t, z;
  int32_t jx = (int32_t)bl_f2u(x), ix = jx & 0x7fffffff;
  if (ix >= 0x7f800000) {
    if (jx >= 0) return one / x + one;
    return one / x - one;
  }
  if (ix < 0x41b00000) {
    if (ix == 0) return x;
    if (ix < 0x24000000) {
      float s = one + x;
      return x * s;
    }
    float ax = bl_u2f((uint32_t)ix);
    if (ix >= 0x3f800000) {
      t = bl_expm1f(2.0f * ax);
      float d = t + 2.0f;
      d = 2.0f / d;
      z = one - d;
    } else {
      t = bl_expm1f(-2.0f * ax);
      float d = t + 2.0f;
      z = -t / d;
    }
  } else {
    z = one - tiny;
  }
  return (jx >= 0) ? z : -z;
}

/* ---------------- RNG: xorshift64 (13, 7, 17) and its [0,1) float ---------------- */
BL_FN uint64_t bl_xorshift(uint64_t x) {
  x ^= x << 13;
  x ^= x >> 7;
  x ^= x << 17;
  return x;
}

/* u64 -> binary32, round to nearest even, integer operations only */
BL_FN float bl_u64_to_f32(uint64_t x) {
  if (x == 0) return 0.0f;
#if defined(__HIP_DEVICE_COMPILE__)
  int e = 63 - __clzll((long long)x);
#else
  int e = 63 - __builtin_clzll(x);
#endif
  if (e <= 23) return bl_u2f(((uint32_t)(e + 127) << 23) | ((uint32_t)(x << (23 - e)) & 0x7fffffu));
  int sh = e - 23;
  uint64_t m = x >> sh;
  uint64_t rem = x & ((1ull << sh) - 1), half = 1ull << (sh - 1);
  if (rem > half || (rem == half && (m & 1))) m++;
  if (m == (1ull << 24)) {
    m >>= 1;
    e++;
  }
  return bl_u2f(((uint32_t)(e + 127) << 23) | ((uint32_t)m & 0x7fffffu));
}

/* next uniform draw: advances *state and returns (x as f32) / 2^64 (exact power-of-two scaling) */
BL_FN float bl_rng_f32(uint64_t *state) {
  uint64_t x = bl_xorshift(*state);
  *state = x;
  return bl_u64_to_f32(x) * 5.42101086242752217e-20f; /* 2^-64 */
}

/* order-preserving key of a float for descending selection; -0 is folded into +0 (they compare equal) */
BL_FN uint32_t bl_fkey(float f) {
  uint32_t u = bl_f2u(f + 0.0f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
BL_FN float bl_fkey_inv(uint32_t k) { return bl_u2f((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k); }

#endif /* BL_MATH_H */
