// CPU check of the exact sequential-sum arithmetic (boring-llm_amd/csrc/bl_exact.h, scalar part) and of
// the glibc-identical math (bl_math.h) against the host glibc. Built and run by tests/test_device_math.py.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <random>
#include <vector>

#include "../../boring-llm_amd/csrc/bl_exact.h"
#include "../../boring-llm_amd/csrc/bl_math.h"

// sequential sum by the binade automaton: increments within a binade, one real add at a crossing
static float auto_sum(const std::vector<float> &a) {
  int e = BL_E_MIN;
  uint32_t N = 0;
  for (float x : a) {
    uint32_t Ne = bl_apply(bl_term_inc(x, e), N);
    if (Ne >= BL_N_TOP) {
      float S = bl_make(e, N) + x;
      bl_split(S, e, N);
    } else {
      N = Ne;
    }
  }
  return bl_make(e, N);
}

// the same walk but with 64-term groups composed first (as the device does), element level at crossings
static float group_sum(const std::vector<float> &a) {
  int e = BL_E_MIN;
  uint32_t N = 0;
  size_t n = a.size();
  for (size_t g0 = 0; g0 < n; g0 += 64) {
    size_t g1 = g0 + 64 < n ? g0 + 64 : n;
    bl_inc f = bl_inc_ident();
    for (size_t j = g0; j < g1; j++) f = bl_compose(f, bl_term_inc(a[j], e));
    uint32_t Ne = bl_apply(f, N);
    if (Ne < BL_N_TOP) {
      N = Ne;
      continue;
    }
    for (size_t j = g0; j < g1; j++) {
      uint32_t Nj = bl_apply(bl_term_inc(a[j], e), N);
      if (Nj >= BL_N_TOP) {
        float S = bl_make(e, N) + a[j];
        bl_split(S, e, N);
      } else {
        N = Nj;
      }
    }
  }
  return bl_make(e, N);
}

static float seq_sum(const std::vector<float> &a) {
  float s = 0.0f;
  for (float x : a) s += x;
  return s;
}

int main() {
  std::mt19937_64 rng(12345);
  long bad = 0, trials = 0;
  // 1) exact sums over many distributions, including tie-heavy and sorted orders
  for (int trial = 0; trial < 3000; trial++) {
    int n = 1 + (int)(rng() % 5000);
    std::vector<float> a(n);
    int kind = trial % 6;
    std::normal_distribution<float> nd(0.0f, kind == 5 ? 10.0f : 3.0f);
    float mx = -1e30f;
    std::vector<float> x(n);
    for (int i = 0; i < n; i++) {
      x[i] = nd(rng);
      if (kind == 2) x[i] = (float)((int)(x[i] * 4)) * 0.25f;  // coarse grid: many exact ties
      if (kind == 3) x[i] = -(float)(rng() % 120);              // wide range incl. subnormal/zero terms
      mx = x[i] > mx ? x[i] : mx;
    }
    for (int i = 0; i < n; i++) a[i] = bl_expf(x[i] - mx);
    if (kind == 1) std::sort(a.begin(), a.end(), [](float p, float q) { return p > q; });
    if (kind == 4) for (int i = 0; i < n; i++) a[i] = ldexpf((float)(rng() % 4096), -(int)(rng() % 40));  // half-ulp ties
    float s1 = seq_sum(a), s2 = auto_sum(a), s3 = group_sum(a);
    trials++;
    if (bl_f2u(s1) != bl_f2u(s2) || bl_f2u(s1) != bl_f2u(s3)) {
      if (bad < 5) printf("mismatch trial %d kind %d n %d: %a %a %a\n", trial, kind, n, s1, s2, s3);
      bad++;
    }
  }
  printf("exact-sum mismatches: %ld of %ld\n", bad, trials);
  // 2) glibc-identical expf / tanhf / logf on a strided sample of all float bit patterns (logf: NaN
  // results compared as NaN, the payload is not part of the path)
  long me = 0, mt = 0, ml = 0, n = 0;
  for (uint64_t u = 0; u <= 0xffffffffull; u += 4093) {
    float x = bl_u2f((uint32_t)u);
    if (x != x) continue;
    n++;
    if (bl_f2u(bl_expf(x)) != bl_f2u(expf(x))) me++;
    if (bl_f2u(bl_tanhf(x)) != bl_f2u(tanhf(x))) mt++;
    const float la = bl_logf(x), lb = logf(x);
    if (!(la != la && lb != lb) && bl_f2u(la) != bl_f2u(lb)) ml++;
  }
  // logf densely over (0, 1], the probabilities it is applied to (every 3rd pattern)
  for (uint32_t u = 1; u <= 0x3f800000u; u += 3) {
    const float x = bl_u2f(u);
    if (bl_f2u(bl_logf(x)) != bl_f2u(logf(x))) ml++;
  }
  printf("expf mismatches %ld, tanhf mismatches %ld, logf mismatches %ld, of %ld sampled inputs\n", me, mt, ml, n);
  // 3) u64 -> f32 rounding against the C conversion
  long mc = 0;
  for (int i = 0; i < 2000000; i++) {
    uint64_t v = rng() >> (rng() % 64);
    if (bl_f2u(bl_u64_to_f32(v)) != bl_f2u((float)v)) mc++;
  }
  printf("u64->f32 mismatches %ld\n", mc);
  // 4) glibc-identical powf: random bit patterns of x and y, and x in [1, 101) with y in [-100, 100)
  long mp = 0, np_ = 0;
  for (int i = 0; i < 4000000; i++) {
    const uint64_t a = rng(), b = rng();
    float x = bl_u2f((uint32_t)a), y = bl_u2f((uint32_t)(b >> 32));
    if (i % 3 == 0) {
      x = 1.0f + (float)(a % 100000) / 1000.0f;
      y = ((float)((b >> 20) % 20000) - 10000.0f) / 100.0f;
    } else if (i % 3 == 1) {
      x = bl_u2f((uint32_t)a & 0x3fffffffu); /* (0, 2) and subnormals */
      y = (float)((int)(b % 41) - 20) * 0.5f; /* integers and halves, with negative x below */
      if (b & (1ull << 40)) x = -x;
    }
    const float pa = bl_powf(x, y), pb = powf(x, y);
    np_++;
    if (!(pa != pa && pb != pb) && bl_f2u(pa) != bl_f2u(pb)) {
      if (mp < 5) printf("powf mismatch x=%a y=%a mine=%a glibc=%a\n", x, y, pa, pb);
      mp++;
    }
  }
  printf("powf mismatches %ld of %ld\n", mp, np_);
  return (bad || me || mt || ml || mc || mp) ? 1 : 0;
}
