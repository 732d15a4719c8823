/*
 * bl_synth.h — portable, integer-only synthetic inputs for the five token-selection workloads.
 *
 * Every value here is a pure function of (workload, seed, step, row, purpose, index), computed with
 * 64-bit integer hashing and exact double arithmetic, so the host (oracle, CPU baseline) and the
 * device (benchmark input pools) produce bit-identical inputs. The one exception is the Zipf(1.1)
 * history sampler, which uses the host libm and therefore runs on the host only; its ids are handed
 * to both sides through the same host arrays.
 *
 * This header is test/benchmark input generation, not part of the token-selection path.
 */
#ifndef BL_SYNTH_H
#define BL_SYNTH_H

#include <stdint.h>

#if defined(__HIPCC__)
#define BL_HD __host__ __device__ inline
#else
#define BL_HD static inline
#endif

/* purposes: separate hash streams per kind of input */
enum {
  BL_P_LOGIT = 1,   /* dense logits */
  BL_P_BUMP = 2,    /* config 1: ids that receive +8 */
  BL_P_HIST = 3,    /* uniform history ids */
  BL_P_BIAS_ID = 4, /* logit_bias ids */
  BL_P_BIAS_VAL = 5,
  BL_P_DRAFT = 6,   /* speculative drafts */
  BL_P_VOCAB = 7,   /* synthetic vocabulary bytes */
  BL_P_ZIPF = 8
};

BL_HD uint64_t bl_splitmix(uint64_t x) {
  x += 0x9e3779b97f4a7c15ull;
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}

/* Stream key for one (workload, seed, step, row, purpose). */
BL_HD uint64_t bl_stream(uint32_t cfg, int64_t seed, int64_t step, int64_t row, uint32_t purpose) {
  uint64_t k = bl_splitmix(((uint64_t)cfg << 56) ^ (uint64_t)seed);
  k = bl_splitmix(k ^ ((uint64_t)step * 0x9e3779b97f4a7c15ull));
  k = bl_splitmix(k ^ ((uint64_t)row * 0xc2b2ae3d27d4eb4full));
  return bl_splitmix(k ^ ((uint64_t)purpose * 0x165667b19e3779f9ull));
}

/* i-th 64-bit draw of a stream */
BL_HD uint64_t bl_draw(uint64_t stream, uint64_t i) { return bl_splitmix(stream + i * 0xd6e8feb86659fd93ull); }

/* uniform integer in [0, n) by 64x64 multiply-high */
BL_HD uint64_t bl_below(uint64_t h, uint64_t n) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __umul64hi(h, n);
#else
  return (uint64_t)(((unsigned __int128)h * n) >> 64);
#endif
}

/*
 * Approximate N(0, sigma^2) by Irwin-Hall(12): twelve exact 24-bit uniforms (two per hash), their
 * integer sum scaled by 2^-24 minus 6 (exact in double), times an integer sigma (exact), rounded once
 * to float32 (round to nearest even). No libm involved.
 */
BL_HD float bl_normal(uint64_t stream, uint64_t idx, int sigma) {
  uint64_t s = 0;
  for (int k = 0; k < 6; k++) {
    uint64_t h = bl_draw(stream, idx * 6 + (uint64_t)k);
    s += (h & 0xffffffull) + ((h >> 24) & 0xffffffull);
  }
  double z = (double)s * (1.0 / 16777216.0) - 6.0;
  return (float)(z * (double)sigma);
}

/* uniform float in [lo, hi) from a 24-bit draw: lo + (hi-lo)*u/2^24 in double, rounded once */
BL_HD float bl_uniform_f(uint64_t h, double lo, double hi) {
  double u = (double)(h & 0xffffffull) * (1.0 / 16777216.0);
  return (float)(lo + (hi - lo) * u);
}

/* ---------------- workload constants (the five BASELINE configurations) ---------------- */

#define BL_V_QWEN 151936
#define BL_V_GEMMA 262144

/* Workload 2 row table: T = {0, 0.7, 1.0}[r%3], top_k = {0, 20, 64}[r/3], top_p = {1.0, 0.9}[r%2]. */
BL_HD float bl_c2_temperature(int r) { return r % 3 == 0 ? 0.0f : (r % 3 == 1 ? 0.7f : 1.0f); }
BL_HD int bl_c2_top_k(int r) { return (r / 3) == 0 ? 0 : ((r / 3) == 1 ? 20 : 64); }
BL_HD float bl_c2_top_p(int r) { return r % 2 == 0 ? 1.0f : 0.9f; }

/* Dense logits row for a workload step. Workload 1 adds +8 to 20 distinct ids afterwards (host side,
 * bl_c1_bump_ids); workload 5 rows are indexed row = seq*(k+1)+position. */
BL_HD int bl_cfg_sigma(int cfg) { return cfg == 2 ? 4 : (cfg == 4 ? 10 : 3); }

BL_HD float bl_logit(int cfg, int64_t seed, int64_t step, int64_t row, uint64_t idx) {
  return bl_normal(bl_stream((uint32_t)cfg, seed, step, row, BL_P_LOGIT), idx, bl_cfg_sigma(cfg));
}

#endif /* BL_SYNTH_H */
