/*
 * bl_kernels.hip — HIP kernels of one token-selection step for B slots (gfx950, wave64).
 *
 *   bl_k_rowpass  grid (chunks, B) x 256: reads each logits row once (float4), applies the model tail
 *                 (logit_mul, soft-cap), then the server's per-token stages at the chunk's records
 *                 (logit_bias -> ignore_eos suppression -> frequency/presence -> repeat penalty,
 *                 src/server.br:940-944, src/sampling.br:65-107,175-237), writes the transformed
 *                 row, and per chunk: max + first argmax, an approximate exp-sum, and the chunk's
 *                 top-K by (value desc, index asc) via a three-pass LDS radix select.
 *   bl_k_exppass  grid (1 + V/1024, B) x 256: workgroup 0 merges a row's chunk top-K lists into its
 *                 sorted top K (top-k sampling and logprob alternatives); the others, for rows with
 *                 logprobs or full-vocabulary sampling, compute the exact exp(x - max) terms
 *                 (glibc-identical expf), the sequential-sum group records of the index-order normaliser
 *                 (src/sampling.br:254-266), and the candidates of a full-vocabulary rank (every token
 *                 within 17.5*max(T,1) of the max; the rest cannot change any float32 sum of the chain).
 *   bl_k_select   grid (B) x 1024: greedy / top-k / full-vocabulary candidate sampling with exact
 *                 sequential sums (src/sampling.br:490-607), the draw from the slot's xorshift stream,
 *                 the exact index-order normaliser of logprob rows (src/sampling.br:254-273),
 *                 alternatives (src/server.br:1027-1035) and the history commit (src/server.br:1004, :1037).
 * No MFMA: the work is bandwidth- and latency-bound scanning, selection and integer arithmetic.
 */
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>

#include <type_traits>

#include "bl_exact.h"
#include "bl_internal.h"
#include "bl_math.h"
#include "bl_synth.h"

#define BL_NEG_INF (-__builtin_inff())

__device__ __forceinline__ const bl_slot_dev &slot_of(const bl_dev &d, int s) { return d.slots[s]; }

/* candidate order keys: (fkey(value) << 32) | ~index, larger = earlier in (value desc, index asc) */
__device__ __forceinline__ uint64_t ckey(float v, int32_t id) {
  return ((uint64_t)bl_fkey(v) << 32) | (uint64_t)(0xffffffffu - (uint32_t)id);
}
__device__ __forceinline__ float ckey_v(uint64_t k) { return bl_fkey_inv((uint32_t)(k >> 32)); }
__device__ __forceinline__ int32_t ckey_i(uint64_t k) { return (int32_t)(0xffffffffu - (uint32_t)k); }

/* ------------------------------------------------------------------ block reductions (256 threads) */
__device__ __forceinline__ void argmax_merge(float &m, int &mi, float m2, int mi2) {
  if (m2 > m || (m2 == m && mi2 < mi)) {
    m = m2;
    mi = mi2;
  }
}

/* keys of a[0..n) (LDS) greater than k, U reads in flight at a time */
template <int U = 8>
__device__ __forceinline__ int count_gt(const uint64_t *a, int n, uint64_t k) {
  int r = 0, j = 0;
  for (; j + U <= n; j += U) {
    uint64_t x[U];
#pragma unroll
    for (int u = 0; u < U; u++) x[u] = a[j + u];
#pragma unroll
    for (int u = 0; u < U; u++) r += x[u] > k ? 1 : 0;
  }
  for (; j < n; j++) r += a[j] > k ? 1 : 0;
  return r;
}

template <int NT>
__device__ __forceinline__ void block_argmax(float &m, int &mi, float *sm, int *si) {
  int t = threadIdx.x, lane = t & 63, w = t >> 6;
#pragma unroll
  for (int k = 32; k >= 1; k >>= 1) {
    float m2 = __shfl_xor(m, k, 64);
    int i2 = __shfl_xor(mi, k, 64);
    argmax_merge(m, mi, m2, i2);
  }
  if (lane == 0) {
    sm[w] = m;
    si[w] = mi;
  }
  __syncthreads();
  if (t == 0) {
    for (int k = 1; k < NT / 64; k++) argmax_merge(m, mi, sm[k], si[k]);
    sm[0] = m;
    si[0] = mi;
  }
  __syncthreads();
  m = sm[0];
  mi = si[0];
  __syncthreads();
}

template <int NT>
__device__ __forceinline__ double block_sum_d(double x, double *sd) {
  int t = threadIdx.x, lane = t & 63, w = t >> 6;
  x = bl_wave_sum_d(x);
  if (lane == 0) sd[w] = x;
  __syncthreads();
  double r = 0.0;
  for (int k = 0; k < NT / 64; k++) r += sd[k];
  __syncthreads();
  return r;
}

/*
 * Histogram bin search from the top over bins [0, nb) (nb a multiple of NT): res[0] = the bin b where
 * the count of keys in bins >= b first reaches `need`, res[1] = the count in bins above b, res[2] = the
 * count in b, res[3] = the total (res[0..2] = 0, total, 0 when the total is below `need`). Thread t
 * owns the nb/NT consecutive bins ending at nb - t*nb/NT.
 */
template <int NT>
__device__ void block_find_bin(const uint32_t *hist, int nb, uint32_t need, uint32_t *res, uint32_t *wsum) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int per = nb / NT;
  uint32_t local = 0u;
  for (int q = 0; q < per; q++) local += hist[nb - 1 - (t * per + q)];
  uint32_t inc = local;
#pragma unroll
  for (int k = 1; k < 64; k <<= 1) {
    uint32_t o = __shfl_up(inc, k, 64);
    if (lane >= k) inc += o;
  }
  if (lane == 63) wsum[w] = inc;
  __syncthreads();
  uint32_t above = inc - local, total = 0u;
  for (int k = 0; k < NT / 64; k++) {
    if (k < w) above += wsum[k];
    total += wsum[k];
  }
  if (t == 0) {
    res[3] = total;
    if (total < need) {
      res[0] = 0u;
      res[1] = total;
      res[2] = 0u;
    }
  }
  if (above < need && above + local >= need) {
    uint32_t acc = above;
    for (int q = 0; q < per; q++) {
      const int b = nb - 1 - (t * per + q);
      const uint32_t h = hist[b];
      if (acc + h >= need) {
        res[0] = (uint32_t)b;
        res[1] = acc;
        res[2] = h;
        break;
      }
      acc += h;
    }
  }
  __syncthreads();
}

/* exclusive scan of a double over the block (NT threads); returns this thread's prefix, *total */
template <int NT>
__device__ double block_excl_scan_d(double x, double *sd, double *total) {
  int t = threadIdx.x, lane = t & 63, w = t >> 6;
  double ex = bl_wave_excl_scan_d(x, lane);
  if (lane == 63) sd[w] = ex + x;
  __syncthreads();
  double base = 0.0, tot = 0.0;
  for (int k = 0; k < NT / 64; k++) {
    if (k < w) base += sd[k];
    tot += sd[k];
  }
  __syncthreads();
  *total = tot;
  return base + ex;
}

/* ------------------------------------------------------------------ server stages */
/* frequency/presence over the reply count, then the repeat penalty over the window count
 * (src/sampling.br:91-107, :65-85) */
__device__ __forceinline__ float stage_counts(const bl_slot_dev &sp, float v, int cc, int wc) {
  if (cc > 0) {
    const float tcf = (float)cc * sp.frequency_penalty;
    v = v - tcf;
    v = v - sp.presence_penalty;
  }
  if (wc > 0) v = v > 0.0f ? v / sp.repeat_penalty : v * sp.repeat_penalty;
  return v;
}
/* then DRY's penalty of a token the last update flagged: multiplier * base^exponent (src/sampling.br:163-170) */
__device__ __forceinline__ float stage_dry(const bl_slot_dev &sp, float v, uint32_t wf) {
  if ((wf >> BL_WF_SHIFT) & BL_TF_DRY) {
    const float pw = bl_powf(sp.dry_base, (float)(int)(wf >> BL_DRY_ESHIFT));
    const float tt = sp.dry_mult * pw;
    v = v - tt;
  }
  return v;
}

/*
 * The decode loop's per-token stages (src/server.br:940-944: logit_bias, ignore_eos suppression,
 * frequency/presence, then sampling_logits' repeat penalty, src/sampling.br:65-107, :175-237) over the
 * row positions [lo, lo + n) held in LDS `vals` (lo a multiple of BL_EB, n <= BL_CH), by the whole
 * workgroup. The buckets' records are read contiguously; the end-of-generation registry is read live.
 * A speculative row (SPEC) adds its count corrections: a corrected token with a record is handled with it,
 * one without by the first correction that names it. The caller writes `vals` before and reads them after.
 */
template <bool SPEC>
__device__ void apply_stages(const bl_dev &d, const bl_slot_dev &sp, const bl_rows &rows, int row, int slot, int lo,
                             int n, float *vals, uint32_t *sup, uint32_t *done) {
  const int t = threadIdx.x, NT = (int)blockDim.x;
  const int b0 = lo / BL_EB, nbk = (n + BL_EB - 1) / BL_EB;
  int pre[BL_SUBS + 1];
  pre[0] = 0;
#pragma unroll
  for (int q = 0; q < BL_SUBS; q++) pre[q + 1] = pre[q] + (q < nbk ? d.rcnt[(int64_t)slot * d.nb + b0 + q] : 0);
  const int nrec = pre[BL_SUBS];
  const bool eog_on = sp.ignore_eos && d.n_eog > 0;
  const int nd = SPEC && rows.delta ? rows.delta_n[row] : 0;
  /* the model tail (src/model.br:973-984) first: logit_mul, then the final soft-cap cap * tanh(x / cap) */
  const float lmul = sp.logit_mul, cap = sp.final_softcap;
  const bool tail = lmul != 1.0f || cap > 0.0f;
  if (nrec == 0 && !eog_on && nd == 0 && !tail) return; /* uniform: nothing in this range changes */
  const bl_sdelta *dl = SPEC && rows.delta ? rows.delta + (int64_t)row * BL_SPEC_DCAP : nullptr;
  const bool fp = sp.fp_on && sp.n_reply > 0, rp = sp.rep_on && sp.n_tokens > 0;
  const int nw = (n + 31) / 32;
  for (int i = t; i < nw; i += NT) {
    sup[i] = 0u;
    if (SPEC) done[i] = 0u;
  }
  __syncthreads(); /* the caller's values and the cleared marks */
  if (tail) {
#pragma unroll 1
    for (int p = t; p < n; p += NT) {
      float x = vals[p];
      if (lmul != 1.0f) x = x * lmul;
      if (cap > 0.0f) {
        const float q = x / cap;
        x = cap * bl_tanhf(q);
      }
      vals[p] = x;
    }
    __syncthreads();
  }
  if (eog_on) {
    for (int e = t; e < d.n_eog; e += NT) {
      const int p = d.eog[e] - lo;
      if (p >= 0 && p < n) {
        vals[p] = -1000000000.0f; /* suppress_token (src/sampling.br:236) */
        atomicOr(&sup[p >> 5], 1u << (p & 31));
      }
    }
    __syncthreads();
  }
  const bl_rec *rb = d.rec + ((int64_t)slot * d.nb + b0) * BL_EB;
  constexpr int RU = 4; /* records in flight per thread */
  for (int base = t; base < nrec; base += RU * NT) {
    bl_rec rr[RU];
#pragma unroll
    for (int u = 0; u < RU; u++) {
      const int i = base + u * NT;
      const int q = (i >= pre[1] ? 1 : 0) + (i >= pre[2] ? 1 : 0) + (i >= pre[3] ? 1 : 0);
      rr[u] = i < nrec ? rb[(int64_t)q * BL_EB + (i - pre[q])] : bl_rec{lo, 0.0f, 0, 0u};
    }
#pragma unroll
    for (int u = 0; u < RU; u++) {
    if (base + u * NT >= nrec) break;
    const bl_rec r = rr[u];
    const int p = r.tok - lo;
    int cc = fp ? r.cnt : 0, wc = rp ? (int)(r.wf & BL_WF_WMASK) : 0;
    if (SPEC) {
      for (int e = 0; e < nd; e++)
        if (dl[e].tok == r.tok) {
          if (sp.fp_on) cc += dl[e].dcnt;
          if (sp.rep_on) wc += dl[e].dwcnt;
        }
      atomicOr(&done[p >> 5], 1u << (p & 31));
    }
    float v = vals[p];
    if (!((sup[p >> 5] >> (p & 31)) & 1u) && ((r.wf >> BL_WF_SHIFT) & BL_TF_BIAS)) v = v + r.bias;
    vals[p] = stage_dry(sp, stage_counts(sp, v, cc, wc), r.wf);
    }
  }
  if (SPEC && nd > 0) {
    __syncthreads(); /* record marks */
    for (int e = t; e < nd; e += NT) {
      const int32_t tok = dl[e].tok;
      const int p = tok - lo;
      if (p < 0 || p >= n || ((done[p >> 5] >> (p & 31)) & 1u)) continue;
      bool first = true;
      int cc = 0, wc = 0;
      for (int e2 = 0; e2 < nd; e2++)
        if (dl[e2].tok == tok) {
          first = first && e2 >= e;
          cc += dl[e2].dcnt;
          wc += dl[e2].dwcnt;
        }
      if (first) vals[p] = stage_counts(sp, vals[p], sp.fp_on ? cc : 0, sp.rep_on ? wc : 0);
    }
  }
  __syncthreads(); /* before the caller reads `vals` back */
}

/* One token's value after the model tail and the server stages: apply_stages' arithmetic for a single
 * token, its record found through the slot's token index. For the places that need a handful of tokens (the
 * normaliser's fallback walk, grammar maxima, the forced end-of-sequence token). */
__device__ __forceinline__ float bl_row_value(const bl_dev &d, const bl_slot_dev &sp, const bl_rows &rows, int row, int slot,
                              const float *logits, int64_t ld, int32_t tok) {
  float x = logits[(int64_t)row * ld + tok];
  const float lmul = sp.logit_mul, cap = sp.final_softcap;
  if (lmul != 1.0f) x = x * lmul;
  if (cap > 0.0f) {
    const float q = x / cap;
    x = cap * bl_tanhf(q);
  }
  bool sup = false;
  if (sp.ignore_eos)
    for (int k = 0; k < d.n_eog; k++) sup |= d.eog[k] == tok;
  if (sup) x = -1000000000.0f;
  const bool fp = sp.fp_on && sp.n_reply > 0, rp = sp.rep_on && sp.n_tokens > 0;
  int cc = 0, wc = 0;
  uint32_t wf = 0u;
  const int ri = d.ridx[(int64_t)slot * d.vocab + tok];
  if (ri >= 0) {
    const bl_rec r = d.rec[((int64_t)slot * d.nb + tok / BL_EB) * BL_EB + ri];
    if (!sup && ((r.wf >> BL_WF_SHIFT) & BL_TF_BIAS)) x = x + r.bias;
    cc = fp ? r.cnt : 0;
    wc = rp ? (int)(r.wf & BL_WF_WMASK) : 0;
    wf = r.wf;
  }
  if (rows.delta) {
    const int nd = rows.delta_n[row];
    const bl_sdelta *dl = rows.delta + (int64_t)row * BL_SPEC_DCAP;
    for (int e = 0; e < nd; e++)
      if (dl[e].tok == tok) {
        if (sp.fp_on) cc += dl[e].dcnt;
        if (sp.rep_on) wc += dl[e].dwcnt;
      }
  }
  return stage_dry(sp, stage_counts(sp, x, cc, wc), wf);
}

/* ------------------------------------------------------------------ K1: row pass */
/* SPEC: the rows may carry speculative count corrections (compiled separately) */
template <bool SPEC>
__device__ __forceinline__ void rowpass_body(const bl_dev &d, const float *__restrict__ logits, int64_t ld,
                                             const bl_rows &rows) {
  const int V = d.vocab, nc = d.nc;
  const int c = blockIdx.x, row = blockIdx.y, t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int slot = bl_row_slot(rows, row);
  const bl_slot_dev &sp = slot_of(d, slot);
  /* LDS kept under 20 KB so that eight workgroups fit a CU. The chunk's values (logprob sums, then the
   * radix fallback) and the compacted keys (the counting rank) are never live together. */
  __shared__ union {
    float xs[BL_CH];
    uint64_t tkeys[BL_TK_CAP]; /* keys at or above the bound */
  } lds;
  static_assert(BL_TK_CAP * 8 <= BL_CH * 4, "the key list fits in the value area");
  float *const xs = lds.xs;
  uint64_t *const tkeys = lds.tkeys;
  __shared__ uint32_t hist[256];
  __shared__ float red_m[4];
  __shared__ int red_i[4];
  __shared__ uint32_t sel[4];
  __shared__ int out_n;
  __shared__ uint32_t tk_wb[BL_RP_THREADS / 64];
  __shared__ int tk_n;
  __shared__ uint32_t st_sup[BL_CH / 32], st_done[SPEC ? BL_CH / 32 : 1];

  const int i0 = c * BL_CH;
  const int cnt = min(BL_CH, V - i0);
  const float *src = logits + (int64_t)row * ld + i0;
  if (c == 0 && t == 0) {
    /* consumed by the kernels that run after this one */
    d.gamb[row] = 0;
    d.ncrit[row] = 0;
  }
  /* thread t owns the chunk positions j*1024 + 4t + q (j, q < 4): one float4 per 1024; positions past
   * the row hold -inf */
  constexpr int NV = BL_CH / (4 * BL_RP_THREADS);
  auto pos_of = [&](int k) { return (k >> 2) * (4 * BL_RP_THREADS) + 4 * t + (k & 3); };
  const bool vec = cnt == BL_CH && (((uintptr_t)src) & 15) == 0;
  float x[4 * NV];
  if (vec) {
#pragma unroll
    for (int j = 0; j < NV; j++) {
      const float4 v = reinterpret_cast<const float4 *>(src)[j * BL_RP_THREADS + t];
      x[4 * j] = v.x;
      x[4 * j + 1] = v.y;
      x[4 * j + 2] = v.z;
      x[4 * j + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int k = 0; k < 4 * NV; k++) x[k] = pos_of(k) < cnt ? src[pos_of(k)] : BL_NEG_INF;
  }
  /* model tail and server stages at the chunk's modified tokens, in LDS (thread t's positions keep their
   * float4 layout) */
  {
    float4 *xv = reinterpret_cast<float4 *>(xs);
#pragma unroll
    for (int j = 0; j < NV; j++) xv[j * BL_RP_THREADS + t] = make_float4(x[4 * j], x[4 * j + 1], x[4 * j + 2], x[4 * j + 3]);
    apply_stages<SPEC>(d, sp, rows, row, slot, i0, cnt, xs, st_sup, st_done);
#pragma unroll
    for (int j = 0; j < NV; j++) {
      const float4 v = xv[j * BL_RP_THREADS + t];
      x[4 * j] = v.x;
      x[4 * j + 1] = v.y;
      x[4 * j + 2] = v.z;
      x[4 * j + 3] = v.w;
    }
    /* a row with a model tail leaves its values for the exponent pass */
    if (bl_tail_on(sp)) {
      float *dst = d.eff + (int64_t)row * V + i0;
      if (cnt == BL_CH && (((uintptr_t)dst) & 15) == 0) {
#pragma unroll
        for (int j = 0; j < NV; j++)
          reinterpret_cast<float4 *>(dst)[j * BL_RP_THREADS + t] = make_float4(x[4 * j], x[4 * j + 1], x[4 * j + 2], x[4 * j + 3]);
      } else {
#pragma unroll
        for (int k = 0; k < 4 * NV; k++)
          if (pos_of(k) < cnt) dst[pos_of(k)] = x[k];
      }
    }
  }
  /* max and first argmax; then, for logprob rows, approximate sums of exp(x - chunk max) over each BL_EB
   * positions, from which the exponent pass predicts the binades of the normaliser's running sum
   * (wavefront j reduces sub-block j) */
  static_assert(NV == BL_SUBS && BL_RP_THREADS / 64 == BL_SUBS, "thread positions j*1024 + ... cover sub-block j");
  {
    float m = BL_NEG_INF;
    int mi = 0x7fffffff;
#pragma unroll
    for (int k = 0; k < 4 * NV; k++) /* positions ascend with k: the first maximum is kept */
      if (x[k] > m) {
        m = x[k];
        mi = pos_of(k);
      }
    bl_wargmax(m, mi, lane);
    if (lane == 0) {
      red_m[w] = m;
      red_i[w] = mi;
    }
    __syncthreads();
    float cm = red_m[0];
    int ci = red_i[0];
#pragma unroll
    for (int k = 1; k < BL_RP_THREADS / 64; k++) argmax_merge(cm, ci, red_m[k], red_i[k]);
    const int64_t o = (int64_t)row * nc + c;
    if (sp.mode & (BL_M_LOGPROBS | BL_M_ADAPT)) {
      float *red_s = xs; /* [BL_SUBS][BL_RP_THREADS]; the value area is free until the key list */
#pragma unroll
      for (int j = 0; j < NV; j++) {
        float sj = 0.0f;
        if (cm > BL_NEG_INF) {
#pragma unroll
          for (int q = 0; q < 4; q++) sj += __expf(x[4 * j + q] - cm);
        }
        red_s[j * BL_RP_THREADS + t] = sj;
      }
      __syncthreads();
      double v = 0.0;
#pragma unroll
      for (int i = 0; i < BL_RP_THREADS / 64; i++) v += (double)red_s[w * BL_RP_THREADS + lane + 64 * i];
      v = bl_wave_sum_d(v);
      if (lane == 0) d.c_bsum[o * BL_SUBS + w] = (float)v;
      __syncthreads(); /* red_s (xs) is read before the fallback reuses it */
    }
    if (t == 0) {
      d.c_max[o] = cm;
      d.c_arg[o] = ci == 0x7fffffff ? i0 : i0 + ci;
    }
    if (sp.mode & BL_M_TNS) {
      /* top-n-sigma's statistics over the chunk's values above -1e29 (src/sampling.br:383-393): the sums of
       * x and x^2 (a float32 square is exact in float64) as double-doubles, the sum of |x| and the count */
      bl_dd ts{0.0, 0.0}, tq{0.0, 0.0};
      double ta = 0.0, tn = 0.0;
#pragma unroll
      for (int k = 0; k < 4 * NV; k++)
        if (x[k] > -1.0e29f) {
          const double v = (double)x[k];
          ts = bl_dd_add_d(ts, v);
          tq = bl_dd_add_d(tq, v * v);
          ta += v < 0.0 ? -v : v;
          tn += 1.0;
        }
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        ts = bl_dd_add(ts, bl_dd{__shfl_xor(ts.hi, off, 64), __shfl_xor(ts.lo, off, 64)});
        tq = bl_dd_add(tq, bl_dd{__shfl_xor(tq.hi, off, 64), __shfl_xor(tq.lo, off, 64)});
        ta += __shfl_xor(ta, off, 64);
        tn += __shfl_xor(tn, off, 64);
      }
      __shared__ double tns_w[BL_RP_THREADS / 64][BL_TNS_W];
      if (lane == 0) {
        tns_w[w][0] = ts.hi;
        tns_w[w][1] = ts.lo;
        tns_w[w][2] = tq.hi;
        tns_w[w][3] = tq.lo;
        tns_w[w][4] = ta;
        tns_w[w][5] = tn;
      }
      __syncthreads();
      if (t == 0) {
        for (int q = 1; q < BL_RP_THREADS / 64; q++) {
          ts = bl_dd_add(ts, bl_dd{tns_w[q][0], tns_w[q][1]});
          tq = bl_dd_add(tq, bl_dd{tns_w[q][2], tns_w[q][3]});
          ta += tns_w[q][4];
          tn += tns_w[q][5];
        }
        double *out = d.c_tns + o * BL_TNS_W;
        out[0] = ts.hi;
        out[1] = ts.lo;
        out[2] = tq.hi;
        out[3] = tq.lo;
        out[4] = ta;
        out[5] = tn;
      }
    }
  }

  /* chunk top-K by (value desc, index asc) over values > -1e30 (src/sampling.br:280-296). Order keys
   * (value, then lower index) are distinct integers. A lower bound on the chunk's K-th value: wavefront w
   * takes the s_w-th largest of its threads' maxima (each of those threads holds a value at or above
   * it), with shares s_w proportional to its threads that hold positions of the row and summing to at
   * least K, and the smallest of the bounds is the chunk's, so at least K values reach it. The keys of
   * those values (typically K to 2K) are compacted and ranked by counting. A wavefront with fewer valid
   * maxima than its share sets no bound; when too many values reach the bound, three radix passes find
   * the K-th key instead. */
  const int K = sp.k_sel;
  if (K <= 0) return;
  const int64_t cbase = ((int64_t)row * nc + c) * BL_KSEL_MAX;
  {
    uint32_t best = 0u; /* this thread's largest valid value as an order key; 0: none */
#pragma unroll
    for (int k = 0; k < 4 * NV; k++)
      if (x[k] > -1.0e30f) {
        const uint32_t fk = bl_fkey(x[k]);
        best = fk > best ? fk : best;
      }
    /* threads holding a position of the row: 4t < cnt */
    const int n_all = min((cnt + 3) >> 2, BL_RP_THREADS);
    const int n_w = min(max(n_all - 64 * w, 0), 64);
    const int share = n_all >= K ? (K * n_w + n_all - 1) / n_all : 64 + 1; /* > 64: no bound */
    /* the share-th largest of the wavefront's maxima: the largest key v with at least `share` maxima >= v,
     * bit by bit from the top (0 when fewer than `share` threads hold a valid value) */
    uint32_t wb = 0u;
#pragma unroll
    for (int bit = 31; bit >= 0; bit--) {
      const uint32_t cand = wb | (1u << bit);
      if (__popcll(__ballot(best >= cand)) >= share) wb = cand;
    }
    if (share == 0) wb = 0xFFFFFFFFu; /* no threads of the row: no part in the bound */
    if (lane == 0) tk_wb[w] = wb;
    if (t == 0) tk_n = 0;
    __syncthreads();
    uint32_t tau = tk_wb[0];
#pragma unroll
    for (int k = 1; k < BL_RP_THREADS / 64; k++) tau = tk_wb[k] < tau ? tk_wb[k] : tau;
    /* compaction of the keys >= tau, in no particular order; one LDS atomic per wavefront */
    int mine = 0;
#pragma unroll
    for (int k = 0; k < 4 * NV; k++) mine += (x[k] > -1.0e30f && bl_fkey(x[k]) >= tau) ? 1 : 0;
    const int incl = bl_wscan_add(mine, lane);
    const int wtot = (int)bl_bcast((uint32_t)incl, 63);
    int wbase = 0;
    if (lane == 0 && wtot > 0) wbase = atomicAdd(&tk_n, wtot);
    int pos = (int)bl_bcast((uint32_t)wbase, 0) + incl - mine;
#pragma unroll
    for (int k = 0; k < 4 * NV; k++)
      if (x[k] > -1.0e30f && bl_fkey(x[k]) >= tau) {
        if (pos < BL_TK_CAP) tkeys[pos] = ckey(x[k], i0 + pos_of(k));
        pos++;
      }
    __syncthreads();
    const int nk = tk_n;
    if (nk <= BL_TK_CAP) {
      /* rank by counting; the K largest go out in order */
      for (int q = t; q < nk; q += BL_RP_THREADS) {
        const uint64_t kk = tkeys[q];
        const int rr = count_gt(tkeys, nk, kk);
        if (rr < K) {
          d.cand_v[cbase + rr] = ckey_v(kk);
          d.cand_i[cbase + rr] = ckey_i(kk);
        }
      }
      for (int q = nk + t; q < K; q += BL_RP_THREADS) {
        d.cand_v[cbase + q] = BL_NEG_INF;
        d.cand_i[cbase + q] = -1;
      }
      return;
    }
    __syncthreads();
  }
  /* fallback: the values go to LDS for the radix passes */
#pragma unroll
  for (int j = 0; j < NV; j++)
    reinterpret_cast<float4 *>(xs)[j * BL_RP_THREADS + t] = make_float4(x[4 * j], x[4 * j + 1], x[4 * j + 2], x[4 * j + 3]);
  __syncthreads();
  uint32_t prefix = 0u, pmask = 0u;
  int need = K;
  bool take_all = false;
  for (int pass = 0; pass < 4; pass++) { /* 8 bits of the order key per pass, from the top */
    const int shift = 24 - 8 * pass;
    constexpr int nb = 256;
    for (int b = t; b < nb; b += BL_RP_THREADS) hist[b] = 0u;
    __syncthreads();
    for (int i = t; i < cnt; i += BL_RP_THREADS) {
      float x = xs[i];
      if (x > -1.0e30f) {
        uint32_t k = bl_fkey(x);
        if ((k & pmask) == prefix) atomicAdd(&hist[(k >> shift) & (nb - 1)], 1u);
      }
    }
    __syncthreads();
    /* bins from the top: thread t owns [nb - (t+1)*per, nb - t*per) */
    const int per = nb / BL_RP_THREADS;
    uint32_t local = 0u;
    for (int q = 0; q < per; q++) local += hist[nb - 1 - (t * per + q)];
    /* exclusive scan of `local` over threads 0..255 */
    uint32_t inc = local;
#pragma unroll
    for (int k = 1; k < 64; k <<= 1) {
      uint32_t o = __shfl_up(inc, k, 64);
      if (lane >= k) inc += o;
    }
    __shared__ uint32_t wsum[4];
    if (lane == 63) wsum[w] = inc;
    __syncthreads();
    uint32_t above = inc - local;
    for (int k = 0; k < w; k++) above += wsum[k];
    uint32_t total = wsum[0] + wsum[1] + wsum[2] + wsum[3];
    if (pass == 0 && total <= (uint32_t)need) {
      take_all = true;
    } else if (above < (uint32_t)need && above + local >= (uint32_t)need) {
      uint32_t acc = above;
      for (int q = 0; q < per; q++) {
        int b = nb - 1 - (t * per + q);
        uint32_t h = hist[b];
        if (acc + h >= (uint32_t)need) {
          sel[0] = (uint32_t)b;
          sel[1] = acc;
          sel[2] = h;
          break;
        }
        acc += h;
      }
    }
    __syncthreads();
    if (take_all) break;
    prefix |= sel[0] << shift;
    pmask |= (uint32_t)(nb - 1) << shift;
    need -= (int)sel[1];
    __syncthreads();
  }
  /* take_all is uniform: every thread saw the same total */
  if (t == 0) out_n = 0;
  __syncthreads();
  const uint32_t kth = prefix;
  const bool cut_ties = !take_all && (int)sel[2] > need;
  int eq_before = 0; /* ties of kth at smaller indices, for the index-order cut */
  for (int s0 = 0; s0 < cnt; s0 += BL_RP_THREADS) {
    int i = s0 + t;
    bool ok = false;
    bool eq = false;
    if (i < cnt) {
      float x = xs[i];
      if (x > -1.0e30f) {
        uint32_t k = bl_fkey(x);
        if (take_all || k > kth) ok = true;
        else if (k == kth) eq = true;
      }
    }
    if (cut_ties) {
      unsigned long long bm = __ballot(eq);
      __shared__ int wcnt_eq[4];
      if (lane == 0) wcnt_eq[w] = __popcll(bm);
      __syncthreads();
      int before = eq_before + __popcll(bm & ((1ull << lane) - 1ull));
      for (int k = 0; k < w; k++) before += wcnt_eq[k];
      if (eq && before < need) ok = true;
      eq_before += wcnt_eq[0] + wcnt_eq[1] + wcnt_eq[2] + wcnt_eq[3];
      __syncthreads();
    } else if (eq) {
      ok = true;
    }
    if (ok) {
      int pos = atomicAdd(&out_n, 1);
      if (pos < K) {
        d.cand_v[cbase + pos] = xs[i];
        d.cand_i[cbase + pos] = i0 + i;
      }
    }
  }
  __syncthreads();
  for (int p = min(out_n, K) + t; p < K; p += BL_RP_THREADS) {
    d.cand_v[cbase + p] = BL_NEG_INF;
    d.cand_i[cbase + p] = -1;
  }
}

__global__ __launch_bounds__(BL_RP_THREADS) void bl_k_rowpass(bl_dev d, const float *__restrict__ logits, int64_t ld,
                                                              bl_rows rows) {
  rowpass_body<false>(d, logits, ld, rows);
}
__global__ __launch_bounds__(BL_RP_THREADS) void bl_k_rowpass_spec(bl_dev d, const float *__restrict__ logits,
                                                                   int64_t ld, bl_rows rows) {
  rowpass_body<true>(d, logits, ld, rows);
}

/* ------------------------------------------------------------------ K2: exponent pass */
/*
 * grid (ceil(V / BL_EB), B) x 256, rows with logprobs or a full-vocabulary rank: thread t holds the block's
 * positions 4t..4t+3 (one float4 of the logits), a 64-term group is 16 threads. The block re-reads its
 * logits, applies the model tail and the server stages at its bucket's records (the row pass's values,
 * recomputed: no transformed row is stored), then writes
 *   - per 64-term group, the exact terms' composed automaton at the binade of the group's approximate start
 *     (bl_grec1), and per block a summary (bl_grec1 + a mask of critical groups);
 *   - per critical group (the sum may cross a power of two inside it), an entry of the row's critical list:
 *     the terms, their prefix compositions at the start binade, suffix compositions at the end binade, and
 *     the block's group records, so that the selection resolves the crossing without re-deriving anything;
 *   - the candidates of a full-vocabulary rank (within bl_cand_span of the row maximum).
 * The critical list is appended with one device-scope atomic per critical group (a few per row); no
 * workgroup waits for another: the selection kernel, a later launch, reads the list.
 */
#define BL_MU_MAX 256 /* the exponent pass's merge: first keys of the chunk lists held in LDS */
#define BL_MSURV 512  /* the exponent pass's merge: survivors of the cut held in LDS */
/* the exponent pass's LDS shared by its two roles: a block's values, or the merge's keys */
#define BL_K2_LDS_U64 (BL_MU_MAX + BL_MSURV)
static_assert(BL_K2_LDS_U64 * 8 >= BL_EB * 4, "a block's values fit the shared area");
#define BL_MREG 8     /* the exponent pass's merge: list entries per thread loaded at once */

/*
 * The exponent pass's first workgroup of each row, beside the row's exponent blocks: the row maximum and its
 * first index (d.rmax, d.rarg) from the chunk statistics, and the row's top K keys in (value desc, index asc)
 * order (top_k_select, src/sampling.br:280-296) merged from the row pass's chunk lists into
 * d.mkeys[row][0..K) (0 past the valid keys). The cut is the selection's merge's: the K-th largest of the
 * lists' first L = ceil(K/nc) keys is at most the row's K-th key, so the row's top K are among the keys at
 * or above it, which are ranked by counting (keys are distinct: they carry the index). d.mstat[row] = 1 once
 * done; 0 when the first keys or the survivors exceed this workgroup's LDS, and the selection then merges the
 * lists itself.
 */
template <int NT>
__device__ __forceinline__ void exp_merge_role(const bl_dev &d, const bl_rows &rows, int row, uint64_t *lds) {
  const int t = threadIdx.x, lane = t & 63, nc = d.nc;
  uint64_t *const m_u = lds, *const m_sv = lds + BL_MU_MAX;
  __shared__ uint64_t m_tau;
  __shared__ int m_n;
  const int K = d.slots[bl_row_slot(rows, row)].k_sel;
  if (t < 64) {
    float M = BL_NEG_INF;
    int Mi = 0x7fffffff;
    for (int k = lane; k < nc; k += 64) argmax_merge(M, Mi, d.c_max[(int64_t)row * nc + k], d.c_arg[(int64_t)row * nc + k]);
    bl_wargmax(M, Mi, lane);
    if (t == 0) {
      d.rmax[row] = M;
      d.rarg[row] = Mi;
    }
  }
  const int L = K > 0 ? (K + nc - 1) / nc : 0, nu = nc * L, total = nc * K;
  if (K <= 0 || nu > BL_MU_MAX) {
    if (t == 0) d.mstat[row] = K <= 0 ? 1 : 0;
    return;
  }
  auto gkey = [&](int c, int q) -> uint64_t {
    const int64_t o = ((int64_t)row * nc + c) * BL_KSEL_MAX + q;
    const int32_t id = d.cand_i[o];
    const float v = d.cand_v[o]; /* loaded with the id, not after it */
    return id >= 0 ? ckey(v, id) : 0ull;
  };
  if (t == 0) {
    m_tau = 1ull; /* every valid key, when fewer than K exist */
    m_n = 0;
  }
  /* every list entry up to BL_MREG * NT of them in registers, all loads in flight at once; the lists' first
   * L keys among them go to LDS */
  constexpr int PU = BL_MREG;
  uint64_t kr[PU];
#pragma unroll
  for (int u = 0; u < PU; u++) {
    const int i = t + u * NT;
    const int c = i / K;
    kr[u] = i < total ? gkey(c, i - c * K) : 0ull;
  }
  if (total <= PU * NT) {
#pragma unroll
    for (int u = 0; u < PU; u++) {
      const int i = t + u * NT;
      const int c = i / K, q = i - c * K;
      if (i < total && q < L) m_u[c * L + q] = kr[u];
    }
  } else {
    for (int i = t; i < nu; i += NT) m_u[i] = gkey(i / L, i - (i / L) * L);
  }
  __syncthreads();
  for (int i = t; i < nu; i += NT) {
    const uint64_t k = m_u[i];
    if (k && count_gt<4>(m_u, nu, k) == K - 1) m_tau = k;
  }
  __syncthreads();
  const uint64_t tau = m_tau;
  auto keep = [&](uint64_t k) {
    if (k >= tau) {
      const int p = atomicAdd(&m_n, 1);
      if (p < BL_MSURV) m_sv[p] = k;
    }
  };
#pragma unroll
  for (int u = 0; u < PU; u++) keep(kr[u]);
  for (int i0 = PU * NT; i0 < total; i0 += PU * NT) { /* longer lists: the next PU keys per thread at once */
#pragma unroll
    for (int u = 0; u < PU; u++) {
      const int i = i0 + t + u * NT;
      const int c = i / K;
      kr[u] = i < total ? gkey(c, i - c * K) : 0ull;
    }
#pragma unroll
    for (int u = 0; u < PU; u++) keep(kr[u]);
  }
  __syncthreads();
  const int C = m_n;
  if (C > BL_MSURV) {
    if (t == 0) d.mstat[row] = 0;
    return;
  }
  uint64_t *out = d.mkeys + (int64_t)row * BL_KSEL_MAX;
  for (int i = t; i < C; i += NT) {
    const uint64_t k = m_sv[i];
    const int r = count_gt<4>(m_sv, C, k);
    if (r < K) out[r] = k;
  }
  for (int q = C + t; q < K; q += NT) out[q] = 0ull;
  if (t == 0) d.mstat[row] = 1;
}

template <bool SPEC>
__device__ __forceinline__ void exppass_body(const bl_dev &d, const float *__restrict__ logits, int64_t ld,
                                             const bl_rows &rows) {
  const int V = d.vocab, nc = d.nc;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  /* workgroup 0 of each row merges (dispatched first: it takes longer than a block), 1 + b computes block b */
  const int b = (int)blockIdx.x - 1, row = blockIdx.y;
  __shared__ uint64_t k2_lds[BL_K2_LDS_U64];
  if (b < 0) {
    exp_merge_role<BL_RP_THREADS>(d, rows, row, k2_lds);
    return;
  }
  const int slot = bl_row_slot(rows, row);
  const bl_slot_dev &sp = slot_of(d, slot);
  const int mode = sp.mode;
  if (!(mode & (BL_M_LOGPROBS | BL_M_FULL | BL_M_GFULL | BL_M_ADAPT))) return;
  __shared__ uint64_t s_tab[BL_EXP2_N]; /* expf's 2^(i/32) table */
  float *const vals = reinterpret_cast<float *>(k2_lds); /* [BL_EB] */
  __shared__ uint32_t st_sup[BL_EB / 32], st_done[SPEC ? BL_EB / 32 : 1];
  __shared__ double wtot[BL_RP_THREADS / 64];
  __shared__ uint32_t bs_crit[BL_RP_THREADS / 64];
  __shared__ int bs_E[BL_RP_THREADS / 64];
  __shared__ bool bs_same[BL_RP_THREADS / 64];
  __shared__ bl_inc bs_v[BL_RP_THREADS / 64];
  __shared__ bl_grec1 s_grp[BL_EB / 64];
  if (t < BL_EXP2_N) s_tab[t] = bl_exp2_tab[t];
  const int i0 = b * BL_EB;
  const int cnt = min(BL_EB, V - i0);
  const int j0 = 4 * t;
  float x[4];
  /* a row with a model tail reads the values the row pass left (the tail's tanhf is not worth computing twice);
   * the others re-read their logits and apply the sparse stages again */
  const bool from_eff = bl_tail_on(sp);
  const float *src = from_eff ? d.eff + (int64_t)row * V + i0 + j0 : logits + (int64_t)row * ld + i0 + j0;
  if (j0 + 4 <= cnt && (((uintptr_t)src) & 15) == 0) {
    const float4 v = *reinterpret_cast<const float4 *>(src);
    x[0] = v.x;
    x[1] = v.y;
    x[2] = v.z;
    x[3] = v.w;
  } else {
#pragma unroll
    for (int k = 0; k < 4; k++) x[k] = j0 + k < cnt ? src[k] : BL_NEG_INF;
  }
  /* the row maximum and its first index, by every wavefront from the chunk statistics; lane k also keeps
   * chunk k's maximum and sub-block sums (the first 64 chunks), loaded with them for the prefix below */
  float M = BL_NEG_INF;
  int Mi = 0x7fffffff;
  float cm0 = BL_NEG_INF;
  float4 cb0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (lane < nc) {
    cm0 = d.c_max[(int64_t)row * nc + lane];
    cb0 = *reinterpret_cast<const float4 *>(d.c_bsum + ((int64_t)row * nc + lane) * BL_SUBS);
    argmax_merge(M, Mi, cm0, d.c_arg[(int64_t)row * nc + lane]);
  }
  for (int k = lane + 64; k < nc; k += 64) argmax_merge(M, Mi, d.c_max[(int64_t)row * nc + k], d.c_arg[(int64_t)row * nc + k]);
  /* model tail and server stages, as the row pass applied them */
  if (!from_eff) {
    *reinterpret_cast<float4 *>(vals + j0) = make_float4(x[0], x[1], x[2], x[3]);
    apply_stages<SPEC>(d, sp, rows, row, slot, i0, cnt, vals, st_sup, st_done);
    const float4 v = *reinterpret_cast<const float4 *>(vals + j0);
    x[0] = v.x;
    x[1] = v.y;
    x[2] = v.z;
    x[3] = v.w;
  }
  bl_wargmax(M, Mi, lane);

  if (mode & (BL_M_LOGPROBS | BL_M_ADAPT)) {
    /* lane k: chunk k's sub-blocks before this block, scaled by the hardware exponential (a prediction:
     * its error, ~1e-7 relative, is far inside the 2^-20 margin of the critical-group test, and a wrong
     * binade is caught on the exact state) */
    static_assert(BL_SUBS == 4, "one float4 of sub-block sums per chunk");
    const int nsub = i0 / BL_EB;
    double part = 0.0;
    for (int k = lane; k * BL_SUBS < nsub; k += 64) {
      const float cm = k < 64 ? cm0 : d.c_max[(int64_t)row * nc + k];
      const float4 cb = k < 64 ? cb0 : *reinterpret_cast<const float4 *>(d.c_bsum + ((int64_t)row * nc + k) * BL_SUBS);
      if (cm > BL_NEG_INF) {
        const int lim = nsub - k * BL_SUBS;
        const double cs = (double)cb.x + (lim > 1 ? (double)cb.y : 0.0) + (lim > 2 ? (double)cb.z : 0.0) +
                          (lim > 3 ? (double)cb.w : 0.0);
        part += cs * (double)__expf(cm - M);
      }
    }
    const double S0 = bl_wave_sum_d(part);
    __syncthreads(); /* s_tab */
    float a[4];
    double sa = 0.0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      a[k] = j0 + k < cnt ? bl_expf_tab(x[k] - M, [&](uint32_t i) { return s_tab[i]; }) : 0.0f;
      sa += (double)a[k];
    }
    const double ex = bl_wave_excl_scan_d(sa, lane);
    if (lane == 63) wtot[w] = ex + sa;
    __syncthreads();
    double before = S0 + ex;
    for (int q = 0; q < BL_RP_THREADS / 64; q++)
      if (q < w) before += wtot[q];
    /* group of 64 terms = 16 threads (one row of the wavefront); its approximate start is its first
     * thread's prefix, raised to the exact floor 1.0 once the row maximum's term exp(0) = 1 is behind it.
     * The row's last lane holds the group's composed automaton (row scan) and its approximate end (its own
     * inclusive prefix), and writes the record. */
    const int gl = lane & ~15, tail_l = gl | 15, r16 = lane & 15;
    const int gs = i0 + 4 * (t & ~15);
    const double floor1 = gs > Mi ? 1.0 : 0.0;
    const double gs0 = __shfl(before, gl, 64);
    const double gstart = gs0 > floor1 ? gs0 : floor1;
    const int E = bl_binade_of(gstart);
    const bl_inc tc = bl_thread_compose<4>(a, E);
    const bl_inc gv = bl_row_scan(tc, lane);
    const bool tail = r16 == 15;
    const bool gex = 4 * (t & ~15) < cnt;
    const int g = gs >> 6;
    bl_grec1 *rec = reinterpret_cast<bl_grec1 *>(reinterpret_cast<bl_grec *>(d.grec) + (int64_t)row * 2 * (V / 64 + 64));
    const double gend = before + sa;
    const double gend_f = gend > floor1 ? gend : floor1;
    const bool crit = gex && bl_group_critical((float)gstart, (float)gend_f, E, floor1);
    if (tail && gex) {
      bl_grec1 r;
      r.E = E;
      r.pad = 0;
      r.v = gv;
      rec[g] = r;
      s_grp[g & 15] = r;
    }
    /* block summary for the normaliser: the critical groups (approximate start or end not safely inside
     * the predicted binade), and, when there is none and every group has the same binade, the block's
     * automaton composed in order (wavefront w holds groups 4w..4w+3) */
    const unsigned long long cb = __ballot(crit && tail);
    const unsigned long long eb = __ballot(gex && tail);
    const int E0 = (int)bl_bcast((uint32_t)E, 15);
    const unsigned long long db = __ballot(gex && tail && E != E0);
    bl_inc f = bl_inc_ident();
#pragma unroll
    for (int q = 0; q < 4; q++)
      if ((eb >> (16 * q + 15)) & 1ull) f = bl_compose(f, bl_inc{bl_bcast(gv.d0, 16 * q + 15), bl_bcast(gv.d1, 16 * q + 15)});
    if (lane == 0) {
      bs_crit[w] = (uint32_t)(((cb >> 15) & 1ull) | ((cb >> 30) & 2ull) | ((cb >> 45) & 4ull) | ((cb >> 60) & 8ull));
      bs_E[w] = ((eb >> 15) & 1ull) ? E0 : BL_E_NONE; /* BL_E_NONE: the wavefront holds no group */
      bs_same[w] = db == 0ull;
      bs_v[w] = f;
    }
    __syncthreads(); /* summaries and s_grp */
    if (t == 0) {
      uint32_t mask = 0u;
      const int Eb = bs_E[0];
      bool clean = true;
      bl_inc v = bl_inc_ident();
      for (int q = 0; q < BL_RP_THREADS / 64; q++) {
        mask |= bs_crit[q] << (4 * q);
        if (bs_E[q] == BL_E_NONE) continue;
        clean = clean && bs_same[q] && bs_E[q] == Eb;
        v = bl_compose(v, bs_v[q]);
      }
      bl_grec1 br;
      br.E = clean && mask == 0u ? Eb : BL_E_NONE;
      br.pad = 0;
      br.v = v;
      reinterpret_cast<bl_grec1 *>(d.brec)[(int64_t)row * d.nb + b] = br;
      d.bcrit[(int64_t)row * d.nb + b] = mask;
    }
    /* critical groups: an entry of the row's critical list each (wavefront-uniform branch; the lanes of
     * other groups compute alongside and write nothing) */
    if (cb) {
      const bool gcrit = __shfl(crit ? 1 : 0, tail_l, 64) != 0;
      const int e1 = bl_binade_of(__shfl(gend_f, tail_l, 64));
      int slot_i = 0;
      if (gcrit && tail) slot_i = atomicAdd(&d.ncrit[row], 1);
      slot_i = __shfl(slot_i, tail_l, 64);
      /* prefix compositions at E: the row scan's exclusive prefix (identity at the row's first lane), then
       * the thread's own terms */
      const uint32_t x0 = bl_dpp<BL_DPP_ROW_SHR(1), 0xF>(0u, gv.d0), x1 = bl_dpp<BL_DPP_ROW_SHR(1), 0xF>(0u, gv.d1);
      bl_inc px = r16 == 0 ? bl_inc_ident() : bl_inc{x0, x1};
      bl_inc cp[4];
#pragma unroll
      for (int q = 0; q < 4; q++) {
        px = bl_compose(px, bl_term_inc(a[q], E));
        cp[q] = px;
      }
      /* suffix compositions at e1: the thread's own suffixes, then the following threads of the group in
       * order (a reversed scan over the row's 16 lanes) */
      bl_inc sfx[4];
      bl_inc acc = bl_inc_ident();
#pragma unroll
      for (int q = 3; q >= 0; q--) {
        acc = bl_compose(bl_term_inc(a[q], e1), acc);
        sfx[q] = acc;
      }
      bl_inc rv = acc; /* composition of this thread's four terms at e1, then those after it */
#pragma unroll
      for (int k = 1; k < 16; k <<= 1) {
        const bl_inc o = bl_inc{(uint32_t)__shfl_down((int)rv.d0, k, 64), (uint32_t)__shfl_down((int)rv.d1, k, 64)};
        if (r16 + k < 16) rv = bl_compose(rv, o);
      }
      const bl_inc nx = bl_inc{(uint32_t)__shfl_down((int)rv.d0, 1, 64), (uint32_t)__shfl_down((int)rv.d1, 1, 64)};
      const bl_inc after = r16 == 15 ? bl_inc_ident() : nx;
      if (gcrit && slot_i < BL_CRIT_MAX) {
        bl_crit &ce = d.crit[(int64_t)row * BL_CRIT_MAX + slot_i];
#pragma unroll
        for (int q = 0; q < 4; q++) {
          ce.terms[4 * r16 + q] = a[q];
          ce.cp[4 * r16 + q] = cp[q];
          ce.cs[4 * r16 + q] = bl_compose(sfx[q], after);
        }
        ce.blk[r16] = s_grp[r16];
        if (tail) {
          ce.g = g;
          ce.e0 = E;
          ce.e1 = e1;
          ce.ng = min(BL_EB / 64, (cnt + 63) / 64);
        }
      }
    }
  }
  if (mode & (BL_M_FULL | BL_M_GFULL)) {
    /* candidates of a full-vocabulary rank (within bl_cand_span of the maximum). The block writes them
     * in index order to its own BL_EB-entry region, and their count: no counter is shared between
     * workgroups. A sampled full-vocabulary grammar row ranks its allowed tokens only (src/server.br:334-357):
     * the mask filters them, and the span counts from the allowed maximum (the grammar pass's block maxima);
     * a sampled top-k grammar row lists every candidate, for its widening levels */
    __shared__ int f_w[BL_RP_THREADS / 64];
    const float T = sp.temperature;
    const bool filt = bl_probs_on(sp);
    const bool gsel = (mode & BL_M_GRAMMAR) && (mode & BL_M_FULL) && T > 0.0f;
    float Mc = M;
    uint32_t amask = 0xFu; /* this thread's four tokens: allowed */
    if (gsel) {
      __shared__ float g_m[BL_RP_THREADS / 64];
      float gm = BL_NEG_INF;
      for (int k = t; k < d.gm_blocks; k += BL_RP_THREADS) gm = fmaxf(gm, d.gm_max[(int64_t)row * d.gm_blocks + k]);
      int gi = 0;
      bl_wargmax(gm, gi, lane);
      if (lane == 0) g_m[w] = gm;
      __syncthreads();
      Mc = g_m[0];
#pragma unroll
      for (int q = 1; q < BL_RP_THREADS / 64; q++) Mc = fmaxf(Mc, g_m[q]);
      const int64_t words = 2 * (((int64_t)V + 63) / 64);
      const int tk = i0 + j0;
      amask = tk < V ? (d.gmask[(int64_t)row * words + (tk >> 6) * 2 + ((tk >> 5) & 1)] >> (tk & 31)) & 0xFu : 0u;
    }
    /* a top-k grammar row's widening levels read the first ranks of the whole row: four spans deep */
    const float thr = Mc - ((mode & BL_M_FULL) ? 1.0f : 4.0f) * bl_cand_span(sp);
    auto keep_k = [&](int k) { return j0 + k < cnt && x[k] >= thr && ((amask >> k) & 1u); };
    int mine = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) mine += keep_k(k) ? 1 : 0;
    const int incl = bl_wscan_add(mine, lane);
    if (lane == 63) f_w[w] = incl;
    __syncthreads();
    int pos = incl - mine, tot = 0;
#pragma unroll
    for (int q = 0; q < BL_RP_THREADS / 64; q++) {
      if (q < w) pos += f_w[q];
      tot += f_w[q];
    }
    const int64_t ro = ((int64_t)row * d.nb + b) * BL_EB;
#pragma unroll
    for (int k = 0; k < 4; k++)
      if (keep_k(k)) {
        d.full_v[ro + pos] = x[k];
        d.full_i[ro + pos] = i0 + j0 + k;
        pos++;
      }
    if (t == 0) d.full_cnt[(int64_t)row * d.nb + b] = tot;
    if (!filt && T > 0.0f) {
      /* the block's share of the tempered sum, approximately (hardware exponential, double partials):
       * the selection derives a lower bound on the draw's running sum from it */
      const float rT = 1.0f / T;
      float ps = 0.0f;
#pragma unroll
      for (int k = 0; k < 4; k++)
        if (keep_k(k)) ps += __expf((x[k] - Mc) * rT);
      const double ws = bl_wave_sum_d((double)ps);
      __shared__ double f_s[BL_RP_THREADS / 64];
      if (lane == 0) f_s[w] = ws;
      __syncthreads();
      if (t == 0) {
        double bs = 0.0;
#pragma unroll
        for (int q = 0; q < BL_RP_THREADS / 64; q++) bs += f_s[q];
        d.full_s[(int64_t)row * d.nb + b] = bs;
      }
    }
  }
}

__global__ __launch_bounds__(BL_RP_THREADS) void bl_k_exppass(bl_dev d, const float *__restrict__ logits, int64_t ld,
                                                              bl_rows rows) {
  exppass_body<false>(d, logits, ld, rows);
}
__global__ __launch_bounds__(BL_RP_THREADS) void bl_k_exppass_spec(bl_dev d, const float *__restrict__ logits,
                                                                   int64_t ld, bl_rows rows) {
  exppass_body<true>(d, logits, ld, rows);
}

/* ------------------------------------------------------------------ K2g: grammar allow-mask */
/*
 * grid (ceil(V/256), B) x 256 over the rows of grammar slots; one lane per token. The allowed
 * predicate of sample_grammar_token (src/server.br:334-350): an end-of-generation token when the
 * frontier is complete and ignore_eos is off, any other token when grammar_advance_text(frontier,
 * piece) is not empty. Writes the packed allow-bitmask (a __ballot per wavefront), the frontier's
 * status (src/server.br:311-321), and, with `with_values`, each block's allowed maximum of the row after
 * the model tail and server stages (bl_row_value of the allowed tokens: a grammar leaves few) with its
 * lowest index and the number of allowed tokens equal to it (the first allowed candidate in rank order of
 * a greedy step, src/server.br:351-356).
 */
__global__ __launch_bounds__(BL_GM_THREADS) void bl_k_gmask(bl_dev d, const float *__restrict__ logits, int64_t ld,
                                                            bl_rows rows, int with_values) {
  const int V = d.vocab, row = blockIdx.y, t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int slot = bl_row_slot(rows, row);
  const bl_slot_dev &sp = d.slots[slot];
  if (!sp.g_on) return;
  __shared__ float red_m[BL_GM_THREADS / 64];
  __shared__ int red_i[BL_GM_THREADS / 64];
  __shared__ int red_n[BL_GM_THREADS / 64];
  const bl_gram_view g = d.gram[slot];
  const bl_gram_pos pos = sp.gpos;
  const bool js = sp.g_kind == 1;
  const bl_json_pos jp = sp.jpos;
  const uint8_t *jst = d.jstack + (int64_t)slot * BL_JSON_DEPTH;
  const int32_t front = js ? 0 : bl_gw_frontier(g, pos);
  const int64_t tok = (int64_t)blockIdx.x * BL_GM_THREADS + t;
  bool allowed = false, ambig = false;
  if (js && tok < V) {
    /* json_object_decoded_candidate_allowed (src/json.br:420-426): an end-of-generation token only when the
     * reply is a complete object, where the step forces it (src/server.br:266-269); any other token when
     * the reply with its piece stays viable */
    bool eog = false;
    for (int k = 0; k < d.n_eog; k++) eog |= d.eog[k] == (int32_t)tok;
    if (!eog) {
      const uint32_t o0 = d.voff[tok], o1 = d.voff[tok + 1];
      const uint8_t *b = d.vblob + o0;
      bool over = false;
      allowed = bl_js_walk(jp, jst, [&](int i) { return (uint32_t)b[i]; }, (int)(o1 - o0), &over);
      ambig = over;
    } else {
      allowed = !sp.ignore_eos && bl_js_complete(jp, jp.depth > 0 ? (int)jst[jp.depth - 1] : -1);
    }
  } else if (front >= 0 && tok < V) {
    bool eog = false;
    for (int k = 0; k < d.n_eog; k++) eog |= d.eog[k] == (int32_t)tok;
    if (eog) {
      allowed = (g.flags[front] & BL_GS_COMPLETE) && !sp.ignore_eos;
    } else {
      const uint32_t o0 = d.voff[tok], o1 = d.voff[tok + 1];
      const uint8_t *b = d.vblob + o0;
      int32_t st = bl_gw_walk(g, pos, front, [&](int i) { return (uint32_t)b[i]; }, (int)(o1 - o0));
      allowed = st >= 0;
      ambig = st == BL_GT_AMBIG;
    }
  }
  const unsigned long long bm = __ballot(allowed);
  const unsigned long long am = __ballot(ambig);
  const int64_t words = 2 * (((int64_t)V + 63) / 64);
  if (lane == 0) {
    const int64_t wi = (tok >> 6) * 2; /* lane 0 holds a multiple of 64 */
    if (wi < words) {
      d.gmask[(int64_t)row * words + wi] = (uint32_t)bm;
      d.gmask[(int64_t)row * words + wi + 1] = (uint32_t)(bm >> 32);
    }
    if (am) atomicOr(&d.gamb[row], js ? 2 : 1); /* 2: a JSON walk outgrew its stack overlay */
  }
  if (js && blockIdx.x == 0 && t == 0) {
    /* should_stop (src/server.br:266-269); a slot stack past its capacity leaves the row undecided */
    const int top = jp.depth > 0 ? (int)jst[jp.depth - 1] : -1;
    d.gstat[row] = bl_js_complete(jp, top) && !sp.ignore_eos ? BL_GR_FORCED : 0;
    if (jp.dead == 2) atomicOr(&d.gamb[row], 2);
  }
  if (!js && blockIdx.x == 0 && t == 0) {
    int st = 0;
    if (front == BL_GT_AMBIG) st |= BL_GR_FAMBIG;
    else if (front < 0) st |= BL_GR_DEAD;
    else if ((g.flags[front] & BL_GS_COMPLETE) && !(g.flags[front] & BL_GS_CONTINUE) && !sp.ignore_eos)
      st |= BL_GR_FORCED;
    d.gstat[row] = st;
  }
  if (!with_values) return;
  /* allowed maximum of this block, lowest index, and its multiplicity */
  float m = BL_NEG_INF;
  int mi = 0x7fffffff;
  const float v = allowed ? bl_row_value(d, sp, rows, row, slot, logits, ld, (int32_t)tok) : BL_NEG_INF;
  if (allowed) {
    m = v;
    mi = (int)tok;
  }
  block_argmax<BL_GM_THREADS>(m, mi, red_m, red_i);
  const bool eq = allowed && v == m;
  int n_eq = __popcll(__ballot(eq));
  if (lane == 0) red_n[w] = n_eq;
  __syncthreads();
  if (t == 0) {
    int tot = 0;
    for (int k = 0; k < BL_GM_THREADS / 64; k++) tot += red_n[k];
    const int64_t o = (int64_t)row * d.gm_blocks + blockIdx.x;
    d.gm_max[o] = m;
    d.gm_arg[o] = mi;
    d.gm_eq[o] = tot;
  }
}

/* ------------------------------------------------------------------ K3: per-row selection */
#define SEL_NW (BL_SEL_THREADS / 64)


__device__ __forceinline__ void bitonic_desc(uint64_t *s, int P) {
  for (int k = 2; k <= P; k <<= 1)
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < P; i += blockDim.x) {
        int ixj = i ^ j;
        if (ixj > i) {
          uint64_t a = s[i], b = s[ixj];
          bool desc = (i & k) == 0;
          if (desc ? (a < b) : (a > b)) {
            s[i] = b;
            s[ixj] = a;
          }
        }
      }
      __syncthreads();
    }
}

/* Phase A over a list of n terms term(val(j)), records into `recs`, approximate sums through `gsum`; the
 * terms are kept in `tbuf` for the walks. A record composes only the predicted binade's variant when the
 * float running sum before its group, g*64 terms, is within g*64*2^-24 (recursive summation bound, with
 * a 1% margin) of the approximate prefix and that interval lies in one binade. */
template <class ValF, class TermF>
__device__ __forceinline__ void block_records(int64_t n, ValF val, TermF term, bl_grec *recs, double *gsum, float *tbuf) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t G = (n + 63) / 64;
  /* each loop loads the next group's inputs before this group's stores: global stores share the
   * in-order load counter, so a load issued after a store would wait for the store as well */
  auto vload = [&](int64_t g) -> float {
    const int64_t j = g * 64 + lane;
    return g < G && j < n ? val(j) : 0.0f;
  };
  float vn = vload(w);
  for (int64_t g = w; g < G; g += SEL_NW) {
    const float vc = vn;
    vn = vload(g + SEL_NW);
    const bool in = g * 64 + lane < n;
    const float a = in ? term(vc) : 0.0f;
    if (in) tbuf[g * 64 + lane] = a;
    const double sg = bl_wave_sum_d((double)a);
    if (lane == 0) gsum[g] = sg;
  }
  __syncthreads();
  if (w == 0) {
    double run = 0.0;
    for (int64_t g0 = 0; g0 < G; g0 += 64) {
      int64_t g = g0 + lane;
      double v = g < G ? gsum[g] : 0.0;
      double ex = bl_wave_excl_scan_d(v, lane);
      double tot = __shfl(ex + v, 63, 64);
      if (g < G) gsum[g] = run + ex;
      run += tot;
    }
  }
  __syncthreads();
  /* a group's terms were stored by this same lane */
  auto aload = [&](int64_t g) -> float {
    const int64_t j = g * 64 + lane;
    return g < G && j < n ? tbuf[j] : 0.0f;
  };
  float an = aload(w);
  double sn = w < G ? gsum[w] : 0.0;
  for (int64_t g = w; g < G; g += SEL_NW) {
    const float a = an;
    const double sc = sn;
    an = aload(g + SEL_NW);
    sn = g + SEL_NW < G ? gsum[g + SEL_NW] : 0.0;
    const double margin = (double)(g * 64) * 0x1.02p-24 + 0x1p-40;
    bl_grec r = bl_group_record_pred(a, sc, margin, lane);
    if (lane == 0) recs[g] = r;
  }
  __syncthreads();
}

/* the fast normaliser's working set */
struct sel_norm {
  int32_t bE[BL_STAGE_B];              /* each block's binade, BL_E_NONE when not composable as a whole */
  bl_inc bV[BL_STAGE_B];               /* each block's composed automaton */
  float terms[BL_CRIT_MAX * 64];       /* the critical groups' terms */
  bl_inc cp[BL_CRIT_MAX * 64];         /* their prefix compositions at the predicted start binade */
  bl_inc cs[BL_CRIT_MAX * 64];         /* their suffix compositions at the predicted end binade */
  bl_grec1 blk[BL_CRIT_MAX * (BL_EB / 64)]; /* the group records of each critical group's block */
  int ce0[BL_CRIT_MAX], ce1[BL_CRIT_MAX]; /* those binades */
  int eg[BL_CRIT_MAX], epos[BL_CRIT_MAX]; /* the entries' groups, and their positions in group order */
  int crit[BL_CRIT_MAX];               /* critical groups, ascending */
  int r_E[BL_CRIT_MAX + 1];            /* runs between them: predicted binade */
  int r_st[BL_CRIT_MAX + 1];           /* 0 empty, 1 composed in one binade, 2 not composable */
  bl_inc r_f[BL_CRIT_MAX + 1];         /* composed automaton */
  int cw[SEL_NW];
  int ncrit;                           /* critical groups kept (at most BL_CRIT_MAX) */
  float S;                             /* the normaliser */
};
/* a sampled row's ranked candidate list */
struct sel_cand {
  uint64_t keys[BL_LDS_SORT];          /* the merged top-K keys, or the sorted full-vocabulary candidates */
  uint64_t tmp[BL_RANK_MAX];           /* full-vocabulary candidates before ranking by counting */
  bl_grec recs[BL_LDS_SORT / 64];
  double gsum[BL_LDS_SORT / 64];
};
/* the bucket sort of a long full-vocabulary list keeps the region offsets, then a tile of the bucketed
 * list, in the normaliser's LDS (free until norm_prep) */
#define BL_BOFF_BYTES (((BL_MAX_CHUNKS * BL_SUBS + 1) * 4 + 15) / 16 * 16)
#define BL_RTILE 4096 /* keys per rank tile */
#define BL_SPLIT_TIES 8 /* halfway tail terms a plain draw's head/tail split resolves */
#define BL_SPLIT_HEAD_MAX 2048 /* longest head the split ranks (its sum is added by one wavefront) */
#define BL_CAND_U 8   /* candidate loads in flight per lane */
static_assert(BL_BOFF_BYTES + BL_RTILE * 8 <= sizeof(sel_norm), "rank tile");
static_assert(BL_RTILE % BL_SEL_THREADS == 0, "rank tile");
/* the draw of a ranked list: the chosen position (-2: a cut would need a candidate past the materialised
 * list), the drawn range [first, cut) and its renormalised sum, whose terms the list's term array holds
 * from `first` (src/sampling.br:576-607) */
struct sel_draw {
  int pos, first, cut;
  float S;
};

struct sel_shared {
  sel_norm n; /* both live at once: the normaliser's chain runs beside the draw */
  sel_cand c;
  uint64_t rng_out;                    /* the RNG state after a draw */
  float ser_e[BL_SERIAL_MAX];          /* short-list terms exp(v - v0) */
  float ser_r[BL_SERIAL_MAX];          /* short-list terms exp((v - v0) / T), from the draw's first candidate */
  float ser_v[BL_SERIAL_MAX];          /* short-list values */
  int16_t ser_o[BL_SERIAL_MAX];        /* after the typical filter: a kept candidate's list position */
  sel_draw draw;                        /* the draw's range and sum */
  float fres[8];
  int ires[8];
  float red_m[SEL_NW];
  int red_i[SEL_NW];
  int32_t eog[BL_EOG_LDS];             /* the first end-of-generation ids */
  uint64_t mkeys[BL_KSEL_MAX];         /* the merged top-K keys */
  uint64_t mtau;                       /* the merge's lower bound on the K-th key */
  int mcnt;                            /* the merge's survivors */
  uint64_t etab[BL_EXP2_N];            /* expf's 2^(i/32) table (a global table read is a dependent load) */
  double ltab[32];                     /* logf's (1/c, log c) table */
  float tns_thr;                       /* top-n-sigma's threshold */
  int tns_st;                          /* its sigma undecided */
  int split_h;                         /* a plain draw's last ranked bucket */
  float split_s;                       /* the ranked head's exact sum */
  int split_nt;                        /* its tail's terms halfway between multiples of u: count, */
  uint32_t split_par;                  /* parities of the other tail terms before each, */
  uint64_t split_tk[BL_SPLIT_TIES];    /* keys, */
  double split_tf[BL_SPLIT_TIES];      /* floor(t / u), */
  uint32_t split_ti[BL_SPLIT_TIES];    /* the u-multiples each adds */
  int split_cb;                        /* a draw in the tail: u-multiples before its bucket, */
  int split_ne;                        /* that bucket's candidates, */
  uint64_t split_key;                  /* the drawn key */
};
/* expf and logf through the selection's LDS copies of their tables */
#define SEL_EXPF(x) bl_expf_tab((x), [&](uint32_t i_) { return sh.etab[i_]; })
#define SEL_LOGF(x) bl_logf_tab((x), [&](int j_) { return sh.ltab[j_]; })

/* sample_candidates_with_probs (src/sampling.br:490-607) for T > 0: the stages without a device path, and
 * a min_keep that reaches past the materialised list, leave the row unsupported */
__device__ __forceinline__ bool ranked_supported(const bl_slot_dev &sp, int64_t n_list, int64_t n_logical,
                                                 int64_t &keep) {
  keep = sp.min_keep > 1 ? sp.min_keep : 1;
  if (keep > n_logical) keep = n_logical;
  return !(keep > n_list);
}

/* a short ranked list (n_list <= BL_SERIAL_MAX), by every thread: the values, the terms exp(v - v0) of
 * the untempered softmax (when formed) and exp((v - v0) / T) of the draw */
template <class ValF>
__device__ __forceinline__ void ranked_terms(const bl_slot_dev &sp, ValF val, int64_t n_list, sel_shared &sh) {
  const float T = sp.temperature;
  const bool filt = bl_probs_on(sp);
  const float v0 = val(0);
  for (int j = threadIdx.x; j < n_list; j += BL_SEL_THREADS) {
    const float x = val(j);
    sh.ser_v[j] = x;
    sh.ser_e[j] = filt ? SEL_EXPF(x - v0) : 0.0f;
    const float dd = x - v0;
    const float q = dd / T;
    sh.ser_r[j] = SEL_EXPF(q);
  }
}

/* lane k's float as a wavefront-uniform value */
__device__ __forceinline__ float sel_rl(float x, int k) {
  return bl_u2f((uint32_t)__builtin_amdgcn_readlane((int)bl_f2u(x), k));
}

/* ... then the reference's sequential float32 loops over those terms, by one wavefront: softmax sum, top-p
 * prefix, min-p cut, XTC, tempered sum and the draw (src/sampling.br:505-607). Each loop's per-term work
 * (a division, a logarithm, a comparison) runs in the lanes, 64 terms at a time; the running sums add the
 * lanes' values in list order, every lane computing the same sum, so they are the reference's float32
 * sums. *rng_out = the state after the draw (written by lane 0) */
__device__ __forceinline__ sel_draw ranked_serial(const bl_slot_dev &sp, int n, int64_t n_logical, int64_t keep, uint64_t rng,
                                 int rng_skip, bool pre, float S_whole, sel_shared &sh, uint64_t *rng_out) {
  const int lane = threadIdx.x & 63;
  const float *ser_e = sh.ser_e, *ser_v = sh.ser_v;
  float *ser_r = sh.ser_r;
  constexpr int NBAT = BL_SERIAL_MAX / 64;
  float pv[NBAT]; /* the draw's running sum after term b*64 + lane, in batch b (when kept: have_p) */
  const bool xtc = bl_xtc_on(sp);
  const bool filt = bl_probs_on(sp);
  int64_t cut = n_logical;
  bool unsup = false;
  float sum_exp = 0.0f;
  /* term j of a batch: lane j - b0 */
  auto at = [&](const float *arr, int j) { return j < n ? arr[j] : 0.0f; };
  /* without XTC or a dynamic temperature the draw's terms run from position 0 at T: their running sums
   * (the tempered sum's and the draw's walk, the same float additions) are kept in pv, formed beside the
   * softmax sum as a second chain of additions; the tempered sum is then one entry and the draw a ballot */
  const bool pfx = !xtc && !(sp.dynatemp_range > 0.0f) && !pre;
  bool have_p = false;
#pragma unroll
  for (int b = 0; b < NBAT; b++) pv[b] = 0.0f;
  if (filt) {
    /* `pre`: ser_e already holds the probabilities (after the typical filter), divided here by 1 */
    if (pre) {
      sum_exp = 1.0f;
    } else {
      float tp = 0.0f;
#pragma unroll
      for (int b = 0; b < NBAT; b++) {
        const int b0 = b * 64;
        if (b0 >= n) break;
        const float e = at(ser_e, b0 + lane);
        const float r = pfx ? at(ser_r, b0 + lane) : 0.0f;
        const int m = n - b0 < 64 ? n - b0 : 64;
        float mine = 0.0f;
        for (int k = 0; k < m; k++) {
          sum_exp += sel_rl(e, k);
          if (pfx) {
            tp += sel_rl(r, k);
            mine = lane == k ? tp : mine;
          }
        }
        pv[b] = mine;
      }
      have_p = pfx;
    }
    if (sp.top_p < 1.0f) {
      float cum = 0.0f;
      bool done = false;
      for (int b0 = 0; b0 < n && !done; b0 += 64) {
        const float pj = at(ser_e, b0 + lane) / sum_exp;
        const int m = n - b0 < 64 ? n - b0 : 64;
        for (int k = 0; k < m; k++) {
          cum += sel_rl(pj, k);
          const int j = b0 + k;
          if (j >= keep - 1 && cum >= sp.top_p) {
            cut = j + 1;
            done = true;
            break;
          }
        }
      }
    }
    if (sp.min_p > 0.0f) {
      const float p0 = ser_e[0] / sum_exp;
      const float threshold = p0 * sp.min_p;
      const int64_t lim = cut < n ? cut : n;
      int64_t first_small = -1;
      for (int64_t b0 = keep; b0 < lim && first_small < 0; b0 += 64) {
        const int64_t j = b0 + lane;
        const bool small = j < lim && ser_e[j] / sum_exp < threshold;
        const unsigned long long bm = __ballot(small);
        if (bm) first_small = b0 + __ffsll((long long)bm) - 1;
      }
      if (first_small < 0) {
        if (lim < cut) {
          /* the next, unmaterialised candidate is below 2^-25 of the top one */
          if (threshold <= p0 * 5.9604645e-8f) unsup = true;
          first_small = lim;
        } else {
          first_small = cut;
        }
      }
      cut = keep > first_small ? keep : first_small;
    }
  }
  uint64_t st = rng;
  for (int k = 0; k < rng_skip; k++) st = bl_xorshift(st);
  int first = 0;
  if (xtc && cut >= 2) {
    const float chance = bl_rng_f32(&st);
    if (chance <= sp.xtc_probability) {
      /* the sum of the probabilities before the cut, then the last of the leading run at or above the
       * threshold (candidates past the materialised list are below it, by the candidate span) */
      const int lim = (int)(cut < n ? cut : n);
      float xs = 0.0f;
      for (int b0 = 0; b0 < lim; b0 += 64) {
        const float pj = (b0 + lane < lim ? ser_e[b0 + lane] : 0.0f) / sum_exp;
        const int m = lim - b0 < 64 ? lim - b0 : 64;
        for (int k = 0; k < m; k++) xs += sel_rl(pj, k);
      }
      int64_t pos_last = 0;
      bool ended = false;
      for (int b0 = 0; b0 < lim && !ended; b0 += 64) {
        const int j = b0 + lane;
        const bool stop = j < lim && !((ser_e[j] / sum_exp) / xs >= sp.xtc_threshold);
        const unsigned long long bm = __ballot(stop);
        if (bm) {
          const int f = b0 + __ffsll((long long)bm) - 1;
          if (f > 0) pos_last = f - 1;
          ended = true;
        } else {
          pos_last = (b0 + 64 < lim ? b0 + 64 : lim) - 1;
        }
      }
      if (pos_last > 0 && cut - pos_last >= keep) first = (int)pos_last;
    }
  }
  const int n_eff = (int)(cut < n ? cut : n);
  /* dynamic_temperature (src/sampling.br:467-488): the entropy of the renormalised probabilities over
   * [first, cut) against that of a uniform choice, raised to the exponent */
  float Teff = sp.temperature;
  if (sp.dynatemp_range > 0.0f && cut - first > 1) {
    if (cut > n) {
      unsup = true; /* the entropy would need candidates past the materialised list */
    } else {
      float ss = 0.0f;
      for (int b0 = first; b0 < n_eff; b0 += 64) {
        const float pj = (b0 + lane < n_eff ? ser_e[b0 + lane] : 0.0f) / sum_exp;
        const int m = n_eff - b0 < 64 ? n_eff - b0 : 64;
        for (int k = 0; k < m; k++) ss += sel_rl(pj, k);
      }
      float ent = 0.0f;
      for (int b0 = first; b0 < n_eff; b0 += 64) {
        const float q = ((b0 + lane < n_eff ? ser_e[b0 + lane] : 0.0f) / sum_exp) / ss;
        const float tq = q > 0.0f ? q * bl_logf(q) : 0.0f;
        const int m = n_eff - b0 < 64 ? n_eff - b0 : 64;
        for (int k = 0; k < m; k++) {
          if (sel_rl(q, k) > 0.0f) ent -= sel_rl(tq, k);
        }
      }
      const float maxe = bl_logf((float)(cut - first));
      const float ne = bl_powf(ent / maxe, sp.dynatemp_exponent);
      const float T = sp.temperature, rg = sp.dynatemp_range;
      const float tmin = T > rg ? T - rg : 0.0f, tmax = T + rg;
      Teff = tmin + (tmax - tmin) * ne;
    }
  }
  sel_draw r;
  if (!(Teff > 0.0f)) {
    /* no draw: the first candidate, probability 1 (src/sampling.br:581-582) */
    if (lane == 0) {
      ser_r[first] = 1.0f;
      *rng_out = st;
    }
    r.pos = unsup ? -2 : first;
    r.first = first;
    r.cut = first + 1;
    r.S = 1.0f;
    return r;
  }
  if (first > 0 || Teff != sp.temperature) {
    /* the draw's terms from the first candidate at the effective temperature */
    const float vf = ser_v[first];
    for (int j = first + lane; j < n_eff; j += 64) {
      const float dd = ser_v[j] - vf;
      const float q = dd / Teff;
      ser_r[j] = SEL_EXPF(q);
    }
  }
  float S = 0.0f;
  if (have_p) { /* first = 0: the running sums are pv's */
    const int last = n_eff - 1;
#pragma unroll
    for (int b = 0; b < NBAT; b++)
      if (last >= 0 && b == (last >> 6)) S = sel_rl(pv[b], last & 63);
  } else if (pfx) { /* the same with the terms added here (no softmax sum was formed): first = 0 */
#pragma unroll
    for (int b = 0; b < NBAT; b++) {
      const int b0 = b * 64;
      if (b0 >= n_eff) break;
      const float e = b0 + lane < n_eff ? ser_r[b0 + lane] : 0.0f;
      const int m = n_eff - b0 < 64 ? n_eff - b0 : 64;
      float mine = 0.0f;
      for (int k = 0; k < m; k++) {
        S += sel_rl(e, k);
        mine = lane == k ? S : mine;
      }
      pv[b] = mine;
    }
    have_p = true;
  } else {
    for (int b0 = first; b0 < n_eff; b0 += 64) {
      const float e = b0 + lane < n_eff ? ser_r[b0 + lane] : 0.0f;
      const int m = n_eff - b0 < 64 ? n_eff - b0 : 64;
      for (int k = 0; k < m; k++) S += sel_rl(e, k);
    }
  }
  if (S_whole > 0.0f) S = S_whole; /* the list is the head of a longer one whose sum is known */
  const float target = bl_rng_f32(&st) * S;
  int64_t f = -1;
  if (have_p) { /* the first position whose running sum reaches the target (the sums never decrease) */
#pragma unroll
    for (int b = 0; b < NBAT; b++) {
      const int b0 = b * 64;
      if (b0 < n_eff) {
        const unsigned long long bm = __ballot(b0 + lane < n_eff && pv[b] >= target);
        if (bm && f < 0) f = b0 + __ffsll((long long)bm) - 1;
      }
    }
  } else {
    float run = 0.0f;
    for (int b0 = first; b0 < n_eff && f < 0; b0 += 64) {
      const float e = b0 + lane < n_eff ? ser_r[b0 + lane] : 0.0f;
      const int m = n_eff - b0 < 64 ? n_eff - b0 : 64;
      for (int k = 0; k < m; k++) {
        run += sel_rl(e, k);
        if (run >= target) {
          f = b0 + k;
          break;
        }
      }
    }
  }
  if (lane == 0) *rng_out = st;
  r.pos = unsup ? -2 : (int)(f >= 0 ? f : cut - 1);
  r.first = first;
  r.cut = (int)cut;
  r.S = S;
  return r;
}

/*
 * typical_filter (src/sampling.br:424-465) on a complete short list, by the block. The probabilities
 * p = e / sum_exp and the entropy -sum p ln p are the reference's float loops (the sums by one thread,
 * in order); candidates are taken by distance |-ln p - entropy|, ties by position (the loop's strict
 * `<`), until their probabilities, added in that order, reach typical_p and min_keep is met. The kept
 * candidates, in list order, replace the short list: values, probabilities in ser_e (ranked_serial then
 * divides by 1: the later stages read the unrenormalised probabilities) and the draw's terms from the
 * new first value; ser_o maps a kept position to its list position. Returns the kept count. On a
 * full-vocabulary rank a cut between equal distances picks among equal values by the heap's order:
 * reported as a tie.
 */
__device__ __forceinline__ int typical_filter(const bl_slot_dev &sp, int n, bool full, sel_shared &sh, int &status) {
  const int t = threadIdx.x;
  float *tp = reinterpret_cast<float *>(&sh.n); /* the normaliser's LDS is free until norm_prep */
  float *tq = tp + BL_SERIAL_MAX;
  float *tl = tq + BL_SERIAL_MAX;
  uint64_t *tk = reinterpret_cast<uint64_t *>(tl + BL_SERIAL_MAX);
  int *ord = reinterpret_cast<int *>(tk + BL_SERIAL_MAX);
  __syncthreads(); /* the short list's terms */
  if (t == 0) {
    float se = 0.0f;
    for (int j = 0; j < n; j++) se += sh.ser_e[j];
    sh.fres[4] = se;
  }
  __syncthreads();
  const float se = sh.fres[4];
  for (int j = t; j < n; j += BL_SEL_THREADS) {
    const float p = sh.ser_e[j] / se;
    const float l = p > 0.0f ? bl_logf(p) : 0.0f;
    tp[j] = p;
    tl[j] = l;
    tq[j] = p * l;
  }
  __syncthreads();
  if (t == 0) {
    float ent = 0.0f;
    for (int j = 0; j < n; j++)
      if (tp[j] > 0.0f) ent -= tq[j];
    sh.fres[5] = ent;
  }
  __syncthreads();
  const float ent = sh.fres[5];
  for (int j = t; j < n; j += BL_SEL_THREADS) {
    const float dist = fabsf(-tl[j] - ent);
    tk[j] = (uint64_t)(tp[j] > 0.0f ? bl_f2u(dist) : 0xffffffffu) << 32 | (uint32_t)j;
  }
  __syncthreads();
  for (int j = t; j < n; j += BL_SEL_THREADS) {
    const uint64_t k = tk[j];
    int r = 0;
    for (int q = 0; q < n; q++) r += tk[q] < k ? 1 : 0;
    ord[r] = j;
  }
  __syncthreads();
  if (t == 0) {
    const int req = sp.min_keep > 1 ? sp.min_keep : 1;
    float cum = 0.0f;
    int m = 0;
    while (m < n && (cum < sp.typical_p || m < req)) {
      const int j = ord[m];
      if (!(tp[j] > 0.0f)) break; /* nothing selectable is left */
      cum += tp[j];
      m++;
    }
    sh.ires[7] = m;
  }
  __syncthreads();
  const int m = sh.ires[7];
  const uint64_t klast = tk[ord[m - 1]];
  if (full && m < n && (uint32_t)(tk[ord[m]] >> 32) == (uint32_t)(klast >> 32)) status |= BL_SE_TIE; /* uniform */
  /* compaction in list order (one candidate per thread: n <= BL_SERIAL_MAX < the block) */
  const bool sel = t < n && tk[t] <= klast;
  int ni = 0;
  if (sel)
    for (int q = 0; q < t; q++) ni += tk[q] <= klast ? 1 : 0;
  const float v = t < n ? sh.ser_v[t] : 0.0f, p = t < n ? tp[t] : 0.0f;
  __syncthreads();
  if (sel) {
    sh.ser_v[ni] = v;
    sh.ser_e[ni] = p;
    sh.ser_o[ni] = (int16_t)t;
  }
  __syncthreads();
  const float v0 = sh.ser_v[0], T = sp.temperature;
  for (int j = t; j < m; j += BL_SEL_THREADS) {
    const float dd = sh.ser_v[j] - v0;
    const float q = dd / T;
    sh.ser_r[j] = SEL_EXPF(q);
  }
  __syncthreads();
  return m;
}

/*
 * A long ranked list (more than BL_SERIAL_MAX entries) by the whole block: the sequential sums of
 * sample_candidates_with_probs (src/sampling.br:490-607) through the exact-sum records. n_list entries are
 * materialised; n_logical >= n_list is the reference's candidate count, the entries past n_list being too
 * small to change any float32 sum. Returns the draw (pos -1 with `status` set on failure); `tbuf` then
 * holds the draw's terms from its first candidate (tbuf[j - first]).
 */
template <class ValF>
__device__ __forceinline__ sel_draw sample_ranked_long(const bl_slot_dev &sp, ValF val, int64_t &n_list, int64_t n_logical,
                                      int64_t keep, uint64_t &rng, int rng_skip, float S_whole, bl_grec *recs,
                                      double *gsum, float *tbuf, sel_shared &sh, int &status, uint64_t *keys_w = nullptr,
                                      int32_t *tmerged = nullptr, int32_t *trank = nullptr) {
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const float T = sp.temperature;
  const float v0 = val(0);
  const bool xtc = bl_xtc_on(sp);
  int64_t cutoff = n_logical;
  float sum_exp = 1.0f;
  auto termPv = [&](float v) { return SEL_EXPF(v - v0) / sum_exp; };
  auto termS = [&](int64_t j) { return tbuf[j]; };
  sel_draw out;
  out.pos = -1;
  out.first = 0;
  out.cut = 0;
  out.S = 0.0f;
  if (bl_probs_on(sp)) {
    block_records(n_list, val, [&](float v) { return SEL_EXPF(v - v0); }, recs, gsum, tbuf);
    if (w == 0) {
      float S;
      bl_seq_walk(n_list, termS, [&](int64_t g) { return recs[g]; }, false, 0.0f, 0, S, lane);
      if (lane == 0) sh.fres[0] = S;
    }
    __syncthreads();
    sum_exp = sh.fres[0];
    __syncthreads();
    if (keys_w) {
      /* typical_filter (src/sampling.br:424-465) over the whole list (every value whose term exp(v - v0) is
       * not 0; the later ones have probability 0 and take no part). Along the list -ln p only grows, so the
       * distance |-ln p - H| falls until -ln p reaches H (positions [0, m)) and grows after it ([m, n)): the
       * order of the selection (distance, then position) merges the two runs, each element's place found by
       * binary search in the other run (and, in the falling run, among its equal distances). The probabilities
       * added in that order reach typical_p (and min_keep) at the walk's stop; the kept entries are compacted
       * in list order, the list's first value and sum staying those of the whole list */
      int64_t lo = 0, hi = n_list; /* n = first position whose probability is 0 */
      while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (termPv(val(mid)) > 0.0f) lo = mid + 1;
        else hi = mid;
      }
      const int64_t n = lo;
      block_records(n, val, [&](float v) {
        const float q = termPv(v);
        return q > 0.0f ? -(q * bl_logf(q)) : 0.0f;
      }, recs, gsum, tbuf);
      if (w == 0) {
        float S;
        bl_seq_walk(n, termS, [&](int64_t g) { return recs[g]; }, false, 0.0f, 0, S, lane);
        if (lane == 0) sh.fres[3] = S;
      }
      __syncthreads();
      const float H = sh.fres[3];
      __syncthreads();
      /* tbuf[j] = -ln p_j - H (its magnitude is the reference's distance) */
      for (int64_t j = t; j < n; j += blockDim.x) tbuf[j] = -bl_logf(termPv(val(j))) - H;
      __syncthreads();
      lo = 0;
      hi = n;
      while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (tbuf[mid] < 0.0f) lo = mid + 1;
        else hi = mid;
      }
      const int64_t m = lo;
      for (int64_t j = t; j < n; j += blockDim.x) {
        const float dj = fabsf(tbuf[j]);
        int64_t rank;
        if (j >= m) {
          /* rising run: its own earlier entries, and the falling run's entries at distance <= dj (a suffix) */
          int64_t a = 0, b = m;
          while (a < b) {
            const int64_t c = (a + b) >> 1;
            if (fabsf(tbuf[c]) <= dj) b = c;
            else a = c + 1;
          }
          rank = (j - m) + (m - a);
        } else {
          /* falling run: its entries at a smaller distance (after its run of distance dj), its equal ones
           * before j, and the rising run's entries at a smaller distance (a prefix) */
          int64_t a = 0, b = m; /* first position of distance dj */
          while (a < b) {
            const int64_t c = (a + b) >> 1;
            if (fabsf(tbuf[c]) <= dj) b = c;
            else a = c + 1;
          }
          const int64_t first_eq = a;
          a = j;
          b = m; /* first position past the run of distance dj */
          while (a < b) {
            const int64_t c = (a + b) >> 1;
            if (fabsf(tbuf[c]) < dj) b = c;
            else a = c + 1;
          }
          const int64_t past_eq = a;
          a = m;
          b = n; /* first rising position at distance >= dj */
          while (a < b) {
            const int64_t c = (a + b) >> 1;
            if (fabsf(tbuf[c]) < dj) a = c + 1;
            else b = c;
          }
          rank = (m - past_eq) + (j - first_eq) + (a - m);
        }
        tmerged[rank] = (int32_t)j;
        trank[j] = (int32_t)rank;
      }
      __syncthreads();
      /* the probabilities in selection order, added until they reach typical_p with at least min_keep */
      const int64_t req = keep > 1 ? keep : 1;
      block_records(n, [&](int64_t k) { return val(tmerged[k]); }, termPv, recs, gsum, tbuf);
      if (w == 0) {
        float S;
        const int f = bl_seq_walk(n, termS, [&](int64_t g) { return recs[g]; }, true, sp.typical_p, req - 1, S, lane);
        if (lane == 0) sh.ires[0] = f;
      }
      __syncthreads();
      const int f = sh.ires[0];
      const int64_t nk = f >= 0 ? f + 1 : n;
      /* equal values on both sides of the stop: which of them the reference keeps is the heap's order */
      if (nk < n && val(tmerged[nk - 1]) == val(tmerged[nk])) status |= BL_SE_TIE;
      __syncthreads();
      /* stable compaction of the kept entries to the list's front, a tile at a time */
      int64_t off = 0;
      for (int64_t base = 0; base < n; base += blockDim.x) {
        const int64_t j = base + t;
        const uint64_t k = j < n ? keys_w[j] : 0ull;
        const int fl = j < n && trank[j] < nk ? 1 : 0;
        const int incl = bl_wscan_add(fl, lane);
        if (lane == 63) sh.red_i[w] = incl;
        __syncthreads();
        int before = incl - fl, tot = 0;
        for (int q = 0; q < SEL_NW; q++) {
          if (q < w) before += sh.red_i[q];
          tot += sh.red_i[q];
        }
        if (fl) keys_w[off + before] = k;
        off += tot;
        __syncthreads();
      }
      n_list = nk;
      cutoff = nk;
      if (keep > nk) keep = nk;
      if (status) return out;
    }
    if (sp.top_p < 1.0f) {
      block_records(n_list, val, termPv, recs, gsum, tbuf);
      if (w == 0) {
        float S;
        int f = bl_seq_walk(n_list, termS, [&](int64_t g) { return recs[g]; }, true, sp.top_p, keep - 1, S, lane);
        if (lane == 0) sh.ires[0] = f;
      }
      __syncthreads();
      if (sh.ires[0] >= 0) cutoff = sh.ires[0] + 1;
      __syncthreads();
    }
    if (sp.min_p > 0.0f) {
      const float p0 = termPv(v0);
      const float threshold = p0 * sp.min_p;
      /* first j in [keep, cutoff) with probs[j] < threshold */
      if (t == 0) sh.ires[1] = 0x7fffffff;
      __syncthreads();
      int64_t lim = cutoff < n_list ? cutoff : n_list;
      for (int64_t j = keep + t; j < lim; j += blockDim.x)
        if (termPv(val(j)) < threshold) atomicMin(&sh.ires[1], (int)j);
      __syncthreads();
      int64_t first_small = sh.ires[1];
      if (first_small == 0x7fffffff) {
        if (lim < cutoff) {
          /* the next, unmaterialised candidate is below 2^-25 of the top one */
          if (threshold <= p0 * 5.9604645e-8f) status |= BL_SE_UNSUPPORTED;
          first_small = lim;
        } else {
          first_small = cutoff;
        }
      }
      cutoff = keep > first_small ? keep : first_small;
      __syncthreads();
    }
  }
  if (status) return out;
  /* the RNG after the rows drawn before this one, then XTC's chance (every thread) */
  uint64_t st = rng;
  for (int k = 0; k < rng_skip; k++) st = bl_xorshift(st);
  int64_t first = 0;
  if (xtc && cutoff >= 2) {
    const float chance = bl_rng_f32(&st);
    if (chance <= sp.xtc_probability) {
      /* the sum of the probabilities before the cut (candidates past the list add nothing), then the
       * last of the leading run at or above the threshold (past the list all are below it) */
      const int64_t nx = cutoff < n_list ? cutoff : n_list;
      block_records(nx, val, termPv, recs, gsum, tbuf);
      if (w == 0) {
        float S;
        bl_seq_walk(nx, termS, [&](int64_t g) { return recs[g]; }, false, 0.0f, 0, S, lane);
        if (lane == 0) {
          sh.fres[2] = S;
          sh.ires[1] = 0x7fffffff;
        }
      }
      __syncthreads();
      const float xs = sh.fres[2];
      for (int64_t j = t; j < nx; j += blockDim.x)
        if (!(tbuf[j] / xs >= sp.xtc_threshold)) atomicMin(&sh.ires[1], (int)j);
      __syncthreads();
      const int64_t ff = sh.ires[1] == 0x7fffffff ? nx : sh.ires[1];
      const int64_t pos_last = ff > 0 ? ff - 1 : 0;
      if (pos_last > 0 && cutoff - pos_last >= keep) first = pos_last;
      __syncthreads();
    }
  }
  const int64_t n_eff = cutoff < n_list ? cutoff : n_list;
  const int64_t m = n_eff - first;
  const float vf = val(first);
  auto valF = [&](int64_t j) { return val(first + j); };
  /* dynamic_temperature (src/sampling.br:467-488): the surviving probabilities' sum, then the entropy of
   * the renormalised ones (entropy -= q ln q adds the non-negative -(q ln q)), raised to the exponent */
  float Teff = T;
  if (sp.dynatemp_range > 0.0f && cutoff - first > 1) {
    if (cutoff > n_list) { /* the entropy would need candidates past the materialised list */
      status |= BL_SE_UNSUPPORTED;
      return out;
    }
    block_records(m, valF, termPv, recs, gsum, tbuf);
    if (w == 0) {
      float S;
      bl_seq_walk(m, termS, [&](int64_t g) { return recs[g]; }, false, 0.0f, 0, S, lane);
      if (lane == 0) sh.fres[3] = S;
    }
    __syncthreads();
    const float ss = sh.fres[3];
    __syncthreads();
    block_records(m, valF, [&](float v) {
      const float q = termPv(v) / ss;
      return q > 0.0f ? -(q * bl_logf(q)) : 0.0f;
    }, recs, gsum, tbuf);
    if (w == 0) {
      float S;
      bl_seq_walk(m, termS, [&](int64_t g) { return recs[g]; }, false, 0.0f, 0, S, lane);
      if (lane == 0) sh.fres[3] = S;
    }
    __syncthreads();
    const float ent = sh.fres[3];
    __syncthreads();
    const float maxe = bl_logf((float)(cutoff - first));
    const float ne = bl_powf(ent / maxe, sp.dynatemp_exponent);
    const float rg = sp.dynatemp_range;
    const float tmin = T > rg ? T - rg : 0.0f, tmax = T + rg;
    Teff = tmin + (tmax - tmin) * ne;
  }
  if (!(Teff > 0.0f)) {
    /* no draw: the first candidate, probability 1 (src/sampling.br:581-582) */
    if (t == 0) tbuf[0] = 1.0f;
    __syncthreads();
    rng = st;
    out.pos = (int)first;
    out.first = (int)first;
    out.cut = (int)first + 1;
    out.S = 1.0f;
    return out;
  }
  auto termRv = [&](float v) {
    float dd = v - vf;
    float q = dd / Teff;
    return SEL_EXPF(q);
  };
  block_records(m, valF, termRv, recs, gsum, tbuf);
  if (w == 0) {
    float S;
    bl_seq_walk(m, termS, [&](int64_t g) { return recs[g]; }, false, 0.0f, 0, S, lane);
    if (S_whole > 0.0f) S = S_whole; /* the list is the head of a longer one whose sum is known */
    float r01 = bl_rng_f32(&st);
    float target = r01 * S;
    float S2;
    int f = bl_seq_walk(m, termS, [&](int64_t g) { return recs[g]; }, true, target, 0, S2, lane);
    if (lane == 0) {
      sh.ires[2] = f >= 0 ? (int)(first + f) : (int)(cutoff - 1);
      sh.fres[1] = S;
      sh.rng_out = st;
    }
  }
  __syncthreads();
  int chosen = sh.ires[2];
  rng = sh.rng_out;
  out.S = sh.fres[1];
  __syncthreads();
  out.first = (int)first;
  out.cut = (int)cutoff;
  if (chosen >= n_list) {
    status |= BL_SE_UNSUPPORTED;
    return out;
  }
  out.pos = chosen;
  return out;
}

/*
 * sample_mirostat_v2 (src/sampling.br:663-674, draw_mirostat_prefix :643-659) and sample_mirostat_v1
 * (:676-700) over the full-vocabulary list, by the block: scaled values v/T, the softmax of exp(v/T - v0/T)
 * over every candidate (the terms past the list are below half an ulp of the sum), the prefix (v2: while
 * the surprise -ln p / ln 2 stays within mu; v1: the length predicted by a Zipf fit), the softmax and draw
 * over that prefix, and mu - eta (surprise - tau) for the slot (sh.fres[6]). `mk` is this thread's key of
 * the row's merged top-K list (v1 reads the first min(V, 100)).
 */
template <class ValF>
__device__ __forceinline__ sel_draw sample_mirostat(const bl_slot_dev &sp, ValF val, int64_t n_list, int64_t n_logical,
                                    uint64_t mk, uint64_t &rng, int rng_skip, bl_grec *recs, double *gsum,
                                    float *tbuf, sel_shared &sh, int &status) {
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const float T = sp.temperature;
  const float s0 = val(0) / T;
  auto termE = [&](float v) { return SEL_EXPF(v / T - s0); };
  auto termS = [&](int64_t j) { return tbuf[j]; };
  sel_draw out;
  out.pos = -1;
  out.first = 0;
  out.cut = 0;
  out.S = 0.0f;
  const bool v1 = sp.mirostat == 1;
  const int m1 = n_logical < 100 ? (int)n_logical : 100; /* v1's fitted ranks */
  if (v1 && t < m1) sh.ser_v[t] = ckey_v(mk);             /* short-list LDS: unused by these rows */
  /* softmax_prefix over the whole rank */
  block_records(n_list, val, termE, recs, gsum, tbuf);
  if (w == 0) {
    float S;
    bl_seq_walk(n_list, termS, [&](int64_t g) { return recs[g]; }, false, 0.0f, 0, S, lane);
    if (lane == 0) {
      sh.fres[0] = S;
      sh.ires[1] = 0x7fffffff;
    }
  }
  __syncthreads();
  const float total = sh.fres[0];
  const float ln2 = bl_logf(2.0f), mu = sp.mu;
  bool past;   /* the prefix runs past the list */
  int64_t cut; /* the prefix within the list */
  if (v1) {
    /* the fit (src/sampling.br:683-699): lane l of wavefront 0 forms pairs l and l + 64 of
     * t_i = ln((i + 2) / (i + 1)), b_i = ln(p_i / p_(i+1)); every lane then adds t_i b_i and t_i^2 in order */
    if (w == 0) {
      float a[2], q[2];
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const int i = lane + 64 * h;
        a[h] = q[h] = 0.0f;
        if (i < m1 - 1) {
          const float ti = SEL_LOGF((float)(i + 2) / (float)(i + 1));
          const float pi = termE(sh.ser_v[i]) / total, pn = termE(sh.ser_v[i + 1]) / total;
          const float bi = SEL_LOGF(pi / pn);
          a[h] = ti * bi;
          q[h] = ti * ti;
        }
      }
      float sa = 0.0f, sq = 0.0f;
#pragma unroll
      for (int h = 0; h < 2; h++)
#pragma unroll
        for (int l = 0; l < 64; l++)
          if (64 * h + l < m1 - 1) {
            sa += bl_u2f((uint32_t)__builtin_amdgcn_readlane((int)bl_f2u(a[h]), l));
            sq += bl_u2f((uint32_t)__builtin_amdgcn_readlane((int)bl_f2u(q[h]), l));
          }
      if (lane == 0) {
        const float s_hat = sa / sq;
        const float eps = s_hat - 1.0f;
        const float num = eps * bl_powf(2.0f, mu);
        const float den = 1.0f - bl_powf((float)n_logical, -eps);
        const float est = bl_powf(num / den, 1.0f / s_hat);
        /* `as int`: truncation, saturating, NaN to 0; then clamped to [1, V] */
        int64_t e = est != est ? 0 : est >= 0x1p63f ? INT64_MAX : est <= -0x1p63f ? INT64_MIN : (int64_t)est;
        if (e < 1) e = 1;
        if (e > n_logical) e = n_logical;
        sh.ires[1] = (int)e;
      }
    }
    __syncthreads();
    past = sh.ires[1] > n_list;
    cut = past ? n_list : sh.ires[1];
  } else {
    /* the cutoff: the first candidate whose surprise exceeds mu */
    for (int64_t j = t; j < n_list; j += BL_SEL_THREADS) {
      const float p = tbuf[j] / total;
      if (!((-bl_logf(p)) / ln2 <= mu)) atomicMin(&sh.ires[1], (int)j);
    }
    __syncthreads();
    past = sh.ires[1] == 0x7fffffff && n_list < n_logical;
    cut = sh.ires[1] == 0x7fffffff ? n_list : sh.ires[1];
    if (cut == 0) cut = 1;
  }
  __syncthreads();
  /* softmax_prefix over the cut, then the draw (draw_mirostat_prefix) */
  block_records(cut, val, termE, recs, gsum, tbuf);
  if (w == 0) {
    float S;
    bl_seq_walk(cut, termS, [&](int64_t g) { return recs[g]; }, false, 0.0f, 0, S, lane);
    if (lane == 0) sh.fres[2] = S;
  }
  __syncthreads();
  const float total2 = sh.fres[2];
  __syncthreads();
  block_records(cut, val, [&](float v) { return termE(v) / total2; }, recs, gsum, tbuf);
  uint64_t st = rng;
  for (int k = 0; k < rng_skip; k++) st = bl_xorshift(st);
  const float draw = bl_rng_f32(&st);
  if (w == 0) {
    float S2;
    const int f = bl_seq_walk(cut, termS, [&](int64_t g) { return recs[g]; }, true, draw, 0, S2, lane);
    if (lane == 0) sh.ires[2] = f;
  }
  __syncthreads();
  const int f = sh.ires[2];
  __syncthreads();
  if (f < 0 && past) { /* the default, last candidate of the prefix lies past the list */
    status |= BL_SE_UNSUPPORTED;
    return out;
  }
  const int64_t sel = f >= 0 ? f : cut - 1;
  const float nl = -bl_logf(tbuf[sel]);
  const float surprise = nl / ln2;
  const float dd = surprise - sp.mirostat_tau;
  const float tt = sp.mirostat_eta * dd;
  if (t == 0) sh.fres[6] = mu - tt;
  rng = st;
  out.pos = (int)sel;
  out.cut = (int)cut;
  out.S = 1.0f;
  return out;
}

/* wavefront-level resolution of the terms [start, 64) of one 64-term group from state (e, N): the group
 * crosses a binade (or its prediction failed), so its terms are added one at a time in float32 from the
 * exact running sum, as the reference's loop does (src/sampling.br:262-264). `a` is this lane's term and
 * `in` whether it exists (the existing terms are a prefix of the lanes). */
__device__ __forceinline__ void elem_resolve(float a, bool in, int &e, uint32_t &N, int lane, int start = 0) {
  (void)lane;
  const int n_in = __popcll(__ballot(in));
  float S = bl_make(e, N);
  /* unrolled: the broadcasts do not depend on the running sum and issue ahead of the adds */
#pragma unroll
  for (int j = 0; j < 64; j++) {
    const float x = bl_bcastf(a, j);
    if (j >= start && j < n_in) S = S + x;
  }
  bl_split(S, e, N);
}

/* groups [g_lo, g_hi) from the exact state (e, N), one wavefront: 64 group records per composed scan,
 * element level where a group crosses a binade or lacks the needed binade */
template <class TermF, class RecF>
__device__ void walk_groups(int64_t g_lo, int64_t g_hi, int64_t n, TermF term, RecF rec, int &e, uint32_t &N,
                            int lane) {
  int64_t g = g_lo;
  while (g < g_hi) {
    const int64_t gl = g + lane;
    bool valid = gl < g_hi;
    bl_inc f = bl_inc_ident();
    if (valid) {
      const bl_grec r = rec(gl);
      const int k = e - (r.E - 1);
      if (k >= 0 && k <= 2 && e >= BL_E_MIN) f = k == 0 ? r.v[0] : (k == 1 ? r.v[1] : r.v[2]); /* selects: no dynamic index into private memory */
      else valid = false;
    }
    const uint32_t Nend = bl_apply(bl_wave_scan(f, lane), N);
    const unsigned long long m = __ballot(!valid || Nend >= BL_N_TOP);
    const int first = m ? __ffsll((long long)m) - 1 : 64;
    if (first > 0) {
      N = bl_bcast(Nend, first - 1);
      g += first;
    }
    if (g >= g_hi) break;
    if (first == 64) continue;
    const int64_t j = g * 64 + lane;
    elem_resolve(j < n ? term(j) : 0.0f, j < n, e, N, lane);
    g += 1;
  }
}

/*
 * Exact index-order sum of exp(x[j] - M), j < V (logprob_normalizer, src/sampling.br:254-266), by the whole
 * block (norm_prep) and one wavefront (norm_chain). The exponent pass left, per 64-term group, the composed
 * automaton at the binade of its approximate start, per 1024-term block the groups where the sum may cross a
 * power of two ("critical") and, for a block without them, the block's composed automaton, and for each
 * critical group an entry with its terms, prefix compositions at the binade of its start, suffix
 * compositions at the binade of its end and its block's group records. The groups between two critical
 * groups form a run in one binade; the wavefronts compose the runs (edge groups from the entries, whole
 * blocks from the summaries). One wavefront then chains runs and critical groups: a run applies at once when
 * the exact state is in its binade and stays there; a critical group needs one ballot for the crossing, one
 * real float add and the suffix. Every prediction is checked on the exact state; a run or group whose
 * prediction fails is walked group by group and element by element (terms recomputed from the logits).
 * With more critical groups than BL_CRIT_MAX the whole row is walked that way.
 */
__device__ __forceinline__ void norm_prep(const bl_dev &d, int row, float M, sel_shared &sh, uint32_t m_pre, bl_grec1 br_pre,
                          int n_ent) {
  const int V = d.vocab, t = threadIdx.x, w = t >> 6, lane = t & 63;
  const int G = (V + 63) / 64, NB = d.nb;
  const bl_grec1 *rec =
      reinterpret_cast<const bl_grec1 *>(reinterpret_cast<const bl_grec *>(d.grec) + (int64_t)row * 2 * (V / 64 + 64));
  const bl_grec1 *brec = reinterpret_cast<const bl_grec1 *>(d.brec) + (int64_t)row * NB;
  const uint32_t *bcrit = d.bcrit + (int64_t)row * NB;
  const bl_crit *ent = d.crit + (int64_t)row * BL_CRIT_MAX;
  sel_norm &nm = sh.n;
  /* the entries to LDS in their order of arrival (slot i); nm.epos maps a critical group's rank to its slot */
  const int ne = n_ent < BL_CRIT_MAX ? n_ent : BL_CRIT_MAX;
  for (int idx = t; idx < ne * 64; idx += BL_SEL_THREADS) {
    const int i = idx >> 6, l = idx & 63;
    nm.terms[idx] = ent[i].terms[l];
    nm.cp[idx] = ent[i].cp[l];
    nm.cs[idx] = ent[i].cs[l];
    if (l < BL_EB / 64) nm.blk[i * (BL_EB / 64) + l] = ent[i].blk[l];
    if (l == 0) {
      nm.eg[i] = ent[i].g;
      nm.ce0[i] = ent[i].e0;
      nm.ce1[i] = ent[i].e1;
    }
  }
  /* 1. critical groups in order (a block-wide scan of the per-block counts); block summaries to LDS */
  int ncrit_all = 0;
  for (int b0 = 0; b0 < NB; b0 += BL_SEL_THREADS) {
    const int b = b0 + t;
    uint32_t m = 0u;
    if (b < NB) {
      m = b0 == 0 ? m_pre : bcrit[b]; /* the first BL_SEL_THREADS blocks were loaded by the caller */
      if (b < BL_STAGE_B) {
        const bl_grec1 br = b0 == 0 ? br_pre : brec[b];
        nm.bE[b] = br.E;
        nm.bV[b] = br.v;
      }
    }
    const int pc = __popc(m);
    const int inc = bl_wscan_add(pc, lane);
    if (lane == 63) nm.cw[w] = inc;
    __syncthreads();
    int off = ncrit_all + inc - pc, tot = 0;
    for (int q = 0; q < SEL_NW; q++) {
      if (q < w) off += nm.cw[q];
      tot += nm.cw[q];
    }
    while (m) {
      const int j = __ffs(m) - 1;
      m &= m - 1u;
      if (off < BL_CRIT_MAX) nm.crit[off] = b * (BL_EB / 64) + j;
      off++;
    }
    ncrit_all += tot;
    __syncthreads();
  }
  /* every critical group has its entry when they number at most BL_CRIT_MAX; past that the row is walked */
  const bool have = ncrit_all <= BL_CRIT_MAX && ne == ncrit_all;
  const int ncrit = have ? ncrit_all : 0;
  /* 2. the slot of each critical group's entry (its rank among the entries' groups) */
  if (have) {
    if (w == 0) { /* lane j holds entry j's group; the others are broadcast from their lanes */
      const int g = lane < ncrit ? nm.eg[lane] : 0x7fffffff;
      int p = 0;
      for (int j = 0; j < ncrit; j++) p += (int)bl_bcast((uint32_t)g, j) < g ? 1 : 0;
      if (lane < ncrit) nm.epos[p] = lane;
    }
    __syncthreads();
  }
  auto run_lo = [&](int r) { return r == 0 ? 0 : nm.crit[r - 1] + 1; };
  auto run_hi = [&](int r) { return r == ncrit ? G : nm.crit[r]; };
  auto blk_E = [&](int b) -> int { return b < BL_STAGE_B ? nm.bE[b] : brec[b].E; };
  auto blk_v = [&](int b) -> bl_inc { return b < BL_STAGE_B ? nm.bV[b] : brec[b].v; };
  /* a group record of a block holding critical group r (from its entry) */
  auto edge = [&](int r, int g) -> bl_grec1 { return nm.blk[nm.epos[r] * (BL_EB / 64) + (g & (BL_EB / 64 - 1))]; };
  /* 3. runs (edge groups and whole blocks), one per wavefront at a time */
  const int nrun = ncrit + 1;
  for (int it = w; it < nrun; it += SEL_NW) {
    const int lo = run_lo(it), hi = run_hi(it);
    int st = 0, Er = BL_E_NONE;
    bl_inc acc = bl_inc_ident();
    if (lo < hi) {
      const int gb0 = min((lo + 15) & ~15, hi);
      /* whole blocks from their summaries, the row's short last block included (its summary covers its groups) */
      const int gb1 = (hi == G && (hi & 15) && gb0 <= (hi & ~15)) ? hi : max(hi & ~15, gb0);
      const int npre = gb0 - lo, nblk = (gb1 - gb0 + 15) >> 4, nit = npre + nblk + (hi - gb1);
      /* a group of a critical group's block from that entry; others (a short last block that a critical group
       * cuts) from the exponent pass's records */
      auto grp = [&](int g) -> bl_grec1 {
        const int bg = g >> 4;
        if (it > 0 && (nm.crit[it - 1] >> 4) == bg) return edge(it - 1, g);
        if (it < ncrit && (nm.crit[it] >> 4) == bg) return edge(it, g);
        return rec[g];
      };
      Er = npre > 0 ? grp(lo).E : (nblk > 0 ? blk_E(gb0 >> 4) : grp(gb1).E);
      bool bad = false;
      for (int i0 = 0; i0 < nit; i0 += 64) {
        const int i = i0 + lane;
        bl_inc f = bl_inc_ident();
        if (i < nit) {
          int Ei;
          if (i < npre || i >= npre + nblk) {
            const bl_grec1 gr = grp(i < npre ? lo + i : gb1 + (i - npre - nblk));
            Ei = gr.E;
            f = gr.v;
          } else {
            const int bb = (gb0 >> 4) + (i - npre);
            Ei = blk_E(bb);
            f = blk_v(bb);
          }
          bad |= Ei != Er;
        }
        acc = bl_compose(acc, bl_wave_reduce(f, lane));
      }
      st = __ballot(bad) ? 2 : 1;
    }
    if (lane == 0) {
      nm.r_E[it] = Er;
      nm.r_st[it] = st;
      nm.r_f[it] = acc;
    }
  }
  if (t == 0) nm.ncrit = ncrit;
  __syncthreads();
}

/*
 * The chain of the index-order normaliser, by one whole wavefront after norm_prep; nm.S = the sum. Lane r
 * holds run r's composed automaton and critical group r's index and predicted binades, so the walk reads
 * them with readlane; a critical group's per-lane term, prefix and suffix compositions are read one group
 * ahead. `term(j)` recomputes term j for the fallback walks.
 */
template <class TermF>
__device__ __forceinline__ void norm_chain(const bl_dev &d, int row, sel_shared &sh, TermF term) {
  const int V = d.vocab, lane = threadIdx.x & 63;
  const int G = (V + 63) / 64;
  const bl_grec1 *rec =
      reinterpret_cast<const bl_grec1 *>(reinterpret_cast<const bl_grec *>(d.grec) + (int64_t)row * 2 * (V / 64 + 64));
  const sel_norm &nm = sh.n;
  const int ncrit = nm.ncrit, nrun = ncrit + 1;
  static_assert(BL_CRIT_MAX + 1 <= 64, "one lane per run and per critical group");
  const int rl = lane < nrun ? lane : 0;
  const int rE = nm.r_E[rl], rst = nm.r_st[rl];
  const bl_inc rf = nm.r_f[rl];
  const int cl = lane < ncrit ? lane : 0;
  const int cslot = lane < ncrit ? nm.epos[cl] : 0; /* critical group cl's entry slot (none without entries) */
  const int cg = nm.crit[cl], ce0 = nm.ce0[cslot], ce1 = nm.ce1[cslot];
  auto slot_of_r = [&](int r) { return (int)bl_bcast((uint32_t)cslot, r); };
  auto crit_of = [&](int r) { return (int)bl_bcast((uint32_t)cg, r); };
  auto run_lo = [&](int r) { return r == 0 ? 0 : crit_of(r - 1) + 1; };
  auto run_hi = [&](int r) { return r == ncrit ? G : crit_of(r); };
  int e = BL_E_MIN;
  uint32_t N = 0u;
  /* a record holds its own binade only: a neighbouring binade reads as saturated (element level) */
  auto recf = [&](int64_t g) {
    const bl_grec1 r1 = rec[g];
    return bl_grec{r1.E, 0u, {bl_inc{BL_SAT, BL_SAT}, r1.v, bl_inc{BL_SAT, BL_SAT}}};
  };
  /* lane c holds term c, the composition of terms 0..c, and that of the terms after c */
  auto cs_after = [&](int r) {
    const int sr = slot_of_r(r); /* the broadcast runs in every lane */
    return lane < 63 ? nm.cs[sr * 64 + lane + 1] : bl_inc_ident();
  };
  float a = 0.0f;
  bl_inc cp = bl_inc_ident(), cs = bl_inc_ident();
  if (ncrit > 0) {
    a = nm.terms[slot_of_r(0) * 64 + lane];
    cp = nm.cp[slot_of_r(0) * 64 + lane];
    cs = cs_after(0);
  }
  for (int r = 0; r <= ncrit; r++) {
    float a_nx = 0.0f;
    bl_inc cp_nx = bl_inc_ident(), cs_nx = bl_inc_ident();
    if (r + 1 < ncrit) {
      const int sn = slot_of_r(r + 1);
      a_nx = nm.terms[sn * 64 + lane];
      cp_nx = nm.cp[sn * 64 + lane];
      cs_nx = cs_after(r + 1);
    }
    const int st = (int)bl_bcast((uint32_t)rst, r);
    if (st != 0) {
      const bl_inc f = bl_inc{bl_bcast(rf.d0, r), bl_bcast(rf.d1, r)};
      const uint32_t N2 = bl_apply(f, N);
      if (st == 1 && (int)bl_bcast((uint32_t)rE, r) == e && N2 < BL_N_TOP) N = N2;
      else walk_groups(run_lo(r), run_hi(r), V, term, recf, e, N, lane);
    }
    if (r == ncrit) break;
    const bool in = (int64_t)crit_of(r) * 64 + lane < V;
    if (e != (int)bl_bcast((uint32_t)ce0, r)) {
      elem_resolve(a, in, e, N, lane, 0);
    } else {
      const uint32_t Ne = bl_apply(cp, N);
      const unsigned long long ms = __ballot(in && Ne >= BL_N_TOP);
      if (!ms) {
        N = bl_bcast(Ne, 63);
      } else {
        const int c = __ffsll((long long)ms) - 1;
        const uint32_t Nbefore = c > 0 ? bl_bcast(Ne, c - 1) : N;
        const float Sn = bl_make(e, Nbefore) + bl_bcastf(a, c); /* the one real float add at the crossing */
        bl_split(Sn, e, N);
        if (c < 63) {
          const uint32_t N2 = bl_apply(bl_inc{bl_bcast(cs.d0, c), bl_bcast(cs.d1, c)}, N);
          if (e == (int)bl_bcast((uint32_t)ce1, r) && N2 < BL_N_TOP) N = N2;
          else elem_resolve(a, in, e, N, lane, c + 1);
        }
      }
    }
    a = a_nx;
    cp = cp_nx;
    cs = cs_nx;
  }
  if (lane == 0) sh.n.S = bl_make(e, N);
}

/*
 * The heap rank's order among equal values (all_candidates_sorted, src/sampling.br:301-365), for a
 * full-vocabulary draw that landed on position `pos` of the sorted list whose value has equal neighbours.
 * The drawn position depends only on the values (equal terms sum alike in any order); which token sits
 * there is the heap's choice. Elements below the tied value never move an element at or above it: a sift
 * compares them only with each other or loses to it, and below the current level the sub-heaps hold only
 * smaller values under a smaller root. So the heap is simulated on the nb elements >= the tied value (the
 * sorted prefix), every other position reading as smaller than all of them:
 *   - occupancy (position -> element of the prefix, or -1) in `occ_g`, V entries of global scratch; the
 *     bottom-up build runs level by level, the parents of one level owning disjoint subtrees;
 *   - after the build the prefix forms a rooted subtree; one lane replays the extractions up to `pos` on
 *     an LDS copy of that occupancy: the first BL_TIE_OCC positions densely, the subtree's positions past
 *     them in an open-addressing table (BL_TIE_HASH slots, filled to at most 3/4). An extraction moves
 *     elements of the prefix only into positions that held one, so the table needs no insertion later.
 * Returns the token id, or -1 when the prefix exceeds BL_TIE_MAX elements or its deep positions the table
 * (the caller then reports the tie).
 */
static_assert(BL_NBUCKET * sizeof(uint32_t) <= sizeof(sel_cand::keys), "bucket counters live in the list's LDS");
static_assert(BL_NBUCKET % BL_SEL_THREADS == 0, "whole buckets per thread");
#define BL_TIE_MAX 8192                                     /* elements >= the tied value */
#define BL_TIE_OCC ((int)(sizeof(sel_norm) / sizeof(int16_t))) /* positions copied to LDS */
#define BL_TIE_HASH BL_RANK_MAX /* slots of the deep-position table (the counting sort's LDS, free by now) */
static_assert((BL_TIE_HASH & (BL_TIE_HASH - 1)) == 0, "table size is a power of two");
__device__ __forceinline__ uint32_t tie_slot(int p) { return ((uint32_t)p * 2654435761u) >> 22 & (BL_TIE_HASH - 1); }
/* the heap's extractions over the sorted prefix key(0..nb) (every element below it reads as smaller than all
 * of it): the first extraction i whose element o (a prefix index) satisfies stop(i, o), as that element's
 * token; -1 when none does or the simulation does not fit */
template <class KeyF, class StopF>
__device__ __forceinline__ int heap_extract_until(KeyF key, bool keys_in_lds, int nb, int V, int32_t *occ_g, sel_shared &sh,
                                                  StopF stop) {
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  if (nb > BL_TIE_MAX) return -1;
  /* the prefix's values, in LDS (the list itself when it is there, else a float copy in its place) */
  float *bval = reinterpret_cast<float *>(sh.c.keys);
  if (!keys_in_lds)
    for (int k = t; k < nb; k += BL_SEL_THREADS) bval[k] = ckey_v(key(k));
  auto vbig = [&](int k) -> float { return keys_in_lds ? ckey_v(key(k)) : bval[k]; };
  /* k above j (-1: a position below the whole prefix) */
  auto above = [&](int k, int j) -> bool {
    if (k < 0) return false;
    if (j < 0) return true;
    return vbig(k) > vbig(j);
  };
  for (int p = t; p < V; p += BL_SEL_THREADS) occ_g[p] = -1;
  __syncthreads();
  for (int k = t; k < nb; k += BL_SEL_THREADS) occ_g[ckey_i(key(k))] = k;
  __syncthreads();
  /* sift-down with a strict `>` on the larger child and on the root, as the reference */
  auto sift = [&](int root, int size, auto get, auto set) {
    while (true) {
      const int l = 2 * root + 1;
      if (l >= size) return;
      const int r = l + 1;
      const int ol = get(l), orr = r < size ? get(r) : -1;
      int c = l, oc = ol;
      if (r < size && above(orr, ol)) {
        c = r;
        oc = orr;
      }
      const int oroot = get(root);
      if (!above(oc, oroot)) return;
      set(root, oc);
      set(c, oroot);
      root = c;
    }
  };
  auto gget = [&](int p) -> int { return occ_g[p]; };
  auto gset = [&](int p, int v) { occ_g[p] = v; };
  const int depth_max = 31 - __clz(V);
  for (int L = depth_max; L >= 0; L--) {
    const int p0 = (1 << L) - 1, p1 = min((2 << L) - 1, V / 2); /* the parents of level L: 2p + 1 < V */
    for (int p = p0 + t; p < p1; p += BL_SEL_THREADS) sift(p, V, gget, gset);
    __syncthreads();
  }
  /* the prefix's positions past the dense copy go to the table: (position + 1) << 32 | element, 0 empty */
  const int n_occ = min(V, BL_TIE_OCC);
  uint64_t *htab = sh.c.tmp;
  for (int i = t; i < BL_TIE_HASH; i += BL_SEL_THREADS) htab[i] = 0ull;
  __syncthreads();
  int deep = 0;
  for (int p = n_occ + t; p < V; p += BL_SEL_THREADS)
    if (occ_g[p] >= 0) deep++;
  deep = bl_wscan_add(deep, lane);
  if (lane == 63) sh.red_i[w] = deep;
  __syncthreads();
  deep = 0;
  for (int q = 0; q < SEL_NW; q++) deep += sh.red_i[q];
  if (deep > BL_TIE_HASH * 3 / 4) return -1; /* uniform */
  if (deep > 0)
    for (int p = n_occ + t; p < V; p += BL_SEL_THREADS) {
      const int o = occ_g[p];
      if (o < 0) continue;
      const uint64_t e = (uint64_t)(uint32_t)(p + 1) << 32 | (uint32_t)o;
      for (uint32_t h = tie_slot(p);; h = (h + 1) & (BL_TIE_HASH - 1))
        if (atomicCAS(reinterpret_cast<unsigned long long *>(&htab[h]), 0ull, (unsigned long long)e) == 0ull) break;
    }
  int16_t *occ_l = reinterpret_cast<int16_t *>(&sh.n);
  for (int p = t; p < n_occ; p += BL_SEL_THREADS) occ_l[p] = (int16_t)occ_g[p];
  __syncthreads();
  if (t == 0) {
    /* the table slot of position p (past the dense copy), or -1 when p holds no prefix element */
    auto hfind = [&](int p) -> int {
      for (uint32_t h = tie_slot(p);; h = (h + 1) & (BL_TIE_HASH - 1)) {
        const uint64_t e = htab[h];
        if (e == 0ull) return -1;
        if ((uint32_t)(e >> 32) == (uint32_t)(p + 1)) return (int)h;
      }
    };
    auto lget = [&](int p) -> int {
      if (p < n_occ) return (int)occ_l[p];
      const int h = hfind(p);
      return h < 0 ? -1 : (int)(int32_t)(uint32_t)htab[h];
    };
    auto lset = [&](int p, int v) { /* only positions that held prefix elements after the build */
      if (p < n_occ) {
        occ_l[p] = (int16_t)v;
      } else {
        const int h = hfind(p);
        if (h >= 0) htab[h] = (htab[h] & 0xffffffff00000000ull) | (uint32_t)v;
      }
    };
    int size = V, res = -1;
    for (int i = 0; i < nb; i++) {
      const int o = lget(0);
      if (stop(i, o)) {
        res = o;
        break;
      }
      size -= 1;
      if (size > 0) {
        lset(0, lget(size));
        sift(0, size, lget, lset);
      }
    }
    sh.ires[4] = res;
  }
  __syncthreads();
  const int res = sh.ires[4];
  __syncthreads();
  return res >= 0 ? ckey_i(key(res)) : -1;
}
/* the token the heap extracts at position `pos` of the sorted list, whose value has equal neighbours */
template <class KeyF>
__device__ __forceinline__ int heap_tie_id(KeyF key, bool keys_in_lds, int64_t n_list, int64_t pos, int V, int32_t *occ_g,
                           sel_shared &sh) {
  const float vp = ckey_v(key(pos));
  /* nb = first index past pos whose value is below vp (the list is sorted: binary search, every thread) */
  int64_t lo = pos + 1, hi = n_list;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (ckey_v(key(mid)) == vp) lo = mid + 1;
    else hi = mid;
  }
  return heap_extract_until(key, keys_in_lds, (int)lo, V, occ_g, sh, [&](int i, int) { return (int64_t)i == pos; });
}

/*
 * K3: grid (B) x 1024, one workgroup per row. The row maximum and first argmax come from the chunk
 * statistics. A sampled row's ranked list is the merged top-K (exponent pass, workgroup 0) or the
 * full-vocabulary candidates, sorted here. A logprob row's exact index-order normaliser is prepared by
 * every wavefront and chained by wavefront 0 while wavefront 1 runs a short list's sequential float32
 * loops. Then the outputs (the token, its logprob (x - max) - ln(normaliser) and the alternatives,
 * src/server.br:1027-1035) and the history commit (src/server.br:1004, :1037): counts and bitmap bits by
 * atomics that nothing waits for, the slot's scalar state read at the start.
 */
/*
 * The row's top K keys in (value desc, index asc) order (top_k_select, src/sampling.br:280-296) from the row
 * pass's chunk lists (each sorted, K long, unfilled entries id -1), into sh.mkeys[0..K) (0 = unfilled), by
 * the block. The lists are staged in LDS. The first L = ceil(K/nc) keys of all the lists hold at least K keys;
 * their K-th largest, tau, is at most the row's K-th key, so the row's top K are among the keys >= tau: in
 * each list a prefix, whose length one thread per list finds by binary search. The prefixes are packed by a
 * prefix sum of their lengths and ranked by counting (keys are distinct: they carry the index). Lists too
 * large to stage find the K-th key itself by bisection over the key bits (a slower path).
 */
__device__ __forceinline__ void sel_merge(const bl_dev &d, int row, int K, sel_shared &sh) {
  constexpr int NT = BL_SEL_THREADS;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, nc = d.nc;
  const int L = (K + nc - 1) / nc, nu = nc * L, total = nc * K;
  auto gkey = [&](int i) -> uint64_t {
    const int c = i / K, q = i - c * K;
    const int64_t o = ((int64_t)row * nc + c) * BL_KSEL_MAX + q;
    const int32_t id = d.cand_i[o];
    return id >= 0 ? ckey(d.cand_v[o], id) : 0ull;
  };
  uint64_t *stage = sh.c.keys, *ua = sh.c.tmp;
  uint64_t *surv = reinterpret_cast<uint64_t *>(&sh.n); /* the normaliser's LDS is free until norm_prep */
  int *lc = reinterpret_cast<int *>(sh.c.tmp);         /* per-list prefix lengths, after the first selection */
  static_assert(sizeof(sel_norm) >= BL_LDS_SORT * sizeof(uint64_t), "survivors fit the normaliser's LDS");
  static_assert(BL_RANK_MAX * 2 >= BL_MAX_CHUNKS + 1, "per-list lengths fit the rank area");
  const bool fits = total <= BL_LDS_SORT && nu <= BL_RANK_MAX;
  if (t == 0) {
    sh.mtau = 1ull; /* every valid key, when fewer than K exist */
    sh.mcnt = 0;
  }
  if (fits) {
    for (int i = t; i < total; i += NT) {
      const uint64_t k = gkey(i);
      stage[i] = k;
      const int c = i / K, q = i - c * K;
      if (q < L) ua[c * L + q] = k;
    }
    __syncthreads();
    for (int i = t; i < nu; i += NT) {
      const uint64_t k = ua[i];
      if (k && count_gt(ua, nu, k) == K - 1) sh.mtau = k;
    }
    __syncthreads();
    const uint64_t tau = sh.mtau;
    /* list c's keys >= tau: a prefix (lists are sorted, unfilled keys 0 < tau); offsets by a block scan */
    for (int c0 = 0; c0 < nc; c0 += NT) {
      const int c = c0 + t;
      int n = 0;
      if (c < nc) {
        int lo = 0, hi = K;
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (stage[c * K + mid] >= tau) lo = mid + 1;
          else hi = mid;
        }
        n = lo;
      }
      const int incl = bl_wscan_add(n, lane);
      if (lane == 63) sh.red_i[w] = incl;
      __syncthreads();
      int off = sh.mcnt + incl - n, tot = 0;
      for (int q = 0; q < NT / 64; q++) {
        if (q < w) off += sh.red_i[q];
        tot += sh.red_i[q];
      }
      if (c < nc) {
        lc[2 * c] = off;
        lc[2 * c + 1] = n;
      }
      __syncthreads();
      if (t == 0) sh.mcnt += tot;
      __syncthreads();
    }
    for (int i = t; i < total; i += NT) {
      const int c = i / K, q = i - c * K;
      if (q < lc[2 * c + 1]) surv[lc[2 * c] + q] = stage[i];
    }
  } else {
    /* bisection: the largest tau with at least K keys >= tau */
    uint64_t tau = 0ull;
    for (int bit = 63; bit >= 0; bit--) {
      const uint64_t cand = tau | (1ull << bit);
      int c = 0;
      for (int i = t; i < total; i += NT) c += gkey(i) >= cand ? 1 : 0;
      c = bl_wscan_add(c, lane);
      if (lane == 63) sh.red_i[w] = c;
      __syncthreads();
      int tot = 0;
      for (int q = 0; q < NT / 64; q++) tot += sh.red_i[q];
      __syncthreads();
      if (tot >= K) tau = cand;
    }
    if (t == 0 && tau) sh.mtau = tau;
    __syncthreads();
    const uint64_t tau2 = sh.mtau;
    for (int i = t; i < total; i += NT) {
      const uint64_t k = gkey(i);
      if (k && k >= tau2) {
        const int p = atomicAdd(&sh.mcnt, 1);
        if (p < BL_LDS_SORT) surv[p] = k;
      }
    }
  }
  __syncthreads();
  const int C = min(sh.mcnt, BL_LDS_SORT);
  for (int i = t; i < C; i += NT) {
    const uint64_t k = surv[i];
    const int r = count_gt(surv, C, k);
    if (r < K) sh.mkeys[r] = k;
  }
  for (int q = C + t; q < K; q += NT) sh.mkeys[q] = 0ull;
  __syncthreads();
}

/* ------------------------------------------------------------------ adaptive-p */
/*
 * sample_adaptive_p (src/sampling.br:705-740) by the block, after the row's normaliser (M, lse): the
 * adapted target 2 target - average (clamped to [0, 1]); each value's probability exp(x - M - lse) and its
 * transform 5 - 10 d^2 / (1 + d), d = |p - target'| / 0.3 (values <= -1e29 kept), over the row in
 * chunks through the server stages; the transform's maximum and its sum of exp(t - tmax) in index order
 * (exact: the group records and the walk of the sequential float32 sums); then the draw's running sum of
 * exp(t - tmax - ln sum) in index order up to the uniform draw. Returns the token; ws / tw = the slot's
 * next weighted sum and total weight.
 */
__device__ __forceinline__ int32_t sample_adaptive(const bl_dev &d, const bl_slot_dev &sp, const bl_rows &rows, int row,
                                                int slot, const float *__restrict__ logits, int64_t ld, float M,
                                                float lse, uint64_t &rng, sel_shared &sh, float &ws, float &tw) {
  const int V = d.vocab, t = threadIdx.x, w = t >> 6, lane = t & 63;
  float *tbuf = reinterpret_cast<float *>(d.sortk + (int64_t)row * 2 * V); /* terms [V] */
  float *tv = tbuf + 2 * (int64_t)V;                                      /* transformed values [V] */
  bl_grec *recs = reinterpret_cast<bl_grec *>(d.grec) + (int64_t)row * 2 * (V / 64 + 64) + (V / 64 + 64);
  double *gsum = d.gsum + (int64_t)row * (V / 64 + 64);
  const float avg = sp.adapt_tw == 0.0f ? sp.adapt_target : sp.adapt_ws / sp.adapt_tw;
  float at = 2.0f * sp.adapt_target - avg;
  if (at < 0.0f) at = 0.0f;
  if (at > 1.0f) at = 1.0f;
  float *vals = reinterpret_cast<float *>(sh.c.keys); /* [BL_CH] */
  uint32_t *sup = reinterpret_cast<uint32_t *>(sh.c.tmp), *done = sup + BL_CH / 32;
  static_assert(BL_CH * 4 <= sizeof(sh.c.keys) && (BL_CH / 32 + 1) * 4 <= sizeof(sh.c.tmp), "adaptive-p scratch");
  float tm = BL_NEG_INF;
  for (int i0 = 0; i0 < V; i0 += BL_CH) {
    const int cnt = V - i0 < BL_CH ? V - i0 : BL_CH;
    for (int p = t; p < cnt; p += BL_SEL_THREADS) vals[p] = logits[(int64_t)row * ld + i0 + p];
    apply_stages<false>(d, sp, rows, row, slot, i0, cnt, vals, sup, done);
    for (int p = t; p < cnt; p += BL_SEL_THREADS) {
      const float x = vals[p];
      float tt = x;
      if (!(x <= -1.0e29f)) {
        const float a = x - M;
        const float pr = SEL_EXPF(a - lse);
        const float dist = fabsf(pr - at) / 0.3f;
        float num = 10.0f * dist;
        num = num * dist;
        tt = 5.0f - num / (1.0f + dist);
      }
      tv[i0 + p] = tt;
      tm = fmaxf(tm, tt);
    }
    __syncthreads();
  }
  int ti = 0;
  bl_wargmax(tm, ti, lane);
  if (lane == 0) sh.red_m[w] = tm;
  __syncthreads();
  float tmax = sh.red_m[0];
  for (int q = 1; q < SEL_NW; q++) tmax = fmaxf(tmax, sh.red_m[q]);
  __syncthreads();
  auto tval = [&](int64_t j) { return tv[j]; };
  auto termS = [&](int64_t j) { return tbuf[j]; };
  /* logprob_normalizer(transformed) (src/sampling.br:725): sum of exp(t - tmax), index order */
  block_records(V, tval, [&](float v) { return SEL_EXPF(v - tmax); }, recs, gsum, tbuf);
  if (w == 0) {
    float S;
    bl_seq_walk(V, termS, [&](int64_t g) { return recs[g]; }, false, 0.0f, 0, S, lane);
    if (lane == 0) sh.fres[4] = S;
  }
  __syncthreads();
  const float tsum = SEL_LOGF(sh.fres[4]);
  __syncthreads();
  /* the draw (:726-736): the first index whose running sum of exp(t - tmax - tsum) reaches it */
  uint64_t st = rng;
  const float draw = bl_rng_f32(&st);
  block_records(V, tval, [&](float v) {
    const float a = v - tmax;
    return SEL_EXPF(a - tsum);
  }, recs, gsum, tbuf);
  if (w == 0) {
    float S;
    const int f = bl_seq_walk(V, termS, [&](int64_t g) { return recs[g]; }, true, draw, 0, S, lane);
    if (lane == 0) sh.ires[5] = f >= 0 ? f : V - 1;
  }
  __syncthreads();
  const int32_t sel = sh.ires[5];
  __syncthreads();
  rng = st;
  /* the chosen token's original probability, then the running sums (:737-740) */
  const float xs = bl_row_value(d, sp, rows, row, slot, logits, ld, sel);
  const float a = xs - M;
  const float psel = SEL_EXPF(a - lse);
  const float wsd = sp.adapt_decay * sp.adapt_ws, twd = sp.adapt_decay * sp.adapt_tw;
  ws = psel + wsd;
  tw = 1.0f + twd;
  return sel;
}

/* ------------------------------------------------------------------ DRY's penalty map */
/* the segment of single-token breaker `tok` (the longer breakers listed before its first occurrence), or -1 */
__device__ __forceinline__ int dry_single_seg(const bl_slot_dev &sp, int32_t tok) {
  int lo = 0, hi = sp.n_bsingle;
  const uint64_t want = (uint64_t)(uint32_t)tok << 32;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (sp.bsingle[mid] < want) lo = mid + 1;
    else hi = mid;
  }
  return lo < sp.n_bsingle && (sp.bsingle[lo] >> 32) == (uint64_t)(uint32_t)tok ? (int)(uint32_t)sp.bsingle[lo] : -1;
}

#define BL_DRY_LDS (BL_DRY_WCAP * 4 + BL_DRY_WCAP * 8 + (2 * BL_DRY_MMAX + 16) * 4)
/*
 * apply_dry_penalty's map (src/sampling.br:114-171) for the slot's next step, from its last dh_len history
 * tokens, by one workgroup with `lds` (BL_DRY_LDS bytes) as scratch:
 *   1. the previous update's flags are cleared;
 *   2. the suffix start (:121-134): each breaker, in list order, moves the start past its last occurrence
 *      at or after the start. A single token's step is a maximum, so the singles between two longer breakers
 *      reduce to one maximum per segment; a longer breaker's step needs its last occurrence;
 *   3. per candidate position, the match between the tokens before it and the context tail (:143-151);
 *      positions matching at least allowed_length tokens give (token + 1, length) keys, sorted in descending
 *      order, so that a token's first key holds its maximum repeat;
 *   4. each such token that is not a single-token breaker gets the flag and the exponent
 *      min(maximum repeat - allowed_length, cap) in its record (:157-170), and joins the flagged list.
 * The slot's state is read after the caller's barrier.
 */
__device__ __forceinline__ void dry_update(const bl_dev &d, bl_slot_dev &sp, int slot, unsigned char *lds) {
  const int t = threadIdx.x, NT = (int)blockDim.x;
  int32_t *lw = reinterpret_cast<int32_t *>(lds);
  uint64_t *lk = reinterpret_cast<uint64_t *>(lds + BL_DRY_WCAP * 4);
  int32_t *lseg = reinterpret_cast<int32_t *>(lds + BL_DRY_WCAP * 12); /* [BL_DRY_MMAX + 1] */
  int32_t *lam = lseg + BL_DRY_MMAX + 1;                           /* [BL_DRY_MMAX] */
  int32_t *lsc = lam + BL_DRY_MMAX;                                /* start, flagged count */
  int32_t *dl = d.dlist + (int64_t)slot * BL_DRY_WCAP;
  auto rec_of = [&](int32_t tok) -> bl_rec * {
    const int ri = d.ridx[(int64_t)slot * d.vocab + tok];
    return ri >= 0 ? d.rec + ((int64_t)slot * d.nb + tok / BL_EB) * BL_EB + ri : nullptr;
  };
  const uint32_t keep = (1u << (BL_WF_SHIFT + 1)) - 1u; /* window count and the bias flag */
  const int n_old = sp.dry_cnt, W = sp.dh_len, A = sp.dry_allowed, nm = sp.n_bmulti;
  for (int i = t; i < n_old; i += NT) {
    bl_rec *r = rec_of(dl[i]);
    if (r) r->wf &= keep;
  }
  const int32_t *ring = d.dring + (int64_t)slot * BL_DRY_WCAP;
  for (int p = t; p < W; p += NT) lw[p] = ring[(sp.dh_head + p) % sp.dry_n];
  for (int m = t; m <= nm; m += NT) lseg[m] = 0;
  for (int m = t; m < nm; m += NT) lam[m] = -1;
  if (t == 0) {
    lsc[0] = 0;
    lsc[1] = 0;
  }
  __syncthreads();
  if (W > A) { /* window <= allowed_length: no penalty (:120) */
    for (int p = t; p < W; p += NT) {
      const int sg = dry_single_seg(sp, lw[p]);
      if (sg >= 0) atomicMax(&lseg[sg], p + 1);
    }
    for (int idx = t; idx < nm * W; idx += NT) {
      const int m = idx / W, p = idx - m * W;
      const int32_t *b = sp.bmulti + (int64_t)m * (BL_DRY_MLEN + 1);
      const int L = b[0];
      if (p + L <= W) {
        bool eq = true;
        for (int q = 0; q < L && eq; q++) eq = lw[p + q] == b[1 + q];
        if (eq) atomicMax(&lam[m], p);
      }
    }
    __syncthreads();
    if (t == 0) {
      int s = 0;
      for (int m = 0; m < nm; m++) {
        s = max(s, lseg[m]);
        if (lam[m] >= s) s = lam[m] + sp.bmulti[(int64_t)m * (BL_DRY_MLEN + 1)];
      }
      lsc[0] = max(s, lseg[nm]);
    }
    __syncthreads();
    const int s = lsc[0], suffix = W - s;
    if (suffix >= A) {
      int P = 64;
      while (P < W) P <<= 1;
      for (int c = t; c < P; c += NT) {
        uint64_t key = 0ull;
        if (c > s && c < W) {
          int r = 0;
          while (r < suffix && c - r - 1 >= s && lw[c - r - 1] == lw[W - r - 1]) r++;
          if (r >= A) key = ((uint64_t)((uint32_t)lw[c] + 1u) << 16) | (uint64_t)r;
        }
        lk[c] = key;
      }
      __syncthreads();
      bitonic_desc(lk, P);
      for (int i = t; i < P; i += NT) {
        const uint64_t k = lk[i];
        if (!k || (i > 0 && (lk[i - 1] >> 16) == (k >> 16))) continue;
        const int32_t tok = (int32_t)((k >> 16) - 1u);
        if (dry_single_seg(sp, tok) >= 0) continue; /* a one-token breaker is exempt */
        int e = (int)(k & 0xFFFFu) - A;
        if (e > sp.dry_maxexp) e = sp.dry_maxexp;
        bl_rec *r = rec_of(tok);
        if (r) {
          r->wf = (r->wf & keep) | (BL_TF_DRY << BL_WF_SHIFT) | ((uint32_t)e << BL_DRY_ESHIFT);
          dl[atomicAdd(&lsc[1], 1)] = tok;
        }
      }
    }
  }
  __syncthreads();
  if (t == 0) sp.dry_cnt = lsc[1];
}

/* the penalty map of one slot from its window (after bl_slot_reset, bl_slot_dry_breakers and bl_slot_commit) */
__global__ __launch_bounds__(BL_SEL_THREADS) void bl_k_dry_prime(bl_dev d, int slot) {
  __shared__ __align__(16) unsigned char lds[BL_DRY_LDS];
  dry_update(d, d.slots[slot], slot, lds);
}

__global__ __launch_bounds__(BL_SEL_THREADS) void bl_k_select(bl_dev d, const float *__restrict__ logits, int64_t ld,
                                                              bl_rows rows) {
  const int V = d.vocab, nc = d.nc;
  const int row = blockIdx.x, t = threadIdx.x, w = t >> 6, lane = t & 63;
  __shared__ sel_shared sh;
  /* loads that need only the row index go out first: the exponent pass's row maximum and merged top-K keys
   * (thread t keeps the t-th); without that pass, wavefront 0 reduces the maximum from the chunk statistics */
  const bool pre = rows.merged != 0;
  float M = BL_NEG_INF;
  int Mi = 0x7fffffff;
  int mst = 0;
  uint64_t mk_pre = 0ull;
  if (pre) {
    M = d.rmax[row];
    Mi = d.rarg[row];
    mst = d.mstat[row];
    if (t < BL_KSEL_MAX) mk_pre = d.mkeys[(int64_t)row * BL_KSEL_MAX + t];
  } else if (w == 0) {
    for (int k = lane; k < nc; k += 64) argmax_merge(M, Mi, d.c_max[(int64_t)row * nc + k], d.c_arg[(int64_t)row * nc + k]);
    bl_wargmax(M, Mi, lane);
    if (lane == 0) {
      sh.red_m[0] = M;
      sh.red_i[0] = Mi;
    }
  }
  uint32_t m_pre = 0u; /* the normaliser's first block flags and summaries (used by logprob rows) */
  bl_grec1 br_pre{};
  const int n_ent = d.ncrit[row]; /* the normaliser's critical-group entries */

  if (t < d.nb) {
    m_pre = d.bcrit[(int64_t)row * d.nb + t];
    br_pre = reinterpret_cast<const bl_grec1 *>(d.brec)[(int64_t)row * d.nb + t];
  }
  const int slot = bl_row_slot(rows, row);
  bl_slot_dev &sp = d.slots[slot];
  const int mode = sp.mode, K = sp.k_sel;
  const float T = sp.temperature;
  const bool lp_row = (mode & BL_M_LOGPROBS) && rows.lp;
  const bool adapt = (mode & BL_M_ADAPT) != 0;
  const bool norm_row = lp_row || adapt; /* the row's normaliser is formed */
  /* slot state the commit updates */
  const int rl = sp.repeat_last_n, win_len = sp.win_len, win_head = sp.win_head;
  const int n_tokens0 = sp.n_tokens, n_reply0 = sp.n_reply;
  const bool rep_on = sp.rep_on != 0, fp_on = sp.fp_on != 0, g_on = sp.g_on != 0;
  const bool ring_full = rep_on && rl > 0 && win_len == rl;
  const int32_t ring_old = (t == 0 && rows.commit && ring_full) ? d.ring[(int64_t)slot * BL_WCAP + win_head] : 0;
  const int n_eog = d.n_eog;
  if (t < n_eog && t < BL_EOG_LDS) sh.eog[t] = d.eog[t];
  if (t < BL_EXP2_N) sh.etab[t] = bl_exp2_tab[t];
  if (t >= 64 && t < 96) sh.ltab[t - 64] = bl_log_tab[t - 64];
  __syncthreads();
  if (!pre) {
    M = sh.red_m[0];
    Mi = sh.red_i[0];
  }
  if (Mi == 0x7fffffff) Mi = 0;
  /* the row's top K keys: thread t keeps the t-th (used when K > t) */
  const bool merged = pre && mst;
  if (K > 0 && !merged) sel_merge(d, row, K, sh);
  const uint64_t mk = t < K ? (merged ? mk_pre : sh.mkeys[t]) : 0ull;

  int status = 0;
  uint64_t rng = sp.rng;
  const int skip = rows.rng_skip ? rows.rng_skip[row] : 0;
  int32_t tok = Mi;
  float tokv = M;
  const bool gram = (mode & BL_M_GRAMMAR) != 0;
  /* a grammar row with T > 0 samples from its allowed candidates (src/server.br:323-362) unless its frontier
   * is dead, ambiguous or forces the end of sequence (then the grammar block below decides) */
  const int gst0 = gram ? d.gstat[row] : 0;
  const bool sampled = !(mode & BL_M_ADAPT) && T > 0.0f &&
                       (!gram || (!(gst0 & (BL_GR_FAMBIG | BL_GR_DEAD | BL_GR_FORCED)) && d.gamb[row] == 0));
  /* top-n-sigma (src/sampling.br:376-407): the threshold max - n * sigma, by wavefront 0 from the row pass's
   * chunk statistics; candidates below it leave the ranked list (the reference sets them to -1e30, which
   * ranks them after every other value and gives them no weight) */
  float tns_thr = BL_NEG_INF;
  if (sampled && (mode & BL_M_TNS)) {
    if (w == 0) {
      bl_dd S{0.0, 0.0}, Q{0.0, 0.0};
      double n = 0.0, es = 0.0, eq = 0.0, off_s = 0.0, off_q = 0.0;
      for (int c0 = 0; c0 < nc; c0 += 64) {
        const int c = c0 + lane;
        double p[BL_TNS_W];
#pragma unroll
        for (int k = 0; k < BL_TNS_W; k++) p[k] = c < nc ? d.c_tns[((int64_t)row * nc + c) * BL_TNS_W + k] : 0.0;
        const double cs = p[0] + p[1], cq = p[2] + p[3];
        /* the reference's additions over chunk c err by at most half an ulp of each partial sum, and a partial
         * sum there is at most |the earlier chunks' sum| + the chunk's sum of magnitudes (approximate prefixes:
         * only the bound reads them) */
        const double ps = off_s + bl_wave_excl_scan_d(cs, lane), pq = off_q + bl_wave_excl_scan_d(cq, lane);
        es += bl_wave_sum_d(p[5] * ((ps < 0.0 ? -ps : ps) + p[4]));
        eq += bl_wave_sum_d(p[5] * (pq + cq));
        off_s += bl_wave_sum_d(cs);
        off_q += bl_wave_sum_d(cq);
        bl_dd sd{p[0], p[1]}, qd{p[2], p[3]};
        double nn = p[5];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
          sd = bl_dd_add(sd, bl_dd{__shfl_xor(sd.hi, off, 64), __shfl_xor(sd.lo, off, 64)});
          qd = bl_dd_add(qd, bl_dd{__shfl_xor(qd.hi, off, 64), __shfl_xor(qd.lo, off, 64)});
          nn += __shfl_xor(nn, off, 64);
        }
        S = bl_dd_add(S, sd);
        Q = bl_dd_add(Q, qd);
        n += nn;
      }
      float sigma = 0.0f;
      const int r = n > 1.0 ? bl_tns_sigma(n, S, Q, es * 0x1p-53 * 1.001, eq * 0x1p-53 * 1.001, sigma) : 0;
      if (lane == 0) {
        sh.tns_thr = r == 1 ? M - sp.top_n_sigma * sigma : BL_NEG_INF;
        sh.tns_st = r < 0 ? 1 : 0;
      }
    }
    __syncthreads();
    tns_thr = sh.tns_thr;
    if (sh.tns_st) status |= BL_SE_SIGMA;
  }
  /* the ranked candidate list of a sampled row */
  uint64_t *keys = sh.c.keys;
  int64_t n_list = 0, n_logical = 0;
  const int64_t gwords = 2 * (((int64_t)V + 63) / 64);
  const uint32_t *gmk = d.gmask + (int64_t)row * gwords;
  auto g_allowed = [&](int32_t id) { return ((gmk[(id >> 6) * 2 + ((id >> 5) & 1)] >> (id & 31)) & 1u) != 0u; };
  float Mc = M; /* the top of the ranked list: the row maximum, or a grammar row's allowed maximum */
  float split_S = 0.0f; /* > 0: the list is a plain draw's ranked head, and this the whole list's sum */
  int split_tail_pos = -1; /* >= 0: the draw landed in the tail, its key stored at this list position */
  uint64_t split_rng = 0ull; /* then the RNG after the draw */
  bool gfull = false; /* a top-k grammar row's widening went past the merged list */
  int gk = 0;         /* its next level */
  if (sampled && gram && (mode & BL_M_TOPK)) {
    /* sample_grammar_token's levels (src/server.br:323-362): the allowed entries of top_k_select(k) in rank
     * order, k widened 4-fold while none is allowed. The merged list holds the first K ranks; a level past
     * it is left unsupported */
    const int32_t my_id = mk ? ckey_i(mk) : 0; /* an unfilled entry reads (-1e30, 0), as in top_k_select */
    const bool a_me = t < K && g_allowed(my_id);
    int kk = sp.top_k < V ? sp.top_k : V;
    for (;;) {
      if (kk > K || kk >= V) { /* past the merged list: the levels continue on the sorted full list below */
        gfull = true;
        gk = kk;
        break;
      }
      const int f = a_me && t < kk ? 1 : 0;
      const int incl = bl_wscan_add(f, lane);
      if (lane == 63) sh.red_i[w] = incl;
      __syncthreads();
      int before = incl - f, tot = 0;
      for (int q = 0; q < SEL_NW; q++) {
        if (q < w) before += sh.red_i[q];
        tot += sh.red_i[q];
      }
      __syncthreads();
      if (tot > 0) {
        if (f) keys[before] = mk;
        n_list = n_logical = tot;
        break;
      }
      kk = kk * 4 < V ? kk * 4 : V;
    }
  } else if (sampled && (mode & BL_M_TOPK)) {
    /* top_k_select list: kk = min(top_k, V) <= K entries, unfilled slots are (-1e30, 0) */
    const int kk = sp.top_k < V ? sp.top_k : V;
    if (t < kk) keys[t] = (mk && ckey_v(mk) >= tns_thr) ? mk : 0ull; /* top-n-sigma: unfilled past its threshold */
    n_list = n_logical = kk;
  }
  if (sampled && (gfull || !(mode & BL_M_TOPK))) {
    /* full-vocabulary rank (src/sampling.br:301-365): the exponent blocks' candidates (block b's at
     * [b*BL_EB, b*BL_EB + count)), concatenated by the prefix sum of the counts, then sorted. A grammar
     * row's candidates are its allowed tokens near the allowed maximum, and its list counts every allowed
     * token */
    const int NB = d.nb;
    if (gram && !(mode & BL_M_TOPK)) {
      float gm = BL_NEG_INF;
      int ga = 0;
      for (int k = t; k < d.gm_blocks; k += BL_SEL_THREADS) gm = fmaxf(gm, d.gm_max[(int64_t)row * d.gm_blocks + k]);
      double na = 0.0;
      for (int64_t q = t; q < gwords; q += BL_SEL_THREADS) na += (double)__popc(gmk[q]);
      bl_wargmax(gm, ga, lane);
      if (lane == 0) sh.red_m[w] = gm;
      na = block_sum_d<BL_SEL_THREADS>(na, sh.c.gsum); /* synchronises */
      Mc = sh.red_m[0];
      for (int q = 1; q < SEL_NW; q++) Mc = fmaxf(Mc, sh.red_m[q]);
      __syncthreads();
      if (na < 1.0) status |= sp.g_kind == 1 ? BL_SE_JREJECT : BL_SE_GREJECT;
      n_logical = (int64_t)na;
    }
    const float *fv = d.full_v + (int64_t)row * NB * BL_EB;
    const int32_t *fi = d.full_i + (int64_t)row * NB * BL_EB;
    int *boff = reinterpret_cast<int *>(&sh.n); /* [NB + 1]; the normaliser's LDS is free until norm_prep */
    const bool filt = bl_probs_on(sp) || (mode & BL_M_MIRO) != 0; /* the draw-aware cut: plain draws only */
    int nf = 0;
    double s_ap = 0.0; /* the exponent blocks' approximate tempered sum (unfiltered rows) */
    for (int b0 = 0; b0 < NB; b0 += BL_SEL_THREADS) {
      const int bb = b0 + t;
      const int c = bb < NB ? d.full_cnt[(int64_t)row * NB + bb] : 0;
      const double bsum = (!filt && bb < NB) ? d.full_s[(int64_t)row * NB + bb] : 0.0;
      const int incl = bl_wscan_add(c, lane);
      const double ws = bl_wave_sum_d(bsum);
      if (lane == 63) {
        sh.red_i[w] = incl;
        sh.c.gsum[w] = ws;
      }
      __syncthreads();
      int base = nf + incl - c, tot = 0;
      for (int q = 0; q < SEL_NW; q++) {
        if (q < w) base += sh.red_i[q];
        tot += sh.red_i[q];
        s_ap += sh.c.gsum[q];
      }
      if (bb < NB) boff[bb] = base;
      nf += tot;
      __syncthreads();
    }
    if (t == 0) boff[NB] = nf;
    __syncthreads();
    /* f(flat index, value, id) over every candidate; candidate i lies in the region lo with
     * boff[lo] <= i < boff[lo + 1] (binary search in LDS, so every thread's loads are independent) */
    auto each_cand = [&](auto f) {
      for (int i = t; i < nf; i += BL_SEL_THREADS) {
        int lo = 0, hi = NB;
        while (hi - lo > 1) {
          const int mid = (lo + hi) >> 1;
          if (boff[mid] <= i) lo = mid;
          else hi = mid;
        }
        const int64_t src = (int64_t)lo * BL_EB + (i - boff[lo]);
        f(i, fv[src], fi[src]);
      }
    };
    int nl = nf;
    /* top-n-sigma's survivors (key 0 for the others, which rank last) */
    auto tns_key = [&](float v, int32_t id) { return v >= tns_thr ? ckey(v, id) : 0ull; };
    auto tns_count = [&]() {
      int c = 0;
      for (int i = t; i < nf; i += BL_SEL_THREADS) c += sh.c.tmp[i] != 0ull ? 1 : 0;
      return (int)block_sum_d<BL_SEL_THREADS>((double)c, sh.c.gsum);
    };
    if (nf <= BL_RANK_MAX) {
      each_cand([&](int i, float v, int32_t id) { sh.c.tmp[i] = tns_key(v, id); });
      __syncthreads();
      if (mode & BL_M_TNS) nl = tns_count();
      /* rank by counting (keys are distinct: they carry the index) */
      for (int i = t; i < nf; i += BL_SEL_THREADS) {
        const uint64_t k = sh.c.tmp[i];
        if (k) keys[count_gt(sh.c.tmp, nf, k)] = k;
      }
    } else if (nf <= BL_LDS_SORT) {
      int P = 1;
      while (P < nf) P <<= 1;
      for (int i = nf + t; i < P; i += BL_SEL_THREADS) keys[i] = 0ull;
      each_cand([&](int i, float v, int32_t id) { keys[i] = tns_key(v, id); });
      __syncthreads();
      if (mode & BL_M_TNS) {
        int c = 0;
        for (int i = t; i < nf; i += BL_SEL_THREADS) c += keys[i] != 0ull ? 1 : 0;
        nl = (int)block_sum_d<BL_SEL_THREADS>((double)c, sh.c.gsum);
      }
      bitonic_desc(keys, P);
    } else {
      /* a large list: the candidates the draw can still see (below), bucketed by value (larger values in
       * lower buckets, equal values in one bucket), scattered by bucket, then ranked by counting within
       * each bucket, one LDS tile of the bucketed list at a time */
      const float T = sp.temperature;
      /* the exponent pass's candidates (four spans deep for a top-k grammar row), top-n-sigma's survivors */
      float thr = fmaxf(Mc - (gram && (mode & BL_M_TOPK) ? 4.0f : 1.0f) * bl_cand_span(sp), tns_thr);
      /* typical_p keeps every value: those below Mc - 104 have exp(v - v0) = 0, probability 0 */
      if (sp.typical_p < 1.0f && !gram) thr = fmaxf(thr, Mc - 104.0f);
      if (!filt && !(gram && (mode & BL_M_TOPK))) { /* a top-k grammar row draws from a subset: no cut */
        /* the draw adds exp((v - M) / T) in descending order. With u = 2^-24 and m <= V terms, the float
         * running sum past every term >= 2^(k-24) is at least (1 - g) (S - V 2^(k-24)), g = m u / (1 - m u)
         * (recursive summation bound), S the exact sum; that is >= 2^k when S >= 2^k (1 / (1 - g) + V u).
         * A term below half an ulp of the running sum leaves it unchanged, and so does every later
         * (smaller) term: the terms below 2^(k-24) are never seen by the draw. S is bounded from below by
         * the exponent blocks' approximate sum with a 10^-3 margin, the cut in logit space with a 10^-3
         * margin on the exponent (both far above the hardware exponential's error) */
        const double mu = (double)V * 0x1p-24;
        const double g = mu / (1.0 - mu);
        const double need = 1.0 / (1.0 - g) + mu;
        const double s_lo = s_ap * 0.999 / need;
        if (mu < 0.5 && s_lo > 0.0) {
          const int k = (int)((bl_d2u(s_lo) >> 52) & 0x7ff) - 1023; /* floor(log2 s_lo), s_lo normal */
          const float cut = Mc + T * ((float)((double)(k - 24) * 0.6931471805599453) - 1.0e-3f);
          thr = fmaxf(thr, cut);
        }
      }
      uint64_t *A = d.sortk + (int64_t)row * (2 * (int64_t)V), *Bk = A + V;
      uint32_t *cnt = reinterpret_cast<uint32_t *>(sh.c.keys); /* BL_NBUCKET counters; the list is in memory */
      const float span = Mc - thr;
      const float scale = span > 0.0f ? (float)BL_NBUCKET / span : 0.0f;
      auto bucket = [&](float v) -> int {
        const float q = (Mc - v) * scale;
        return q >= 0.0f ? (q < (float)(BL_NBUCKET - 1) ? (int)q : BL_NBUCKET - 1) : 0;
      };
      /* wavefront w reads regions w, w + SEL_NW, ... in batches of 64 * BL_CAND_U candidates; each lane
       * keeps BL_CAND_U loads (values, and ids when asked) in flight, the next batch's issued before this
       * batch's stores (stores share the in-order load counter) */
      auto next_batch = [&](int &bb, int &j0) {
        j0 += 64 * BL_CAND_U;
        while (bb < NB && j0 >= boff[bb + 1] - boff[bb]) {
          bb += SEL_NW;
          j0 = 0;
        }
      };
      auto each_region = [&](auto with_id, auto f) {
        constexpr bool WID = decltype(with_id)::value;
        float v[BL_CAND_U], vn[BL_CAND_U];
        int32_t id[BL_CAND_U], idn[BL_CAND_U];
        auto load = [&](int bb, int j0, float *vv, int32_t *ii) {
          const int c = bb < NB ? boff[bb + 1] - boff[bb] : 0;
          const float *pv = fv + (int64_t)bb * BL_EB;
          const int32_t *pi = fi + (int64_t)bb * BL_EB;
#pragma unroll
          for (int u = 0; u < BL_CAND_U; u++) {
            const int j = j0 + lane + 64 * u;
            vv[u] = j < c ? pv[j] : BL_NEG_INF;
            if (WID) ii[u] = j < c ? pi[j] : 0;
          }
        };
        int bb = w, j0 = -64 * BL_CAND_U;
        next_batch(bb, j0);
        load(bb, j0, vn, idn);
        while (bb < NB) {
#pragma unroll
          for (int u = 0; u < BL_CAND_U; u++) {
            v[u] = vn[u];
            id[u] = idn[u];
          }
          next_batch(bb, j0);
          load(bb, j0, vn, idn);
          f(v, id);
        }
      };
      /* A plain draw (no probability filter) needs the list's order only down to where its float running sum
       * has entered the binade [2^K, 2^(K+1)) of the final sum S: within one binade each later addition is
       * s + u round(t / u) (u = 2^(K-23), the rounding of s + t, an exact multiple of u, at any s there),
       * whatever the order, unless t / u lies exactly halfway. So only the head of the bucketed list is ranked,
       * down to a bucket whose lower-bounded mass passes both 2^K and the draw's target (with the
       * approximate sum's margins), and the tail's sum(round(t / u)) is counted in one pass. The head's exact
       * sum then decides: S = s_head + u sum(round(t / u)) when s_head lies in binade K, S < 2^(K+1) and the
       * target lies within the head; otherwise every bucket is ranked. A tail term t = u (f + 1/2) rounds to
       * the even multiple of u: it adds u (f + (N + f) mod 2), N = s / u before it, whose parity is s_head's,
       * the other tail terms' with larger values (a second pass) and the earlier such terms' (in key order). */
      bool split = !filt && !gram && !(mode & BL_M_TNS) && T > 0.0f && span > 0.0f;
      const bool tail_draw_ok = !((mode & BL_M_PSP) && rows.lp); /* post-sampling probabilities read the head */
      int Kb = 0;
      float r01 = 0.0f;
      double need = 0.0;
      if (split) {
        const double lo = s_ap * (1.0 - 4.0e-3), hi = s_ap * (1.0 + 4.0e-3);
        const int klo = (int)((bl_d2u(lo) >> 52) & 0x7ff) - 1023, khi = (int)((bl_d2u(hi) >> 52) & 0x7ff) - 1023;
        split = lo >= 1.0 && klo == khi && khi < 60;
        if (split) {
          Kb = klo;
          uint64_t st = rng;
          for (int k = 0; k < skip; k++) st = bl_xorshift(st);
          r01 = bl_rng_f32(&st);
          split_rng = st;
          /* the head also covers the target unless it lies far down (then it is found in the tail) */
          const float rcov = tail_draw_ok && r01 > 0.9f ? 0.9f : r01;
          need = fmax(bl_u2d((uint64_t)(Kb + 1023) << 52), (double)rcov * hi) * (1.0 + 4.0e-3);
        }
      }
      const int need_c = (sp.min_keep > sp.n_probs ? sp.min_keep : sp.n_probs) + 2;
      /* a lower bound on a term of bucket b (its values exceed Mc - (b + 1) span / BL_NBUCKET) */
      const float bstep = span / (float)BL_NBUCKET / T;
      int nk = 0;
      for (int pass = split ? 0 : 1;; pass++) {
        const bool head = pass == 0;
        for (int b = t; b < BL_NBUCKET; b += BL_SEL_THREADS) cnt[b] = 0u;
        if (t == 0) {
          sh.split_h = BL_NBUCKET;
          sh.split_nt = 0;
          sh.split_par = 0u;
        }
        __syncthreads();
        each_region(std::false_type{}, [&](const float *v, const int32_t *) {
#pragma unroll
          for (int u = 0; u < BL_CAND_U; u++)
            if (v[u] >= thr) atomicAdd(&cnt[bucket(v[u])], 1u);
        });
        __syncthreads();
        /* exclusive offsets: thread t owns buckets [t*PB, (t+1)*PB) */
        constexpr int PB = BL_NBUCKET / BL_SEL_THREADS;
        uint32_t loc[PB], own = 0u;
        double om = 0.0;
#pragma unroll
        for (int q = 0; q < PB; q++) {
          loc[q] = cnt[t * PB + q];
          own += loc[q];
          const int b = t * PB + q;
          if (head && b < BL_NBUCKET - 1 && loc[q]) om += (double)loc[q] * (double)__expf(-(float)(b + 1) * bstep * 1.001f) * 0.999;
        }
        const uint32_t incl = (uint32_t)bl_wscan_add((int)own, lane);
        const double mincl = head ? bl_wscan_add_d(om, lane) : 0.0;
        if (lane == 63) {
          sh.red_i[w] = (int)incl;
          sh.c.gsum[w] = mincl;
        }
        __syncthreads();
        uint32_t run = incl - own;
        double mrun = mincl - om;
        int nall = 0;
        for (int q = 0; q < SEL_NW; q++) {
          if (q < w) {
            run += (uint32_t)sh.red_i[q];
            mrun += sh.c.gsum[q];
          }
          nall += sh.red_i[q];
        }
        if (head) { /* the first bucket where the lower-bounded mass and the count both suffice */
          uint32_t cc = run;
#pragma unroll
          for (int q = 0; q < PB; q++) {
            const int b = t * PB + q;
            cc += loc[q];
            if (b < BL_NBUCKET - 1 && loc[q]) mrun += (double)loc[q] * (double)__expf(-(float)(b + 1) * bstep * 1.001f) * 0.999;
            if (mrun >= need && (int)cc >= need_c) {
              atomicMin(&sh.split_h, b);
              break;
            }
          }
        }
#pragma unroll
        for (int q = 0; q < PB; q++) {
          cnt[t * PB + q] = run;
          run += loc[q];
        }
        __syncthreads();
        int h_end = head && sh.split_h < BL_NBUCKET - 1 ? sh.split_h + 1 : BL_NBUCKET;
        bool tail = h_end < BL_NBUCKET;
        nk = tail ? (int)cnt[h_end] : nall; /* the ranked head's length */
        if (tail && nk > BL_SPLIT_HEAD_MAX) { /* a long head: every bucket is ranked (and summed by the draw) */
          h_end = BL_NBUCKET;
          tail = false;
          nk = nall;
        }
        /* the head scattered by bucket; the tail's ulps of 2^K counted (every thread's own sum is exact: at most
         * 2^23 per term) */
        const double tsc = bl_u2d((uint64_t)(23 - Kb + 1023) << 52);
        double tI = 0.0;
        if (tail) { /* a tail bucket's counter becomes its sum of u-multiples (below 2^24 when the split holds) */
          __syncthreads(); /* every thread has read nk from cnt[h_end] */
          for (int b = h_end + t; b < BL_NBUCKET; b += BL_SEL_THREADS) cnt[b] = 0u;
          __syncthreads();
        }
        each_region(std::true_type{}, [&](const float *v, const int32_t *id) {
#pragma unroll
          for (int u = 0; u < BL_CAND_U; u++)
            if (v[u] >= thr) {
              const int bk = bucket(v[u]);
              if (bk < h_end) {
                A[atomicAdd(&cnt[bk], 1u)] = ckey(v[u], id[u]);
              } else {
                const float dd = v[u] - Mc;
                const float qq = dd / T;
                const double x = (double)SEL_EXPF(qq) * tsc;
                const double fl = floor(x), fr = x - fl;
                if (fr == 0.5) {
                  const int k = atomicAdd(&sh.split_nt, 1);
                  if (k < BL_SPLIT_TIES) {
                    sh.split_tk[k] = ckey(v[u], id[u]);
                    sh.split_tf[k] = fl;
                  }
                } else {
                  const double inc = fr > 0.5 ? fl + 1.0 : fl;
                  tI += inc;
                  if (inc != 0.0) atomicAdd(&cnt[bk], (uint32_t)inc);
                }
              }
            }
        });
        __syncthreads(); /* cnt[b] is now the end of bucket b (of the head) */
        const int nt = sh.split_nt;
        if (tail) tI = block_sum_d<BL_SEL_THREADS>(tI, sh.c.gsum);
        if (tail && nt > 0 && nt <= BL_SPLIT_TIES) {
          /* bit k: the parity of the other tail terms' u-multiples before halfway term k (larger values; a
           * value equal to a halfway term's is one itself) */
          uint32_t bits = 0u;
          each_region(std::false_type{}, [&](const float *v, const int32_t *) {
#pragma unroll
            for (int u = 0; u < BL_CAND_U; u++)
              if (v[u] >= thr && bucket(v[u]) >= h_end) {
                const float dd = v[u] - Mc;
                const float qq = dd / T;
                const double x = (double)SEL_EXPF(qq) * tsc;
                const double fl = floor(x), fr = x - fl;
                if (fr != 0.5 && ((fr > 0.5 ? (uint64_t)fl + 1u : (uint64_t)fl) & 1u))
                  for (int k = 0; k < nt; k++)
                    if (v[u] > ckey_v(sh.split_tk[k])) bits ^= 1u << k;
              }
          });
          uint32_t wb = 0u;
#pragma unroll
          for (int k = 0; k < BL_SPLIT_TIES; k++) wb |= (uint32_t)(__popcll(__ballot((bits >> k) & 1u)) & 1) << k;
          if (lane == 0) sh.red_i[w] = (int)wb;
          __syncthreads();
          if (t == 0) {
            uint32_t pb = 0u;
            for (int q = 0; q < SEL_NW; q++) pb ^= (uint32_t)sh.red_i[q];
            sh.split_par = pb;
          }
          __syncthreads();
        }
        uint64_t *tile = reinterpret_cast<uint64_t *>(reinterpret_cast<char *>(&sh.n) + BL_BOFF_BYTES);
        constexpr int TU = BL_RTILE / BL_SEL_THREADS;
        uint64_t pre[TU]; /* the next tile, loaded before this tile's stores */
#pragma unroll
        for (int u = 0; u < TU; u++) pre[u] = t + u * BL_SEL_THREADS < nk ? A[t + u * BL_SEL_THREADS] : 0ull;
        for (int base = 0; base < nk; base += BL_RTILE) {
          const int n_t = min(BL_RTILE, nk - base);
#pragma unroll
          for (int u = 0; u < TU; u++) tile[t + u * BL_SEL_THREADS] = pre[u];
          __syncthreads();
#pragma unroll
          for (int u = 0; u < TU; u++) {
            const int i = base + BL_RTILE + t + u * BL_SEL_THREADS;
            pre[u] = i < nk ? A[i] : 0ull;
          }
#pragma unroll
          for (int u = 0; u < TU; u++) {
            const int i = t + u * BL_SEL_THREADS;
            if (i < n_t) {
              const uint64_t k = tile[i];
              const int bk = bucket(ckey_v(k));
              const int s0 = bk > 0 ? (int)cnt[bk - 1] : 0, e0 = (int)cnt[bk];
              int r = 0;
              if (s0 >= base && e0 <= base + n_t) {
                for (int j = s0 - base; j < e0 - base; j++) r += tile[j] > k ? 1 : 0;
              } else { /* a bucket across the tile's edge */
                for (int j = s0; j < e0; j++) r += A[j] > k ? 1 : 0;
              }
              Bk[s0 + r] = k;
            }
          }
          __syncthreads();
        }
        if (!tail) break;
        /* the head's exact sum (the draw's terms exp((v - v0) / T), v0 = Mc the first value), by wavefront 0:
         * each lane's term, 64 at a time, added in list order through readlane (every lane alike); the head
         * holds at most BL_SPLIT_HEAD_MAX entries */
        if (w == 0) {
          float Sh = 0.0f;
          for (int b0 = 0; b0 < nk; b0 += 64) {
            const int j = b0 + lane;
            float e = 0.0f;
            if (j < nk) {
              const float dd = ckey_v(Bk[j]) - Mc;
              const float qq = dd / T;
              e = SEL_EXPF(qq);
            }
            const int m = nk - b0 < 64 ? nk - b0 : 64;
            for (int k = 0; k < m; k++) Sh += sel_rl(e, k);
          }
          if (lane == 0) sh.split_s = Sh;
        }
        __syncthreads();
        const float s_head = sh.split_s;
        const double uK = bl_u2d((uint64_t)(Kb - 23 + 1023) << 52);
        bool ok = nt <= BL_SPLIT_TIES && ckey_v(Bk[0]) == Mc && (double)s_head >= bl_u2d((uint64_t)(Kb + 1023) << 52);
        if (ok && nt > 0) { /* the halfway terms in rank order (every thread alike) */
          uint32_t done = 0u, par = (uint32_t)((uint64_t)((double)s_head / uK) & 1u);
          for (int r = 0; r < nt; r++) {
            int kb = -1;
            for (int k = 0; k < nt; k++)
              if (!((done >> k) & 1u) && (kb < 0 || sh.split_tk[k] > sh.split_tk[kb])) kb = k;
            done |= 1u << kb;
            const double fl = sh.split_tf[kb];
            const uint32_t pN = par ^ ((sh.split_par >> kb) & 1u); /* N mod 2 before this term */
            const uint64_t inc = (uint64_t)fl + (((uint64_t)fl + pN) & 1u);
            tI += (double)inc;
            par ^= (uint32_t)(inc & 1u);
            if (t == 0) {
              sh.split_ti[kb] = (uint32_t)inc;
              cnt[bucket(ckey_v(sh.split_tk[kb]))] += (uint32_t)inc;
            }
          }
          __syncthreads();
        }
        const double Sfull = (double)s_head + uK * tI;
        ok = ok && Sfull < bl_u2d((uint64_t)(Kb + 1 + 1023) << 52);
        const float target = r01 * (float)Sfull;
        if (ok && target <= s_head) { /* the draw stops within the head */
          split_S = (float)Sfull;
          break;
        }
        if (ok && tail_draw_ok) {
          /* the draw stops in the tail, where the running sum is s_head + u c: at the first candidate that
           * brings c to cstar = (target - s_head) / u (an integer: both lie in binade K). The bucket where the
           * tail's prefix of u-multiples reaches cstar, then its candidates ranked in LDS and walked */
          const uint32_t cstar = (uint32_t)(((double)target - (double)s_head) / uK);
          constexpr int PB = BL_NBUCKET / BL_SEL_THREADS;
          uint32_t ls = 0u;
#pragma unroll
          for (int q = 0; q < PB; q++) ls += t * PB + q >= h_end ? cnt[t * PB + q] : 0u;
          const uint32_t li = (uint32_t)bl_wscan_add((int)ls, lane);
          if (lane == 63) sh.red_i[w] = (int)li;
          if (t == 0) {
            sh.split_h = -1;
            sh.split_ne = 0;
            sh.split_key = 0ull;
          }
          __syncthreads();
          uint32_t run = li - ls;
          for (int q = 0; q < w; q++) run += (uint32_t)sh.red_i[q];
#pragma unroll
          for (int q = 0; q < PB; q++) {
            const int b = t * PB + q;
            if (b >= h_end) {
              const uint32_t c = cnt[b];
              if (run < cstar && run + c >= cstar) {
                sh.split_h = b;
                sh.split_cb = (int)run;
              }
              run += c;
            }
          }
          __syncthreads();
          const int bs = sh.split_h;
          uint64_t *ek = tile, *sk = tile + 1536;
          uint32_t *ei = reinterpret_cast<uint32_t *>(tile + 1024), *si = reinterpret_cast<uint32_t *>(tile + 2560);
          if (bs >= 0) {
            each_region(std::true_type{}, [&](const float *v, const int32_t *id) {
#pragma unroll
              for (int u = 0; u < BL_CAND_U; u++)
                if (v[u] >= thr && bucket(v[u]) == bs) {
                  const int k = atomicAdd(&sh.split_ne, 1);
                  if (k < 1024) {
                    const uint64_t key = ckey(v[u], id[u]);
                    const float dd = v[u] - Mc;
                    const float qq = dd / T;
                    const double x = (double)SEL_EXPF(qq) * tsc;
                    const double fl = floor(x), fr = x - fl;
                    uint32_t inc = (uint32_t)(fr > 0.5 ? fl + 1.0 : fl);
                    if (fr == 0.5)
                      for (int j = 0; j < nt; j++)
                        if (sh.split_tk[j] == key) inc = sh.split_ti[j];
                    ek[k] = key;
                    ei[k] = inc;
                  }
                }
            });
            __syncthreads();
            const int ne = sh.split_ne;
            if (ne <= 1024) {
              for (int i = t; i < ne; i += BL_SEL_THREADS) {
                const uint64_t k = ek[i];
                int r = 0;
                for (int j = 0; j < ne; j++) r += ek[j] > k ? 1 : 0;
                sk[r] = k;
                si[r] = ei[i];
              }
              __syncthreads();
              if (t == 0) {
                uint32_t c = (uint32_t)sh.split_cb;
                for (int r = 0; r < ne; r++) {
                  c += si[r];
                  if (c >= cstar) {
                    const float vr = ckey_v(sk[r]);
                    /* equal values: the heap's order among them is not simulated here */
                    const bool tie = (r > 0 && ckey_v(sk[r - 1]) == vr) || (r + 1 < ne && ckey_v(sk[r + 1]) == vr);
                    if (!tie) sh.split_key = sk[r];
                    break;
                  }
                }
              }
            }
          }
          __syncthreads();
          const uint64_t ck = sh.split_key;
          __syncthreads();
          if (ck) {
            Bk[nk] = ck;
            split_tail_pos = nk;
            split_S = (float)Sfull;
            break;
          }
        }
        __syncthreads();
      }
      keys = Bk;
      nl = nk;
    }
    n_list = nl;
    if (!gram) n_logical = V;
  }
  __syncthreads();
  bool glevel_v = gram && !(mode & BL_M_TOPK); /* the list ranks the whole vocabulary (heap order of ties) */
  if (sampled && gram && gfull && !status) {
    /* the widening levels past the merged list, on the sorted candidates (every value within the span of
     * the row maximum): level k's entries are the allowed ones among the first k. A level past the list's
     * end would need tokens beyond the span: unsupported, as is the whole-vocabulary level when an allowed
     * token lies beyond the span */
    double na = 0.0;
    for (int64_t q = t; q < gwords; q += BL_SEL_THREADS) na += (double)__popc(gmk[q]);
    na = block_sum_d<BL_SEL_THREADS>(na, sh.c.gsum);
    int kk = gk;
    if (na < 1.0) { /* no level holds an allowed token: the widening ends in the rejection */
      status |= sp.g_kind == 1 ? BL_SE_JREJECT : BL_SE_GREJECT;
      kk = -1;
    }
    for (; kk >= 0;) {
      const bool vlevel = kk >= V;
      if (!vlevel && kk > n_list) {
        status |= BL_SE_UNSUPPORTED;
        break;
      }
      const int64_t lim = vlevel ? n_list : kk;
      double c = 0.0;
      for (int64_t j = t; j < lim; j += BL_SEL_THREADS) c += g_allowed(keys[j] ? ckey_i(keys[j]) : 0) ? 1.0 : 0.0;
      c = block_sum_d<BL_SEL_THREADS>(c, sh.c.gsum);
      if (c > 0.0) {
        if (vlevel && c != na) {
          status |= BL_SE_UNSUPPORTED;
          break;
        }
        glevel_v = vlevel;
        /* stable compaction of the level's allowed entries to the list's front, a tile at a time */
        int64_t off = 0;
        for (int64_t base = 0; base < lim; base += BL_SEL_THREADS) {
          const int64_t j = base + t;
          const uint64_t k = j < lim ? keys[j] : 0ull;
          const int f = j < lim && g_allowed(k ? ckey_i(k) : 0) ? 1 : 0;
          const int incl = bl_wscan_add(f, lane);
          if (lane == 63) sh.red_i[w] = incl;
          __syncthreads();
          int before = incl - f, tot = 0;
          for (int q = 0; q < SEL_NW; q++) {
            if (q < w) before += sh.red_i[q];
            tot += sh.red_i[q];
          }
          if (f) keys[off + before] = k;
          off += tot;
          __syncthreads();
        }
        n_list = n_logical = (int64_t)c;
        break;
      }
      if (vlevel) {
        status |= BL_SE_UNSUPPORTED;
        break;
      }
      kk = kk * 4 < V ? kk * 4 : V;
    }
  }
  auto val = [&](int64_t j) -> float { return keys[j] ? ckey_v(keys[j]) : -1.0e30f; };
  int64_t keep = 1;
  const bool miro = sampled && (mode & BL_M_MIRO) != 0;
  bool short_list = !miro && n_list <= BL_SERIAL_MAX;
  if (sampled && !miro) {
    if (!ranked_supported(sp, n_list, n_logical, keep)) status |= BL_SE_UNSUPPORTED;
    if (!status && short_list) ranked_terms(sp, val, n_list, sh);
  }
  /* the typical filter: complete short lists by the block (typical_filter); a full-vocabulary list, which
   * holds every value whose probability is not 0 (the candidate span keeps every value for it), inside the
   * long draw */
  bool typ = false, typ_long = false;
  int n_draw = (int)n_list;
  int64_t nlog_draw = n_logical;
  if (sampled && !miro && !status && sp.typical_p < 1.0f && n_logical > 1) {
    if (short_list && n_list == n_logical) {
      typ = true;
      n_draw = typical_filter(sp, (int)n_list, (mode & BL_M_FULL) != 0, sh, status);
      nlog_draw = n_draw;
      if (keep > n_draw) keep = n_draw;
    } else if ((mode & BL_M_FULL) && !gram) {
      typ_long = true;
      short_list = false;
    } else {
      status |= BL_SE_UNSUPPORTED;
    }
  }
  /* a draw position -> its list position */
  auto lpos = [&](int64_t j) -> int64_t { return typ ? (int64_t)sh.ser_o[j] : j; };

  if (gram && !sampled) {
    /* sample_grammar_token, greedy (src/server.br:308-361): the frontier's status, then the first
     * allowed candidate in rank order = the allowed maximum; the lowest index among equal allowed
     * maxima is top_k_select's order but not the heap rank's, so a tie is reported */
    const int gst = d.gstat[row];
    if (gst & BL_GR_FAMBIG) {
      status |= BL_SE_GAMBIG;
    } else if (gst & BL_GR_DEAD) {
      status |= BL_SE_GDEAD;
    } else if (gst & BL_GR_FORCED) {
      tok = d.eos_id;
      tokv = bl_row_value(d, sp, rows, row, slot, logits, ld, tok);
    } else if (d.gamb[row]) {
      status |= d.gamb[row] & 2 ? BL_SE_UNSUPPORTED : BL_SE_GAMBIG;
    } else {
      float gm = BL_NEG_INF;
      int gi = 0x7fffffff;
      const int64_t go = (int64_t)row * d.gm_blocks;
      for (int k = t; k < d.gm_blocks; k += BL_SEL_THREADS) argmax_merge(gm, gi, d.gm_max[go + k], d.gm_arg[go + k]);
      block_argmax<BL_SEL_THREADS>(gm, gi, sh.red_m, sh.red_i);
      double n_eq = 0.0;
      if (gi != 0x7fffffff)
        for (int k = t; k < d.gm_blocks; k += BL_SEL_THREADS)
          if (d.gm_arg[go + k] != 0x7fffffff && d.gm_max[go + k] == gm) n_eq += (double)d.gm_eq[go + k];
      n_eq = block_sum_d<BL_SEL_THREADS>(n_eq, sh.c.gsum);
      if (gi == 0x7fffffff) {
        status |= sp.g_kind == 1 ? BL_SE_JREJECT : BL_SE_GREJECT;
      } else {
        tok = gi;
        tokv = gm;
        if (n_eq > 1.0) {
          /* equal allowed maxima g: the levels rank by top_k_select (value desc, index asc) while k < V, where
           * the first allowed is the lowest index gi, found at the first level past its rank r (the keys
           * above (g, gi)); a level of V ranks by the heap (all_candidates_sorted), whose first allowed
           * among the values g comes from the extraction replay over every value >= g (sorted in LDS) */
          int res = -1;
          if (!(sp.top_n_sigma > 0.0f)) {
            uint64_t *lst = d.sortk + (int64_t)row * 2 * V;
            if (t == 0) sh.ires[5] = 0;
            __syncthreads();
            double c_gt = 0.0, c_eq = 0.0;
            for (int j = t; j < V; j += BL_SEL_THREADS) {
              const float x = bl_row_value(d, sp, rows, row, slot, logits, ld, j);
              if (x > gm) c_gt += 1.0;
              else if (x == gm && j < gi) c_eq += 1.0;
              if (x >= gm) {
                const int k = atomicAdd(&sh.ires[5], 1);
                if (k < BL_LDS_SORT) lst[k] = ckey(x, j);
              }
            }
            c_gt = block_sum_d<BL_SEL_THREADS>(c_gt, sh.c.gsum);
            c_eq = block_sum_d<BL_SEL_THREADS>(c_eq, sh.c.gsum);
            const int nge = sh.ires[5];
            const int64_t r = (int64_t)(c_gt + c_eq);
            int64_t k = sp.top_k > 0 && sp.top_k < V ? sp.top_k : V;
            while (k <= r && k < V) k = k * 4 < V ? k * 4 : V;
            if (k < V) {
              res = gi;
            } else if (nge <= BL_LDS_SORT) {
              uint64_t *hk = sh.c.keys;
              int P = 1;
              while (P < nge) P <<= 1;
              for (int i = t; i < P; i += BL_SEL_THREADS) hk[i] = i < nge ? lst[i] : 0ull;
              __syncthreads();
              bitonic_desc(hk, P);
              const int p0 = (int)c_gt; /* the values g follow every larger value */
              res = heap_extract_until([&](int64_t j) { return hk[j]; }, true, nge, V,
                                       d.full_i + (int64_t)row * d.nb * BL_EB, sh,
                                       [&](int i, int o) { return i >= p0 && g_allowed(ckey_i(hk[o])); });
            }
          }
          if (res >= 0) tok = res;
          else status |= BL_SE_TIE;
        }
      }
    }
  }

  /* the normaliser, prepared by every wavefront; then wavefront 0 chains it while wavefront 1 runs the
   * short list's sequential loops */
  if (norm_row) norm_prep(d, row, M, sh, m_pre, br_pre, n_ent);
  __syncthreads();
  if (norm_row && w == 0)
    norm_chain(d, row, sh, [&](int64_t j) { return SEL_EXPF(bl_row_value(d, sp, rows, row, slot, logits, ld, (int32_t)j) - M); });
  if (sampled && !status && short_list && split_tail_pos < 0 && w == 1) {
    const sel_draw r = ranked_serial(sp, n_draw, nlog_draw, keep, rng, skip, typ, split_S, sh, &sh.rng_out);
    if (lane == 0) sh.draw = r;
  }
  __syncthreads();
  const float S_norm = sh.n.S; /* the normaliser's LDS is scratch from here on (heap ties) */
  float ad_ws = 0.0f, ad_tw = 0.0f; /* adaptive-p's next running sums */
  if (adapt && !status) {
    __syncthreads();
    const float lse1 = SEL_LOGF(S_norm);
    tok = sample_adaptive(d, sp, rows, row, slot, logits, ld, M, lse1, rng, sh, ad_ws, ad_tw);
    tokv = bl_row_value(d, sp, rows, row, slot, logits, ld, tok);
  }
  sel_draw dr;
  dr.pos = -1;
  dr.first = dr.cut = 0;
  dr.S = 0.0f;
  const float *dterm = sh.ser_r; /* the draw's term of position j: dterm[j - dshift] */
  int64_t dshift = 0;
  if (sampled && !status) {
    int pos;
    if (split_tail_pos >= 0) { /* drawn in the tail of a plain draw's list (above) */
      dr.pos = pos = split_tail_pos;
      dr.first = 0;
      dr.cut = (int)n_logical;
      dr.S = split_S;
      rng = split_rng;
    } else if (short_list) {
      dr = sh.draw;
      pos = dr.pos;
      if (pos == -2 || pos >= n_draw) {
        status |= BL_SE_UNSUPPORTED;
        pos = dr.pos = -1;
      } else {
        rng = sh.rng_out;
        pos = (int)lpos(pos);
      }
    } else {
      bl_grec *recs = sh.c.recs;
      double *gsum = sh.c.gsum;
      if ((n_list + 63) / 64 > BL_LDS_SORT / 64) {
        recs = reinterpret_cast<bl_grec *>(d.grec) + (int64_t)row * 2 * (V / 64 + 64) + (V / 64 + 64);
        gsum = d.gsum + (int64_t)row * (V / 64 + 64);
      }
      float *tbuf = reinterpret_cast<float *>(d.sortk + (int64_t)row * 2 * V); /* free once the list is sorted */
      dr = miro ? sample_mirostat(sp, val, n_list, n_logical, mk, rng, skip, recs, gsum, tbuf, sh, status)
                : sample_ranked_long(sp, val, n_list, n_logical, keep, rng, skip, split_S, recs, gsum, tbuf, sh, status,
                                     typ_long ? keys : nullptr, reinterpret_cast<int32_t *>(d.full_v) + (int64_t)row * d.nb * BL_EB,
                                     d.full_i + (int64_t)row * d.nb * BL_EB);
      pos = dr.pos;
      dterm = tbuf;
      dshift = dr.first;
    }
    /* dr.pos stays a draw position; pos is the list position */
    if (pos >= 0) {
      const uint64_t kp = keys[pos];
      tok = kp ? ckey_i(kp) : 0;
      tokv = kp ? ckey_v(kp) : bl_row_value(d, sp, rows, row, slot, logits, ld, tok);
      /* the heap rank orders equal values its own way (src/sampling.br:310-364): a draw on a tie takes
       * the heap's token (or reports the tie when the simulation does not fit) */
      if ((mode & BL_M_FULL) || glevel_v) {
        const float vp = val(pos);
        if ((pos > 0 && val(pos - 1) == vp) || (pos + 1 < n_list && val(pos + 1) == vp)) {
          int hid = -1;
          if (gram) {
            /* a grammar row's list is the heap order of the whole row restricted to its allowed tokens: the
             * (pos - a0)-th allowed token among the values vp in the extraction order of every value >= vp
             * (collected and sorted in LDS, at most 4096), a0 the list's first position of value vp */
            int64_t lo = 0, hi = pos;
            while (lo < hi) {
              const int64_t mid = (lo + hi) >> 1;
              if (val(mid) == vp) hi = mid;
              else lo = mid + 1;
            }
            const int q = (int)(pos - lo);
            uint64_t *lst = d.sortk + (int64_t)row * 2 * V; /* the list itself is past it, or in LDS */
            __syncthreads();
            if (t == 0) sh.ires[5] = 0;
            __syncthreads();
            double c_gt = 0.0;
            for (int j = t; j < V; j += BL_SEL_THREADS) {
              const float x = bl_row_value(d, sp, rows, row, slot, logits, ld, j);
              if (x > vp) c_gt += 1.0;
              if (x >= vp) {
                const int k = atomicAdd(&sh.ires[5], 1);
                if (k < BL_LDS_SORT) lst[k] = ckey(x, j);
              }
            }
            c_gt = block_sum_d<BL_SEL_THREADS>(c_gt, sh.c.gsum);
            const int nge = sh.ires[5];
            if (nge <= BL_LDS_SORT) {
              uint64_t *hk = sh.c.keys; /* the list is not read again */
              int P = 1;
              while (P < nge) P <<= 1;
              __syncthreads();
              for (int i = t; i < P; i += BL_SEL_THREADS) hk[i] = i < nge ? lst[i] : 0ull;
              __syncthreads();
              bitonic_desc(hk, P);
              const int p0 = (int)c_gt;
              int seen = 0; /* the replay runs on one lane */
              hid = heap_extract_until([&](int64_t j) { return hk[j]; }, true, nge, V,
                                       d.full_i + (int64_t)row * d.nb * BL_EB, sh, [&](int i, int o) {
                                         if (i < p0 || !g_allowed(ckey_i(hk[o]))) return false;
                                         if (seen == q) return true;
                                         seen++;
                                         return false;
                                       });
            }
          } else if (!typ_long) { /* a typical row's list is compacted: the heap's prefix is gone (a tie) */
            hid = heap_tie_id([&](int64_t j) { return keys[j]; }, keys == sh.c.keys, n_list, pos, V,
                              d.full_i + (int64_t)row * d.nb * BL_EB, sh);
          }
          if (hid >= 0) tok = hid;
          else status |= BL_SE_TIE;
        }
      }
    }
  }

  /* post-sampling probabilities (src/server.br:1015-1025): the drawn token's and those of the first
   * n_probs candidates of the drawn range, each its term over the range's sum (src/sampling.br:600-607);
   * a greedy row has the one probability 1 (src/sampling.br:753-755), a grammar row none. Equal values
   * next to the listed positions of a full-vocabulary rank stand in the heap's order: reported as a tie */
  const bool psp_row = (mode & BL_M_PSP) && rows.lp;
  const int n_alt = sp.n_probs < rows.top_stride ? sp.n_probs : rows.top_stride;
  int psp_n = 0;
  float psp_tok = 0.0f;
  if (psp_row) {
    if (sampled && !gram) {
      if (!status) {
        const int64_t avail = (int64_t)dr.cut - dr.first;
        psp_n = (int)(avail < n_alt ? avail : n_alt);
        if (dr.first + psp_n > (typ ? n_draw : n_list)) status |= BL_SE_UNSUPPORTED;
      }
      if (t == 0) sh.ires[6] = 0;
      __syncthreads();
      if (!status && (mode & BL_M_FULL) && t <= psp_n) {
        const int64_t j = dr.first + t;
        if (j >= 1 && j < (typ ? n_draw : n_list) && val(lpos(j - 1)) == val(lpos(j))) sh.ires[6] = 1;
      }
      __syncthreads();
      if (sh.ires[6]) status |= BL_SE_TIE;
      if (!status) psp_tok = dterm[dr.pos - dshift] / dr.S;
    } else if (!gram) {
      psp_n = n_alt > 0 ? 1 : 0;
      psp_tok = 1.0f;
    }
    if (t < n_alt) {
      int32_t id = -1;
      float pv = 0.0f;
      if (t < psp_n && !status) {
        if (sampled) {
          const int64_t j = dr.first + t, lj = lpos(j);
          id = keys[lj] ? ckey_i(keys[lj]) : 0;
          pv = dterm[j - dshift] / dr.S;
        } else {
          id = tok;
          pv = 1.0f;
        }
      }
      rows.top_ids[(int64_t)row * rows.top_stride + t] = id;
      rows.top_lp[(int64_t)row * rows.top_stride + t] = pv;
    }
  }

  /* outputs, logprobs (src/server.br:1027-1035): alternatives = the first n_probs of the merged list */
  const float lse = lp_row ? SEL_LOGF(S_norm) : 0.0f; /* sum_exp.ln(), glibc's logf (src/sampling.br:265) */
  if (lp_row) {
    const int n = sp.n_probs < rows.top_stride ? sp.n_probs : rows.top_stride;
    if (t < n) {
      const uint64_t k = t < K ? mk : 0ull;
      const float v = k ? ckey_v(k) : -1.0e30f;
      rows.top_ids[(int64_t)row * rows.top_stride + t] = k ? ckey_i(k) : 0;
      rows.top_lp[(int64_t)row * rows.top_stride + t] = (v - M) - lse;
    }
  }
  /* the rest of the row's alternatives (past its n_probs, or all of a row without logprobs): id -1, 0 */
  if (rows.lp && t < rows.top_stride && !(lp_row && t < sp.n_probs) && !(psp_row && t < n_alt)) {
    rows.top_ids[(int64_t)row * rows.top_stride + t] = -1;
    rows.top_lp[(int64_t)row * rows.top_stride + t] = 0.0f;
  }
  if (t == 0) {
    rows.tok[row] = status ? -1 : tok; /* a failed row has no token; its status stays sticky in the slot */
    if (rows.status) rows.status[row] = status;
    if (rows.lp) rows.lp[row] = lp_row ? (tokv - M) - lse : psp_row ? psp_tok : 0.0f;
    bool is_eog = false;
    for (int k = 0; k < n_eog; k++) is_eog |= (k < BL_EOG_LDS ? sh.eog[k] : d.eog[k]) == tok;
    if (rows.commit && status == 0) {
      /* tokens.push (src/server.br:1004): repeat window; reply_tokens.push unless EOG (:1037) */
      sp.n_tokens = n_tokens0 + 1;
      if (rep_on) {
        if (rl > 0) {
          int32_t *ring = d.ring + (int64_t)slot * BL_WCAP;
          if (ring_full) {
            bl_rec_get(d, slot, ring_old)->wf -= 1u;
            ring[win_head] = tok;
            sp.win_head = (win_head + 1) % rl;
          } else {
            ring[(win_head + win_len) % rl] = tok;
            sp.win_len = win_len + 1;
          }
        }
        bl_rec_get(d, slot, tok)->wf += 1u;
      }
      if (!is_eog) {
        sp.n_reply = n_reply0 + 1;
        if (fp_on) bl_rec_get(d, slot, tok)->cnt += 1;
        if (g_on) grammar_commit(d, sp, d.gram[slot], tok, slot);
      }
      bl_dry_push(d, sp, slot, tok);
      sp.rng = rng;
      if (mode & BL_M_MIRO) sp.mu = sh.fres[6];
      if (adapt) {
        sp.adapt_ws = ad_ws;
        sp.adapt_tw = ad_tw;
      }
      sh.ires[7] = 1;
    } else {
      sh.ires[7] = 0;
    }
    if (status) sp.err |= status;
  }
  if (sp.dry_on) { /* the next step's DRY penalties, from the window with this step's token */
    __syncthreads();
    const bool pushed = sh.ires[7] != 0;
    __syncthreads();
    static_assert(sizeof(sel_shared) >= BL_DRY_LDS, "DRY scratch");
    if (pushed) dry_update(d, sp, slot, reinterpret_cast<unsigned char *>(&sh));
  }
}

/* ------------------------------------------------------------------ synthetic inputs for the benchmark */
__global__ void bl_k_synth(float *out, int64_t ld, int cfg, int64_t seed, int64_t step0, int rows, int V) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int r = blockIdx.y;
  if (i >= V) return;
  int64_t step = step0;
  uint64_t st = bl_stream((uint32_t)cfg, seed, step, r, BL_P_LOGIT);
  out[(int64_t)r * ld + i] = bl_normal(st, (uint64_t)i, bl_cfg_sigma(cfg));
}

/* ------------------------------------------------------------------ host-side launchers */
/* one kernel of the step; with a pair of timing events, an extended launch that records the kernel's own
 * start and end (its execution alone, as a profiler's kernel trace reports it) */
template <typename F, typename... Args>
static void step_launch(F k, dim3 g, dim3 b, hipStream_t s, hipEvent_t *ev, Args... args) {
  if (ev)
    hipExtLaunchKernelGGL(k, g, b, 0, s, ev[0], ev[1], 0, args...);
  else
    hipLaunchKernelGGL(k, g, b, 0, s, args...);
}

/* ev: optional 6 events, the start and end of the row pass, the exponent pass and the selection kernel
 * (kernel timing for the benchmark) */
void bl_launch_step(const bl_dev &d, const float *logits, int64_t ld, const bl_rows &rows_in, int B, bool need_pass2,
                    bool need_gram, hipStream_t s, hipEvent_t *ev) {
  bl_rows rows = rows_in;
  rows.merged = need_pass2 ? 1 : 0;
  const dim3 g1(d.nc, B), g2(d.nb + 1, B), t1(BL_RP_THREADS);
  if (rows.delta)
    step_launch(bl_k_rowpass_spec, g1, t1, s, ev, d, logits, ld, rows);
  else
    step_launch(bl_k_rowpass, g1, t1, s, ev, d, logits, ld, rows);
  if (need_gram) hipLaunchKernelGGL(bl_k_gmask, dim3(d.gm_blocks, B), dim3(BL_GM_THREADS), 0, s, d, logits, ld, rows, 1);
  if (need_pass2) {
    if (rows.delta)
      step_launch(bl_k_exppass_spec, g2, t1, s, ev ? ev + 2 : nullptr, d, logits, ld, rows);
    else
      step_launch(bl_k_exppass, g2, t1, s, ev ? ev + 2 : nullptr, d, logits, ld, rows);
  }
  step_launch(bl_k_select, dim3(B), dim3(BL_SEL_THREADS), s, ev ? ev + 4 : nullptr, d, logits, ld, rows);
}

/* the allow-mask of one slot's current position, without a step (bl_grammar_mask); rows.slot[0] is
 * the slot, row 0's mask and status are written */
__global__ void bl_k_gclear(bl_dev d) {
  if (threadIdx.x == 0) d.gamb[0] = 0;
}
void bl_launch_gmask(const bl_dev &d, const bl_rows &rows, hipStream_t s) {
  hipLaunchKernelGGL(bl_k_gclear, dim3(1), dim3(64), 0, s, d);
  hipLaunchKernelGGL(bl_k_gmask, dim3(d.gm_blocks, 1), dim3(BL_GM_THREADS), 0, s, d, (const float *)nullptr, (int64_t)0,
                     rows, 0);
}

void bl_launch_dry_prime(const bl_dev &d, int slot, hipStream_t s) {
  hipLaunchKernelGGL(bl_k_dry_prime, dim3(1), dim3(BL_SEL_THREADS), 0, s, d, slot);
}

void bl_launch_synth(float *out, int64_t ld, int cfg, int64_t seed, int64_t step, int rows, int V, hipStream_t s) {
  dim3 g((V + 255) / 256, rows);
  hipLaunchKernelGGL(bl_k_synth, g, dim3(256), 0, s, out, ld, cfg, seed, step, rows, V);
}

/* ------------------------------------------------------------------ math self-test */
/* Digest of f over input bit patterns [b*2^20, (b+1)*2^20): sum of splitmix(u << 32 | bits(f(u))). */
/* exponent of the two-argument powf family: a multiple of 1/512 in [-8, 8] hashed from the input */
__device__ inline float bl_digest_pow_y(uint32_t u) {
  return (float)((int)((bl_splitmix(u) >> 40) % 8193u) - 4096) * 0x1p-9f;
}
__global__ void bl_k_math_digest(int fn, uint32_t first_block, unsigned long long *out) {
  const uint32_t blk = first_block + blockIdx.y;
  const uint32_t base = blk << 20;
  uint64_t h = 0;
  for (int k = 0; k < 16; k++) {
    uint32_t u = base + (uint32_t)(blockIdx.x * 4096 + k * 256 + threadIdx.x);
    float x = bl_u2f(u);
    float y;
    if (fn == 0) y = bl_expf(x);
    else if (fn == 1) y = bl_tanhf(x);
    else if (fn == 2) y = bl_logf(x);
    else if (fn == 3) y = bl_powf(x, 0.7f);
    else if (fn == 4) y = bl_powf(2.0f, x);
    else y = bl_powf(x, bl_digest_pow_y(u));
    uint32_t yb = y != y ? 0x7fc00000u : bl_f2u(y); /* NaN payloads are not part of the path */
    h += bl_splitmix(((uint64_t)u << 32) | yb);
  }
#pragma unroll
  for (int k = 32; k >= 1; k >>= 1) h += (uint64_t)__shfl_xor((long long)h, k, 64);
  if ((threadIdx.x & 63) == 0) atomicAdd(out + blockIdx.y, (unsigned long long)h);
}

__global__ void bl_k_zero_u64(unsigned long long *p, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0ull;
}

void bl_launch_math_digest(int fn, uint32_t first_block, int n_blocks, unsigned long long *out, hipStream_t s) {
  hipLaunchKernelGGL(bl_k_zero_u64, dim3((n_blocks + 255) / 256), dim3(256), 0, s, out, n_blocks);
  hipLaunchKernelGGL(bl_k_math_digest, dim3(256, n_blocks), dim3(256), 0, s, fn, first_block, out);
}
