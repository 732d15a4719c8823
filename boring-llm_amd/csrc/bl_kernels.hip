/*
 * bl_kernels.hip — HIP kernels of one token-selection step for B slots (gfx950, wave64).
 *
 *   bl_k_rowpass  grid (chunks, B) x 256: reads each logits row once (float4), applies the model tail
 *                 (logit_mul, soft-cap), then the server's per-token stages at the touched bits
 *                 (logit_bias -> ignore_eos suppression -> frequency/presence -> repeat penalty,
 *                 src/server.br:940-944, src/sampling.br:65-107,175-237), writes the transformed
 *                 row, and per chunk: max + first argmax, an approximate exp-sum, and a candidate
 *                 superset of the chunk's top-K (one 12-bit histogram pass; exact refinement only
 *                 when one bin is crowded).
 *   bl_k_exppass  grid (chunks, B) x 256, rows with logprobs or full-vocabulary sampling: exact
 *                 exp(x - max) terms (glibc-identical expf), the sequential-sum records of the
 *                 index-order normaliser (src/sampling.br:254-266) per 64-term group and per chunk,
 *                 each thread composing 16 consecutive terms in registers; and the candidates of a
 *                 full-vocabulary rank (every token within 17.5*max(T,1) of the max: the others cannot
 *                 change any float32 sum of the chain).
 *   bl_k_select   grid (B, 2) x 1024: workgroup 0 of a row samples (greedy / top-k / full-vocabulary
 *                 candidate sampling with exact sequential sums, src/sampling.br:490-607, the draw from
 *                 the slot's xorshift stream, the history commit of src/server.br:1004, :1037);
 *                 workgroup 1 walks the normaliser and writes the logprob alternatives
 *                 (src/server.br:1027-1035). Whichever finishes second writes the chosen token's
 *                 logprob (a counter hand-off; neither waits for the other).
 * No MFMA: the work is bandwidth- and latency-bound scanning, selection and integer arithmetic.
 */
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bl_exact.h"
#include "bl_internal.h"
#include "bl_math.h"
#include "bl_synth.h"

#define BL_NEG_INF (-__builtin_inff())

__device__ __forceinline__ const bl_slot_dev &slot_of(const bl_dev &d, int s) { return d.slots[s]; }

/* ------------------------------------------------------------------ block helpers */
__device__ __forceinline__ void argmax_merge(float &m, int &mi, float m2, int mi2) {
  if (m2 > m || (m2 == m && mi2 < mi)) {
    m = m2;
    mi = mi2;
  }
}

template <int NT>
__device__ void block_argmax(float &m, int &mi, float *sm, int *si) {
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
__device__ double block_sum_d(double x, double *sd) {
  int t = threadIdx.x, lane = t & 63, w = t >> 6;
  x = bl_wave_sum_d(x);
  if (lane == 0) sd[w] = x;
  __syncthreads();
  double r = 0.0;
  for (int k = 0; k < NT / 64; k++) r += sd[k];
  __syncthreads();
  return r;
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

/*
 * Histogram bin search from the top: bins [0, nb) of `hist`; writes res[0] = the bin b where the count
 * of keys in bins >= b first reaches `need`, res[1] = the count in bins above b, res[2] = the count in
 * b, res[3] = the total. NT threads, each owning nb/NT consecutive bins (thread 0 the highest).
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
  if (t == 0) res[3] = total;
  if (above < need && above + local >= need) {
    uint32_t acc = above;
    for (int q = 0; q < per; q++) {
      int b = nb - 1 - (t * per + q);
      uint32_t h = hist[b];
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

/* ------------------------------------------------------------------ K1: row pass */
__global__ __launch_bounds__(BL_RP_THREADS) void bl_k_rowpass(bl_dev d, const float *__restrict__ logits, int64_t ld,
                                                              bl_rows rows) {
  const int V = d.vocab, nc = d.nc;
  const int c = blockIdx.x, row = blockIdx.y, t = threadIdx.x;
  const int slot = rows.slot[row];
  const bl_slot_dev &sp = slot_of(d, slot);
  __shared__ float xs[BL_CH];
  __shared__ uint32_t hist[4096];
  __shared__ float red_m[4];
  __shared__ int red_i[4];
  __shared__ double red_d[4];
  __shared__ uint32_t res[4], wsum[4];
  __shared__ int out_n, wcnt_eq[4];

  const int i0 = c * BL_CH;
  const int cnt = min(BL_CH, V - i0);
  const float *src = logits + (int64_t)row * ld + i0;
  if (c == 0 && t == 0) {
    /* consumed by later kernels of this step */
    d.full_n[row] = 0;
    d.done[row] = 0;
    if (rows.status) rows.status[row] = 0;
  }
  /* model tail (src/model.br:973-984), applied in registers by the thread that loads the value */
  const float lmul = sp.logit_mul, cap = sp.final_softcap;
  const bool tail = lmul != 1.0f || cap > 0.0f;
  auto finish = [&](float x) {
    if (lmul != 1.0f) x = x * lmul;
    if (cap > 0.0f) {
      float q = x / cap;
      x = cap * bl_tanhf(q);
    }
    return x;
  };
  if (cnt == BL_CH && (((uintptr_t)src) & 15) == 0) {
#pragma unroll
    for (int j = 0; j < BL_CH / (4 * BL_RP_THREADS); j++) {
      float4 v = reinterpret_cast<const float4 *>(src)[j * BL_RP_THREADS + t];
      if (tail) {
        v.x = finish(v.x);
        v.y = finish(v.y);
        v.z = finish(v.z);
        v.w = finish(v.w);
      }
      reinterpret_cast<float4 *>(xs)[j * BL_RP_THREADS + t] = v;
    }
  } else {
    for (int i = t; i < cnt; i += BL_RP_THREADS) xs[i] = tail ? finish(src[i]) : src[i];
  }
  __syncthreads();
  /* server stages at the touched tokens of this chunk */
  {
    const uint32_t *tw = d.touched + (int64_t)slot * d.words + (i0 >> 5);
    const int nwords = (cnt + 31) >> 5;
    const int64_t so = (int64_t)slot * V;
    const bool fp = sp.fp_on && sp.n_reply > 0;
    const bool rp = sp.rep_on && sp.n_tokens > 0;
    for (int w = t; w < nwords; w += BL_RP_THREADS) {
      uint32_t bits = tw[w];
      while (bits) {
        int b = __ffs(bits) - 1;
        bits &= bits - 1;
        int li = w * 32 + b;
        if (li >= cnt) break;
        int64_t id = so + i0 + li;
        float x = xs[li];
        uint32_t f = d.flags[id];
        if (f & BL_TF_BIAS) x = x + d.bias[id];
        if (f & BL_TF_SUPPRESS) x = -1000000000.0f;
        if (fp) {
          int cc = d.cnt[id];
          if (cc > 0) {
            float tcf = (float)cc * sp.frequency_penalty;
            x = x - tcf;
            x = x - sp.presence_penalty;
          }
        }
        if (rp && d.wcnt[id] > 0) x = x > 0.0f ? x / sp.repeat_penalty : x * sp.repeat_penalty;
        xs[li] = x;
      }
    }
  }
  __syncthreads();
  /* transformed row */
  {
    float *dst = d.eff + (int64_t)row * V + i0;
    if (cnt == BL_CH) {
#pragma unroll
      for (int j = 0; j < BL_CH / (4 * BL_RP_THREADS); j++)
        reinterpret_cast<float4 *>(dst)[j * BL_RP_THREADS + t] = reinterpret_cast<float4 *>(xs)[j * BL_RP_THREADS + t];
    } else {
      for (int i = t; i < cnt; i += BL_RP_THREADS) dst[i] = xs[i];
    }
  }
  /* max, first argmax, approximate exp-sum */
  float m = BL_NEG_INF;
  int mi = 0x7fffffff;
  for (int i = t; i < cnt; i += BL_RP_THREADS) {
    float x = xs[i];
    if (x > m) {
      m = x;
      mi = i;
    }
  }
  block_argmax<BL_RP_THREADS>(m, mi, red_m, red_i);
  double s = 0.0;
  if (m > BL_NEG_INF)
    for (int i = t; i < cnt; i += BL_RP_THREADS) s += (double)__expf(xs[i] - m);
  s = block_sum_d<BL_RP_THREADS>(s, red_d);
  const int64_t o = (int64_t)row * nc + c;
  if (t == 0) {
    d.c_max[o] = m;
    d.c_arg[o] = mi == 0x7fffffff ? i0 : i0 + mi;
    d.c_sum[o] = (float)s;
  }

  /*
   * Candidates for top_k_select (src/sampling.br:280-296: values > -1e30, (value desc, index asc)).
   * Emit every element of the chunk whose order key reaches the edge of the histogram bin holding the
   * K-th largest: at least K elements, so the row's top-K lies in the union of the chunks' emissions
   * that reach the largest edge. A crowded bin is refined to the exact K-th key and cut by index.
   */
  const int K = sp.k_sel;
  if (K <= 0) return;
  const int64_t cbase = o * BL_CCAP;
  for (int b = t; b < 4096; b += BL_RP_THREADS) hist[b] = 0u;
  if (t == 0) out_n = 0;
  __syncthreads();
  for (int i = t; i < cnt; i += BL_RP_THREADS) {
    float x = xs[i];
    if (x > -1.0e30f) atomicAdd(&hist[bl_fkey(x) >> 20], 1u);
  }
  __syncthreads();
  block_find_bin<BL_RP_THREADS>(hist, 4096, (uint32_t)K, res, wsum);
  const uint32_t total = res[3];
  if (total <= (uint32_t)K || res[1] + res[2] <= (uint32_t)(K + 32)) {
    /* every valid key (total <= K) or every key in bins >= b */
    const uint32_t edge = total <= (uint32_t)K ? 1u : (res[0] << 20);
    for (int i = t; i < cnt; i += BL_RP_THREADS) {
      float x = xs[i];
      if (x > -1.0e30f && bl_fkey(x) >= edge) {
        int pos = atomicAdd(&out_n, 1);
        if (pos < BL_CCAP) {
          d.cand_v[cbase + pos] = x;
          d.cand_i[cbase + pos] = i0 + i;
        }
      }
    }
    __syncthreads();
    if (t == 0) {
      d.c_cnt[o] = min(out_n, BL_CCAP);
      d.c_edge[o] = edge;
    }
    return;
  }
  /* crowded bin: the exact K-th key by two more 10-bit passes within bin res[0] */
  uint32_t prefix = res[0] << 20, pmask = 0xfff00000u;
  int need = K - (int)res[1];
  for (int pass = 0; pass < 2; pass++) {
    const int shift = pass == 0 ? 10 : 0;
    __syncthreads();
    for (int b = t; b < 1024; b += BL_RP_THREADS) hist[b] = 0u;
    __syncthreads();
    for (int i = t; i < cnt; i += BL_RP_THREADS) {
      float x = xs[i];
      if (x > -1.0e30f) {
        uint32_t k = bl_fkey(x);
        if ((k & pmask) == prefix) atomicAdd(&hist[(k >> shift) & 1023u], 1u);
      }
    }
    __syncthreads();
    block_find_bin<BL_RP_THREADS>(hist, 1024, (uint32_t)need, res, wsum);
    prefix |= res[0] << shift;
    pmask |= 1023u << shift;
    need -= (int)res[1];
  }
  const uint32_t kth = prefix;
  const bool cut_ties = (int)res[2] > need;
  int eq_before = 0;
  for (int s0 = 0; s0 < cnt; s0 += BL_RP_THREADS) {
    int i = s0 + t;
    bool ok = false, eq = false;
    if (i < cnt) {
      float x = xs[i];
      if (x > -1.0e30f) {
        uint32_t k = bl_fkey(x);
        if (k > kth) ok = true;
        else if (k == kth) eq = true;
      }
    }
    if (cut_ties) {
      unsigned long long bm = __ballot(eq);
      int lane = t & 63, w = t >> 6;
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
      if (pos < BL_CCAP) {
        d.cand_v[cbase + pos] = xs[i];
        d.cand_i[cbase + pos] = i0 + i;
      }
    }
  }
  __syncthreads();
  if (t == 0) {
    d.c_cnt[o] = min(out_n, BL_CCAP);
    d.c_edge[o] = kth;
  }
}

/* ------------------------------------------------------------------ K2: exponent pass */
#define XPAD(i) ((i) + ((i) >> 4)) /* 16 consecutive terms per thread without LDS bank conflicts */

__global__ __launch_bounds__(BL_RP_THREADS) void bl_k_exppass(bl_dev d, bl_rows rows) {
  const int V = d.vocab, nc = d.nc;
  const int c = blockIdx.x, row = blockIdx.y, t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int slot = rows.slot[row];
  const bl_slot_dev &sp = slot_of(d, slot);
  const int mode = sp.mode;
  if (!(mode & (BL_M_LOGPROBS | BL_M_FULL))) return;
  __shared__ float xs[BL_CH + BL_CH / 16];
  __shared__ float red_m[4];
  __shared__ int red_i[4];
  __shared__ double red_d[4];
  __shared__ bl_inc wred[4][2];
  const int i0 = c * BL_CH;
  const int cnt = min(BL_CH, V - i0);
  const float *src = d.eff + (int64_t)row * V + i0;
  if (cnt == BL_CH) {
#pragma unroll
    for (int j = 0; j < BL_CH / (4 * BL_RP_THREADS); j++) {
      int p = (j * BL_RP_THREADS + t) * 4;
      float4 v = reinterpret_cast<const float4 *>(src)[j * BL_RP_THREADS + t];
      int q = XPAD(p);
      xs[q] = v.x;
      xs[q + 1] = v.y;
      xs[q + 2] = v.z;
      xs[q + 3] = v.w;
    }
  } else {
    for (int i = t; i < BL_CH; i += BL_RP_THREADS) xs[XPAD(i)] = i < cnt ? src[i] : BL_NEG_INF;
  }
  /* row max from the chunk statistics; its barriers also publish xs */
  float M = BL_NEG_INF;
  int Mi = 0x7fffffff;
  for (int k = t; k < nc; k += BL_RP_THREADS) argmax_merge(M, Mi, d.c_max[(int64_t)row * nc + k], k);
  block_argmax<BL_RP_THREADS>(M, Mi, red_m, red_i);

  if (mode & BL_M_LOGPROBS) {
    /* approximate sum before this chunk, from the row pass statistics */
    double part = 0.0;
    for (int k = t; k < c; k += BL_RP_THREADS) {
      float cm = d.c_max[(int64_t)row * nc + k];
      if (cm > BL_NEG_INF) part += (double)d.c_sum[(int64_t)row * nc + k] * exp((double)cm - (double)M);
    }
    const double S0 = block_sum_d<BL_RP_THREADS>(part, red_d);
    /* this thread's 16 consecutive exact terms */
    float a[16];
    double sa = 0.0;
#pragma unroll
    for (int k = 0; k < 16; k++) {
      int i = t * 16 + k;
      a[k] = i < cnt ? bl_expf(xs[XPAD(i)] - M) : 0.0f;
      sa += (double)a[k];
    }
    double tot;
    double before = S0 + block_excl_scan_d<BL_RP_THREADS>(sa, red_d, &tot);
    /* group record (4 threads per group; the group starts at its first thread's prefix) */
    double gstart = __shfl(before, lane & ~3, 64);
    uint32_t gmask;
    int E = bl_choose_binades(gstart, &gmask);
    bl_grec r;
    r.E = E;
    r.mask = gmask;
#pragma unroll
    for (int k = 0; k < 2; k++) {
      bl_inc f = ((gmask >> k) & 1u) ? bl_thread_compose<16>(a, E + k) : bl_inc_ident();
      r.v[k] = bl_quad_compose(f, lane);
    }
    bl_grec *grec = reinterpret_cast<bl_grec *>(d.grec) + (int64_t)row * 2 * (V / 64 + 64) + (int64_t)c * 64;
    if ((lane & 3) == 0 && i0 + t * 16 < V) grec[t >> 2] = r;
    /* chunk record: ordered composition of the 256 thread runs */
    uint32_t cmask;
    int Ec = bl_choose_binades(S0, &cmask);
    bl_inc fc[2];
#pragma unroll
    for (int k = 0; k < 2; k++) {
      bl_inc f = ((cmask >> k) & 1u) ? bl_thread_compose<16>(a, Ec + k) : bl_inc_ident();
      fc[k] = bl_wave_reduce(f, lane);
    }
    if (lane == 0) {
      wred[w][0] = fc[0];
      wred[w][1] = fc[1];
    }
    __syncthreads();
    if (t == 0) {
      bl_grec cr;
      cr.E = Ec;
      cr.mask = cmask;
      for (int k = 0; k < 2; k++) {
        bl_inc f = wred[0][k];
        for (int q = 1; q < BL_RP_THREADS / 64; q++) f = bl_compose(f, wred[q][k]);
        cr.v[k] = f;
      }
      reinterpret_cast<bl_grec *>(d.crec)[(int64_t)row * nc + c] = cr;
    }
  }
  if (mode & BL_M_FULL) {
    float T = sp.temperature;
    float span = 17.5f * (T > 1.0f ? T : 1.0f);
    float thr = M - span;
    for (int i = t; i < cnt; i += BL_RP_THREADS) {
      float x = xs[XPAD(i)];
      if (x >= thr) {
        int pos = atomicAdd(&d.full_n[row], 1);
        if (pos < V) {
          d.full_v[(int64_t)row * V + pos] = x;
          d.full_i[(int64_t)row * V + pos] = i0 + i;
        }
      }
    }
  }
}

/* ------------------------------------------------------------------ K3: per-row selection */
#define SEL_NW (BL_SEL_THREADS / 64)
#define SEL_LIST 4096 /* merged / full candidate lists held in LDS */

/* candidate list order: composite key (fkey(value) << 32) | ~index, sorted descending */
__device__ __forceinline__ uint64_t ckey(float v, int32_t id) {
  return ((uint64_t)bl_fkey(v) << 32) | (uint64_t)(0xffffffffu - (uint32_t)id);
}
__device__ __forceinline__ float ckey_v(uint64_t k) { return bl_fkey_inv((uint32_t)(k >> 32)); }
__device__ __forceinline__ int32_t ckey_i(uint64_t k) { return (int32_t)(0xffffffffu - (uint32_t)k); }

__device__ void bitonic_desc(uint64_t *s, int P) {
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

struct sel_shared {
  uint64_t keys[SEL_LIST]; /* merged top-K list, or a full-vocabulary list */
  bl_grec recs[SEL_LIST / 64];
  double sd[SEL_NW];
  float fres[4];
  int ires[4];
  uint64_t ures[2];
  uint32_t ucnt;
  float red_m[SEL_NW];
  int red_i[SEL_NW];
};

/* the row's top-K by (value desc, index asc) from the row pass candidates; returns its length */
__device__ int merge_topk(const bl_dev &d, int row, sel_shared &sh, int &status) {
  const int nc = d.nc, t = threadIdx.x;
  const int64_t ro = (int64_t)row * nc;
  /* largest edge: every key of the row's top-K reaches it */
  uint32_t tau = 0u;
  for (int k = t; k < nc; k += BL_SEL_THREADS)
    if (d.c_cnt[ro + k] > 0) tau = max(tau, d.c_edge[ro + k]);
#pragma unroll
  for (int k = 32; k >= 1; k >>= 1) tau = max(tau, (uint32_t)__shfl_xor((int)tau, k, 64));
  if ((t & 63) == 0) sh.red_i[t >> 6] = (int)tau;
  if (t == 0) sh.ucnt = 0u;
  __syncthreads();
  tau = 0u;
  for (int k = 0; k < SEL_NW; k++) tau = max(tau, (uint32_t)sh.red_i[k]);
  for (int f = t; f < nc * BL_CCAP; f += BL_SEL_THREADS) {
    int ch = f / BL_CCAP, q = f - ch * BL_CCAP;
    if (q < d.c_cnt[ro + ch]) {
      int64_t o = (ro + ch) * BL_CCAP + q;
      float v = d.cand_v[o];
      if (bl_fkey(v) >= tau) {
        uint32_t pos = atomicAdd(&sh.ucnt, 1u);
        if (pos < SEL_LIST) sh.keys[pos] = ckey(v, d.cand_i[o]);
      }
    }
  }
  __syncthreads();
  int n = (int)sh.ucnt;
  if (n > SEL_LIST) {
    status |= BL_SE_CAND_FULL;
    n = SEL_LIST;
  }
  int P = 1;
  while (P < n) P <<= 1;
  for (int i = n + t; i < P; i += BL_SEL_THREADS) sh.keys[i] = 0ull;
  __syncthreads();
  bitonic_desc(sh.keys, P);
  return n;
}

/* Phase A (block): 2-variant records of n terms into recs; 16 consecutive terms per thread */
template <class TermF>
__device__ void block_records(int64_t n, TermF term, bl_grec *recs, double *sd) {
  const int t = threadIdx.x, lane = t & 63;
  const int64_t G = (n + 63) / 64;
  double base = 0.0;
  for (int64_t p0 = 0; p0 < n; p0 += 16 * BL_SEL_THREADS) {
    float a[16];
    double sa = 0.0;
#pragma unroll
    for (int k = 0; k < 16; k++) {
      int64_t j = p0 + t * 16 + k;
      a[k] = j < n ? term(j) : 0.0f;
      sa += (double)a[k];
    }
    double tot;
    double before = base + block_excl_scan_d<BL_SEL_THREADS>(sa, sd, &tot);
    double gstart = __shfl(before, lane & ~3, 64);
    uint32_t mask;
    int E = bl_choose_binades(gstart, &mask);
    bl_grec r;
    r.E = E;
    r.mask = mask;
#pragma unroll
    for (int k = 0; k < 2; k++) {
      bl_inc f = ((mask >> k) & 1u) ? bl_thread_compose<16>(a, E + k) : bl_inc_ident();
      r.v[k] = bl_quad_compose(f, lane);
    }
    int64_t g = (p0 + t * 16) / 64;
    if ((lane & 3) == 0 && g < G) recs[g] = r;
    base += tot;
  }
  __syncthreads();
}

struct no_rec {
  __device__ bl_grec operator()(int64_t) const {
    bl_grec r;
    r.E = BL_E_NONE;
    r.mask = 0u;
    return r;
  }
};

/*
 * sample_candidates_with_probs (src/sampling.br:490-607) for T > 0 on the ranked list val(j)
 * (n_list entries materialised; n_logical >= n_list is the reference's candidate count, the entries
 * past n_list being too small to change any float32 sum). Lists of up to 256 entries are walked by
 * wavefront 0 alone at element level; larger ones get group records from the whole block. Every
 * thread of the block must call it. Returns the chosen position, or -1 with `status` set.
 */
template <class ValF>
__device__ int sample_ranked(const bl_slot_dev &sp, ValF val, int64_t n_list, int64_t n_logical, uint64_t &rng,
                             int rng_skip, bl_grec *recs, sel_shared &sh, int &status) {
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const float T = sp.temperature;
  const bool small = n_list <= 256;
  int64_t keep = sp.min_keep > 1 ? sp.min_keep : 1;
  if (keep > n_logical) keep = n_logical;
  if (keep > n_list) {
    status |= BL_SE_UNSUPPORTED;
    return -1;
  }
  const float v0 = val(0);
  auto grec_of = [&](int64_t g) { return recs[g]; };
  auto walk = [&](int64_t n, auto term, bool thr_on, float thr, int64_t min_idx, float &S) -> int {
    if (small) return bl_seq_walk(n, term, no_rec(), no_rec(), false, thr_on, thr, min_idx, S, lane);
    return bl_seq_walk(n, term, grec_of, no_rec(), false, thr_on, thr, min_idx, S, lane);
  };
  int64_t cutoff = n_logical;
  if (sp.top_p < 1.0f || sp.min_p > 0.0f) {
    auto termE = [&](int64_t j) { return bl_expf(val(j) - v0); };
    if (!small) block_records(n_list, termE, recs, sh.sd);
    if (w == 0) {
      float S;
      walk(n_list, termE, false, 0.0f, 0, S);
      if (lane == 0) sh.fres[0] = S;
    }
    __syncthreads();
    const float sum_exp = sh.fres[0];
    auto termP = [&](int64_t j) { return bl_expf(val(j) - v0) / sum_exp; };
    if (sp.top_p < 1.0f) {
      if (!small) block_records(n_list, termP, recs, sh.sd);
      if (w == 0) {
        float S;
        int f = walk(n_list, termP, true, sp.top_p, keep - 1, S);
        if (lane == 0) sh.ires[0] = f;
      }
      __syncthreads();
      if (sh.ires[0] >= 0) cutoff = sh.ires[0] + 1;
    }
    if (sp.min_p > 0.0f) {
      const float p0 = termP(0);
      const float threshold = p0 * sp.min_p;
      /* first j in [keep, cutoff) with probs[j] < threshold */
      const int64_t lim = cutoff < n_list ? cutoff : n_list;
      if (w == 0) {
        int64_t first = -1;
        for (int64_t j0 = keep; j0 < lim && first < 0; j0 += 64) {
          int64_t j = j0 + lane;
          unsigned long long b = __ballot(j < lim && termP(j) < threshold);
          if (b) first = j0 + __ffsll((long long)b) - 1;
        }
        if (lane == 0) sh.ires[1] = (int)first;
      }
      __syncthreads();
      int64_t first_small = sh.ires[1];
      if (first_small < 0) {
        if (lim < cutoff) {
          /* the next, unmaterialised candidate is below 2^-25 of the top one */
          if (threshold <= p0 * 5.9604645e-8f) status |= BL_SE_UNSUPPORTED;
          first_small = lim;
        } else {
          first_small = cutoff;
        }
      }
      cutoff = keep > first_small ? keep : first_small;
    }
    __syncthreads();
  }
  if (status) return -1;
  const int64_t n_eff = cutoff < n_list ? cutoff : n_list;
  auto termR = [&](int64_t j) {
    float dd = val(j) - v0;
    float q = dd / T;
    return bl_expf(q);
  };
  if (!small) block_records(n_eff, termR, recs, sh.sd);
  if (w == 0) {
    float S;
    walk(n_eff, termR, false, 0.0f, 0, S);
    uint64_t st = rng;
    for (int k = 0; k < rng_skip; k++) st = bl_xorshift(st);
    float r01 = bl_rng_f32(&st);
    float target = r01 * S;
    float S2;
    int f = walk(n_eff, termR, true, target, 0, S2);
    if (lane == 0) {
      sh.ires[2] = f >= 0 ? f : (int)(cutoff - 1);
      sh.ures[0] = st;
    }
  }
  __syncthreads();
  int chosen = sh.ires[2];
  rng = sh.ures[0];
  __syncthreads();
  if (chosen >= n_list) {
    status |= BL_SE_UNSUPPORTED;
    return -1;
  }
  return chosen;
}

/* hand-off: the second of the row's two workgroups to arrive writes the chosen token's logprob */
__device__ void handoff(const bl_dev &d, const bl_rows &rows, int row, float M) {
  __threadfence();
  int old = atomicAdd(&d.done[row], 1);
  if (old == 1) {
    __threadfence();
    int tok = atomicAdd(&rows.tok[row], 0);
    float lse = atomicAdd(&d.lse[row], 0.0f);
    float a = d.eff[(int64_t)row * d.vocab + tok] - M;
    rows.lp[row] = a - lse;
  }
}

__global__ __launch_bounds__(BL_SEL_THREADS) void bl_k_select(bl_dev d, bl_rows rows) {
  const int V = d.vocab, nc = d.nc;
  const int row = blockIdx.x, role = blockIdx.y, t = threadIdx.x, w = t >> 6, lane = t & 63;
  const int slot = rows.slot[row];
  bl_slot_dev &sp = d.slots[slot];
  const int mode = sp.mode;
  const bool logprobs = (mode & BL_M_LOGPROBS) && rows.lp;
  if (role == 1 && !logprobs) return;
  __shared__ sel_shared sh;
  int status = 0;

  /* row max and first argmax from the chunk statistics */
  float M = BL_NEG_INF;
  int Mi = 0x7fffffff;
  for (int k = t; k < nc; k += BL_SEL_THREADS)
    argmax_merge(M, Mi, d.c_max[(int64_t)row * nc + k], d.c_arg[(int64_t)row * nc + k]);
  block_argmax<BL_SEL_THREADS>(M, Mi, sh.red_m, sh.red_i);
  if (Mi == 0x7fffffff) Mi = 0;
  const float *eff = d.eff + (int64_t)row * V;

  if (role == 1) {
    /* logprobs: exact index-order normaliser, then the n_probs alternatives (the row pass emitted
     * candidates only when k_sel > 0, which n_probs > 0 implies) */
    int n_top = sp.n_probs > 0 ? merge_topk(d, row, sh, status) : 0;
    if (w == 0) {
      const bl_grec *gr = reinterpret_cast<const bl_grec *>(d.grec) + (int64_t)row * 2 * (V / 64 + 64);
      const bl_grec *cr = reinterpret_cast<const bl_grec *>(d.crec) + (int64_t)row * nc;
      float S;
      bl_seq_walk((int64_t)V, [&](int64_t j) { return bl_expf(eff[j] - M); }, [&](int64_t g) { return gr[g]; },
                  [&](int64_t c) { return cr[c]; }, true, false, 0.0f, 0, S, lane);
      if (lane == 0) sh.fres[0] = (float)log((double)S);
    }
    __syncthreads();
    const float lse = sh.fres[0];
    for (int q = t; q < sp.n_probs && q < rows.top_stride; q += BL_SEL_THREADS) {
      uint64_t k = q < n_top ? sh.keys[q] : 0ull;
      int32_t id = k ? ckey_i(k) : 0;
      float v = k ? ckey_v(k) : -1.0e30f;
      rows.top_ids[(int64_t)row * rows.top_stride + q] = id;
      float b = v - M;
      rows.top_lp[(int64_t)row * rows.top_stride + q] = b - lse;
    }
    if (t == 0) {
      d.lse[row] = lse;
      if (status) {
        if (rows.status) atomicOr(&rows.status[row], status);
        sp.err |= status;
      }
      handoff(d, rows, row, M);
    }
    return;
  }

  /* role 0: sampling */
  uint64_t rng = sp.rng;
  const int skip = rows.rng_skip ? rows.rng_skip[row] : 0;
  int32_t tok = Mi;
  const float T = sp.temperature;
  if (T <= 0.0f) {
    tok = Mi; /* sample_greedy over the full penalised row (src/sampling.br:752-754) */
  } else if (mode & BL_M_TOPK) {
    /* top_k_select list: kk = min(top_k, V) entries, unfilled slots are (-1e30, 0) */
    int n = merge_topk(d, row, sh, status);
    int64_t kk = sp.top_k < V ? sp.top_k : V;
    auto val = [&](int64_t j) -> float { return j < n ? ckey_v(sh.keys[j]) : -1.0e30f; };
    int pos = sample_ranked(sp, val, kk, kk, rng, skip, sh.recs, sh, status);
    if (pos >= 0) tok = pos < n ? ckey_i(sh.keys[pos]) : 0;
  } else {
    /* full-vocabulary rank (src/sampling.br:301-365): candidates from the exponent pass */
    int nf = d.full_n[row];
    if (nf > V) {
      nf = V;
      status |= BL_SE_CAND_FULL;
    }
    int P = 1;
    while (P < nf) P <<= 1;
    uint64_t *keys = P <= SEL_LIST ? sh.keys : d.sortk + (int64_t)row * (2 * (int64_t)V);
    for (int i = t; i < P; i += BL_SEL_THREADS)
      keys[i] = i < nf ? ckey(d.full_v[(int64_t)row * V + i], d.full_i[(int64_t)row * V + i]) : 0ull;
    __syncthreads();
    bitonic_desc(keys, P);
    bl_grec *recs = sh.recs;
    if ((nf + 63) / 64 > SEL_LIST / 64)
      recs = reinterpret_cast<bl_grec *>(d.grec) + (int64_t)row * 2 * (V / 64 + 64) + (V / 64 + 64);
    auto val = [&](int64_t j) -> float { return ckey_v(keys[j]); };
    int pos = sample_ranked(sp, val, nf, (int64_t)V, rng, skip, recs, sh, status);
    if (pos >= 0) {
      tok = ckey_i(keys[pos]);
      /* the heap rank orders equal values its own way (src/sampling.br:310-364): a tie at the chosen
       * position is reported instead of guessed */
      float vp = val(pos);
      if ((pos > 0 && val(pos - 1) == vp) || (pos + 1 < nf && val(pos + 1) == vp)) status |= BL_SE_TIE;
    }
  }

  if (t == 0) {
    rows.tok[row] = tok;
    if (rows.status && status) atomicOr(&rows.status[row], status);
    bool is_eog = false;
    for (int k = 0; k < d.n_eog; k++) is_eog |= d.eog[k] == tok;
    if (rows.commit && status == 0) {
      /* tokens.push (src/server.br:1004): repeat window; reply_tokens.push unless EOG (:1037) */
      const int64_t so = (int64_t)slot * V;
      uint32_t *tw = d.touched + (int64_t)slot * d.words;
      sp.n_tokens += 1;
      if (sp.rep_on) {
        int rl = sp.repeat_last_n;
        if (rl > 0) {
          int32_t *ring = d.ring + (int64_t)slot * BL_WCAP;
          if (sp.win_len == rl) {
            int32_t old = ring[sp.win_head];
            d.wcnt[so + old] -= 1;
            ring[sp.win_head] = tok;
            sp.win_head = (sp.win_head + 1) % rl;
          } else {
            ring[(sp.win_head + sp.win_len) % rl] = tok;
            sp.win_len += 1;
          }
        }
        d.wcnt[so + tok] += 1;
        tw[tok >> 5] |= 1u << (tok & 31);
      }
      if (!is_eog) {
        sp.n_reply += 1;
        if (sp.fp_on) {
          d.cnt[so + tok] += 1;
          tw[tok >> 5] |= 1u << (tok & 31);
        }
      }
      sp.rng = rng;
    }
    if (status) sp.err |= status;
    if (logprobs) handoff(d, rows, row, M);
  }
}

/* ------------------------------------------------------------------ host-side launch of a step */
/* ev: optional 4 events recorded before/after the three kernels (kernel timing for the benchmark) */
void bl_launch_step(const bl_dev &d, const float *logits, int64_t ld, const bl_rows &rows, int B, bool need_exp,
                    hipStream_t s, hipEvent_t *ev) {
  dim3 g1(d.nc, B);
  if (ev) (void)hipEventRecord(ev[0], s);
  hipLaunchKernelGGL(bl_k_rowpass, g1, dim3(BL_RP_THREADS), 0, s, d, logits, ld, rows);
  if (ev) (void)hipEventRecord(ev[1], s);
  if (need_exp) hipLaunchKernelGGL(bl_k_exppass, g1, dim3(BL_RP_THREADS), 0, s, d, rows);
  if (ev) (void)hipEventRecord(ev[2], s);
  hipLaunchKernelGGL(bl_k_select, dim3(B, 2), dim3(BL_SEL_THREADS), 0, s, d, rows);
  if (ev) (void)hipEventRecord(ev[3], s);
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

void bl_launch_synth(float *out, int64_t ld, int cfg, int64_t seed, int64_t step, int rows, int V, hipStream_t s) {
  dim3 g((V + 255) / 256, rows);
  hipLaunchKernelGGL(bl_k_synth, g, dim3(256), 0, s, out, ld, cfg, seed, step, rows, V);
}

/* ------------------------------------------------------------------ math self-test */
/* Digest of f over input bit patterns [b*2^20, (b+1)*2^20): sum of splitmix(u << 32 | bits(f(u))). */
__global__ void bl_k_math_digest(int fn, uint32_t first_block, unsigned long long *out) {
  const uint32_t blk = first_block + blockIdx.y;
  const uint32_t base = blk << 20;
  uint64_t h = 0;
  for (int k = 0; k < 16; k++) {
    uint32_t u = base + (uint32_t)(blockIdx.x * 4096 + k * 256 + threadIdx.x);
    float x = bl_u2f(u);
    float y = fn == 0 ? bl_expf(x) : bl_tanhf(x);
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
