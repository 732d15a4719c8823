/*
 * bl_exact.h — exact, parallel emulation of a sequential float32 sum of non-negative terms.
 *
 * The reference sums softmax terms one at a time in float32 (src/sampling.br:255-265 in index order;
 * :506-598 in rank order), and logprobs/draws depend on the exact rounded result. A tree reduction
 * does not reproduce it, so the sum is re-derived as integer arithmetic:
 *
 *   While the running sum S stays in one binade [2^e, 2^(e+1)), S = N*u with u = 2^(e-23) and N an
 *   integer in [2^23, 2^24) (the bottom segment e = -126 covers [0, 2^-125) with N in [0, 2^24)).
 *   Adding a term a rounds a/u = q + f to an integer ulps count: q, q+1 when f > 1/2, and on a tie
 *   (f == 1/2) whichever makes N even. The increment therefore depends only on the parity of N, so a
 *   term is a pair (d0, d1) = (increment from even N, increment from odd N) and consecutive terms
 *   compose associatively (an automaton over parity). Sums of 64-term groups are wave reductions;
 *   prefixes are wave scans.
 *   When N would reach 2^24 the sum leaves the binade; that one step is done as a real float add and
 *   the walk continues in the new binade.
 *
 * The walk is split in two phases:
 *   Phase A (many threads): per 64-term group, the composed pair for three binades around the one an
 *            approximate (double) prefix predicts.
 *   Phase B (one wavefront): walks the groups 64 at a time with a composed scan, and drops to
 *            element level only in a group that crosses a binade, lacks the needed binade, or contains
 *            the element a threshold search is looking for. At element level the group's terms are
 *            added one at a time in float32 from the exact running sum (at most 64 adds, each term
 *            broadcast from its lane), which is the reference's own computation.
 */
#ifndef BL_EXACT_H
#define BL_EXACT_H

#include <stdint.h>

#include "bl_math.h"

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define BL_SD __host__ __device__ __forceinline__
#else
#define BL_SD static inline
#endif

#define BL_N_TOP (1u << 24)
#define BL_SAT (1u << 25)
#define BL_E_MIN (-126)
#define BL_E_NONE (-100000) /* no binade */

struct bl_inc {
  uint32_t d0, d1;
};

/* group record: composed pairs for binades E-1, E, E+1 (a variant below BL_E_MIN is unused) */
struct bl_grec {
  int32_t E;
  uint32_t pad;
  bl_inc v[3];
};

/* index-order group record: the composed automaton at the binade of the group's approximate start */
struct bl_grec1 {
  int32_t E;
  uint32_t pad;
  bl_inc v;
};

BL_SD bl_inc bl_inc_ident() { return bl_inc{0u, 0u}; }

/* f then g */
BL_SD bl_inc bl_compose(bl_inc f, bl_inc g) {
  uint32_t a = f.d0 + ((f.d0 & 1u) ? g.d1 : g.d0);
  uint32_t b = f.d1 + (((f.d1 + 1u) & 1u) ? g.d1 : g.d0);
  return bl_inc{a < BL_SAT ? a : BL_SAT, b < BL_SAT ? b : BL_SAT};
}

BL_SD uint32_t bl_apply(bl_inc f, uint32_t N) { return N + ((N & 1u) ? f.d1 : f.d0); }

/* increment of a term a >= 0 at binade e (units of 2^(e-23)) */
BL_SD bl_inc bl_term_inc(float a, int e) {
  uint32_t b = bl_f2u(a) & 0x7fffffffu;
  uint32_t ex = b >> 23, m = b & 0x7fffffu;
  if (b == 0u) return bl_inc{0u, 0u};
  if (ex == 0xffu) return bl_inc{BL_SAT, BL_SAT};
  int ea = ex ? (int)ex - 127 : -126;
  uint32_t M = ex ? (m | 0x800000u) : m;
  int s = e - ea;
  if (s < 0) return bl_inc{BL_SAT, BL_SAT};
  if (s == 0) return bl_inc{M, M};
  if (s >= 25) return bl_inc{0u, 0u};
  uint32_t q = M >> s, rem = M & ((1u << s) - 1u), half = 1u << (s - 1);
  if (rem > half) return bl_inc{q + 1u, q + 1u};
  if (rem < half) return bl_inc{q, q};
  return bl_inc{q + (q & 1u), q + ((q & 1u) ^ 1u)};
}

/* S (>= 0, finite) -> (e, N) */
BL_SD void bl_split(float S, int &e, uint32_t &N) {
  uint32_t b = bl_f2u(S) & 0x7fffffffu;
  uint32_t ex = b >> 23;
  if (ex == 0u) {
    e = BL_E_MIN;
    N = b;
  } else {
    e = (int)ex - 127;
    N = (b & 0x7fffffu) | 0x800000u;
  }
}

/* (e, N) with N < 2^24 -> S, exact */
BL_SD float bl_make(int e, uint32_t N) {
  if (N < 0x800000u) return bl_u2f(N); /* only reachable at e == BL_E_MIN: subnormal or zero */
  return bl_u2f(((uint32_t)(e + 127) << 23) | (N & 0x7fffffu));
}

/* binade index predicted from an approximate sum */
BL_SD int bl_binade_of(double s) {
  float f = (float)s;
  int e;
  uint32_t N;
  bl_split(f < 0.0f ? 0.0f : f, e, N);
  return e;
}

/* a 64-term group whose approximate start ga and end gb are not both safely (2^-20 relative) inside its
 * predicted binade E: the exact sum may cross a power of two within it. `floor` is an exact lower bound
 * of the running sum over the group (a float sum of non-negative terms is never below a term already
 * added), so the lower side of the margin stops there: a sum that a term of exactly 1.0 (the row
 * maximum's exp(0)) has just raised to 1 + tiny stays in binade 0. */
BL_SD bool bl_group_critical(float ga, float gb, int E, double floor) {
  const float lo = 0.99999904632568359375f, hi = 1.00000095367431640625f; /* 1 -+ 2^-20 */
  const double la = (double)ga * lo, lb = (double)gb * lo;
  return bl_binade_of(la > floor ? la : floor) != E || bl_binade_of((double)ga * hi) != E ||
         bl_binade_of(lb > floor ? lb : floor) != E || bl_binade_of((double)gb * hi) != E;
}

/* ---- top-n-sigma's statistics (src/sampling.br:376-400): sums of float32 values in float64 ---- */
/* a + b = s + e exactly (Knuth's two-sum; no contraction, no reassociation) */
BL_SD void bl_two_sum(double a, double b, double &s, double &e) {
  s = a + b;
  const double bb = s - a;
  e = (a - (s - bb)) + (b - bb);
}
/* a double-double: hi + lo, |lo| <= half an ulp of hi */
struct bl_dd {
  double hi, lo;
};
BL_SD bl_dd bl_dd_add(bl_dd x, bl_dd y) {
  double s, e, h, l;
  bl_two_sum(x.hi, y.hi, s, e);
  e += x.lo + y.lo;
  bl_two_sum(s, e, h, l);
  return bl_dd{h, l};
}
BL_SD bl_dd bl_dd_add_d(bl_dd x, double v) { return bl_dd_add(x, bl_dd{v, 0.0}); }

/* [lo, hi] -> an interval that also holds every rounding of a value in it, and the rounding of this
 * computation's own operations (4 ulps relative, plus the smallest normal) */
BL_SD void bl_widen(double &lo, double &hi) {
  const double u4 = 0x1p-51, tiny = 0x1p-1022;
  lo = lo - (lo < 0.0 ? -lo : lo) * u4 - tiny;
  hi = hi + (hi < 0.0 ? -hi : hi) * u4 + tiny;
}

/*
 * The float32 sigma that top_n_sigma_logits computes (src/sampling.br:376-400) from the row's statistics:
 * the count n of values above -1e29, the sums S of the values and Q of their squares (double-doubles, within
 * 2^-100 relative of the exact sums) and bounds Es, Eq on the rounding error of the reference's sequential
 * float64 sums (each addition errs by at most half an ulp of its partial sum). The reference's later float64
 * operations (sum / n, mean * mean, sum_sq / n, their difference, the square root) each round once; the
 * interval of their possible results is carried through them, and the square root goes to float32 by a
 * monotone rounding. Returns 1 with that sigma, 0 when the reference's variance is not positive (no filter),
 * and -1 when the interval holds zero or a float32 rounding boundary (undecided).
 */
BL_SD int bl_tns_sigma(double n, bl_dd S, bl_dd Q, double Es, double Eq, float &sigma) {
  double s_lo = (S.hi + S.lo) - Es, s_hi = (S.hi + S.lo) + Es;
  bl_widen(s_lo, s_hi);
  double m_lo = s_lo / n, m_hi = s_hi / n;
  bl_widen(m_lo, m_hi);
  double mm_lo, mm_hi;
  if (m_lo <= 0.0 && m_hi >= 0.0) {
    mm_lo = 0.0;
    mm_hi = (-m_lo > m_hi ? m_lo * m_lo : m_hi * m_hi);
  } else {
    const double a = m_lo < 0.0 ? -m_hi : m_lo, b = m_lo < 0.0 ? -m_lo : m_hi; /* 0 < a <= b */
    mm_lo = a * a;
    mm_hi = b * b;
  }
  bl_widen(mm_lo, mm_hi);
  double q_lo = ((Q.hi + Q.lo) - Eq) / n, q_hi = ((Q.hi + Q.lo) + Eq) / n;
  bl_widen(q_lo, q_hi);
  double v_lo = q_lo - mm_hi, v_hi = q_hi - mm_lo;
  bl_widen(v_lo, v_hi);
  if (v_hi <= 0.0) return 0;
  if (v_lo <= 0.0) return -1;
  double r_lo = sqrt(v_lo), r_hi = sqrt(v_hi);
  bl_widen(r_lo, r_hi);
  const float f_lo = (float)r_lo, f_hi = (float)r_hi;
  if (f_lo != f_hi) return -1;
  sigma = f_lo;
  return 1;
}

#if defined(__HIPCC__)
/* ---- wave primitives (wavefront of 64) ---- */
__device__ __forceinline__ bl_inc bl_shfl_up(bl_inc v, int k) {
  return bl_inc{(uint32_t)__shfl_up((int)v.d0, k, 64), (uint32_t)__shfl_up((int)v.d1, k, 64)};
}
__device__ __forceinline__ bl_inc bl_shfl(bl_inc v, int l) {
  return bl_inc{(uint32_t)__shfl((int)v.d0, l, 64), (uint32_t)__shfl((int)v.d1, l, 64)};
}
/* DPP move (gfx9 data-parallel primitives): lanes enabled by row_mask read lane `ctrl` selects,
 * others keep `old` */
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t bl_dpp(uint32_t old, uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROW_MASK, 0xF, false);
}
#define BL_DPP_ROW_SHR(k) (0x110 + (k))
#define BL_DPP_ROW_BCAST15 0x142
#define BL_DPP_ROW_BCAST31 0x143

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ bl_inc bl_dpp_inc(bl_inc f) {
  return bl_inc{bl_dpp<CTRL, ROW_MASK>(0u, f.d0), bl_dpp<CTRL, ROW_MASK>(0u, f.d1)};
}

/* inclusive ordered scan of composition across the wavefront: shifts within 16-lane rows, then the
 * row broadcasts of lane 15 (to rows 1, 3) and lane 31 (to rows 2, 3); all in VALU, no LDS. With
 * REV the composition runs the other way (lane l holds f_l then ... then f_0): scanning terms placed in
 * reversed lane order gives their suffix compositions. */
template <bool REV = false>
__device__ __forceinline__ bl_inc bl_wave_scan(bl_inc f, int lane) {
  const int r = lane & 15;
  auto cmp = [](bl_inc earlier, bl_inc later) { return REV ? bl_compose(later, earlier) : bl_compose(earlier, later); };
  bl_inc o;
  o = bl_dpp_inc<BL_DPP_ROW_SHR(1), 0xF>(f);
  if (r >= 1) f = cmp(o, f);
  o = bl_dpp_inc<BL_DPP_ROW_SHR(2), 0xF>(f);
  if (r >= 2) f = cmp(o, f);
  o = bl_dpp_inc<BL_DPP_ROW_SHR(4), 0xF>(f);
  if (r >= 4) f = cmp(o, f);
  o = bl_dpp_inc<BL_DPP_ROW_SHR(8), 0xF>(f);
  if (r >= 8) f = cmp(o, f);
  o = bl_dpp_inc<BL_DPP_ROW_BCAST15, 0xA>(f);
  if (lane & 16) f = cmp(o, f);
  o = bl_dpp_inc<BL_DPP_ROW_BCAST31, 0xC>(f);
  if (lane >= 32) f = cmp(o, f);
  return f;
}
/* inclusive ordered scan of composition within each 16-lane row (lane 16q + 15 holds its row's total) */
__device__ __forceinline__ bl_inc bl_row_scan(bl_inc f, int lane) {
  const int r = lane & 15;
  bl_inc o;
  o = bl_dpp_inc<BL_DPP_ROW_SHR(1), 0xF>(f);
  if (r >= 1) f = bl_compose(o, f);
  o = bl_dpp_inc<BL_DPP_ROW_SHR(2), 0xF>(f);
  if (r >= 2) f = bl_compose(o, f);
  o = bl_dpp_inc<BL_DPP_ROW_SHR(4), 0xF>(f);
  if (r >= 4) f = bl_compose(o, f);
  o = bl_dpp_inc<BL_DPP_ROW_SHR(8), 0xF>(f);
  if (r >= 8) f = bl_compose(o, f);
  return f;
}

/* value of lane l (wave-uniform) in every lane */
__device__ __forceinline__ uint32_t bl_bcast(uint32_t v, int l) { return (uint32_t)__builtin_amdgcn_readlane((int)v, l); }
__device__ __forceinline__ float bl_bcastf(float v, int l) { return bl_u2f(bl_bcast(bl_f2u(v), l)); }

/* lane 63's value of a composed scan, in every lane */
__device__ __forceinline__ bl_inc bl_lane63(bl_inc f) {
  return bl_inc{(uint32_t)__builtin_amdgcn_readlane((int)f.d0, 63), (uint32_t)__builtin_amdgcn_readlane((int)f.d1, 63)};
}
/* ordered reduction; result valid in every lane */
__device__ __forceinline__ bl_inc bl_wave_reduce(bl_inc f, int lane) { return bl_lane63(bl_wave_scan(f, lane)); }

/* inclusive ordered scan with `op` across the wavefront on 32-bit lanes: row shifts, then the row
 * broadcasts of lanes 15 and 31 (DPP, in VALU; no LDS round trip) */
template <class Op>
__device__ __forceinline__ uint32_t bl_wscan_u32(uint32_t v, int lane, Op op) {
  const int r = lane & 15;
  uint32_t o;
  o = bl_dpp<BL_DPP_ROW_SHR(1), 0xF>(0u, v);
  if (r >= 1) v = op(o, v);
  o = bl_dpp<BL_DPP_ROW_SHR(2), 0xF>(0u, v);
  if (r >= 2) v = op(o, v);
  o = bl_dpp<BL_DPP_ROW_SHR(4), 0xF>(0u, v);
  if (r >= 4) v = op(o, v);
  o = bl_dpp<BL_DPP_ROW_SHR(8), 0xF>(0u, v);
  if (r >= 8) v = op(o, v);
  o = bl_dpp<BL_DPP_ROW_BCAST15, 0xA>(0u, v);
  if (lane & 16) v = op(o, v);
  o = bl_dpp<BL_DPP_ROW_BCAST31, 0xC>(0u, v);
  if (lane >= 32) v = op(o, v);
  return v;
}
__device__ __forceinline__ uint32_t bl_wmax_u32(uint32_t v, int lane) {
  return bl_bcast(bl_wscan_u32(v, lane, [](uint32_t a, uint32_t b) { return a > b ? a : b; }), 63);
}
__device__ __forceinline__ uint32_t bl_wmin_u32(uint32_t v, int lane) {
  return bl_bcast(bl_wscan_u32(v, lane, [](uint32_t a, uint32_t b) { return a < b ? a : b; }), 63);
}
/* inclusive prefix sum of an int */
__device__ __forceinline__ int bl_wscan_add(int v, int lane) {
  return (int)bl_wscan_u32((uint32_t)v, lane, [](uint32_t a, uint32_t b) { return a + b; });
}
/* the wavefront's first maximum: the largest value (NaN never wins, -0 equals +0 and comes back as +0)
 * and the lowest index holding it; result in every lane */
__device__ __forceinline__ void bl_wargmax(float &m, int &mi, int lane) {
  const uint32_t k = m != m ? 0u : bl_fkey(m + 0.0f);
  const uint32_t km = bl_wmax_u32(k, lane);
  mi = (int)bl_wmin_u32(k == km ? (uint32_t)mi : 0xFFFFFFFFu, lane);
  m = bl_fkey_inv(km);
}
/* doubles: both halves moved by DPP */
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ double bl_dpp_d(double v) {
  const uint64_t b = bl_d2u(v);
  const uint64_t lo = bl_dpp<CTRL, ROW_MASK>(0u, (uint32_t)b), hi = bl_dpp<CTRL, ROW_MASK>(0u, (uint32_t)(b >> 32));
  return bl_u2d(lo | (hi << 32));
}
__device__ __forceinline__ double bl_wscan_add_d(double v, int lane) {
  const int r = lane & 15;
  double o;
  o = bl_dpp_d<BL_DPP_ROW_SHR(1), 0xF>(v);
  if (r >= 1) v = o + v;
  o = bl_dpp_d<BL_DPP_ROW_SHR(2), 0xF>(v);
  if (r >= 2) v = o + v;
  o = bl_dpp_d<BL_DPP_ROW_SHR(4), 0xF>(v);
  if (r >= 4) v = o + v;
  o = bl_dpp_d<BL_DPP_ROW_SHR(8), 0xF>(v);
  if (r >= 8) v = o + v;
  o = bl_dpp_d<BL_DPP_ROW_BCAST15, 0xA>(v);
  if (lane & 16) v = o + v;
  o = bl_dpp_d<BL_DPP_ROW_BCAST31, 0xC>(v);
  if (lane >= 32) v = o + v;
  return v;
}
__device__ __forceinline__ double bl_bcast_d(double v, int l) {
  const uint64_t b = bl_d2u(v);
  const uint64_t lo = bl_bcast((uint32_t)b, l), hi = bl_bcast((uint32_t)(b >> 32), l);
  return bl_u2d(lo | (hi << 32));
}
/* approximate wave sum (the association is the scan's; used for predictions only), in every lane */
__device__ __forceinline__ double bl_wave_sum_d(double x) {
  const int lane = (int)(threadIdx.x & 63);
  return bl_bcast_d(bl_wscan_add_d(x, lane), 63);
}
__device__ __forceinline__ double bl_wave_excl_scan_d(double x, int lane) { return bl_wscan_add_d(x, lane) - x; }

/* composed pair of NT consecutive terms at binade e, folded in order by one thread */
template <int NT>
__device__ __forceinline__ bl_inc bl_thread_compose(const float *a, int e) {
  if (e < BL_E_MIN) return bl_inc{BL_SAT, BL_SAT};
  bl_inc f = bl_inc_ident();
#pragma unroll
  for (int k = 0; k < NT; k++) f = bl_compose(f, bl_term_inc(a[k], e));
  return f;
}

/* ordered composition across L aligned consecutive lanes (lane L*q + i holds the i-th run); the result
 * is valid in every lane of the L */
template <int L>
__device__ __forceinline__ bl_inc bl_lanes_compose(bl_inc f, int lane) {
#pragma unroll
  for (int k = 1; k < L; k <<= 1) {
    const bl_inc o = bl_inc{(uint32_t)__shfl_xor((int)f.d0, k, 64), (uint32_t)__shfl_xor((int)f.d1, k, 64)};
    f = (lane & k) ? bl_compose(o, f) : bl_compose(f, o);
  }
  return f;
}

/*
 * Phase A for one group, executed by a whole wavefront: `a` is this lane's term (0 beyond the end),
 * `approx_start` the approximate sum before the group. Returns the record (valid in every lane).
 */
__device__ __forceinline__ bl_grec bl_group_record(float a, double approx_start, int lane) {
  bl_grec r;
  r.E = bl_binade_of(approx_start);
  r.pad = 0;
#pragma unroll
  for (int k = 0; k < 3; k++) {
    int e = r.E - 1 + k;
    bl_inc f = e >= BL_E_MIN ? bl_term_inc(a, e) : bl_inc{BL_SAT, BL_SAT};
    r.v[k] = bl_wave_reduce(f, lane);
  }
  return r;
}

/*
 * bl_group_record when the running sum before the group is known to within a relative `margin` of
 * `approx_start`: if both ends of that interval lie in one binade, the sum starts there and only that
 * variant is composed (the others read as saturated, which sends a mistaken prediction to the element
 * level). Otherwise all three.
 */
__device__ __forceinline__ bl_grec bl_group_record_pred(float a, double approx_start, double margin, int lane) {
  const int E = bl_binade_of(approx_start);
  if (bl_binade_of(approx_start * (1.0 - margin)) == E && bl_binade_of(approx_start * (1.0 + margin)) == E) {
    bl_grec r;
    r.E = E;
    r.pad = 0;
    r.v[0] = r.v[2] = bl_inc{BL_SAT, BL_SAT};
    r.v[1] = bl_wave_reduce(bl_term_inc(a, E), lane);
    return r;
  }
  return bl_group_record(a, approx_start, lane);
}

/*
 * Phase B: sequential-sum walk over n terms in groups of 64, by one wavefront.
 *   term(j)   -> float term j (only called for j < n)
 *   rec(g)    -> bl_grec of group g
 * Search mode (thr_on): stops at the first index j >= min_idx whose inclusive sum S_j >= thr and
 * returns j (S holds S_j); otherwise returns -1 with S the full sum. All lanes return the same.
 */
template <class TermF, class RecF>
__device__ int bl_seq_walk(int64_t n, TermF term, RecF rec, bool thr_on, float thr, int64_t min_idx, float &S_out,
                           int lane) {
  int e = BL_E_MIN;
  uint32_t N = 0u;
  int64_t G = (n + 63) / 64;
  int64_t g = 0;
  while (g < G) {
    /* ---- group level over groups g .. g+63 ---- */
    int64_t gl = g + lane;
    bool valid = gl < G;
    bl_inc f = bl_inc_ident();
    if (valid) {
      bl_grec r = rec(gl);
      int k = e - (r.E - 1);
      if (k >= 0 && k <= 2 && e >= BL_E_MIN) f = k == 0 ? r.v[0] : (k == 1 ? r.v[1] : r.v[2]); /* selects: no dynamic index into private memory */
      else valid = false;
    }
    bl_inc sc = bl_wave_scan(f, lane);
    uint32_t Nend = bl_apply(sc, N);
    bool bad = !valid || Nend >= BL_N_TOP;
    if (!bad && thr_on) bad = bl_make(e, Nend) >= thr; /* reaching the threshold: resolve at element level */
    unsigned long long m = __ballot(bad);
    int first = m ? __ffsll((long long)m) - 1 : 64;
    if (first > 0) {
      N = bl_bcast(Nend, first - 1);
      g += first;
    }
    if (g >= G) break;
    if (first == 64) continue;
    /* ---- element level in group g: the group crosses a binade, lacks the needed binade or reaches the
     * threshold, so its terms are added one at a time in float32 from the exact running sum ---- */
    const int64_t j0 = g * 64;
    const int64_t j = j0 + lane;
    const float a = j < n ? term(j) : 0.0f;
    const int n_in = (int)(n - j0 < 64 ? n - j0 : 64);
    float S = bl_make(e, N);
    int hit = -1; /* first index reaching the threshold */
#pragma unroll
    for (int c = 0; c < 64; c++) {
      const float x = bl_bcastf(a, c);
      if (c < n_in && hit < 0) {
        S = S + x;
        if (thr_on && j0 + c >= min_idx && S >= thr) hit = c;
      }
    }
    if (hit >= 0) {
      S_out = S;
      return (int)(j0 + hit);
    }
    bl_split(S, e, N);
    g += 1;
  }
  S_out = bl_make(e, N);
  return -1;
}

#endif /* __HIPCC__ */

#endif /* BL_EXACT_H */
