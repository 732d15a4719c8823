/*
 * bl_internal.h — device data layout shared by the kernels and the host side of libbl_select.
 *
 * Per slot (one request's sampler state, all in HBM, owned by the context):
 *   bl_slot_dev            sampling parameters + scalar state (RNG, history lengths, window ring head)
 *   rec[nb][BL_EB]         the tokens the server stages modify (a logit_bias value, a reply count for the
 *                          frequency / presence penalties, a repeat-window count), one 16-byte bl_rec each,
 *                          grouped by 1024-token bucket and packed at the front of the bucket's area
 *   rcnt[nb]               records in each bucket
 *   ridx[V]                a token's record index within its bucket, or -1 (used by commits only)
 *   ring[WCAP]             the last repeat_last_n tokens, for window eviction
 * A pass over a chunk of the row reads its buckets' counts, then their records contiguously (coalesced, no
 * per-token gather) and applies them in LDS. Committing a token is O(1) writes. ignore_eos suppression
 * reads the context's end-of-generation registry at every step.
 *
 * Per step workspace, rows = B: transformed rows, per-chunk statistics and top-K candidates,
 * sequential-sum group records, full-vocabulary candidate lists and sort scratch.
 */
#ifndef BL_INTERNAL_H
#define BL_INTERNAL_H

#include <stdint.h>

#include "bl_exact.h"
#include "bl_gwalk.h"
#include "bl_jwalk.h"

#define BL_CH 4096          /* vocabulary chunk per workgroup in the row passes */
#define BL_RP_THREADS 256   /* row-pass workgroup */
#define BL_EB 1024          /* exponent pass: terms per workgroup (4 per thread); the row pass sums per BL_EB */
#define BL_SUBS (BL_CH / BL_EB)
#define BL_SEL_THREADS 1024 /* per-row selection workgroup */
#define BL_KSEL_MAX 256     /* largest per-chunk candidate count (top_k / n_probs) */
#define BL_WCAP 8192        /* repeat window ring capacity */
#define BL_LDS_SORT 4096    /* candidate lists sorted in LDS up to this size */
#define BL_MAX_CHUNKS 1024  /* vocabulary up to BL_MAX_CHUNKS * BL_CH tokens */
#define BL_SERIAL_MAX 512   /* candidate lists up to this length are summed by one lane */
#define BL_CRIT_MAX 32      /* critical groups the fast normaliser precomputes (terms + two scans in LDS) */
#define BL_TK_CAP 1024      /* chunk top-K: keys at or above the thread-maximum bound ranked in LDS */
#define BL_STAGE_B 1024     /* block summaries staged in LDS by the fast normaliser (V up to 1M) */
#define BL_RANK_MAX 1024    /* full-vocabulary candidate lists up to this size are sorted by counting */
#define BL_NBUCKET 8192     /* value buckets of the sort of longer lists (more than BL_LDS_SORT) */
#define BL_EOG_LDS 64       /* end-of-generation ids the selection keeps in LDS */
#define BL_TNS_W 6          /* doubles of top-n-sigma statistics per chunk */

/* record flags (bl_rec.wf above BL_WF_SHIFT) */
#define BL_TF_BIAS 1u
#define BL_TF_DRY 2u        /* the token carries this step's DRY penalty; its exponent above BL_DRY_ESHIFT */
#define BL_WF_SHIFT 16
#define BL_WF_WMASK 0xFFFFu /* repeat-window count (at most BL_WCAP) */
#define BL_DRY_ESHIFT 18    /* DRY exponent (at most BL_DRY_WCAP) in the record's top 14 bits */
#define BL_DRY_WCAP 2048    /* DRY window (dry_penalty_last_n) capacity */
#define BL_DRY_MMAX 512     /* DRY sequence breakers of two or more tokens per slot */
#define BL_DRY_MLEN 24      /* tokens of one such breaker */

/* row modes */
#define BL_M_GREEDY 1
#define BL_M_TOPK 2
#define BL_M_FULL 4
#define BL_M_LOGPROBS 8
#define BL_M_GRAMMAR 16
#define BL_M_PSP 32 /* logprobs as post-sampling probabilities (src/server.br:1015-1025) */
#define BL_M_MIRO 64 /* the draw is mirostat v2's */
#define BL_M_TNS 128 /* top-n-sigma filters the ranked candidates (src/sampling.br:376-407) */
#define BL_M_ADAPT 512 /* adaptive-p replaces the chain (src/sampling.br:705-740); the row's normaliser is formed */
#define BL_M_GFULL 256 /* a sampled top-k grammar row: the exponent pass also lists its allowed candidates, for
                          the widening level that ranks the whole vocabulary */

/* grammar mask kernel: tokens per workgroup */
#define BL_GM_THREADS 256

/* per-row grammar status (bl_dev.gstat) */
#define BL_GR_FORCED 1  /* complete and cannot continue: the step returns EOS (src/server.br:319-321) */
#define BL_GR_DEAD 2    /* the reply no longer matches the grammar (src/server.br:318) */
#define BL_GR_FAMBIG 4  /* the reply's own walk hit the 20,000-stack guard (src/grammar.br:354) */

/* per-row status bits (also sticky in the slot) */
#define BL_SE_UNSUPPORTED 1
#define BL_SE_TIE 2
#define BL_SE_CAND_FULL 4
#define BL_SE_EMPTY 8
#define BL_SE_GDEAD 16
#define BL_SE_GREJECT 32
#define BL_SE_GAMBIG 64
#define BL_SE_SIGMA 128 /* top-n-sigma's sigma undecided (at a float32 rounding boundary) */
#define BL_SE_JREJECT 256 /* a JSON-object slot: every vocabulary token rejected (src/server.br:302) */

/* one modified token's server-stage inputs in one slot (src/server.br:940-944, src/sampling.br:65-107,
 * :175-188) */
struct alignas(16) bl_rec {
  int32_t tok;  /* token id */
  float bias;   /* logit_bias value (BL_TF_BIAS) */
  int32_t cnt;  /* occurrences in the reply */
  uint32_t wf;  /* occurrences in the repeat window (low 16 bits), BL_TF_* flags above */
};

/* A speculative row's correction to one token's counts: row i of a sequence is sampled with the drafts
 * before it appended to the history (src/server.br:1173-1216), so each such draft adds to its reply count
 * and window count, and window entries the drafts push out subtract from theirs. */
#define BL_SPEC_DCAP 256 /* corrections per row: drafts before the row plus the entries they evict (2 k) */
struct bl_sdelta {
  int32_t tok;
  int16_t dcnt;  /* reply count */
  int16_t dwcnt; /* repeat-window count */
};

/* One critical 64-term group of a row's index-order normaliser (the running sum may cross a power of two
 * inside it), written by the exponent pass: the exact terms, cp[l] = the composition of terms 0..l at the
 * binade e0 of the group's approximate start, cs[l] = that of terms l..63 at the binade e1 of its approximate
 * end, and the group records of its block (ng groups), from which the selection composes the runs between
 * critical groups. */
struct bl_crit {
  int32_t g, e0, e1, ng;
  float terms[64];
  bl_inc cp[64];
  bl_inc cs[64];
  bl_grec1 blk[BL_EB / 64];
};

struct bl_slot_dev {
  /* parameters (SamplingParams, src/model.br:1565-1584, and server extras) */
  float temperature, dynatemp_range, dynatemp_exponent, top_n_sigma;
  float typical_p, top_p, min_p, xtc_probability, xtc_threshold;
  float repeat_penalty, frequency_penalty, presence_penalty, final_softcap, logit_mul;
  int32_t top_k, min_keep, repeat_last_n, n_probs, ignore_eos, post_sampling_probs;
  /* derived at configuration */
  int32_t mode, k_sel, fp_on, rep_on;
  /* state */
  uint64_t rng;
  int32_t n_tokens, n_reply, win_len, win_head, err, pad;
  /* grammar (src/server.br:309-362): position of the reply in the slot's automaton; or, with g_kind 1,
   * response_format json_object (src/server.br:261-304): the JSON classifier's position (stack in
   * bl_dev.jstack) */
  bl_gram_pos gpos;
  int32_t g_on, g_kind;
  bl_json_pos jpos;
  /* mirostat v1 / v2 (src/sampling.br:663-700): the version, tau, eta and the running mu */
  int32_t mirostat;
  float mirostat_tau, mirostat_eta, mu;
  /* DRY (src/sampling.br:114-171): parameters, the cap on the exponent, the last dry_n history tokens (ring
   * dh_len / dh_head in bl_dev.dring), the tokens flagged by the last update (bl_dev.dlist), and the sequence
   * breakers: single tokens sorted as (token << 32 | segment), where segment = the longer breakers listed
   * before the token's first single occurrence; longer breakers as [length, tokens...] rows in list order */
  /* adaptive-p: target, decay and the running weighted sum and total weight (src/server.br:937-938) */
  float adapt_target, adapt_decay, adapt_ws, adapt_tw;
  int32_t dry_on, dry_allowed, dry_n, dry_maxexp;
  float dry_mult, dry_base;
  int32_t dh_len, dh_head, dry_cnt, n_bsingle, n_bmulti, pad3;
  const uint64_t *bsingle;
  const int32_t *bmulti; /* [n_bmulti][BL_DRY_MLEN + 1] */
};

struct bl_dev {
  int vocab, nc, max_slots, max_rows;
  bl_slot_dev *slots;
  bl_rec *rec;       /* [slots][nb][BL_EB] */
  int32_t *rcnt;     /* [slots][nb] */
  int16_t *ridx;     /* [slots][V] */
  int32_t *ring;     /* [slots][WCAP] */
  int32_t *dring;    /* [slots][DRY_WCAP] DRY's history window */
  int32_t *dlist;    /* [slots][DRY_WCAP] tokens carrying a DRY penalty */
  int32_t *eog;      /* [n_eog] end-of-generation ids */
  int32_t n_eog;
  /* workspace for up to max_rows rows */
  float *eff;       /* [rows][V] the values after the model tail and the server stages, rows with a tail only */
  float *c_max;     /* [rows][nc] */
  int32_t *c_arg;   /* [rows][nc] */
  float *c_bsum;    /* [rows][nc][BL_SUBS] approximate sums of exp(x - c_max) over each BL_EB positions */
  double *c_tns;    /* [rows][nc][BL_TNS_W] top-n-sigma's chunk statistics: sum and sum of squares as
                       double-doubles, sum of magnitudes, count */
  float *cand_v;    /* [rows][nc][KSEL_MAX] */
  int32_t *cand_i;
  void *grec;       /* [rows][2 * (V/64 + 64)] bl_grec: index-order records, then sorted-list records */
  float *full_v;    /* [rows][nb][BL_EB] full-vocabulary candidates, exponent block b's in region b */
  int32_t *full_i;
  int32_t *full_cnt; /* [rows][nb] candidates in each region */
  double *full_s;    /* [rows][nb] approximate tempered sum over each region (rows without top-p/min-p) */
  uint64_t *sortk;  /* [rows][2V]: bucketed keys, then the sorted list; the draw's terms in the first half */
  double *gsum;     /* [rows][V/64 + 64] */
  bl_crit *crit;    /* [rows][BL_CRIT_MAX] the normaliser's critical groups, in order of arrival */
  int32_t *ncrit;   /* [rows] critical groups found (entries past BL_CRIT_MAX are not stored) */
  uint64_t *mkeys;  /* [rows][KSEL_MAX] the row's top-K keys, merged by the exponent pass */
  int32_t *mstat;   /* [rows] 1: mkeys holds the merge; 0: the selection merges the chunk lists itself */
  float *rmax;      /* [rows] the row maximum and its first index, reduced by the exponent pass */
  int32_t *rarg;
  void *brec;       /* [rows][nb] bl_grec1 per BL_EB terms: the block's binade and composed automaton, or
                       BL_E_NONE when it holds a critical group or two binades */
  uint32_t *bcrit;  /* [rows][nb] the block's critical groups (bit i: group 16 b + i) */
  int32_t nb;       /* ceil(V / BL_EB) */
  /* grammar-constrained sampling */
  bl_gram_view *gram; /* [slots] the slot's compiled grammar (device pointers) */
  uint8_t *jstack;    /* [slots][BL_JSON_DEPTH] JSON-object slots' container stacks */
  const uint8_t *vblob;   /* vocabulary piece bytes */
  const uint32_t *voff;   /* [V+1] byte offsets of each token's piece */
  int32_t eos_id;
  int32_t gm_blocks;      /* ceil(V / BL_GM_THREADS) */
  uint32_t *gmask;        /* [rows][2 * ceil(V/64)] allow-bitmask */
  int32_t *gstat;         /* [rows] BL_GR_* of the frontier */
  int32_t *gamb;          /* [rows] a candidate's walk hit the 20,000-stack guard */
  float *gm_max;          /* [rows][gm_blocks] allowed maximum per block */
  int32_t *gm_arg;        /* lowest index reaching it */
  int32_t *gm_eq;         /* allowed tokens equal to it */
};

#define BL_ROWS_INLINE 64 /* rows whose slot index travels in the kernel arguments */

/* one step's row table (device pointers; the first BL_ROWS_INLINE slot indices also by value, so a
 * kernel reads its row's slot without a dependent load) */
struct bl_rows {
  const int32_t *slot;     /* [B] */
  int16_t slot_inline[BL_ROWS_INLINE];
  const int32_t *rng_skip; /* [B] draws consumed before this row's draw (speculative rows), or null */
  int32_t commit;          /* append the chosen token to the slot history */
  int32_t merged;          /* the exponent pass ran: it left each row's maximum and merged top-K keys */
  int32_t *tok;            /* [B] */
  float *lp;               /* [B] */
  int32_t *top_ids;        /* [B][top_stride] */
  float *top_lp;
  int32_t top_stride;
  int32_t *status;         /* [B] */
  const bl_sdelta *delta;  /* [B][BL_SPEC_DCAP] speculative rows' count corrections, or null */
  const int32_t *delta_n;  /* [B] corrections of each row */
};

#if defined(__HIPCC__)
__device__ __forceinline__ int bl_row_slot(const bl_rows &r, int row) {
  return row < BL_ROWS_INLINE ? (int)r.slot_inline[row] : r.slot[row];
}

/* the model tail (src/model.br:973-984) changes the row: logit_mul != 1 or a final soft-cap */
__device__ __forceinline__ bool bl_tail_on(const bl_slot_dev &sp) {
  return sp.logit_mul != 1.0f || sp.final_softcap > 0.0f;
}

/* XTC runs (src/sampling.br:552-572): it draws its chance whenever the candidates reach two */
__device__ __forceinline__ bool bl_xtc_on(const bl_slot_dev &sp) {
  return sp.xtc_probability > 0.0f && sp.xtc_threshold <= 0.5f;
}
/* the untempered softmax is formed (top-p, min-p, XTC, the dynamic temperature or the typical filter
 * read it) */
__device__ __forceinline__ bool bl_probs_on(const bl_slot_dev &sp) {
  return sp.top_p < 1.0f || sp.min_p > 0.0f || bl_xtc_on(sp) || sp.dynatemp_range > 0.0f || sp.typical_p < 1.0f;
}
/* A full-vocabulary rank's candidates: every value within this span of the row maximum. Past it a term
 * exp(v - v0) (untempered, when formed) or exp((v - v0) / T) of the draw is below 2^-25 of the first
 * term, too small to change a float32 sum that holds the first term (17.5 > 25 ln 2). The span is
 * 17.5 max(T, 1) when the untempered softmax is formed and 17.5 T otherwise. XTC may start the draw at a
 * later candidate v_first, whose probability, at least the threshold, puts it within -ln(threshold)
 * (+0.05 for the rounding of the probabilities and their sum) of the maximum: the span grows by that.
 * The dynamic temperature draws at most at T + range. */
__device__ __forceinline__ float bl_cand_span(const bl_slot_dev &sp) {
  /* mirostat's terms exp(v/T - v0/T) (the span allows for the rounding of the two quotients) */
  if (sp.mode & BL_M_MIRO) return 17.6f * sp.temperature;
  const float T = sp.dynatemp_range > 0.0f ? sp.temperature + sp.dynatemp_range : sp.temperature;
  float span = 17.5f * (bl_probs_on(sp) && T < 1.0f ? 1.0f : T);
  if (bl_xtc_on(sp)) span = sp.xtc_threshold > 1.0e-30f ? span + (-__logf(sp.xtc_threshold) + 0.05f) : 3.0e38f;
  /* without a top-p or min-p cut the dynamic temperature's entropy runs over every candidate, where
   * terms -q ln q far below the draw's reach still count: every value is a candidate */
  if (sp.dynatemp_range > 0.0f && !(sp.top_p < 1.0f || sp.min_p > 0.0f)) span = 3.0e38f;
  /* the typical filter needs the whole candidate list */
  if (sp.typical_p < 1.0f) span = 3.0e38f;
  return span;
}

/* the record of `tok` in `slot`, created (zeroed) when the token has none; one thread (commits) */
__device__ inline bl_rec *bl_rec_get(const bl_dev &d, int slot, int32_t tok) {
  const int64_t sb = (int64_t)slot * d.nb + tok / BL_EB;
  int16_t *ri = d.ridx + (int64_t)slot * d.vocab + tok;
  bl_rec *base = d.rec + sb * BL_EB;
  int i = *ri;
  if (i < 0) {
    i = d.rcnt[sb];
    d.rcnt[sb] = i + 1;
    *ri = (int16_t)i;
    base[i] = bl_rec{tok, 0.0f, 0, 0u};
  }
  return base + i;
}

/* the DRY window's tokens.push (src/server.br:1004); one thread. Every window token keeps a record, where
 * the update sets its penalty. */
__device__ inline void bl_dry_push(const bl_dev &d, bl_slot_dev &sp, int slot, int32_t tok) {
  if (!sp.dry_on) return;
  int32_t *ring = d.dring + (int64_t)slot * BL_DRY_WCAP;
  if (sp.dh_len == sp.dry_n) {
    ring[sp.dh_head] = tok;
    sp.dh_head = (sp.dh_head + 1) % sp.dry_n;
  } else {
    ring[(sp.dh_head + sp.dh_len) % sp.dry_n] = tok;
    sp.dh_len += 1;
  }
  bl_rec_get(d, slot, tok);
}

/* appends token `tok`'s bytes to the slot's grammar position (reply_tokens.push of a non-EOG token,
 * src/server.br:1037), or to its JSON classifier's; one thread */
__device__ inline void grammar_commit(const bl_dev &d, bl_slot_dev &sp, const bl_gram_view &g, int32_t tok, int slot) {
  const uint32_t o0 = d.voff[tok], o1 = d.voff[tok + 1];
  const uint8_t *b = d.vblob + o0;
  if (sp.g_kind == 1)
    bl_js_commit(sp.jpos, d.jstack + (int64_t)slot * BL_JSON_DEPTH, [&](int i) { return (uint32_t)b[i]; }, (int)(o1 - o0));
  else
    bl_gw_commit(g, sp.gpos, [&](int i) { return (uint32_t)b[i]; }, (int)(o1 - o0));
}
#endif

#endif /* BL_INTERNAL_H */
