/*
 * capi.cpp — extern "C" surface of the oracle for the Python tests and the benchmark's CPU baseline,
 * plus the five workload drivers. TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Errors: functions returning int return 0 on success and -1 on a reference error path; the message
 * (the reference's throw text) is available from orc_last_error().
 */
#include <string.h>

#include <chrono>
#include <stdexcept>
#include <string>

#include "../boring-llm_amd/csrc/bl_synth.h"
#include "../boring-llm_amd/csrc/bl_workload.h"
#include "oracle.h"

using namespace orc;

static thread_local std::string g_err;

static uint32_t crc32_bytes(const void *data, size_t n) {
  static uint32_t table[256];
  static bool init = false;
  if (!init) {
    for (uint32_t i = 0; i < 256; i++) {
      uint32_t c = i;
      for (int k = 0; k < 8; k++) c = (c & 1) ? 0xEDB88320u ^ (c >> 1) : c >> 1;
      table[i] = c;
    }
    init = true;
  }
  uint32_t c = 0xFFFFFFFFu;
  const uint8_t *p = (const uint8_t *)data;
  for (size_t i = 0; i < n; i++) c = table[(c ^ p[i]) & 0xFF] ^ (c >> 8);
  return c ^ 0xFFFFFFFFu;
}

extern "C" {

const char *orc_last_error(void) { return g_err.c_str(); }
uint32_t orc_crc32(const void *data, size_t n) { return crc32_bytes(data, n); }

/* ---------------- RNG ---------------- */
int64_t orc_resolve_seed(int64_t requested, uint64_t entropy, int64_t counter) {
  return resolve_seed(requested, entropy, counter);
}
uint64_t orc_seed_rng(int64_t seed) { return seed_rng(seed).state; }
uint64_t orc_rng_next_u64(uint64_t *state) {
  Rng r{*state};
  uint64_t x = rng_next_u64(r);
  *state = r.state;
  return x;
}
float orc_rng_next_f32(uint64_t *state) {
  Rng r{*state};
  float f = rng_next_f32(r);
  *state = r.state;
  return f;
}

/* ---------------- row transforms ---------------- */
void orc_apply_repeat_penalty(const float *logits, int64_t n, const int32_t *hist, int64_t nh, float penalty,
                              int64_t last_n, float *out) {
  Row r = apply_repeat_penalty(Row(logits, logits + n), Ids(hist, hist + nh), penalty, last_n);
  memcpy(out, r.data(), n * sizeof(float));
}
void orc_apply_presence_frequency(const float *logits, int64_t n, const int32_t *gen, int64_t ng, float freq,
                                  float pres, float *out) {
  Row r = apply_presence_frequency_penalty(Row(logits, logits + n), Ids(gen, gen + ng), freq, pres);
  memcpy(out, r.data(), n * sizeof(float));
}
/* breakers flattened: lens[i] tokens each, concatenated in flat */
void orc_apply_dry(const float *logits, int64_t n, const int32_t *hist, int64_t nh, float mult, float base,
                   int64_t allowed, int64_t last_n, const int32_t *flat, const int32_t *lens, int64_t nb, float *out) {
  std::vector<Ids> br;
  int64_t at = 0;
  for (int64_t i = 0; i < nb; i++) {
    br.push_back(Ids(flat + at, flat + at + lens[i]));
    at += lens[i];
  }
  Row r = apply_dry_penalty(Row(logits, logits + n), Ids(hist, hist + nh), mult, base, allowed, last_n, br);
  memcpy(out, r.data(), n * sizeof(float));
}
void orc_apply_logit_bias(const float *logits, int64_t n, const int32_t *ids, const float *vals, int64_t nb,
                          float *out) {
  std::map<int32_t, float> m;
  for (int64_t i = 0; i < nb; i++) m[ids[i]] = vals[i];
  Row r = apply_logit_bias(Row(logits, logits + n), m);
  memcpy(out, r.data(), n * sizeof(float));
}
void orc_set_eog_tokens(const int32_t *ids, int64_t n, int32_t close_id) { set_eog_tokens(Ids(ids, ids + n), close_id); }
int orc_is_eog_token(int32_t tok, int32_t eos) { return is_eog_token(tok, eos) ? 1 : 0; }
int32_t orc_turn_close_token(int32_t eos) { return turn_close_token(eos); }
void orc_suppress_eog_tokens(const float *logits, int64_t n, int32_t eos, float *out) {
  Row r = suppress_eog_tokens(Row(logits, logits + n), eos);
  memcpy(out, r.data(), n * sizeof(float));
}
void orc_suppress_token(const float *logits, int64_t n, int32_t tok, float *out) {
  Row r = suppress_token(Row(logits, logits + n), tok);
  memcpy(out, r.data(), n * sizeof(float));
}
void orc_finish_logits(const float *logits, int64_t n, float logit_mul, float cap, float *out) {
  Row r = finish_logits(Row(logits, logits + n), logit_mul, cap);
  memcpy(out, r.data(), n * sizeof(float));
}
/* top_n_sigma_logits' threshold (1) or 0 when the row is kept whole */
int orc_top_n_sigma_threshold(const float *logits, int64_t n, float sig, float *threshold) {
  return top_n_sigma_threshold(Row(logits, logits + n), n, sig, *threshold) ? 1 : 0;
}

void orc_top_n_sigma(const float *logits, int64_t n, float sig, float *out) {
  Row r = top_n_sigma_logits(Row(logits, logits + n), n, sig);
  memcpy(out, r.data(), n * sizeof(float));
}

/* ---------------- ranking ---------------- */
int32_t orc_sample_greedy(const float *logits, int64_t n) { return sample_greedy(Row(logits, logits + n), n); }
void orc_logprob_normalizer(const float *logits, int64_t n, float *mx, float *lse) {
  logprob_normalizer(Row(logits, logits + n), n, *mx, *lse);
}
/* the normaliser's float32 sum itself (sum_exp before its logf) */
float orc_logprob_sum(const float *logits, int64_t n) {
  float mx, lse, sum;
  logprob_normalizer(Row(logits, logits + n), n, mx, lse, &sum);
  return sum;
}
float orc_token_logprob(const float *logits, int64_t n, int32_t tok) { return token_logprob(Row(logits, logits + n), n, tok); }
/* writes min(k, n) entries */
void orc_top_k_select(const float *logits, int64_t n, int64_t k, float *vals, int32_t *ids) {
  Row v;
  Ids i;
  top_k_select(Row(logits, logits + n), n, k, v, i);
  memcpy(vals, v.data(), v.size() * sizeof(float));
  memcpy(ids, i.data(), i.size() * sizeof(int32_t));
}
void orc_all_candidates_sorted(const float *logits, int64_t n, float *vals, int32_t *ids) {
  Row v;
  Ids i;
  all_candidates_sorted(Row(logits, logits + n), n, v, i);
  memcpy(vals, v.data(), n * sizeof(float));
  memcpy(ids, i.data(), n * sizeof(int32_t));
}

/* ---------------- candidate sampling ---------------- */
/* the running sums of one sample_candidates_with_probs call: out_f = {sum_exp, temperature, renorm_sum, target},
 * out_i = {cutoff, first, chosen}; returns the token or -1 */
int32_t orc_sample_candidates_trace(uint64_t rng, const float *vals, const int32_t *ids, int64_t n, float temperature,
                                    float top_p, float min_p, int64_t min_keep, float *out_f, int64_t *out_i) {
  try {
    CandTrace tr{};
    CandResult r = sample_candidates_with_probs(Rng{rng}, Row(vals, vals + n), Ids(ids, ids + n), temperature, 0.0f,
                                                1.0f, 1.0f, top_p, min_p, 0.0f, 0.1f, min_keep, &tr);
    out_f[0] = tr.sum_exp;
    out_f[1] = tr.temperature;
    out_f[2] = tr.renorm_sum;
    out_f[3] = tr.target;
    out_i[0] = tr.cutoff;
    out_i[1] = tr.first;
    out_i[2] = tr.chosen;
    return r.token;
  } catch (const std::exception &e) {
    g_err = e.what();
    return -1;
  }
}
/* returns the token (or -1 on error); probs/ids receive the post-sampling list (cap entries at most) */
int32_t orc_sample_candidates(uint64_t *rng, const float *vals, const int32_t *ids, int64_t n, float temperature,
                              float dyn_range, float dyn_exp, float typical_p, float top_p, float min_p, float xtc_p,
                              float xtc_t, int64_t min_keep, float *probs_out, int32_t *ids_out, int64_t cap,
                              int64_t *n_out) {
  try {
    CandResult r = sample_candidates_with_probs(Rng{*rng}, Row(vals, vals + n), Ids(ids, ids + n), temperature, dyn_range,
                                                dyn_exp, typical_p, top_p, min_p, xtc_p, xtc_t, min_keep);
    *rng = r.rng.state;
    if (n_out) *n_out = (int64_t)r.probs.size();
    for (size_t i = 0; i < r.probs.size() && (int64_t)i < cap; i++) {
      if (probs_out) probs_out[i] = r.probs[i];
      if (ids_out) ids_out[i] = r.ids[i];
    }
    return r.token;
  } catch (const std::exception &e) {
    g_err = e.what();
    return -1;
  }
}
int64_t orc_typical_filter(const float *probs, const float *logits, const int32_t *ids, int64_t n, float typical_p,
                           int64_t min_keep, float *kp, float *kl, int32_t *ki) {
  Row a, b;
  Ids c;
  typical_filter(Row(probs, probs + n), Row(logits, logits + n), Ids(ids, ids + n), typical_p, min_keep, a, b, c);
  memcpy(kp, a.data(), a.size() * sizeof(float));
  memcpy(kl, b.data(), b.size() * sizeof(float));
  memcpy(ki, c.data(), c.size() * sizeof(int32_t));
  return (int64_t)a.size();
}
float orc_dynamic_temperature(const float *probs, int64_t n, int64_t first, int64_t cutoff, float t, float range,
                              float expo) {
  return dynamic_temperature(Row(probs, probs + n), first, cutoff, t, range, expo);
}
int32_t orc_mirostat(int version, uint64_t *rng, const float *logits, int64_t n, float t, float tau, float eta,
                     float *mu) {
  MirostatResult r = version == 1 ? sample_mirostat_v1(Rng{*rng}, Row(logits, logits + n), n, t, tau, eta, *mu)
                                  : sample_mirostat_v2(Rng{*rng}, Row(logits, logits + n), n, t, tau, eta, *mu);
  *rng = r.rng.state;
  *mu = r.mu;
  return r.token;
}
int64_t orc_mirostat_v1_cutoff(const float *logits, int64_t n, float t, float mu, float *s_hat) {
  return mirostat_v1_cutoff_of(Row(logits, logits + n), n, t, mu, *s_hat);
}
int32_t orc_adaptive_p(uint64_t *rng, const float *logits, int64_t n, float target, float decay, float *ws, float *tw) {
  AdaptiveResult r = sample_adaptive_p(Rng{*rng}, Row(logits, logits + n), n, target, decay, *ws, *tw);
  *rng = r.rng.state;
  *ws = r.weighted_sum;
  *tw = r.total_weight;
  return r.token;
}

/* Params in a flat C struct (field meanings = orc::Params) */
typedef struct {
  float temperature, dynatemp_range, dynatemp_exponent, top_n_sigma;
  int64_t top_k;
  float typical_p, top_p, min_p, xtc_probability, xtc_threshold;
  int64_t min_keep;
  float repeat_penalty;
  int64_t repeat_last_n;
  float dry_multiplier, dry_base;
  int64_t dry_allowed_length, dry_penalty_last_n;
  float frequency_penalty, presence_penalty;
  int64_t n_probs;
  int64_t post_sampling_probs, ignore_eos;
  float final_softcap, logit_mul;
} orc_params;

static Params to_params(const orc_params *c) {
  Params p;
  p.temperature = c->temperature;
  p.dynatemp_range = c->dynatemp_range;
  p.dynatemp_exponent = c->dynatemp_exponent;
  p.top_n_sigma = c->top_n_sigma;
  p.top_k = c->top_k;
  p.typical_p = c->typical_p;
  p.top_p = c->top_p;
  p.min_p = c->min_p;
  p.xtc_probability = c->xtc_probability;
  p.xtc_threshold = c->xtc_threshold;
  p.min_keep = c->min_keep;
  p.repeat_penalty = c->repeat_penalty;
  p.repeat_last_n = c->repeat_last_n;
  p.dry_multiplier = c->dry_multiplier;
  p.dry_base = c->dry_base;
  p.dry_allowed_length = c->dry_allowed_length;
  p.dry_penalty_last_n = c->dry_penalty_last_n;
  p.frequency_penalty = c->frequency_penalty;
  p.presence_penalty = c->presence_penalty;
  p.n_probs = (int)c->n_probs;
  p.post_sampling_probs = c->post_sampling_probs != 0;
  p.ignore_eos = c->ignore_eos != 0;
  p.final_softcap = c->final_softcap;
  p.logit_mul = c->logit_mul;
  return p;
}

/* sample() (src/sampling.br:762) with an explicit history */
int32_t orc_sample(uint64_t *rng, const float *logits, int64_t n, const orc_params *cp, const int32_t *hist,
                   int64_t nh) {
  try {
    SampleResult r = sample_with_probs(Rng{*rng}, Row(logits, logits + n), n, to_params(cp), Ids(hist, hist + nh));
    *rng = r.rng.state;
    return r.token;
  } catch (const std::exception &e) {
    g_err = e.what();
    return -1;
  }
}

/* ---------------- UTF-8 ---------------- */
int64_t orc_bytes_to_cps(const uint8_t *b, int64_t n, uint32_t *out, int64_t cap) {
  std::vector<uint32_t> c = bytes_to_cps(b, (size_t)n);
  for (size_t i = 0; i < c.size() && (int64_t)i < cap; i++) out[i] = c[i];
  return (int64_t)c.size();
}
int orc_is_valid_utf8(const uint8_t *b, int64_t n) { return is_valid_utf8(b, (size_t)n) ? 1 : 0; }

/* ---------------- grammar ---------------- */
struct orc_grammar {
  Grammar g;
  std::unique_ptr<Matcher> m;
};
orc_grammar *orc_grammar_new(const char *gbnf) {
  try {
    orc_grammar *h = new orc_grammar;
    h->g = parse_gbnf(gbnf);
    h->m.reset(new Matcher(h->g));
    return h;
  } catch (const std::exception &e) {
    g_err = e.what();
    return nullptr;
  }
}
void orc_grammar_free(orc_grammar *h) { delete h; }
/* 1 complete / 0 not; -1 on error. viable: state non-empty. */
static int grammar_walk(orc_grammar *h, const char *text, int want_complete) {
  try {
    std::vector<uint32_t> cps = bytes_to_cps((const uint8_t *)text, strlen(text));
    State s = h->m->advance_text(h->m->start(), cps);
    return want_complete ? (h->m->complete(s) ? 1 : 0) : (s.empty() ? 0 : 1);
  } catch (const std::exception &e) {
    g_err = e.what();
    return -1;
  }
}
int orc_grammar_accepts(orc_grammar *h, const char *text) { return grammar_walk(h, text, 1); }
int orc_grammar_viable(orc_grammar *h, const char *text) { return grammar_walk(h, text, 0); }
int64_t orc_json_schema_to_gbnf(const char *schema, char *out, int64_t cap) {
  try {
    std::string s = json_schema_to_gbnf(schema);
    if ((int64_t)s.size() + 1 <= cap) memcpy(out, s.c_str(), s.size() + 1);
    return (int64_t)s.size();
  } catch (const std::exception &e) {
    g_err = e.what();
    return -1;
  }
}

int64_t orc_ngram_draft(const int32_t *tokens, int64_t n, int64_t max_draft, int64_t ngram_max, int64_t ngram_min,
                        int32_t *out) {
  Ids d = ngram_draft(Ids(tokens, tokens + n), max_draft, ngram_max, ngram_min);
  memcpy(out, d.data(), d.size() * sizeof(int32_t));
  return (int64_t)d.size();
}

/* ---------------- slots: one request's state, driven step by step ---------------- */
struct orc_slot {
  Slot s;
  Vocab vocab;
  bool has_vocab = false;
};
orc_slot *orc_slot_new(const orc_params *cp, uint64_t rng_state, const int32_t *history, int64_t n_hist,
                       const int32_t *reply, int64_t n_reply, const int32_t *bias_ids, const float *bias_vals,
                       int64_t n_bias) {
  orc_slot *h = new orc_slot;
  h->s.params = to_params(cp);
  h->s.rng = Rng{rng_state};
  h->s.tokens.assign(history, history + n_hist);
  h->s.reply.assign(reply, reply + n_reply);
  for (int64_t i = 0; i < n_bias; i++) h->s.bias[bias_ids[i]] = bias_vals[i];
  return h;
}
void orc_slot_free(orc_slot *h) { delete h; }
/* the request's tokenised DRY breakers (flat + lens, in order) */
void orc_slot_set_breakers(orc_slot *h, const int32_t *flat, const int32_t *lens, int64_t nb) {
  h->s.params.dry_breakers.clear();
  int64_t at = 0;
  for (int64_t i = 0; i < nb; i++) {
    h->s.params.dry_breakers.push_back(Ids(flat + at, flat + at + lens[i]));
    at += lens[i];
  }
}
uint64_t orc_slot_rng(orc_slot *h) { return h->s.rng.state; }
/* a token chosen outside the sampler: tokens.push, and reply_tokens.push unless end-of-generation */
void orc_slot_push(orc_slot *h, int32_t tok, int32_t eos_id) {
  h->s.tokens.push_back(tok);
  if (!is_eog_token(tok, eos_id)) h->s.reply.push_back(tok);
}
int orc_slot_set_grammar(orc_slot *h, const char *gbnf, const uint8_t *blob, const uint32_t *offsets, int64_t n_tokens,
                         int32_t eos_id) {
  try {
    h->s.grammar.reset(new Grammar(parse_gbnf(gbnf)));
    h->s.matcher.reset(new Matcher(*h->s.grammar));
    h->vocab.blob.assign(blob, blob + offsets[n_tokens]);
    h->vocab.offsets.assign(offsets, offsets + n_tokens + 1);
    h->vocab.eos_id = eos_id;
    h->has_vocab = true;
    return 0;
  } catch (const std::exception &e) {
    g_err = e.what();
    return -1;
  }
}
/* clears reply and history (a new request on the same grammar) */
void orc_slot_restart(orc_slot *h) {
  h->s.tokens.clear();
  h->s.reply.clear();
}
/* one decode step; returns 0, or -1 on a reference error (message in orc_last_error) */
int orc_slot_step(orc_slot *h, const float *logits, int64_t V, int wants_logprobs, int fast_grammar, int32_t *token,
                  float *logprob, int32_t *top_ids, float *top_lps, int *eog) {
  try {
    StepOut o = decode_step(h->s, logits, V, h->has_vocab ? &h->vocab : nullptr, wants_logprobs != 0, fast_grammar != 0);
    *token = o.token;
    if (logprob) *logprob = o.logprob;
    for (size_t i = 0; i < o.top_ids.size(); i++) {
      if (top_ids) top_ids[i] = o.top_ids[i];
      if (top_lps) top_lps[i] = o.top_logprobs[i];
    }
    if (eog) *eog = o.eog ? 1 : 0;
    return 0;
  } catch (const std::exception &e) {
    g_err = e.what();
    return -1;
  }
}
/* grammar allow-mask of the current reply; returns 1 ok, 0 dead state, -1 error */
/* response_format json_object on the slot (src/server.br:726), with the vocabulary pieces */
void orc_slot_set_json_object(orc_slot *h, const uint8_t *blob, const uint32_t *offsets, int64_t n_tokens,
                              int32_t eos_id) {
  h->s.json_object = true;
  h->vocab.blob.assign(blob, blob + offsets[n_tokens]);
  h->vocab.offsets.assign(offsets, offsets + n_tokens + 1);
  h->vocab.eos_id = eos_id;
  h->has_vocab = true;
}
/* the classifiers over code points (src/json.br:227, :394) */
int orc_json_prefix_state(const uint32_t *cps, int64_t n, int object) {
  std::vector<uint32_t> cs(cps, cps + n);
  return object ? json_object_prefix_state(cs) : json_prefix_state(cs);
}
int orc_slot_grammar_mask(orc_slot *h, int64_t V, uint32_t *mask, int *forced_eos, int fast) {
  try {
    std::vector<uint32_t> m;
    bool forced = false;
    bool ok = h->s.json_object ? json_object_mask(h->s, h->vocab, V, m, forced)
                               : grammar_mask(h->s, h->vocab, V, m, forced, fast != 0);
    memcpy(mask, m.data(), m.size() * sizeof(uint32_t));
    *forced_eos = forced ? 1 : 0;
    return ok ? 1 : 0;
  } catch (const std::exception &e) {
    g_err = e.what();
    return -1;
  }
}
int orc_slot_spec_verify(orc_slot *h, const float *rows, int64_t V, const int32_t *drafts, int64_t k, int32_t *tokens,
                         int32_t *accepted) {
  try {
    SpecOut o = spec_verify(h->s, rows, V, Ids(drafts, drafts + k));
    memcpy(tokens, o.tokens.data(), o.tokens.size() * sizeof(int32_t));
    *accepted = o.accepted;
    return 0;
  } catch (const std::exception &e) {
    g_err = e.what();
    return -1;
  }
}

/* ---------------- synthetic inputs (identical to the benchmark's) ---------------- */
void orc_synth_logits(int cfg, int64_t seed, int64_t step, int64_t row, int64_t V, float *out) {
  uint64_t st = bl_stream((uint32_t)cfg, seed, step, row, BL_P_LOGIT);
  int sigma = bl_cfg_sigma(cfg);
  for (int64_t i = 0; i < V; i++) out[i] = bl_normal(st, (uint64_t)i, sigma);
  if (cfg == 1) {
    for (int32_t id : blw::c1_bump_ids(seed, step, (int)V)) out[id] = out[id] + 8.0f;
  }
}

/* ---------------- workload drivers ---------------- */
static Params c1_params() {
  Params p;
  p.temperature = 0.8f;
  p.top_k = 40;
  p.top_p = 0.95f;
  p.min_p = 0.05f;
  p.repeat_penalty = 1.1f;
  p.repeat_last_n = 64;
  return p;
}

/* Workload 1: 1000 steps from seed 1234 in the benchmark; returns tokens[steps] */
int orc_run_c1(int64_t seed, int64_t steps, int32_t *tokens, double *usec) {
  const int V = BL_V_QWEN;
  Slot s;
  s.params = c1_params();
  s.rng = seed_rng(seed);
  s.tokens = blw::uniform_ids(1, seed, 0, 512, V);
  std::vector<float> row(V);
  double total = 0.0;
  try {
    for (int64_t t = 0; t < steps; t++) {
      orc_synth_logits(1, seed, t, 0, V, row.data());
      auto a = std::chrono::steady_clock::now();
      StepOut o = decode_step(s, row.data(), V, nullptr, false, true);
      auto b = std::chrono::steady_clock::now();
      total += std::chrono::duration<double, std::micro>(b - a).count();
      tokens[t] = o.token;
    }
  } catch (const std::exception &e) {
    g_err = e.what();
    return -1;
  }
  if (usec) *usec = total;
  return 0;
}

/* Workload 2 row setup shared by the driver and the tests */
static void c2_slot(Slot &s, int64_t seed, int r, int V) {
  Params p;
  p.temperature = bl_c2_temperature(r);
  p.top_k = bl_c2_top_k(r);
  p.top_p = bl_c2_top_p(r);
  p.frequency_penalty = 0.5f;
  p.presence_penalty = 0.3f;
  p.n_probs = 10;
  s.params = p;
  s.rng = seed_rng(seed + r);
  s.reply = blw::zipf_ids(2, seed, r, 4096, V, 1.1);
  s.tokens = s.reply;
  std::vector<int32_t> ids;
  std::vector<float> vals;
  blw::bias_list(2, seed, r, 300, V, -100.0, 100.0, ids, vals);
  for (size_t i = 0; i < ids.size(); i++) s.bias[ids[i]] = vals[i];
}

/* Workload 2: B=8; per step and row: token, logprob, 10 alternatives. `rows` limits the rows run
 * (the CPU baseline's bounded sample); usec receives the summed per-step time. */
int orc_run_c2(int64_t seed, int64_t steps, int rows, int32_t *tokens, float *lps, int32_t *top_ids, float *top_lps,
               double *usec) {
  const int V = BL_V_QWEN, B = 8;
  std::vector<Slot> slots(B);
  for (int r = 0; r < B; r++) c2_slot(slots[r], seed, r, V);
  std::vector<float> row(V);
  double total = 0.0;
  try {
    for (int64_t t = 0; t < steps; t++)
      for (int r = 0; r < rows; r++) {
        orc_synth_logits(2, seed, t, r, V, row.data());
        auto a = std::chrono::steady_clock::now();
        StepOut o = decode_step(slots[r], row.data(), V, nullptr, true, true);
        auto b = std::chrono::steady_clock::now();
        total += std::chrono::duration<double, std::micro>(b - a).count();
        int64_t at = t * B + r;
        tokens[at] = o.token;
        lps[at] = o.logprob;
        for (int i = 0; i < 10; i++) {
          top_ids[at * 10 + i] = i < (int)o.top_ids.size() ? o.top_ids[i] : -1;
          top_lps[at * 10 + i] = i < (int)o.top_logprobs.size() ? o.top_logprobs[i] : 0.0f;
        }
      }
  } catch (const std::exception &e) {
    g_err = e.what();
    return -1;
  }
  if (usec) *usec = total;
  return 0;
}

/* The per-row inputs of workload 2 for the GPU harness: reply history (4096) and bias (300). */
void orc_c2_row_inputs(int64_t seed, int r, int32_t *reply4096, int32_t *bias_ids300, float *bias_vals300) {
  std::vector<int32_t> z = blw::zipf_ids(2, seed, r, 4096, BL_V_QWEN, 1.1);
  memcpy(reply4096, z.data(), z.size() * sizeof(int32_t));
  std::vector<int32_t> ids;
  std::vector<float> vals;
  blw::bias_list(2, seed, r, 300, BL_V_QWEN, -100.0, 100.0, ids, vals);
  memcpy(bias_ids300, ids.data(), 300 * sizeof(int32_t));
  memcpy(bias_vals300, vals.data(), 300 * sizeof(float));
}

/* Workload 3: greedy grammar-constrained decode; per step: token, CRC32 of the allow-mask, forced flag.
 * The reply restarts after an end-of-sequence token. `fast` selects the carry form of the piece. */
int orc_run_c3(int64_t seed, int64_t steps, int fast, int32_t *tokens, uint32_t *mask_crc, int32_t *forced,
               double *usec) {
  const int V = BL_V_QWEN;
  Slot s;
  s.params = Params();  /* greedy, top_k 0 */
  s.rng = seed_rng(seed);
  Vocab v;
  blw::c3_vocab(seed, V, v.blob, v.offsets, v.eos_id);
  std::string gbnf;
  try {
    gbnf = json_schema_to_gbnf(blw::c3_schema());
    s.grammar.reset(new Grammar(parse_gbnf(gbnf)));
    s.matcher.reset(new Matcher(*s.grammar));
  } catch (const std::exception &e) {
    g_err = e.what();
    return -1;
  }
  std::vector<float> row(V);
  std::vector<uint32_t> mask;
  double total = 0.0;
  try {
    for (int64_t t = 0; t < steps; t++) {
      orc_synth_logits(3, seed, t, 0, V, row.data());
      bool fe = false;
      if (mask_crc) {
        grammar_mask(s, v, V, mask, fe, fast != 0);
        mask_crc[t] = crc32_bytes(mask.data(), mask.size() * 4);
      }
      auto a = std::chrono::steady_clock::now();
      StepOut o = decode_step(s, row.data(), V, &v, false, fast != 0);
      auto b = std::chrono::steady_clock::now();
      total += std::chrono::duration<double, std::micro>(b - a).count();
      tokens[t] = o.token;
      if (forced) forced[t] = fe ? 1 : 0;
      if (o.eog) {
        s.tokens.clear();
        s.reply.clear();
      }
    }
  } catch (const std::exception &e) {
    g_err = e.what();
    return -1;
  }
  if (usec) *usec = total;
  return 0;
}

/* Workload 4: B=32, V=262144, soft-cap 30, T 1, top_k 64, top_p 0.95, 20 logprobs. */
int orc_run_c4(int64_t seed, int64_t steps, int rows, int32_t *tokens, float *lps, int32_t *top_ids, float *top_lps,
               double *usec) {
  const int V = BL_V_GEMMA, B = 32;
  std::vector<Slot> slots(B);
  for (int r = 0; r < B; r++) {
    Params p;
    p.temperature = 1.0f;
    p.top_k = 64;
    p.top_p = 0.95f;
    p.n_probs = 20;
    p.final_softcap = 30.0f;
    slots[r].params = p;
    slots[r].rng = seed_rng(seed + r);
  }
  std::vector<float> row(V);
  double total = 0.0;
  try {
    for (int64_t t = 0; t < steps; t++)
      for (int r = 0; r < rows; r++) {
        orc_synth_logits(4, seed, t, r, V, row.data());
        auto a = std::chrono::steady_clock::now();
        StepOut o = decode_step(slots[r], row.data(), V, nullptr, true, true);
        auto b = std::chrono::steady_clock::now();
        total += std::chrono::duration<double, std::micro>(b - a).count();
        int64_t at = t * B + r;
        tokens[at] = o.token;
        lps[at] = o.logprob;
        for (int i = 0; i < 20; i++) {
          top_ids[at * 20 + i] = o.top_ids[i];
          top_lps[at * 20 + i] = o.top_logprobs[i];
        }
      }
  } catch (const std::exception &e) {
    g_err = e.what();
    return -1;
  }
  if (usec) *usec = total;
  return 0;
}

/* Workload 5: 16 sequences x (8 drafts + 1) rows; greedy and sampled (T 0.7, top_k 0) verification.
 * Per step: tokens[16*9] and accepted[16] for each mode. */
int orc_run_c5(int64_t seed, int64_t steps, int seqs, int32_t *g_tokens, int32_t *g_acc, int32_t *s_tokens,
               int32_t *s_acc, double *usec) {
  const int V = BL_V_QWEN, S = 16, K = 8;
  std::vector<Slot> gs(S), ss(S);
  for (int b = 0; b < S; b++) {
    gs[b].params = Params();
    gs[b].rng = seed_rng(seed + b);
    Params p;
    p.temperature = 0.7f;
    ss[b].params = p;
    ss[b].rng = seed_rng(seed + b);
  }
  std::vector<float> rows((size_t)(K + 1) * V);
  double total = 0.0;
  try {
    for (int64_t t = 0; t < steps; t++)
      for (int b = 0; b < seqs; b++) {
        int32_t am[K];
        for (int i = 0; i <= K; i++) {
          orc_synth_logits(5, seed, t, b * (K + 1) + i, V, rows.data() + (size_t)i * V);
          if (i < K) am[i] = sample_greedy(Row(rows.data() + (size_t)i * V, rows.data() + (size_t)(i + 1) * V), V);
        }
        Ids drafts = blw::c5_drafts(seed, t, b, am, K, V);
        auto a = std::chrono::steady_clock::now();
        SpecOut og = spec_verify(gs[b], rows.data(), V, drafts);
        SpecOut os = spec_verify(ss[b], rows.data(), V, drafts);
        auto e = std::chrono::steady_clock::now();
        total += std::chrono::duration<double, std::micro>(e - a).count();
        for (int i = 0; i <= K; i++) {
          g_tokens[(t * S + b) * (K + 1) + i] = og.tokens[i];
          s_tokens[(t * S + b) * (K + 1) + i] = os.tokens[i];
        }
        g_acc[t * S + b] = og.accepted;
        s_acc[t * S + b] = os.accepted;
      }
  } catch (const std::exception &e) {
    g_err = e.what();
    return -1;
  }
  if (usec) *usec = total;
  return 0;
}

/* Workload 3 static inputs for the GPU harness */
int64_t orc_c3_vocab(int64_t seed, uint8_t *blob, int64_t blob_cap, uint32_t *offsets, int32_t *eos) {
  std::vector<uint8_t> b;
  std::vector<uint32_t> o;
  int32_t e;
  blw::c3_vocab(seed, BL_V_QWEN, b, o, e);
  if (blob && (int64_t)b.size() <= blob_cap) memcpy(blob, b.data(), b.size());
  if (offsets) memcpy(offsets, o.data(), o.size() * sizeof(uint32_t));
  if (eos) *eos = e;
  return (int64_t)b.size();
}

} /* extern "C" */
