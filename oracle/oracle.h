/*
 * oracle.h — CPU restatement of boring-llm's per-step token-selection path.
 *
 * TEST INFRASTRUCTURE ONLY. This code is the checker the HIP path is compared against and the CPU
 * baseline the benchmark times. Nothing in the product library (boring-llm_amd/) may include, link
 * or call it; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it.
 *
 * It restates, function by function, the reference's Boring sources (paths relative to the
 * reference checkout):
 *   src/sampling.br        RNG, penalties, bias, greedy, logprobs, top-k, heap rank, candidate sampling,
 *                          typical, dynatemp, XTC, mirostat, adaptive-p, top-n-sigma, DRY
 *   src/io.br:64-147       lossy UTF-8 decoding (bytes_to_str, is_valid_utf8)
 *   src/grammar.br         GBNF parser and stack-machine matcher
 *   src/schema_grammar.br  JSON Schema -> GBNF (+ src/json.br json_parse, src/jinja.br jv_to_json)
 *   src/speculative.br     n-gram drafting
 *   src/server.br          decode-step stage order (:939-1036), grammar-constrained sampling
 *                          (:309-362), response_format json_object (:261-304, with src/json.br:227-426),
 *                          speculative verification (:1173-1216)
 *   src/model.br:973-984   final logit soft-capping
 *
 * Arithmetic follows the reference's lowering: Boring float32 -> Rust f32 -> IEEE binary32 with
 * round-to-nearest-even and no contraction (build with -ffp-contract=off), Rust f32::{exp,ln,tanh,
 * powf} -> the host glibc expf/logf/tanhf/powf, `as float32` from integers -> round to nearest even.
 * That lowering is an assumption about the external `boring` compiler, which is not vendored.
 *
 * What pins each part (tests/test_oracle_*.py, tests/test_device_math.py):
 *   RNG, seed fold, u64->f32      closed form with exact integer/Fraction arithmetic; the reference's
 *                                 determinism tests (test/test_sampling.br:7-13, :29-39)
 *   bias, penalties, greedy,      the reference's known answers (test/test_sampling.br:16, :42-61,
 *   top-k, heap rank (distinct)   :187-264) and lexsort/brute-force rankings on random rows
 *   heap rank among equal values  numpy's heapsort (same bottom-up max-heap and extraction), reversed, on
 *                                 1,200 tied arrays and a bfloat16 row of 151,936 (test_oracle_pinning.py)
 *   logprob normaliser            np.cumsum (a sequential float32 sum) over glibc expf terms, bit for bit,
 *                                 at V up to 262,144, then glibc logf; the reference's approximate known
 *                                 answers (:19-26)
 *   candidate sampling            sum_exp, the top-p running probability, the min-p cut, the tempered sum,
 *                                 the draw target and position restated with numpy sequential sums and glibc
 *                                 expf, bit for bit (full-vocabulary lists of 151,936 and 150 short lists);
 *                                 known answers typical->8, XTC->9, min_p=1 (:112-122, :163-167, :268-272);
 *                                 a chi-square check of the draw distribution
 *   soft-cap                      float64 closed form within float32 rounding (test/test_arch.br); the device
 *                                 tanhf equals glibc's over all 2^32 inputs
 *   grammar, schema, UTF-8,       transliterations of test/test_grammar.br, test_schema_grammar.br,
 *   n-gram drafts                 test_tokenizer.br:52-58, test_speculative.br; the workload-3 GBNF
 *                                 against its hand derivation; the carry form of a candidate piece
 *                                 against the literal whole-reply re-decode
 *   full-vocabulary masks         by composition of pinned parts: each bit is grammar_advance_text over
 *                                 the candidate's piece, the piece is bytes_to_str of the carry form, and the
 *                                 carry form equals the literal whole-reply re-decode (test_oracle_grammar.py)
 *   speculative verification      sequential decoding of the same rows (CHANGELOG.md:92's invariant)
 *   top-n-sigma statistics        numpy's sequential float64 sums, bit for bit (test_oracle_pinning.py)
 *   mirostat v1 fit               a float32 loop over glibc logf/powf, and a Zipf closed form
 *   JSON prefix classifier        the reference's known answers (test/test_json.br:67-99) and the prefixes of
 *                                 documents Python's json module writes (test_oracle_json.py)
 * Every check above fails against a build with a planted mistake where one is listed in oracle/Makefile
 * (`mutants`: sift tie direction, pairwise normaliser, reversed softmax sum, split tempered sum, top-n-sigma
 * float32 sum, mirostat v1 fit without its last pair, a leading zero followed by digits).
 * Assumed, not pinned: that the external `boring` compiler lowers float32 exp/ln/tanh/powf to Rust f32 and
 * so to glibc (it is not vendored); the oracle and the device follow glibc 2.35 exactly.
 */
#ifndef BL_ORACLE_H
#define BL_ORACLE_H

#include <stdint.h>

#include <map>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

namespace orc {

/* ---------------- sampling.br ---------------- */
struct Rng {
  uint64_t state;
};
int64_t resolve_seed(int64_t requested, uint64_t entropy, int64_t request_counter);
Rng seed_rng(int64_t seed);
uint64_t rng_next_u64(Rng &rng);
float rng_next_f32(Rng &rng);

typedef std::vector<float> Row;
typedef std::vector<int32_t> Ids;

Row apply_repeat_penalty(const Row &logits, const Ids &history, float penalty, int64_t repeat_last_n);
Row apply_presence_frequency_penalty(const Row &logits, const Ids &generated, float frequency, float presence);
Row apply_dry_penalty(const Row &logits, const Ids &history, float multiplier, float base, int64_t allowed_length,
                      int64_t penalty_last_n, const std::vector<Ids> &breakers);
/* logit_bias as {id: bias}; std::map iteration order is immaterial (distinct keys) */
Row apply_logit_bias(const Row &logits, const std::map<int32_t, float> &biases);
void set_eog_tokens(const Ids &ids, int32_t close_id);
bool is_eog_token(int32_t token, int32_t eos_id);
int32_t turn_close_token(int32_t eos_id);
Row suppress_eog_tokens(const Row &logits, int32_t eos_id);
Row suppress_token(const Row &logits, int32_t token);
int32_t sample_greedy(const Row &logits, int64_t vocab);
void logprob_normalizer(const Row &logits, int64_t vocab, float &maximum, float &log_sum_exp,
                        float *sum_out = nullptr);
float normalized_token_logprob(const Row &logits, int32_t token, float maximum, float log_sum_exp);
float token_logprob(const Row &logits, int64_t vocab, int32_t token);
void top_k_select(const Row &logits, int64_t vocab, int64_t k, Row &top_val, Ids &top_idx);
void all_candidates_sorted(const Row &logits, int64_t vocab, Row &values, Ids &ids);
void rank_candidates(const Row &logits, int64_t vocab, int64_t top_k, Row &values, Ids &ids);
bool top_n_sigma_threshold(const Row &logits, int64_t vocab, float n, float &threshold);
Row top_n_sigma_logits(const Row &logits, int64_t vocab, float n);
void typical_filter(const Row &probs, const Row &logits, const Ids &ids, float typical_p, int64_t min_keep,
                    Row &kept_probs, Row &kept_logits, Ids &kept_ids);
float dynamic_temperature(const Row &probs, int64_t first, int64_t cutoff, float temperature, float range,
                          float exponent);

struct CandResult {
  int32_t token;
  Rng rng;
  Row probs;
  Ids ids;
};
/* the float32 running sums of one call, for the checks that pin them (tests/test_oracle_pinning.py) */
struct CandTrace {
  float sum_exp;      /* untempered softmax denominator, rank order */
  int64_t cutoff;     /* after top-p and min-p */
  int64_t first;      /* after XTC */
  float temperature;  /* effective (dynamic) temperature */
  float renorm_sum;   /* tempered sum over [first, cutoff) */
  float target;       /* r01 * renorm_sum */
  int64_t chosen;     /* drawn list position */
};
/* throws std::runtime_error("sample_candidates: empty or mismatched candidates") */
CandResult sample_candidates_with_probs(Rng rng, const Row &top_val, const Ids &top_idx, float temperature,
                                        float dynatemp_range, float dynatemp_exponent, float typical_p, float top_p,
                                        float min_p, float xtc_probability, float xtc_threshold, int64_t min_keep,
                                        CandTrace *trace = nullptr);
int32_t sample_candidates(Rng &rng, const Row &top_val, const Ids &top_idx, float temperature, float dynatemp_range,
                          float dynatemp_exponent, float typical_p, float top_p, float min_p, float xtc_probability,
                          float xtc_threshold, int64_t min_keep);

struct MirostatResult {
  int32_t token;
  Rng rng;
  float mu;
};
MirostatResult sample_mirostat_v2(Rng rng, const Row &logits, int64_t vocab, float temperature, float tau, float eta,
                                  float mu);
MirostatResult sample_mirostat_v1(Rng rng, const Row &logits, int64_t vocab, float temperature, float tau, float eta,
                                  float mu);
/* the prefix length sample_mirostat_v1 draws from (temperature > 0), and the fitted exponent s_hat */
int64_t mirostat_v1_cutoff_of(const Row &logits, int64_t vocab, float temperature, float mu, float &s_hat);
struct AdaptiveResult {
  int32_t token;
  Rng rng;
  float weighted_sum, total_weight;
};
AdaptiveResult sample_adaptive_p(Rng rng, const Row &logits, int64_t vocab, float target, float decay,
                                 float weighted_sum, float total_weight);

/* SamplingParams (src/model.br:1565-1584) + the server's extra per-request fields (src/server.br:665-760) */
struct Params {
  float temperature = 0.0f;
  float dynatemp_range = 0.0f;
  float dynatemp_exponent = 1.0f;
  float top_n_sigma = -1.0f;
  int64_t top_k = 0;
  float typical_p = 1.0f;
  float top_p = 1.0f;
  float min_p = 0.0f;
  float xtc_probability = 0.0f;
  float xtc_threshold = 0.1f;
  int64_t min_keep = 0;
  int64_t seed = 0;
  float repeat_penalty = 1.0f;
  int64_t repeat_last_n = 64;
  float dry_multiplier = 0.0f;
  float dry_base = 1.75f;
  int64_t dry_allowed_length = 2;
  int64_t dry_penalty_last_n = 64;
  std::vector<Ids> dry_breakers;
  /* server extras */
  float frequency_penalty = 0.0f;
  float presence_penalty = 0.0f;
  int n_probs = 0;
  bool post_sampling_probs = false;
  bool ignore_eos = false;
  float final_softcap = 0.0f; /* model tail, src/model.br:973-984 */
  float logit_mul = 1.0f;
};

struct SampleResult {
  int32_t token;
  Rng rng;
  Row probs;
  Ids ids;
};
SampleResult sample_with_probs(Rng rng, const Row &logits, int64_t vocab, const Params &p, const Ids &history);
Row sampling_logits(const Row &logits, const Ids &history, float repeat_penalty, int64_t repeat_last_n);

/* ---------------- model.br tail ---------------- */
Row finish_logits(const Row &logits, float logit_mul, float final_softcap);

/* ---------------- io.br ---------------- */
/* decoded code points; U+FFFD for each bad byte */
std::vector<uint32_t> bytes_to_cps(const uint8_t *bytes, size_t n);
bool is_valid_utf8(const uint8_t *bytes, size_t n);
std::string cps_to_utf8(const std::vector<uint32_t> &cps);

/* ---------------- grammar.br ---------------- */
struct GElem {
  int kind; /* 0 charset, 1 rule ref */
  int rule;
  std::vector<int64_t> ranges;
  bool negated;
  std::string key;
};
struct Grammar {
  std::vector<std::vector<std::vector<GElem>>> rules;
  int root = 0;
};
/* throws std::runtime_error with the reference's message */
Grammar parse_gbnf(const std::string &text);

/* A matcher state is the reference's list of stacks. Stacks are interned (an element key sequence);
 * a State keeps the reference's list order. `Matcher` memoises the pure advance function. */
typedef std::vector<int> State; /* interned stack ids */
class Matcher {
 public:
  explicit Matcher(const Grammar &g);
  State start();                                  /* grammar_start */
  State advance(const State &s, uint32_t cp);     /* grammar_advance */
  State advance_text(const State &s, const std::vector<uint32_t> &cps); /* grammar_advance_text */
  bool complete(const State &s);                  /* grammar_complete */
  bool can_continue(const State &s);              /* grammar_can_continue */
  bool allows_non_ascii(const State &s);          /* grammar_allows_non_ascii */
  size_t n_stacks() const { return stacks_.size(); }

 private:
  State expand(const std::vector<std::vector<int>> &stacks);
  int intern_elem(const GElem &e);
  int intern_stack(const std::vector<int> &st);
  const Grammar &g_;
  std::vector<GElem> elems_;
  std::unordered_map<std::string, int> elem_ids_;
  std::vector<std::vector<int>> stacks_;
  std::map<std::vector<int>, int> stack_ids_;
  std::map<std::pair<State, uint32_t>, State> memo_;
};

/* ---------------- schema_grammar.br (+ json.br / jinja.br) ---------------- */
std::string json_schema_to_gbnf(const std::string &schema_json); /* throws */

/* ---------------- speculative.br ---------------- */
Ids ngram_draft(const Ids &tokens, int64_t max_draft, int64_t ngram_max, int64_t ngram_min);

/* ---------------- server.br decode step ---------------- */
struct Vocab {
  std::vector<uint8_t> blob;
  std::vector<uint32_t> offsets; /* n_tokens + 1 */
  int32_t eos_id = -1;
  Ids eog_ids; /* registered EOG ids besides eos */
  std::vector<bool> special;
  int n() const { return (int)offsets.size() - 1; }
};

struct Slot {
  Ids tokens;                     /* prompt + reply (repeat penalty / DRY history) */
  Ids reply;                      /* reply tokens (frequency / presence) */
  std::map<int32_t, float> bias;  /* request logit_bias */
  Rng rng{0};
  Params params;
  std::unique_ptr<Grammar> grammar;
  std::unique_ptr<Matcher> matcher;
  bool json_object = false; /* response_format json_object (src/server.br:726, :985) */
};

struct StepOut {
  int32_t token = -1;
  float logprob = 0.0f;
  Ids top_ids;
  Row top_logprobs;
  bool eog = false;
};

/* One iteration of the decode loop's sampling block (src/server.br:940-1036) for the standard chain
 * or the grammar-constrained sampler, then the pushes of :1004 and :1037. Throws on the reference's
 * error paths. `wants_logprobs` follows :943 (logprobs requested). `vocab` may be null when no
 * grammar is set. `fast_grammar` selects the carry-based piece computation (identical results to
 * re-decoding the whole reply, proven by the tests) instead of the literal per-candidate re-decode. */
/* ---------------- json.br prefix classifier, sample_json_token (json_prefix.cpp) ---------------- */
int json_prefix_state(const std::vector<uint32_t> &cs);
int json_object_prefix_state(const std::vector<uint32_t> &cs);
bool json_object_mask(const Slot &slot, const Vocab &v, int64_t V, std::vector<uint32_t> &mask, bool &forced_eos);
int32_t sample_json_token(Slot &slot, const Vocab &v, const Row &logits, int64_t vocab);

StepOut decode_step(Slot &slot, const float *logits, int64_t V, const Vocab *vocab, bool wants_logprobs,
                    bool fast_grammar);

/* Allow-mask of the grammar-constrained sampler for the current reply: bit t set when candidate t
 * would be kept by src/server.br:336-356 (EOG rule included). Returns false when the state is dead
 * ("the reply no longer matches the grammar"); `forced_eos` reports :321-323. */
bool grammar_mask(Slot &slot, const Vocab &vocab, int64_t V, std::vector<uint32_t> &mask, bool &forced_eos,
                  bool fast);

/* Speculative verification (src/server.br:1173-1216): rows [(k+1) x V]; samples row i under the
 * history extended by drafts[0..i); every row's token is reported (row i as if drafts[0..i) were
 * accepted, RNG advanced i times). accepted = leading matches; the slot commits drafts[0..accepted)
 * plus tokens[accepted] and its RNG advances accepted+1 draws. */
struct SpecOut {
  Ids tokens; /* k+1 */
  int accepted = 0;
};
SpecOut spec_verify(Slot &slot, const float *rows, int64_t V, const Ids &drafts);

} /* namespace orc */

#endif /* BL_ORACLE_H */
