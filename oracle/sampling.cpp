/*
 * sampling.cpp — restatement of the reference's src/sampling.br and src/model.br:973-984.
 * TEST INFRASTRUCTURE ONLY (see oracle.h). Line numbers cite src/sampling.br unless stated.
 */
#include <math.h>

#include <algorithm>
#include <set>
#include <stdexcept>
#include <unordered_map>
#include <unordered_set>

#include "oracle.h"

namespace orc {

static const uint64_t SEED_FOLD = 88172645463325252ull;

/* :21-33 */
int64_t resolve_seed(int64_t requested, uint64_t entropy, int64_t request_counter) {
  if (requested >= 0) return requested;
  uint64_t mixed = entropy ^ ((uint64_t)request_counter << 32) ^ (uint64_t)request_counter;
  mixed = mixed ^ (mixed << 13);
  mixed = mixed ^ (mixed >> 7);
  mixed = mixed ^ (mixed << 17);
  int64_t chosen = (int64_t)(mixed & 2147483647ull);
  return chosen == 0 ? 1 : chosen;
}

/* :35-40 */
Rng seed_rng(int64_t seed) {
  uint64_t s = seed == 0 ? SEED_FOLD : ((uint64_t)seed ^ SEED_FOLD);
  return Rng{s};
}

/* :42-47 xorshift64 (13, 7, 17) */
uint64_t rng_next_u64(Rng &rng) {
  uint64_t x = rng.state;
  x = x ^ (x << 13);
  x = x ^ (x >> 7);
  x = x ^ (x << 17);
  rng.state = x;
  return x;
}

/* :51-54 u64 -> f32 (round to nearest even) divided by 2^64 */
float rng_next_f32(Rng &rng) {
  uint64_t x = rng_next_u64(rng);
  float f = (float)x / 18446744073709551616.0f;
  return f;
}

/* :65-85 */
Row apply_repeat_penalty(const Row &logits, const Ids &history, float penalty, int64_t repeat_last_n) {
  if (penalty == 1.0f || repeat_last_n == 0 || history.empty()) return logits;
  Row out(logits.size());
  for (size_t i = 0; i < logits.size(); i++) out[i] = logits[i];
  int64_t hl = (int64_t)history.size();
  int64_t window = (repeat_last_n > 0 && hl > repeat_last_n) ? repeat_last_n : hl;
  int64_t start = hl - window;
  std::unordered_set<int32_t> seen;
  for (int64_t j = start; j < hl; j++) {
    int32_t tok = history[j];
    if (!seen.count(tok)) {
      seen.insert(tok);
      float v = out[tok];
      out[tok] = v > 0.0f ? v / penalty : v * penalty;
    }
  }
  return out;
}

/* :91-107 */
Row apply_presence_frequency_penalty(const Row &logits, const Ids &generated, float frequency, float presence) {
  if ((frequency == 0.0f && presence == 0.0f) || generated.empty()) return logits;
  Row out(logits.size());
  for (size_t i = 0; i < logits.size(); i++) out[i] = logits[i];
  std::unordered_map<int32_t, int64_t> counts;
  for (int32_t tok : generated) counts[tok] += 1;
  for (auto &kv : counts) {
    int32_t tok = kv.first;
    float c = (float)kv.second;
    float t = c * frequency;
    out[tok] = out[tok] - t - presence;
  }
  return out;
}

/* :114-171 */
Row apply_dry_penalty(const Row &logits, const Ids &history, float multiplier, float base, int64_t allowed_length,
                      int64_t penalty_last_n, const std::vector<Ids> &breakers) {
  if (multiplier == 0.0f || base < 1.0f || penalty_last_n == 0) return logits;
  int64_t hl = (int64_t)history.size();
  int64_t window = hl > penalty_last_n ? penalty_last_n : hl;
  if (window <= allowed_length) return logits;
  int64_t start = hl - window;
  for (const Ids &breaker : breakers) {
    int64_t bl = (int64_t)breaker.size();
    if (bl > 0 && bl <= hl - start) {
      int64_t at = hl - bl;
      while (at >= start) {
        bool matches = true;
        int64_t b = 0;
        while (b < bl && matches) {
          if (history[at + b] != breaker[b]) matches = false;
          b += 1;
        }
        if (matches && at + bl > start) {
          start = at + bl;
          at = start - 1;
        } else {
          at -= 1;
        }
      }
    }
  }
  int64_t suffix_len = hl - start;
  if (suffix_len < allowed_length) return logits;
  Row out(logits.size());
  for (size_t v = 0; v < logits.size(); v++) out[v] = logits[v];
  /* {int=int} map; iteration order of keys is immaterial (each key touched once) */
  std::map<int32_t, int64_t> maximum_repeat;
  int64_t candidate_at = start + 1;
  while (candidate_at < hl) {
    int64_t repeated = 0;
    while (repeated < suffix_len && candidate_at - repeated - 1 >= start &&
           history[candidate_at - repeated - 1] == history[hl - repeated - 1])
      repeated += 1;
    if (repeated >= allowed_length) {
      int32_t token = history[candidate_at];
      auto it = maximum_repeat.find(token);
      int64_t previous = it == maximum_repeat.end() ? -1 : it->second;
      if (repeated > previous) maximum_repeat[token] = repeated;
    }
    candidate_at += 1;
  }
  for (auto &kv : maximum_repeat) {
    int32_t token = kv.first;
    bool exempt = false;
    for (const Ids &breaker : breakers)
      if (breaker.size() == 1 && breaker[0] == token) exempt = true;
    if (!exempt) {
      int64_t repeated = kv.second;
      int64_t exponent = repeated - allowed_length;
      if (base > 1.000001f) {
        /* `(88.7228391 / base.ln()) as int`: Rust float->int casts truncate and saturate */
        float q = 88.7228391f / logf(base);
        int64_t maximum_exponent = (int64_t)q;
        if (exponent > maximum_exponent) exponent = maximum_exponent;
      }
      float pw = powf(base, (float)exponent);
      float t = multiplier * pw;
      out[token] = out[token] - t;
    }
  }
  return out;
}

/* :175-188 */
Row apply_logit_bias(const Row &logits, const std::map<int32_t, float> &biases) {
  if (biases.empty()) return logits;
  Row out(logits.size());
  for (size_t i = 0; i < logits.size(); i++) out[i] = logits[i];
  for (auto &kv : biases) out[kv.first] = out[kv.first] + kv.second;
  return out;
}

/* :200-237 */
static Ids g_eog_ids;
static int32_t g_turn_close = -1;

void set_eog_tokens(const Ids &ids, int32_t close_id) {
  g_eog_ids = ids;
  g_turn_close = close_id;
}

bool is_eog_token(int32_t token, int32_t eos_id) {
  if (token == eos_id) return true;
  for (int32_t id : g_eog_ids)
    if (id == token) return true;
  return false;
}

int32_t turn_close_token(int32_t eos_id) { return g_turn_close >= 0 ? g_turn_close : eos_id; }

Row suppress_eog_tokens(const Row &logits, int32_t eos_id) {
  Row out = suppress_token(logits, eos_id);
  for (int32_t id : g_eog_ids) out = suppress_token(out, id);
  return out;
}

Row suppress_token(const Row &logits, int32_t token) {
  if (token < 0 || token >= (int64_t)logits.size()) return logits;
  Row out(logits.size());
  for (size_t i = 0; i < logits.size(); i++) out[i] = logits[i];
  out[token] = -1000000000.0f;
  return out;
}

/* :239-249 strict `>`: lowest index among equal maxima */
int32_t sample_greedy(const Row &logits, int64_t vocab) {
  int32_t best = 0;
  float best_val = logits[0];
  for (int64_t v = 1; v < vocab; v++) {
    float val = logits[v];
    if (val > best_val) {
      best_val = val;
      best = (int32_t)v;
    }
  }
  return best;
}

/* :254-266 sequential float32 sum in index order */
void logprob_normalizer(const Row &logits, int64_t vocab, float &maximum, float &log_sum_exp, float *sum_out) {
  float mx = logits[0];
  for (int64_t i = 1; i < vocab; i++)
    if (logits[i] > mx) mx = logits[i];
  float sum_exp = 0.0f;
#if ORC_MUTANT == 2 /* planted mistake (tests only): a pairwise sum instead of the sequential one */
  Row t(vocab);
  for (int64_t i = 0; i < vocab; i++) t[i] = expf(logits[i] - mx);
  for (int64_t w = 1; w < vocab; w *= 2)
    for (int64_t i = 0; i + w < vocab; i += 2 * w) t[i] += t[i + w];
  sum_exp = t[0];
#else
  for (int64_t i = 0; i < vocab; i++) sum_exp += expf(logits[i] - mx);
#endif
  maximum = mx;
  log_sum_exp = logf(sum_exp);
  if (sum_out) *sum_out = sum_exp;
}

/* :268-269 */
float normalized_token_logprob(const Row &logits, int32_t token, float maximum, float log_sum_exp) {
  float t = logits[token] - maximum;
  return t - log_sum_exp;
}

/* :271-273 */
float token_logprob(const Row &logits, int64_t vocab, int32_t token) {
  float mx, lse;
  logprob_normalizer(logits, vocab, mx, lse);
  return normalized_token_logprob(logits, token, mx, lse);
}

/* :280-296 insertion selection; values <= -1e30 never enter; unfilled slots stay (-1e30, 0) */
void top_k_select(const Row &logits, int64_t vocab, int64_t k, Row &top_val, Ids &top_idx) {
  int64_t kk = k > vocab ? vocab : k;
  top_val.assign(kk, -1.0e30f);
  top_idx.assign(kk, 0);
  for (int64_t v = 0; v < vocab; v++) {
    float val = logits[v];
    if (val > top_val[kk - 1]) {
      int64_t slot = kk - 1;
      while (slot > 0 && val > top_val[slot - 1]) {
        top_val[slot] = top_val[slot - 1];
        top_idx[slot] = top_idx[slot - 1];
        slot -= 1;
      }
      top_val[slot] = val;
      top_idx[slot] = (int32_t)v;
    }
  }
}

/* :301-365 bottom-up max-heap build, then repeated extraction (the heap's own tie order) */
static void sift_down(Row &hv, Ids &hi, int64_t root, int64_t size) {
  bool placed = false;
  while (!placed) {
    int64_t left = root * 2 + 1;
    if (left >= size) {
      placed = true;
    } else {
      int64_t child = left;
      int64_t right = left + 1;
#if ORC_MUTANT == 1 /* planted mistake (tests only): ties go to the right child */
      if (right < size && hv[right] >= hv[left]) child = right;
#else
      if (right < size && hv[right] > hv[left]) child = right;
#endif
      if (hv[child] <= hv[root]) {
        placed = true;
      } else {
        std::swap(hv[root], hv[child]);
        std::swap(hi[root], hi[child]);
        root = child;
      }
    }
  }
}

void all_candidates_sorted(const Row &logits, int64_t vocab, Row &values, Ids &ids) {
  Row hv(vocab);
  Ids hi(vocab);
  for (int64_t i = 0; i < vocab; i++) {
    hv[i] = logits[i];
    hi[i] = (int32_t)i;
  }
  for (int64_t parent = vocab / 2 - 1; parent >= 0; parent--) sift_down(hv, hi, parent, vocab);
  values.assign(vocab, 0.0f);
  ids.assign(vocab, 0);
  int64_t heap_size = vocab;
  int64_t i = 0;
  while (heap_size > 0) {
    values[i] = hv[0];
    ids[i] = hi[0];
    heap_size -= 1;
    if (heap_size > 0) {
      hv[0] = hv[heap_size];
      hi[0] = hi[heap_size];
      sift_down(hv, hi, 0, heap_size);
    }
    i += 1;
  }
}

/* :367-371 */
void rank_candidates(const Row &logits, int64_t vocab, int64_t top_k, Row &values, Ids &ids) {
  if (top_k > 0 && top_k < vocab) top_k_select(logits, vocab, top_k, values, ids);
  else all_candidates_sorted(logits, vocab, values, ids);
}

/* :376-407 (statistics in float64); the threshold maximum - n * sigma, or false when the row is kept whole */
bool top_n_sigma_threshold(const Row &logits, int64_t vocab, float n, float &threshold) {
  if (n <= 0.0f || vocab <= 1) return false;
  float maximum = -1.0e30f;
  double sum = 0.0, sum_sq = 0.0;
  int64_t count = 0;
  for (int64_t i = 0; i < vocab; i++) {
    float value = logits[i];
    if (value > -1.0e29f) {
      if (value > maximum) maximum = value;
#if ORC_MUTANT == 5 /* planted mistake (tests only): the value sum in float32 */
      sum = (double)((float)sum + value);
#else
      sum += (double)value;
#endif
      double vd = (double)value;
      double sq = vd * vd;
      sum_sq += sq;
      count += 1;
    }
  }
  if (count <= 1) return false;
  double mean = sum / (double)count;
  double msq = mean * mean;
  double variance = sum_sq / (double)count - msq;
  if (variance <= 0.0) return false;
  float sigma = (float)sqrt(variance);
  float ns = n * sigma;
  threshold = maximum - ns;
  return true;
}

Row top_n_sigma_logits(const Row &logits, int64_t vocab, float n) {
  float threshold;
  if (!top_n_sigma_threshold(logits, vocab, n, threshold)) return logits;
  Row filtered(vocab, -1.0e30f);
  for (int64_t i = 0; i < vocab; i++)
    if (logits[i] >= threshold) filtered[i] = logits[i];
  return filtered;
}

/* :424-465 */
void typical_filter(const Row &probs, const Row &logits, const Ids &ids, float typical_p, int64_t min_keep,
                    Row &kept_probs, Row &kept_logits, Ids &kept_ids) {
  if (typical_p >= 1.0f || probs.size() <= 1) {
    kept_probs = probs;
    kept_logits = logits;
    kept_ids = ids;
    return;
  }
  int64_t n = (int64_t)probs.size();
  float entropy = 0.0f;
  for (int64_t i = 0; i < n; i++)
    if (probs[i] > 0.0f) {
      float t = probs[i] * logf(probs[i]);
      entropy -= t;
    }
  std::vector<bool> selected(n, false);
  int64_t required = min_keep > 1 ? min_keep : 1;
  float cumulative = 0.0f;
  int64_t count = 0;
  while (count < n && (cumulative < typical_p || count < required)) {
    int64_t best = -1;
    float best_distance = 3.4028235e38f;
    for (int64_t i = 0; i < n; i++) {
      if (!selected[i] && probs[i] > 0.0f) {
        float nl = -logf(probs[i]);
        float distance = fabsf(nl - entropy);
        if (best < 0 || distance < best_distance) {
          best = i;
          best_distance = distance;
        }
      }
    }
    if (best < 0) {
      count = n;
    } else {
      selected[best] = true;
      cumulative += probs[best];
      count += 1;
    }
  }
  kept_probs.clear();
  kept_logits.clear();
  kept_ids.clear();
  for (int64_t i = 0; i < n; i++)
    if (selected[i]) {
      kept_probs.push_back(probs[i]);
      kept_logits.push_back(logits[i]);
      kept_ids.push_back(ids[i]);
    }
}

/* :467-488 */
float dynamic_temperature(const Row &probs, int64_t first, int64_t cutoff, float temperature, float range,
                          float exponent) {
  if (range <= 0.0f || cutoff - first <= 1) return temperature;
  float surviving_sum = 0.0f;
  for (int64_t i = first; i < cutoff; i++) surviving_sum += probs[i];
  float entropy = 0.0f;
  for (int64_t i = first; i < cutoff; i++) {
    float probability = probs[i] / surviving_sum;
    if (probability > 0.0f) {
      float t = probability * logf(probability);
      entropy -= t;
    }
  }
  int64_t candidate_count = cutoff - first;
  float max_entropy = logf((float)candidate_count);
  float normalized_entropy = entropy / max_entropy;
  float min_temperature = temperature > range ? temperature - range : 0.0f;
  float max_temperature = temperature + range;
  float span = max_temperature - min_temperature;
  float pw = powf(normalized_entropy, exponent);
  float t = span * pw;
  return min_temperature + t;
}

/* :490-607 */
CandResult sample_candidates_with_probs(Rng rng, const Row &top_val, const Ids &top_idx, float temperature,
                                        float dynatemp_range, float dynatemp_exponent, float typical_p, float top_p,
                                        float min_p, float xtc_probability, float xtc_threshold, int64_t min_keep,
                                        CandTrace *trace) {
  if (!(top_val.size() > 0 && top_val.size() == top_idx.size()))
    throw std::runtime_error("sample_candidates: empty or mismatched candidates");
  if (temperature <= 0.0f) return CandResult{top_idx[0], rng, Row{1.0f}, Ids{top_idx[0]}};
  int64_t n = (int64_t)top_val.size();
  int64_t keep = min_keep > 1 ? min_keep : 1;
  if (keep > n) keep = n;

  /* untempered softmax, sequential float32 sum in rank order (:506-517) */
  Row probs(n, 0.0f);
  float sum_exp = 0.0f;
  for (int64_t i = 0; i < n; i++) {
    float e = expf(top_val[i] - top_val[0]);
    probs[i] = e;
#if ORC_MUTANT != 3
    sum_exp += e;
#endif
  }
#if ORC_MUTANT == 3 /* planted mistake (tests only): the softmax sum in reverse rank order */
  for (int64_t i = n - 1; i >= 0; i--) sum_exp += probs[i];
#endif
  for (int64_t i = 0; i < n; i++) probs[i] = probs[i] / sum_exp;

  Row tprobs, tvalues;
  Ids tidx;
  typical_filter(probs, top_val, top_idx, typical_p, keep, tprobs, tvalues, tidx);
  probs = tprobs;
  const Row &candidate_values = tvalues;
  const Ids &candidate_idx = tidx;
  int64_t filtered_n = (int64_t)probs.size();
  if (keep > filtered_n) keep = filtered_n;

  /* top-p (:530-540) */
  int64_t cutoff = filtered_n;
  if (top_p < 1.0f) {
    float cum = 0.0f;
    int64_t j = 0;
    bool cut_found = false;
    while (j < filtered_n && !cut_found) {
      cum += probs[j];
      j += 1;
      if (cum >= top_p && j >= keep) {
        cutoff = j;
        cut_found = true;
      }
    }
  }
  /* min-p (:545-550) */
  if (min_p > 0.0f) {
    float threshold = probs[0] * min_p;
    int64_t min_cutoff = keep;
    while (min_cutoff < cutoff && probs[min_cutoff] >= threshold) min_cutoff += 1;
    cutoff = min_cutoff;
  }
  /* XTC (:555-572) */
  int64_t first = 0;
  Rng sample_rng = rng;
  if (xtc_probability > 0.0f && xtc_threshold <= 0.5f && cutoff >= 2) {
    float chance = rng_next_f32(sample_rng);
    if (chance <= xtc_probability) {
      float xtc_sum = 0.0f;
      for (int64_t i = 0; i < cutoff; i++) xtc_sum += probs[i];
      int64_t pos_last = 0;
      int64_t i = 0;
      while (i < cutoff && probs[i] / xtc_sum >= xtc_threshold) {
        pos_last = i;
        i += 1;
      }
      if (pos_last > 0 && cutoff - pos_last >= keep) first = pos_last;
    }
  }
  float effective_temperature =
      dynamic_temperature(probs, first, cutoff, temperature, dynatemp_range, dynatemp_exponent);
  if (trace) *trace = CandTrace{sum_exp, cutoff, first, effective_temperature, 0.0f, 0.0f, first};
  if (effective_temperature <= 0.0f)
    return CandResult{candidate_idx[first], sample_rng, Row{1.0f}, Ids{candidate_idx[first]}};

  /* tempered renormalisation (:579-584) */
  float renorm_sum = 0.0f;
  for (int64_t i = first; i < cutoff; i++) {
    float d = candidate_values[i] - candidate_values[first];
    float q = d / effective_temperature;
    probs[i] = expf(q);
#if ORC_MUTANT != 4
    renorm_sum += probs[i];
#endif
  }
#if ORC_MUTANT == 4 /* planted mistake (tests only): the tempered sum as two halves added at the end */
  {
    float a = 0.0f, b = 0.0f;
    const int64_t mid = first + (cutoff - first) / 2;
    for (int64_t i = first; i < mid; i++) a += probs[i];
    for (int64_t i = mid; i < cutoff; i++) b += probs[i];
    renorm_sum = a + b;
  }
#endif
  /* draw (:586-598) */
  Rng new_rng = sample_rng;
  float r01 = rng_next_f32(new_rng);
  float target = r01 * renorm_sum;
  int64_t chosen_slot = cutoff - 1;
  float running = 0.0f;
  int64_t s = first;
  bool slot_found = false;
  while (s < cutoff && !slot_found) {
    running += probs[s];
    if (running >= target) {
      chosen_slot = s;
      slot_found = true;
    }
    s += 1;
  }
  if (trace) {
    trace->renorm_sum = renorm_sum;
    trace->target = target;
    trace->chosen = chosen_slot;
  }
  CandResult r{candidate_idx[chosen_slot], new_rng, Row{}, Ids{}};
  for (int64_t i = first; i < cutoff; i++) {
    r.probs.push_back(probs[i] / renorm_sum);
    r.ids.push_back(candidate_idx[i]);
  }
  return r;
}

/* :609-617 */
int32_t sample_candidates(Rng &rng, const Row &top_val, const Ids &top_idx, float temperature, float dynatemp_range,
                          float dynatemp_exponent, float typical_p, float top_p, float min_p, float xtc_probability,
                          float xtc_threshold, int64_t min_keep) {
  CandResult r = sample_candidates_with_probs(rng, top_val, top_idx, temperature, dynatemp_range, dynatemp_exponent,
                                              typical_p, top_p, min_p, xtc_probability, xtc_threshold, min_keep);
  rng = r.rng;
  return r.token;
}

/* :619-627 */
static void temperature_ranked(const Row &logits, int64_t vocab, float temperature, Row &scaled, Ids &ids) {
  Row values;
  all_candidates_sorted(logits, vocab, values, ids);
  float divisor = temperature > 0.0f ? temperature : 1.0f;
  scaled.assign(values.size(), 0.0f);
  for (size_t i = 0; i < values.size(); i++)
    scaled[i] = (temperature <= 0.0f && i > 0) ? -1.0e30f : values[i] / divisor;
}

/* :629-641 */
static Row softmax_prefix(const Row &values, int64_t count, float &total) {
  Row probs(count, 0.0f);
  total = 0.0f;
  for (int64_t i = 0; i < count; i++) {
    probs[i] = expf(values[i] - values[0]);
    total += probs[i];
  }
  for (int64_t i = 0; i < count; i++) probs[i] = probs[i] / total;
  return probs;
}

/* :643-659 */
static MirostatResult draw_mirostat_prefix(Rng rng, const Row &values, const Ids &ids, int64_t count, float tau,
                                           float eta, float mu) {
  float total;
  Row probs = softmax_prefix(values, count, total);
  float draw = rng_next_f32(rng);
  float cumulative = 0.0f;
  int64_t selected = count - 1;
  bool found = false;
  for (int64_t i = 0; i < count && !found; i++) {
    cumulative += probs[i];
    if (cumulative >= draw) {
      selected = i;
      found = true;
    }
  }
  float nl = -logf(probs[selected]);
  float surprise = nl / logf(2.0f);
  float d = surprise - tau;
  float t = eta * d;
  return MirostatResult{ids[selected], rng, mu - t};
}

/* :663-674 */
MirostatResult sample_mirostat_v2(Rng rng, const Row &logits, int64_t vocab, float temperature, float tau, float eta,
                                  float mu) {
  if (temperature <= 0.0f) return MirostatResult{sample_greedy(logits, vocab), rng, mu};
  Row values;
  Ids ids;
  temperature_ranked(logits, vocab, temperature, values, ids);
  float total;
  Row probs = softmax_prefix(values, vocab, total);
  int64_t cutoff = 0;
  while (cutoff < vocab && (-logf(probs[cutoff]) / logf(2.0f)) <= mu) cutoff += 1;
  if (cutoff == 0) cutoff = 1;
  return draw_mirostat_prefix(rng, values, ids, cutoff, tau, eta, mu);
}

/* :683-699: the Zipf exponent s_hat fitted to the first min(vocab, 100) ranked probabilities, and the
 * prefix length it predicts for the target surprise mu */
static int64_t mirostat_v1_cutoff(const Row &probs, int64_t vocab, float mu, float &s_hat_out) {
  int64_t m = vocab < 100 ? vocab : 100;
  float sum_ti_bi = 0.0f, sum_ti_sq = 0.0f;
#if ORC_MUTANT == 6 /* planted mistake (tests only): the fit's last pair dropped */
  m -= 1;
#endif
  for (int64_t i = 0; i < m - 1; i++) {
    float t_i = logf((float)(i + 2) / (float)(i + 1));
    float b_i = logf(probs[i] / probs[i + 1]);
    float a = t_i * b_i;
    sum_ti_bi += a;
    float b = t_i * t_i;
    sum_ti_sq += b;
  }
  float s_hat = sum_ti_bi / sum_ti_sq;
  float epsilon_hat = s_hat - 1.0f;
  float numerator = epsilon_hat * powf(2.0f, mu);
  float denominator = 1.0f - powf((float)vocab, -epsilon_hat);
  float est = powf(numerator / denominator, 1.0f / s_hat);
  /* Rust `as int`: truncation, saturating, NaN -> 0 */
  int64_t estimate = est != est ? 0 : (est >= 9.2e18f ? INT64_MAX : (est <= -9.2e18f ? INT64_MIN : (int64_t)est));
  int64_t cutoff = estimate > 1 ? estimate : 1;
  if (cutoff > vocab) cutoff = vocab;
  s_hat_out = s_hat;
  return cutoff;
}

/* :676-700 */
int64_t mirostat_v1_cutoff_of(const Row &logits, int64_t vocab, float temperature, float mu, float &s_hat) {
  Row values;
  Ids ids;
  temperature_ranked(logits, vocab, temperature, values, ids);
  float total;
  Row probs = softmax_prefix(values, vocab, total);
  return mirostat_v1_cutoff(probs, vocab, mu, s_hat);
}

MirostatResult sample_mirostat_v1(Rng rng, const Row &logits, int64_t vocab, float temperature, float tau, float eta,
                                  float mu) {
  if (temperature <= 0.0f) return MirostatResult{sample_greedy(logits, vocab), rng, mu};
  Row values;
  Ids ids;
  temperature_ranked(logits, vocab, temperature, values, ids);
  float total;
  Row probs = softmax_prefix(values, vocab, total);
  float s_hat;
  const int64_t cutoff = mirostat_v1_cutoff(probs, vocab, mu, s_hat);
  return draw_mirostat_prefix(rng, values, ids, cutoff, tau, eta, mu);
}

/* :705-740 */
AdaptiveResult sample_adaptive_p(Rng rng, const Row &logits, int64_t vocab, float target, float decay,
                                 float weighted_sum, float total_weight) {
  float maximum, log_sum_exp;
  logprob_normalizer(logits, vocab, maximum, log_sum_exp);
  Row original_probs(vocab, 0.0f), transformed(vocab, 0.0f);
  float average = total_weight == 0.0f ? target : weighted_sum / total_weight;
  float adapted_target = 2.0f * target - average;
  if (adapted_target < 0.0f) adapted_target = 0.0f;
  if (adapted_target > 1.0f) adapted_target = 1.0f;
  for (int64_t i = 0; i < vocab; i++) {
    float a = logits[i] - maximum;
    float probability = expf(a - log_sum_exp);
    original_probs[i] = probability;
    if (logits[i] <= -1.0e29f) {
      transformed[i] = logits[i];
    } else {
#if ORC_MUTANT == 8 /* planted mistake (tests only): the distance scaled by 0.25 */
      float distance = fabsf(probability - adapted_target) / 0.25f;
#else
      float distance = fabsf(probability - adapted_target) / 0.3f;
#endif
      float num = 10.0f * distance;
      num = num * distance;
      transformed[i] = 5.0f - num / (1.0f + distance);
    }
  }
  float tmax, tsum;
  logprob_normalizer(transformed, vocab, tmax, tsum);
  float draw = rng_next_f32(rng);
  float cumulative = 0.0f;
  int64_t selected = vocab - 1;
  bool found = false;
  for (int64_t i = 0; i < vocab && !found; i++) {
    float a = transformed[i] - tmax;
    cumulative += expf(a - tsum);
    if (cumulative >= draw) {
      selected = i;
      found = true;
    }
  }
  float ws = decay * weighted_sum;
  float tw = decay * total_weight;
  return AdaptiveResult{(int32_t)selected, rng, original_probs[selected] + ws, 1.0f + tw};
}

/* :778-779 */
Row sampling_logits(const Row &logits, const Ids &history, float repeat_penalty, int64_t repeat_last_n) {
  return apply_repeat_penalty(logits, history, repeat_penalty, repeat_last_n);
}

/* :742-760 */
SampleResult sample_with_probs(Rng rng, const Row &logits, int64_t vocab, const Params &p, const Ids &history) {
  Row repeated = sampling_logits(logits, history, p.repeat_penalty, p.repeat_last_n);
  Row penalized = apply_dry_penalty(repeated, history, p.dry_multiplier, p.dry_base, p.dry_allowed_length,
                                    p.dry_penalty_last_n, p.dry_breakers);
  if (p.temperature <= 0.0f) {
    int32_t token = sample_greedy(penalized, vocab);
    return SampleResult{token, rng, Row{1.0f}, Ids{token}};
  }
  Row sigma_filtered = top_n_sigma_logits(penalized, vocab, p.top_n_sigma);
  Row top_val;
  Ids top_idx;
  rank_candidates(sigma_filtered, vocab, p.top_k, top_val, top_idx);
  CandResult r = sample_candidates_with_probs(rng, top_val, top_idx, p.temperature, p.dynatemp_range,
                                              p.dynatemp_exponent, p.typical_p, p.top_p, p.min_p, p.xtc_probability,
                                              p.xtc_threshold, p.min_keep);
  return SampleResult{r.token, r.rng, r.probs, r.ids};
}

/* src/model.br:973-984: x*logit_mul (when != 1), then cap*tanh(x/cap) when cap > 0 */
Row finish_logits(const Row &logits, float logit_mul, float final_softcap) {
  Row x = logits;
  if (logit_mul != 1.0f)
    for (auto &v : x) v = v * logit_mul;
  if (final_softcap > 0.0f)
    for (auto &v : x) {
      float q = v / final_softcap;
      v = final_softcap * tanhf(q);
    }
  return x;
}

} /* namespace orc */
