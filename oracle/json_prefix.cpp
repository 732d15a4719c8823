/*
 * json_prefix.cpp — restatement of the reference's incremental JSON classifier (src/json.br:227-426) and
 * of sample_json_token, the sampler of `response_format: {type: json_object}` (src/server.br:261-304).
 * TEST INFRASTRUCTURE ONLY: the checker of the device's JSON-object path.
 *
 * Pinned by the reference's own known answers (test/test_json.br:67-99, transliterated in
 * tests/test_oracle_json.py) and by a brute-force property there: every prefix of a document that
 * Python's json module accepts as an object is viable, and the document itself complete.
 */
#include <stdexcept>

#include "oracle.h"

namespace orc {

static bool jws(uint32_t c) { return c == ' ' || c == '\n' || c == '\t' || c == '\r'; }
static bool jhex(uint32_t c) { return (c >= '0' && c <= '9') || (c >= 'a' && c <= 'f') || (c >= 'A' && c <= 'F'); }

/* a string body from position p (after its opening quote): 1 closed (p past the quote), 0 text ended,
 * -1 invalid (:271-301) */
static int scan_string(const std::vector<uint32_t> &cs, size_t &p) {
  while (p < cs.size()) {
    const uint32_t c = cs[p];
    if (c == '"') {
      p += 1;
      return 1;
    }
    if (c == '\\') {
      p += 1;
      if (p >= cs.size()) return 0;
      const uint32_t e = cs[p];
      if (e == 'u') {
        for (int h = 0; h < 4; h++) {
          p += 1;
          if (p >= cs.size()) return 0;
          if (!jhex(cs[p])) return -1;
        }
        p += 1;
      } else if (e == '"' || e == '\\' || e == '/' || e == 'b' || e == 'f' || e == 'n' || e == 'r' || e == 't') {
        p += 1;
      } else {
        return -1;
      }
    } else if (c < 0x20) {
      return -1;
    } else {
      p += 1;
    }
  }
  return 0;
}

/* :227-392. 0 root value, 1 object key/end, 2 colon, 3 object value, 4 object comma/end, 5 array
 * value/end, 6 array comma/end, 7 root done */
int json_prefix_state(const std::vector<uint32_t> &cs) {
  std::vector<int> states{0};
  size_t p = 0;
  while (p < cs.size()) {
    const int state = states.back();
    const uint32_t ch = cs[p];
    if (jws(ch)) {
      p += 1;
    } else if (state == 7) {
      return -1;
    } else if (state == 2) {
      if (ch != ':') return -1;
      states.back() = 3;
      p += 1;
    } else if (state == 4) {
      if (ch == ',') {
        states.back() = 1;
        p += 1;
      } else if (ch == '}') {
        states.pop_back();
        p += 1;
      } else {
        return -1;
      }
    } else if (state == 6) {
      if (ch == ',') {
        states.back() = 5;
        p += 1;
      } else if (ch == ']') {
        states.pop_back();
        p += 1;
      } else {
        return -1;
      }
    } else if (state == 1) {
      if (ch == '}') {
        states.pop_back();
        p += 1;
      } else if (ch != '"') {
        return -1;
      } else {
        p += 1;
        const int r = scan_string(cs, p);
        if (r <= 0) return r;
        states.back() = 2;
      }
    } else {
      if (state != 0 && state != 3 && state != 5) return -1;
      if (ch == ']' && state == 5) {
        states.pop_back();
        p += 1;
      } else {
        states.back() = state == 0 ? 7 : (state == 3 ? 4 : 6);
        if (ch == '{') {
          states.push_back(1);
          p += 1;
        } else if (ch == '[') {
          states.push_back(5);
          p += 1;
        } else if (ch == '"') {
          p += 1;
          const int r = scan_string(cs, p);
          if (r <= 0) return r;
        } else if (ch == 't' || ch == 'f' || ch == 'n') {
          const char *word = ch == 't' ? "true" : (ch == 'f' ? "false" : "null");
          size_t i = 0;
          for (; word[i]; i++) {
            if (p + i >= cs.size()) return 0;
            if (cs[p + i] != (uint32_t)(unsigned char)word[i]) return -1;
          }
          p += i;
        } else {
          size_t q = p;
          auto digit = [&](size_t k) { return cs[k] >= '0' && cs[k] <= '9'; };
          if (cs[q] == '-') {
            q += 1;
            if (q >= cs.size()) return 0;
          }
#if ORC_MUTANT == 7 /* planted mistake (tests only): a leading zero may be followed by digits */
          if (cs[q] >= '0' && cs[q] <= '9') {
#else
          if (cs[q] == '0') {
            q += 1;
          } else if (cs[q] >= '1' && cs[q] <= '9') {
#endif
            q += 1;
            while (q < cs.size() && digit(q)) q += 1;
          } else {
            return -1;
          }
          if (q < cs.size() && cs[q] == '.') {
            q += 1;
            if (q >= cs.size()) return 0;
            if (!digit(q)) return -1;
            while (q < cs.size() && digit(q)) q += 1;
          }
          if (q < cs.size() && (cs[q] == 'e' || cs[q] == 'E')) {
            q += 1;
            if (q >= cs.size()) return 0;
            if (cs[q] == '+' || cs[q] == '-') {
              q += 1;
              if (q >= cs.size()) return 0;
            }
            if (!digit(q)) return -1;
            while (q < cs.size() && digit(q)) q += 1;
          }
          p = q;
        }
      }
    }
    if (states.empty()) states.push_back(7); /* a closed top-level container is a complete root value */
  }
  return states.size() == 1 && states[0] == 7 ? 1 : 0;
}

/* :394-406: only an object at the root, after optional whitespace */
int json_object_prefix_state(const std::vector<uint32_t> &cs) {
  size_t p = 0;
  while (p < cs.size() && jws(cs[p])) p += 1;
  if (p == cs.size()) return 0;
  if (cs[p] != '{') return -1;
  return json_prefix_state(cs);
}

static std::vector<uint32_t> decode_reply(const Vocab &v, const Ids &ids, const int32_t *extra) {
  std::vector<uint8_t> bytes;
  auto put = [&](int32_t id) {
    if (id < 0 || id >= v.n()) return;
    bytes.insert(bytes.end(), v.blob.begin() + v.offsets[id], v.blob.begin() + v.offsets[id + 1]);
  };
  for (int32_t id : ids) put(id);
  if (extra) put(*extra);
  return bytes_to_cps(bytes.data(), bytes.size());
}

/* json_object_decoded_candidate_allowed (:420-426) for candidate `cand` after the reply */
static bool json_allowed(const Slot &slot, const Vocab &v, int before_state, int32_t cand) {
  if (is_eog_token(cand, v.eos_id)) return !slot.params.ignore_eos && before_state == 1;
  return json_object_prefix_state(decode_reply(v, slot.reply, &cand)) >= 0;
}

bool json_object_mask(const Slot &slot, const Vocab &v, int64_t V, std::vector<uint32_t> &mask, bool &forced_eos) {
  mask.assign((V + 31) / 32, 0u);
  const int before = json_object_prefix_state(decode_reply(v, slot.reply, nullptr));
  forced_eos = before == 1 && !slot.params.ignore_eos;
  for (int64_t t = 0; t < V; t++)
    if (json_allowed(slot, v, before, (int32_t)t)) mask[t >> 5] |= 1u << (t & 31);
  return true;
}

/* src/server.br:261-304 (no schema: the schema form is compiled to a grammar, :733-745) */
int32_t sample_json_token(Slot &slot, const Vocab &v, const Row &logits, int64_t vocab) {
  const Params &p = slot.params;
  const int before = json_object_prefix_state(decode_reply(v, slot.reply, nullptr));
  if (before == 1 && !p.ignore_eos) return v.eos_id;
  Row repeated = apply_repeat_penalty(logits, slot.tokens, p.repeat_penalty, p.repeat_last_n);
  Row penalized = apply_dry_penalty(repeated, slot.tokens, p.dry_multiplier, p.dry_base, p.dry_allowed_length,
                                    p.dry_penalty_last_n, p.dry_breakers);
  int64_t k = p.top_k > 0 ? p.top_k : vocab;
  if (k > vocab) k = vocab;
  while (true) {
    Row sigma_filtered = top_n_sigma_logits(penalized, vocab, p.top_n_sigma);
    Row ranked_values;
    Ids ranked_ids;
    rank_candidates(sigma_filtered, vocab, k, ranked_values, ranked_ids);
    Row allowed_values;
    Ids allowed_ids;
    for (size_t i = 0; i < ranked_ids.size(); i++)
      if (json_allowed(slot, v, before, ranked_ids[i])) {
        allowed_values.push_back(ranked_values[i]);
        allowed_ids.push_back(ranked_ids[i]);
      }
    if (!allowed_ids.empty())
      return sample_candidates(slot.rng, allowed_values, allowed_ids, p.temperature, p.dynatemp_range,
                               p.dynatemp_exponent, p.typical_p, p.top_p, p.min_p, p.xtc_probability, p.xtc_threshold,
                               p.min_keep);
    if (!(k < vocab)) throw std::runtime_error("JSON response grammar rejected every vocabulary token");
    k = k * 4 < vocab ? k * 4 : vocab;
  }
}

} /* namespace orc */
