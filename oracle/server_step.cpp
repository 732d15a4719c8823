/*
 * server_step.cpp — restatement of the per-token block of the reference's decode loop
 * (src/server.br:939-1036), its grammar-constrained sampler (src/server.br:309-362), speculative
 * verification (src/server.br:1173-1216) and src/speculative.br. TEST INFRASTRUCTURE ONLY.
 */
#include <stdexcept>

#include "oracle.h"

namespace orc {

/* src/speculative.br:11-34 */
Ids ngram_draft(const Ids &tokens, int64_t max_draft, int64_t ngram_max, int64_t ngram_min) {
  int64_t n = (int64_t)tokens.size();
  int64_t size = ngram_max;
  while (size >= ngram_min && size >= 1) {
    if (n > size) {
      int64_t start = n - size - 1;
      while (start >= 0) {
        bool same = true;
        int64_t j = 0;
        while (same && j < size) {
          if (tokens[start + j] != tokens[n - size + j]) same = false;
          j += 1;
        }
        if (same) {
          Ids draft;
          int64_t k = start + size;
          while (k < n && (int64_t)draft.size() < max_draft) {
            draft.push_back(tokens[k]);
            k += 1;
          }
          if (!draft.empty()) return draft;
        }
        start -= 1;
      }
    }
    size -= 1;
  }
  return Ids{};
}

/* src/tokenizer.br:122-151, :227-240 for a byte vocabulary: ids -> concatenated piece bytes -> bytes_to_str */
static std::vector<uint32_t> decode_ids(const Vocab &v, const Ids &ids, const int32_t *extra) {
  std::vector<uint8_t> bytes;
  auto put = [&](int32_t id) {
    if (id < 0 || id >= v.n()) return;
    bytes.insert(bytes.end(), v.blob.begin() + v.offsets[id], v.blob.begin() + v.offsets[id + 1]);
  };
  for (int32_t id : ids) put(id);
  if (extra) put(*extra);
  return bytes_to_cps(bytes.data(), bytes.size());
}

static std::vector<uint8_t> reply_bytes(const Vocab &v, const Ids &ids) {
  std::vector<uint8_t> bytes;
  for (int32_t id : ids)
    if (id >= 0 && id < v.n()) bytes.insert(bytes.end(), v.blob.begin() + v.offsets[id], v.blob.begin() + v.offsets[id + 1]);
  return bytes;
}

static int utf8_need(uint8_t b) { return b >= 0xF0 ? 4 : (b >= 0xE0 ? 3 : 2); }

/*
 * Carry form of the candidate piece (equivalent to src/server.br:342-351). bytes_to_str decodes left
 * to right and only a truncated trailing sequence can decode differently once bytes are appended,
 * so decode(R ++ T) = decode(R[..p]) ++ decode(R[p..] ++ T) at the last lead byte p (C2..F4) whose
 * following bytes are all continuation bytes but fewer than it needs. Then
 * piece(T) = decode(carry ++ T)[skip..] with carry = R[p..], skip = |carry|-1; without such p,
 * carry is the last byte when decode(R) ends in U+FFFD (skip 0), else empty.
 */
static void reply_carry(const std::vector<uint8_t> &R, const std::vector<uint32_t> &D, std::vector<uint8_t> &carry,
                        size_t &skip) {
  carry.clear();
  skip = 0;
  int64_t n = (int64_t)R.size();
  for (int64_t p = n - 1; p >= 0 && p >= n - 4; p--) {
    uint8_t b = R[p];
    if ((b & 0xC0) == 0x80) continue; /* continuation byte: keep looking left */
    if (b >= 0xC2 && b <= 0xF4 && n - p < utf8_need(b)) {
      carry.assign(R.begin() + p, R.end());
      skip = carry.size() - 1;
      return;
    }
    break;
  }
  if (!D.empty() && D.back() == 0xFFFD) carry.assign(1, R.back());
}

struct GrammarCtx {
  std::vector<uint32_t> before_chars;
  State state;
  bool complete;
  std::vector<uint8_t> carry;
  size_t skip;
  std::vector<uint8_t> R;
};

/* src/server.br:312-320 */
static GrammarCtx grammar_ctx(Slot &slot, const Vocab &v) {
  GrammarCtx c;
  c.R = reply_bytes(v, slot.reply);
  std::vector<uint32_t> D = bytes_to_cps(c.R.data(), c.R.size());
  c.before_chars = D;
  if (!c.before_chars.empty() && c.before_chars.back() == 0xFFFD) c.before_chars.pop_back();
  c.state = slot.matcher->advance_text(slot.matcher->start(), c.before_chars);
  if (c.state.empty()) throw std::runtime_error("the reply no longer matches the grammar");
  c.complete = slot.matcher->complete(c.state);
  reply_carry(c.R, D, c.carry, c.skip);
  return c;
}

/* allowed predicate of src/server.br:339-352 for one candidate */
static bool grammar_allowed(Slot &slot, const Vocab &v, const GrammarCtx &c, int32_t cand, int32_t eos_id, bool fast) {
  if (is_eog_token(cand, eos_id)) return c.complete && !slot.params.ignore_eos;
  std::vector<uint32_t> piece;
  if (fast) {
    std::vector<uint8_t> b = c.carry;
    if (cand >= 0 && cand < v.n()) b.insert(b.end(), v.blob.begin() + v.offsets[cand], v.blob.begin() + v.offsets[cand + 1]);
    std::vector<uint32_t> d = bytes_to_cps(b.data(), b.size());
    if (d.size() > c.skip) piece.assign(d.begin() + c.skip, d.end());
  } else {
    std::vector<uint32_t> after = decode_ids(v, slot.reply, &cand);
    for (size_t i = c.before_chars.size(); i < after.size(); i++) piece.push_back(after[i]);
  }
  return !slot.matcher->advance_text(c.state, piece).empty();
}

bool grammar_mask(Slot &slot, const Vocab &v, int64_t V, std::vector<uint32_t> &mask, bool &forced_eos, bool fast) {
  mask.assign((V + 31) / 32, 0u);
  GrammarCtx c;
  try {
    c = grammar_ctx(slot, v);
  } catch (const std::runtime_error &) {
    return false;
  }
  forced_eos = c.complete && !slot.matcher->can_continue(c.state) && !slot.params.ignore_eos;
  for (int64_t t = 0; t < V; t++)
    if (grammar_allowed(slot, v, c, (int32_t)t, v.eos_id, fast)) mask[t >> 5] |= 1u << (t & 31);
  return true;
}

/* src/server.br:309-362 */
static int32_t sample_grammar_token(Slot &slot, const Vocab &v, const Row &logits, int64_t vocab, bool fast) {
  const Params &p = slot.params;
  GrammarCtx c = grammar_ctx(slot, v);
  if (c.complete && !slot.matcher->can_continue(c.state) && !p.ignore_eos) return v.eos_id;
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
    for (size_t i = 0; i < ranked_ids.size(); i++) {
      int32_t cand = ranked_ids[i];
      if (grammar_allowed(slot, v, c, cand, v.eos_id, fast)) {
        allowed_values.push_back(ranked_values[i]);
        allowed_ids.push_back(cand);
      }
    }
    if (!allowed_ids.empty())
      return sample_candidates(slot.rng, allowed_values, allowed_ids, p.temperature, p.dynatemp_range,
                               p.dynatemp_exponent, p.typical_p, p.top_p, p.min_p, p.xtc_probability, p.xtc_threshold,
                               p.min_keep);
    if (!(k < vocab)) throw std::runtime_error("the grammar rejected every vocabulary token");
    k = k * 4 < vocab ? k * 4 : vocab;
  }
}

/* src/server.br:940-1037 */
StepOut decode_step(Slot &slot, const float *logits, int64_t V, const Vocab *vocab, bool wants_logprobs,
                    bool fast_grammar) {
  const Params &p = slot.params;
  int32_t eos_id = vocab ? vocab->eos_id : -1;
  /* model tail (src/model.br:973-984) produces the logits the server receives */
  Row raw = finish_logits(Row(logits, logits + V), p.logit_mul, p.final_softcap);
  Row request_biased = apply_logit_bias(raw, slot.bias);
  Row biased = p.ignore_eos ? suppress_eog_tokens(request_biased, eos_id) : request_biased;
  Row penalized = apply_presence_frequency_penalty(biased, slot.reply, p.frequency_penalty, p.presence_penalty);
  Row effective;
  if (wants_logprobs) {
    Row repeated = sampling_logits(penalized, slot.tokens, p.repeat_penalty, p.repeat_last_n);
    effective = apply_dry_penalty(repeated, slot.tokens, p.dry_multiplier, p.dry_base, p.dry_allowed_length,
                                  p.dry_penalty_last_n, p.dry_breakers);
  }
  StepOut out;
  Row sampled_probs;
  Ids sampled_ids;
  if (slot.grammar) {
    if (!vocab) throw std::runtime_error("grammar sampling needs a vocabulary");
    out.token = sample_grammar_token(slot, *vocab, penalized, V, fast_grammar);
  } else if (slot.json_object) {
    if (!vocab) throw std::runtime_error("JSON-object sampling needs a vocabulary");
    out.token = sample_json_token(slot, *vocab, penalized, V);
  } else {
    SampleResult r = sample_with_probs(slot.rng, penalized, V, p, slot.tokens);
    slot.rng = r.rng;
    out.token = r.token;
    sampled_probs = r.probs;
    sampled_ids = r.ids;
  }
  slot.tokens.push_back(out.token);
  if (is_eog_token(out.token, eos_id)) {
    out.eog = true;
    return out;
  }
  if (wants_logprobs) {
    if (p.post_sampling_probs) {
      float selected = 0.0f;
      for (size_t i = 0; i < sampled_ids.size(); i++) {
        if (sampled_ids[i] == out.token) selected = sampled_probs[i];
        if ((int64_t)i < p.n_probs) {
          out.top_ids.push_back(sampled_ids[i]);
          out.top_logprobs.push_back(sampled_probs[i]);
        }
      }
      out.logprob = selected;
    } else {
      float mx, lse;
      logprob_normalizer(effective, V, mx, lse);
      out.logprob = normalized_token_logprob(effective, out.token, mx, lse);
      if (p.n_probs > 0) {
        Row tv;
        Ids ti;
        top_k_select(effective, V, p.n_probs, tv, ti);
        for (size_t i = 0; i < ti.size(); i++) {
          out.top_ids.push_back(ti[i]);
          out.top_logprobs.push_back(normalized_token_logprob(effective, ti[i], mx, lse));
        }
      }
    }
  }
  slot.reply.push_back(out.token);
  return out;
}

/* src/server.br:1173-1216: rows are sampled in order; a row's token is compared with its draft */
SpecOut spec_verify(Slot &slot, const float *rows, int64_t V, const Ids &drafts) {
  int k = (int)drafts.size();
  SpecOut out;
  out.tokens.assign(k + 1, -1);
  out.accepted = -1;
  Rng rng = slot.rng;
  Ids base_tokens = slot.tokens, base_reply = slot.reply;
  for (int i = 0; i <= k; i++) {
    Slot s;
    s.tokens = base_tokens;
    s.reply = base_reply;
    for (int j = 0; j < i; j++) {
      s.tokens.push_back(drafts[j]);
      s.reply.push_back(drafts[j]);
    }
    s.bias = slot.bias;
    s.params = slot.params;
    s.rng = rng;
    StepOut st = decode_step(s, rows + (int64_t)i * V, V, nullptr, false, true);
    rng = s.rng;
    out.tokens[i] = st.token;
    if (out.accepted < 0 && (i == k || st.token != drafts[i] || st.eog)) {
      out.accepted = i;
      slot.tokens = s.tokens;
      slot.reply = s.reply;
      slot.rng = s.rng;
    }
  }
  return out;
}

} /* namespace orc */
