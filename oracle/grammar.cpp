/*
 * grammar.cpp — restatement of the reference's src/grammar.br (GBNF parser + stack-machine matcher)
 * and src/io.br:64-147 (lossy UTF-8 decoding). TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * The matcher keeps the reference's data model: a state is the ordered list of stacks produced by
 * expand_stacks, stacks are deduplicated by their element-key sequence. Stacks are interned and the
 * pure function advance(state, cp) is memoised; neither changes any result.
 */
#include <set>
#include <stdexcept>
#include <string>

#include "oracle.h"

namespace orc {

/* ---------------- src/io.br:70-115 bytes_to_str ---------------- */
std::vector<uint32_t> bytes_to_cps(const uint8_t *b, size_t n) {
  std::vector<uint32_t> out;
  const uint32_t bad = 0xFFFD;
  size_t i = 0;
  while (i < n) {
    uint32_t b0 = b[i];
    if (b0 < 0x80) {
      out.push_back(b0);
      i += 1;
    } else if (b0 >= 0xC2 && b0 <= 0xDF) {
      if (i + 1 < n && (b[i + 1] & 0xC0) == 0x80) {
        out.push_back(((b0 & 0x1F) << 6) | (b[i + 1] & 0x3F));
        i += 2;
      } else {
        out.push_back(bad);
        i += 1;
      }
    } else if (b0 >= 0xE0 && b0 <= 0xEF) {
      if (i + 2 < n && (b[i + 1] & 0xC0) == 0x80 && (b[i + 2] & 0xC0) == 0x80) {
        uint32_t cp = ((b0 & 0x0F) << 12) | ((uint32_t)(b[i + 1] & 0x3F) << 6) | (b[i + 2] & 0x3F);
        if (cp < 0x800 || (cp >= 0xD800 && cp <= 0xDFFF)) {
          out.push_back(bad);
          i += 1;
        } else {
          out.push_back(cp);
          i += 3;
        }
      } else {
        out.push_back(bad);
        i += 1;
      }
    } else if (b0 >= 0xF0 && b0 <= 0xF4) {
      if (i + 3 < n && (b[i + 1] & 0xC0) == 0x80 && (b[i + 2] & 0xC0) == 0x80 && (b[i + 3] & 0xC0) == 0x80) {
        uint32_t cp = ((b0 & 0x07) << 18) | ((uint32_t)(b[i + 1] & 0x3F) << 12) | ((uint32_t)(b[i + 2] & 0x3F) << 6) |
                      (b[i + 3] & 0x3F);
        if (cp < 0x10000 || cp > 0x10FFFF) {
          out.push_back(bad);
          i += 1;
        } else {
          out.push_back(cp);
          i += 4;
        }
      } else {
        out.push_back(bad);
        i += 1;
      }
    } else {
      out.push_back(bad);
      i += 1;
    }
  }
  return out;
}

/* src/io.br:120-147 */
bool is_valid_utf8(const uint8_t *b, size_t n) {
  size_t i = 0;
  while (i < n) {
    uint32_t b0 = b[i];
    if (b0 < 0x80) {
      i += 1;
    } else if (b0 >= 0xC2 && b0 <= 0xDF) {
      if (i + 1 >= n || (b[i + 1] & 0xC0) != 0x80) return false;
      i += 2;
    } else if (b0 >= 0xE0 && b0 <= 0xEF) {
      if (i + 2 >= n || (b[i + 1] & 0xC0) != 0x80 || (b[i + 2] & 0xC0) != 0x80) return false;
      uint32_t b1 = b[i + 1];
      if ((b0 == 0xE0 && b1 < 0xA0) || (b0 == 0xED && b1 >= 0xA0)) return false;
      i += 3;
    } else if (b0 >= 0xF0 && b0 <= 0xF4) {
      if (i + 3 >= n || (b[i + 1] & 0xC0) != 0x80 || (b[i + 2] & 0xC0) != 0x80 || (b[i + 3] & 0xC0) != 0x80)
        return false;
      uint32_t b1 = b[i + 1];
      if ((b0 == 0xF0 && b1 < 0x90) || (b0 == 0xF4 && b1 >= 0x90)) return false;
      i += 4;
    } else {
      return false;
    }
  }
  return true;
}

std::string cps_to_utf8(const std::vector<uint32_t> &cps) {
  std::string s;
  for (uint32_t cp : cps) {
    if (cp < 0x80) s.push_back((char)cp);
    else if (cp < 0x800) {
      s.push_back((char)(0xC0 | (cp >> 6)));
      s.push_back((char)(0x80 | (cp & 0x3F)));
    } else if (cp < 0x10000) {
      s.push_back((char)(0xE0 | (cp >> 12)));
      s.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
      s.push_back((char)(0x80 | (cp & 0x3F)));
    } else {
      s.push_back((char)(0xF0 | (cp >> 18)));
      s.push_back((char)(0x80 | ((cp >> 12) & 0x3F)));
      s.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
      s.push_back((char)(0x80 | (cp & 0x3F)));
    }
  }
  return s;
}

/* ---------------- src/grammar.br parser (:45-323) ---------------- */
static const int GRAMMAR_MAX_DEPTH = 64;
static const int GRAMMAR_MAX_REPEAT = 2000;
static const int GRAMMAR_MAX_REPEAT_ELEMS = 200000;

namespace {
struct GParser {
  std::vector<uint32_t> src;
  int64_t pos = 0;
  std::map<std::string, int> names;
  std::vector<std::string> rule_names;
  std::vector<bool> defined;
  std::vector<std::vector<std::vector<GElem>>> rules;
  int depth = 0;
  int64_t elems = 0;
};
}  // namespace

static std::string chr_utf8(uint32_t c) { return cps_to_utf8(std::vector<uint32_t>{c}); }

/* :45-49 */
static GElem charset_elem(const std::vector<int64_t> &ranges, bool negated) {
  std::string key = negated ? "n" : "c";
  for (int64_t r : ranges) key += "," + std::to_string(r);
  return GElem{0, -1, ranges, negated, key};
}
/* :51-52 */
static GElem ref_elem(int rule) { return GElem{1, rule, {}, false, "r" + std::to_string(rule)}; }

/* :54-55 */
static bool is_name_char(uint32_t c) {
  return (c >= 48 && c <= 57) || (c >= 65 && c <= 90) || (c >= 97 && c <= 122) || c == 45 || c == 95;
}

/* :57-61 */
static int64_t hex_value(uint32_t c) {
  if (c >= 48 && c <= 57) return c - 48;
  if (c >= 97 && c <= 102) return c - 87;
  if (c >= 65 && c <= 70) return c - 55;
  throw std::runtime_error("grammar: invalid hex digit");
}

/* :63-73 */
static void skip_space(GParser &p, bool newline_ok) {
  bool going = true;
  while (going && p.pos < (int64_t)p.src.size()) {
    uint32_t c = p.src[p.pos];
    if (c == 32 || c == 9 || (newline_ok && (c == 10 || c == 13))) {
      p.pos += 1;
    } else if (c == 35) {
      while (p.pos < (int64_t)p.src.size() && p.src[p.pos] != 10 && p.src[p.pos] != 13) p.pos += 1;
    } else {
      going = false;
    }
  }
}

/* :75-100 */
static int64_t parse_char(GParser &p) {
  int64_t n = (int64_t)p.src.size();
  if (!(p.pos < n)) throw std::runtime_error("grammar: unexpected end of input");
  uint32_t c = p.src[p.pos];
  if (c != 92) {
    p.pos += 1;
    return c;
  }
  if (!(p.pos + 1 < n)) throw std::runtime_error("grammar: unexpected end of input after '\\'");
  uint32_t e = p.src[p.pos + 1];
  p.pos += 2;
  if (e == 116) return 9;
  if (e == 114) return 13;
  if (e == 110) return 10;
  if (e == 92 || e == 34 || e == 91 || e == 93) return e;
  int digits = 0;
  if (e == 120) digits = 2;
  else if (e == 117) digits = 4;
  else if (e == 85) digits = 8;
  else throw std::runtime_error("grammar: unknown escape \\" + chr_utf8(e));
  int64_t value = 0;
  for (int i = 0; i < digits; i++) {
    if (!(p.pos < n)) throw std::runtime_error("grammar: truncated escape");
    value = value * 16 + hex_value(p.src[p.pos]);
    p.pos += 1;
  }
  return value;
}

/* :102-108 */
static std::string parse_name(GParser &p) {
  std::string name;
  while (p.pos < (int64_t)p.src.size() && is_name_char(p.src[p.pos])) {
    name.push_back((char)p.src[p.pos]);
    p.pos += 1;
  }
  if (name.empty()) throw std::runtime_error("grammar: expected a rule name at offset " + std::to_string(p.pos));
  return name;
}

/* :110-118 */
static int rule_id(GParser &p, const std::string &name) {
  auto it = p.names.find(name);
  if (it != p.names.end()) return it->second;
  int id = (int)p.rules.size();
  p.names[name] = id;
  p.rule_names.push_back(name);
  p.defined.push_back(false);
  p.rules.push_back({});
  return id;
}

/* :120-125 */
static int anonymous_rule(GParser &p) {
  int id = (int)p.rules.size();
  p.rule_names.push_back("(anonymous " + std::to_string(id) + ")");
  p.defined.push_back(true);
  p.rules.push_back({});
  return id;
}

/* :129-163 */
static std::vector<GElem> repeat_symbol(GParser &p, const std::vector<GElem> &sym, int64_t min, int64_t max) {
  int64_t copies = max > min ? max : min;
  if (!(copies <= GRAMMAR_MAX_REPEAT))
    throw std::runtime_error("grammar: a repetition count above " + std::to_string(GRAMMAR_MAX_REPEAT) +
                             " is not supported");
  p.elems += copies * ((int64_t)sym.size() + 1);
  if (!(p.elems <= GRAMMAR_MAX_REPEAT_ELEMS))
    throw std::runtime_error("grammar: repetitions expand to more than " + std::to_string(GRAMMAR_MAX_REPEAT_ELEMS) +
                             " elements");
  std::vector<GElem> out;
  for (int64_t i = 0; i < min; i++)
    for (const GElem &e : sym) out.push_back(e);
  if (max < 0) {
    int r = anonymous_rule(p);
    std::vector<GElem> looped = sym;
    looped.push_back(ref_elem(r));
    p.rules[r] = {looped, {}};
    out.push_back(ref_elem(r));
  } else if (max > min) {
    std::vector<GElem> inner;
    for (int64_t k = 0; k < max - min; k++) {
      int r = anonymous_rule(p);
      std::vector<GElem> step = sym;
      for (const GElem &e : inner) step.push_back(e);
      p.rules[r] = {step, {}};
      inner = {ref_elem(r)};
    }
    for (const GElem &e : inner) out.push_back(e);
  }
  return out;
}

/* :165-174 */
static int64_t parse_int(GParser &p) {
  int64_t value = 0;
  int digits = 0;
  while (p.pos < (int64_t)p.src.size() && p.src[p.pos] >= 48 && p.src[p.pos] <= 57) {
    value = value * 10 + (p.src[p.pos] - 48);
    p.pos += 1;
    digits += 1;
    if (!(digits <= 9))
      throw std::runtime_error("grammar: a repetition count above " + std::to_string(GRAMMAR_MAX_REPEAT) +
                               " is not supported");
  }
  if (!(digits > 0))
    throw std::runtime_error("grammar: expected a number in a repetition at offset " + std::to_string(p.pos));
  return value;
}

static void parse_alternates(GParser &p, int id, bool nested);

/* :176-281 */
static std::vector<GElem> parse_sequence(GParser &p, bool nested) {
  std::vector<GElem> out;
  size_t last_start = 0;
  bool going = true;
  int64_t n = (int64_t)p.src.size();
  while (going && p.pos < n) {
    uint32_t c = p.src[p.pos];
    if (c == 34) {
      p.pos += 1;
      last_start = out.size();
      while (p.pos < n && p.src[p.pos] != 34) {
        int64_t cp = parse_char(p);
        out.push_back(charset_elem({cp, cp}, false));
      }
      if (!(p.pos < n)) throw std::runtime_error("grammar: unterminated string literal");
      p.pos += 1;
      skip_space(p, nested);
    } else if (c == 91) {
      p.pos += 1;
      bool negated = false;
      if (p.pos < n && p.src[p.pos] == 94) {
        negated = true;
        p.pos += 1;
      }
      last_start = out.size();
      std::vector<int64_t> ranges;
      while (p.pos < n && p.src[p.pos] != 93) {
        int64_t lo = parse_char(p);
        int64_t hi = lo;
        if (p.pos + 1 < n && p.src[p.pos] == 45 && p.src[p.pos + 1] != 93) {
          p.pos += 1;
          hi = parse_char(p);
        }
        ranges.push_back(lo);
        ranges.push_back(hi);
      }
      if (!(p.pos < n)) throw std::runtime_error("grammar: unterminated character class");
      p.pos += 1;
      out.push_back(charset_elem(ranges, negated));
      skip_space(p, nested);
    } else if (is_name_char(c)) {
      std::string name = parse_name(p);
      skip_space(p, nested);
      last_start = out.size();
      out.push_back(ref_elem(rule_id(p, name)));
    } else if (c == 40) {
      p.pos += 1;
      skip_space(p, true);
      int sub = anonymous_rule(p);
      if (!(p.depth < GRAMMAR_MAX_DEPTH))
        throw std::runtime_error("grammar: groups are nested deeper than " + std::to_string(GRAMMAR_MAX_DEPTH) +
                                 " levels");
      p.depth += 1;
      parse_alternates(p, sub, true);
      p.depth -= 1;
      if (!(p.pos < n && p.src[p.pos] == 41))
        throw std::runtime_error("grammar: expected ')' at offset " + std::to_string(p.pos));
      p.pos += 1;
      skip_space(p, nested);
      last_start = out.size();
      out.push_back(ref_elem(sub));
    } else if (c == 46) {
      p.pos += 1;
      skip_space(p, nested);
      last_start = out.size();
      out.push_back(charset_elem({}, true));
    } else if (c == 42 || c == 43 || c == 63 || c == 123) {
      if (!(out.size() > last_start))
        throw std::runtime_error("grammar: a repetition needs something to repeat (offset " + std::to_string(p.pos) +
                                 ")");
      std::vector<GElem> sym(out.begin() + last_start, out.end());
      std::vector<GElem> before(out.begin(), out.begin() + last_start);
      int64_t min = 0, max = -1;
      if (c == 42) {
        p.pos += 1;
      } else if (c == 43) {
        min = 1;
        p.pos += 1;
      } else if (c == 63) {
        max = 1;
        p.pos += 1;
      } else {
        p.pos += 1;
        skip_space(p, false);
        min = parse_int(p);
        skip_space(p, false);
        max = min;
        if (p.pos < n && p.src[p.pos] == 44) {
          p.pos += 1;
          skip_space(p, false);
          if (p.pos < n && p.src[p.pos] >= 48 && p.src[p.pos] <= 57) {
            max = parse_int(p);
            skip_space(p, false);
          } else {
            max = -1;
          }
        }
        if (!(p.pos < n && p.src[p.pos] == 125))
          throw std::runtime_error("grammar: expected '}' at offset " + std::to_string(p.pos));
        p.pos += 1;
      }
      if (!(max < 0 || max >= min)) throw std::runtime_error("grammar: repetition maximum is smaller than its minimum");
      std::vector<GElem> rep = repeat_symbol(p, sym, min, max);
      out = before;
      last_start = out.size();
      for (const GElem &e : rep) out.push_back(e);
      skip_space(p, nested);
    } else {
      going = false;
    }
  }
  return out;
}

/* :283-290 */
static void parse_alternates(GParser &p, int id, bool nested) {
  std::vector<std::vector<GElem>> alts;
  alts.push_back(parse_sequence(p, nested));
  while (p.pos < (int64_t)p.src.size() && p.src[p.pos] == 124) {
    p.pos += 1;
    skip_space(p, true);
    alts.push_back(parse_sequence(p, nested));
  }
  p.rules[id] = alts;
}

/* :292-306 */
static void parse_rule(GParser &p) {
  std::string name = parse_name(p);
  skip_space(p, false);
  int64_t n = (int64_t)p.src.size();
  if (!(p.pos + 2 < n && p.src[p.pos] == 58 && p.src[p.pos + 1] == 58 && p.src[p.pos + 2] == 61))
    throw std::runtime_error("grammar: expected '::=' after rule name '" + name + "' at offset " +
                             std::to_string(p.pos));
  p.pos += 3;
  skip_space(p, true);
  int id = rule_id(p, name);
  if (p.defined[id]) throw std::runtime_error("grammar: rule '" + name + "' is defined twice");
  p.defined[id] = true;
  parse_alternates(p, id, false);
  if (p.pos < n && !(p.src[p.pos] == 10 || p.src[p.pos] == 13)) {
    int64_t at = p.pos;
    throw std::runtime_error("grammar: unexpected '" + chr_utf8(p.src[at]) + "' at offset " + std::to_string(at) +
                             " in rule '" + name + "'");
  }
  while (p.pos < n && (p.src[p.pos] == 10 || p.src[p.pos] == 13)) p.pos += 1;
}

/* :309-323 */
Grammar parse_gbnf(const std::string &text) {
  GParser p;
  p.src = bytes_to_cps((const uint8_t *)text.data(), text.size());
  skip_space(p, true);
  while (p.pos < (int64_t)p.src.size()) {
    parse_rule(p);
    skip_space(p, true);
  }
  for (size_t i = 0; i < p.rules.size(); i++)
    if (!p.defined[i]) throw std::runtime_error("grammar: undefined rule '" + p.rule_names[i] + "'");
  auto it = p.names.find("root");
  if (it == p.names.end()) throw std::runtime_error("grammar: there is no `root` rule");
  Grammar g;
  g.rules = p.rules;
  g.root = it->second;
  return g;
}

/* ---------------- matcher (:327-451) ---------------- */
Matcher::Matcher(const Grammar &g) : g_(g) {}

int Matcher::intern_elem(const GElem &e) {
  auto it = elem_ids_.find(e.key);
  if (it != elem_ids_.end()) return it->second;
  int id = (int)elems_.size();
  elems_.push_back(e);
  elem_ids_[e.key] = id;
  return id;
}

int Matcher::intern_stack(const std::vector<int> &st) {
  auto it = stack_ids_.find(st);
  if (it != stack_ids_.end()) return it->second;
  int id = (int)stacks_.size();
  stacks_.push_back(st);
  stack_ids_[st] = id;
  return id;
}

/* :343-376 expand_stacks; stack identity = element-key sequence (stack_key :327-331) */
State Matcher::expand(const std::vector<std::vector<int>> &stacks) {
  std::vector<std::vector<int>> work;
  std::set<std::vector<int>> queued;
  for (const auto &st : stacks)
    if (!queued.count(st)) {
      queued.insert(st);
      work.push_back(st);
    }
  State out;
  size_t i = 0;
  while (i < work.size()) {
    if (!(work.size() < 20000)) throw std::runtime_error("grammar is left-recursive or too ambiguous to match");
    std::vector<int> st = work[i];
    i += 1;
    if (st.empty() || elems_[st.back()].kind == 0) {
      out.push_back(intern_stack(st));
    } else {
      const GElem &top = elems_[st.back()];
      std::vector<int> base(st.begin(), st.end() - 1);
      for (const auto &alt : g_.rules[top.rule]) {
        std::vector<int> next = base;
        for (auto it = alt.rbegin(); it != alt.rend(); ++it) next.push_back(intern_elem(*it));
        if (!queued.count(next)) {
          queued.insert(next);
          work.push_back(next);
        }
      }
    }
  }
  return out;
}

/* :378-382 */
State Matcher::start() {
  std::vector<std::vector<int>> stacks;
  for (const auto &alt : g_.rules[g_.root]) {
    std::vector<int> st;
    for (auto it = alt.rbegin(); it != alt.rend(); ++it) st.push_back(intern_elem(*it));
    stacks.push_back(st);
  }
  return expand(stacks);
}

/* :384-391 */
static bool elem_matches(const GElem &e, uint32_t cp) {
  bool inside = false;
  for (size_t i = 0; i + 1 < e.ranges.size(); i += 2)
    if ((int64_t)cp >= e.ranges[i] && (int64_t)cp <= e.ranges[i + 1]) inside = true;
  return inside != e.negated;
}

/* :394-404 */
State Matcher::advance(const State &s, uint32_t cp) {
  auto key = std::make_pair(s, cp);
  auto it = memo_.find(key);
  if (it != memo_.end()) return it->second;
  std::vector<std::vector<int>> next;
  for (int sid : s) {
    const std::vector<int> &st = stacks_[sid];
    if (!st.empty() && elem_matches(elems_[st.back()], cp)) next.push_back(std::vector<int>(st.begin(), st.end() - 1));
  }
  State r = expand(next);
  memo_[key] = r;
  return r;
}

/* :408-420 */
bool Matcher::allows_non_ascii(const State &s) {
  for (int sid : s) {
    const std::vector<int> &st = stacks_[sid];
    if (!st.empty()) {
      const GElem &top = elems_[st.back()];
      if (top.kind == 0) {
        if (top.negated) return true;
        for (size_t i = 1; i < top.ranges.size(); i += 2)
          if (top.ranges[i] >= 128) return true;
      }
    }
  }
  return false;
}

/* :425-437 */
State Matcher::advance_text(const State &s, const std::vector<uint32_t> &chars) {
  State state = s;
  size_t i = 0;
  while (i < chars.size() && !state.empty()) {
    uint32_t cp = chars[i];
    if (cp == 0xFFFD && i == chars.size() - 1) {
      if (!allows_non_ascii(state)) state.clear();
    } else {
      state = advance(state, cp);
    }
    i += 1;
  }
  return state;
}

/* :440-451 */
bool Matcher::complete(const State &s) {
  for (int sid : s)
    if (stacks_[sid].empty()) return true;
  return false;
}

bool Matcher::can_continue(const State &s) {
  for (int sid : s)
    if (!stacks_[sid].empty()) return true;
  return false;
}

} /* namespace orc */
