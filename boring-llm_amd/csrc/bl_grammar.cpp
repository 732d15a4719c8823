/*
 * bl_grammar.cpp — GBNF text -> stack-set automaton tables (host side of the grammar mask path).
 *
 * Three stages:
 *   1. GbnfReader: the reference's GBNF syntax (src/grammar.br:45-323) into a rule table. Rules are
 *      alternatives of symbol sequences; a symbol is a character set (interned by its ranges and
 *      negation, so equal sets share an id) or a rule reference. Repetitions expand the way the
 *      reference expands them (copies, then a right-nested chain of anonymous rules), because the
 *      20,000-stack guard counts the stacks that structure produces.
 *   2. Frontiers: a stack is a symbol sequence (top last); a frontier is the set of stacks reached by
 *      expanding rule references on top until every top is a character set or the stack is empty
 *      (expand_stacks :343-376). Stacks and frontiers are interned.
 *   3. The automaton: breadth-first from the root frontier, one transition per code-point class;
 *      a class is a maximal set of code points that every character set of the grammar treats alike.
 */
#include "bl_grammar.h"

#include <algorithm>
#include <map>
#include <stdexcept>
#include <unordered_map>

#include "../../include/bl_select.h"

namespace {

const int kMaxDepth = 64;          /* src/grammar.br:39 */
const int64_t kMaxRepeat = 2000;   /* :40 */
const int64_t kMaxRepElems = 200000; /* :41 */
const size_t kStackGuard = 20000;  /* :354 */

struct GrammarError : std::runtime_error {
  int code;
  GrammarError(int c, const std::string &m) : std::runtime_error(m), code(c) {}
};

struct CharSet {
  std::vector<int64_t> ranges; /* lo0, hi0, lo1, hi1, ... */
  bool negated = false;
  bool matches(uint32_t cp) const {
    bool in = false;
    for (size_t k = 0; k + 1 < ranges.size(); k += 2) in |= (int64_t)cp >= ranges[k] && (int64_t)cp <= ranges[k + 1];
    return in != negated;
  }
};

/* symbol: >= 0 character set id, < 0 reference to rule (-sym - 1) */
typedef int32_t Sym;
inline Sym ref_sym(int rule) { return -rule - 1; }
inline int sym_rule(Sym s) { return -s - 1; }

std::string utf8_of(uint32_t c) {
  std::string s;
  if (c < 0x80) s.push_back((char)c);
  else if (c < 0x800) {
    s.push_back((char)(0xC0 | (c >> 6)));
    s.push_back((char)(0x80 | (c & 0x3F)));
  } else if (c < 0x10000) {
    s.push_back((char)(0xE0 | (c >> 12)));
    s.push_back((char)(0x80 | ((c >> 6) & 0x3F)));
    s.push_back((char)(0x80 | (c & 0x3F)));
  } else {
    s.push_back((char)(0xF0 | (c >> 18)));
    s.push_back((char)(0x80 | ((c >> 12) & 0x3F)));
    s.push_back((char)(0x80 | ((c >> 6) & 0x3F)));
    s.push_back((char)(0x80 | (c & 0x3F)));
  }
  return s;
}

/* ------------------------------------------------------------------ 1. GBNF reader */
class GbnfReader {
 public:
  std::vector<std::vector<std::vector<Sym>>> rules;
  std::vector<CharSet> sets;
  int root = -1;

  explicit GbnfReader(const std::string &text) {
    bl_utf8_decode((const uint8_t *)text.data(), text.size(), src_);
    blank(true);
    while (pos_ < src_.size()) {
      rule_definition();
      blank(true);
    }
    for (size_t r = 0; r < rules.size(); r++)
      if (!defined_[r]) fail("grammar: undefined rule '" + names_[r] + "'");
    auto it = by_name_.find("root");
    if (it == by_name_.end()) fail("grammar: there is no `root` rule");
    root = it->second;
  }

 private:
  std::vector<uint32_t> src_;
  size_t pos_ = 0;
  std::map<std::string, int> by_name_;
  std::vector<std::string> names_;
  std::vector<char> defined_;
  std::map<std::pair<std::vector<int64_t>, bool>, int> set_ids_;
  int depth_ = 0;
  int64_t expanded_ = 0;

  [[noreturn]] static void fail(const std::string &m) { throw GrammarError(BL_EGRAMMAR, m); }
  bool more() const { return pos_ < src_.size(); }
  uint32_t peek(size_t k = 0) const { return src_[pos_ + k]; }
  static bool name_char(uint32_t c) {
    return (c >= '0' && c <= '9') || (c >= 'A' && c <= 'Z') || (c >= 'a' && c <= 'z') || c == '-' || c == '_';
  }

  /* spaces, tabs, comments; newlines only where `nl` (inside groups, between rules) — :63-73 */
  void blank(bool nl) {
    while (more()) {
      uint32_t c = peek();
      if (c == ' ' || c == '\t' || (nl && (c == '\n' || c == '\r'))) {
        pos_++;
      } else if (c == '#') {
        while (more() && peek() != '\n' && peek() != '\r') pos_++;
      } else {
        return;
      }
    }
  }

  static int64_t hex_digit(uint32_t c) {
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    if (c >= 'A' && c <= 'F') return c - 'A' + 10;
    fail("grammar: invalid hex digit");
  }

  /* one literal character with escapes — :75-100 */
  int64_t literal_char() {
    if (!more()) fail("grammar: unexpected end of input");
    uint32_t c = peek();
    if (c != '\\') {
      pos_++;
      return c;
    }
    if (pos_ + 1 >= src_.size()) fail("grammar: unexpected end of input after '\\'");
    uint32_t e = peek(1);
    pos_ += 2;
    switch (e) {
      case 't': return 9;
      case 'r': return 13;
      case 'n': return 10;
      case '\\': case '"': case '[': case ']': return e;
      default: break;
    }
    int digits = e == 'x' ? 2 : e == 'u' ? 4 : e == 'U' ? 8 : 0;
    if (!digits) fail("grammar: unknown escape \\" + utf8_of(e));
    int64_t v = 0;
    for (int k = 0; k < digits; k++) {
      if (!more()) fail("grammar: truncated escape");
      v = v * 16 + hex_digit(peek());
      pos_++;
    }
    return v;
  }

  std::string name() {
    std::string n;
    while (more() && name_char(peek())) n.push_back((char)src_[pos_++]);
    if (n.empty()) fail("grammar: expected a rule name at offset " + std::to_string(pos_));
    return n;
  }

  int new_rule(const std::string &nm, bool def) {
    int id = (int)rules.size();
    rules.emplace_back();
    names_.push_back(nm);
    defined_.push_back(def);
    return id;
  }
  int named_rule(const std::string &nm) {
    auto it = by_name_.find(nm);
    if (it != by_name_.end()) return it->second;
    int id = new_rule(nm, false);
    by_name_[nm] = id;
    return id;
  }
  int anonymous() { return new_rule("(anonymous " + std::to_string(rules.size()) + ")", true); }

  Sym charset(const std::vector<int64_t> &ranges, bool negated) {
    auto key = std::make_pair(ranges, negated);
    auto it = set_ids_.find(key);
    if (it != set_ids_.end()) return it->second;
    int id = (int)sets.size();
    sets.push_back(CharSet{ranges, negated});
    set_ids_[key] = id;
    return id;
  }

  /* x{min,max}: min copies, then (max-min) optional copies as right-nested anonymous rules, or one
   * self-referencing rule when unbounded — :129-163 */
  std::vector<Sym> repeat(const std::vector<Sym> &unit, int64_t min, int64_t max) {
    int64_t copies = std::max(max, min);
    if (copies > kMaxRepeat)
      fail("grammar: a repetition count above " + std::to_string(kMaxRepeat) + " is not supported");
    expanded_ += copies * ((int64_t)unit.size() + 1);
    if (expanded_ > kMaxRepElems)
      fail("grammar: repetitions expand to more than " + std::to_string(kMaxRepElems) + " elements");
    std::vector<Sym> out;
    for (int64_t k = 0; k < min; k++) out.insert(out.end(), unit.begin(), unit.end());
    if (max < 0) {
      int r = anonymous();
      std::vector<Sym> loop = unit;
      loop.push_back(ref_sym(r));
      rules[r] = {loop, {}};
      out.push_back(ref_sym(r));
    } else if (max > min) {
      std::vector<Sym> tail;
      for (int64_t k = 0; k < max - min; k++) {
        int r = anonymous();
        std::vector<Sym> seq = unit;
        seq.insert(seq.end(), tail.begin(), tail.end());
        rules[r] = {seq, {}};
        tail = {ref_sym(r)};
      }
      out.insert(out.end(), tail.begin(), tail.end());
    }
    return out;
  }

  int64_t count() {
    int64_t v = 0;
    int digits = 0;
    while (more() && peek() >= '0' && peek() <= '9') {
      v = v * 10 + (peek() - '0');
      pos_++;
      if (++digits > 9) fail("grammar: a repetition count above " + std::to_string(kMaxRepeat) + " is not supported");
    }
    if (!digits) fail("grammar: expected a number in a repetition at offset " + std::to_string(pos_));
    return v;
  }

  /* :176-281 */
  std::vector<Sym> sequence(bool nested) {
    std::vector<Sym> out;
    size_t last = 0; /* start of the most recent symbol (what a repetition applies to) */
    while (more()) {
      uint32_t c = peek();
      if (c == '"') {
        pos_++;
        last = out.size();
        while (more() && peek() != '"') {
          int64_t ch = literal_char();
          out.push_back(charset({ch, ch}, false));
        }
        if (!more()) fail("grammar: unterminated string literal");
        pos_++;
        blank(nested);
      } else if (c == '[') {
        pos_++;
        bool neg = more() && peek() == '^';
        if (neg) pos_++;
        last = out.size();
        std::vector<int64_t> ranges;
        while (more() && peek() != ']') {
          int64_t lo = literal_char(), hi = lo;
          if (pos_ + 1 < src_.size() && peek() == '-' && peek(1) != ']') {
            pos_++;
            hi = literal_char();
          }
          ranges.push_back(lo);
          ranges.push_back(hi);
        }
        if (!more()) fail("grammar: unterminated character class");
        pos_++;
        out.push_back(charset(ranges, neg));
        blank(nested);
      } else if (name_char(c)) {
        std::string n = name();
        blank(nested);
        last = out.size();
        out.push_back(ref_sym(named_rule(n)));
      } else if (c == '(') {
        pos_++;
        blank(true);
        int sub = anonymous();
        if (depth_ >= kMaxDepth)
          fail("grammar: groups are nested deeper than " + std::to_string(kMaxDepth) + " levels");
        depth_++;
        alternatives(sub, true);
        depth_--;
        if (!(more() && peek() == ')')) fail("grammar: expected ')' at offset " + std::to_string(pos_));
        pos_++;
        blank(nested);
        last = out.size();
        out.push_back(ref_sym(sub));
      } else if (c == '.') {
        pos_++;
        blank(nested);
        last = out.size();
        out.push_back(charset({}, true));
      } else if (c == '*' || c == '+' || c == '?' || c == '{') {
        if (out.size() <= last)
          fail("grammar: a repetition needs something to repeat (offset " + std::to_string(pos_) + ")");
        std::vector<Sym> unit(out.begin() + last, out.end());
        out.resize(last);
        int64_t min = 0, max = -1;
        pos_++;
        if (c == '+') {
          min = 1;
        } else if (c == '?') {
          max = 1;
        } else if (c == '{') {
          blank(false);
          min = max = count();
          blank(false);
          if (more() && peek() == ',') {
            pos_++;
            blank(false);
            if (more() && peek() >= '0' && peek() <= '9') {
              max = count();
              blank(false);
            } else {
              max = -1;
            }
          }
          if (!(more() && peek() == '}')) fail("grammar: expected '}' at offset " + std::to_string(pos_));
          pos_++;
        }
        if (max >= 0 && max < min) fail("grammar: repetition maximum is smaller than its minimum");
        std::vector<Sym> rep = repeat(unit, min, max);
        out.insert(out.end(), rep.begin(), rep.end());
        blank(nested);
      } else {
        break;
      }
    }
    return out;
  }

  void alternatives(int rule, bool nested) {
    std::vector<std::vector<Sym>> alts;
    alts.push_back(sequence(nested));
    while (more() && peek() == '|') {
      pos_++;
      blank(true);
      alts.push_back(sequence(nested));
    }
    rules[rule] = alts;
  }

  void rule_definition() {
    std::string n = name();
    blank(false);
    if (!(pos_ + 2 < src_.size() && peek() == ':' && peek(1) == ':' && peek(2) == '='))
      fail("grammar: expected '::=' after rule name '" + n + "' at offset " + std::to_string(pos_));
    pos_ += 3;
    blank(true);
    int id = named_rule(n);
    if (defined_[id]) fail("grammar: rule '" + n + "' is defined twice");
    defined_[id] = 1;
    alternatives(id, false);
    if (more() && peek() != '\n' && peek() != '\r') {
      size_t at = pos_;
      fail("grammar: unexpected '" + utf8_of(src_[at]) + "' at offset " + std::to_string(at) + " in rule '" + n + "'");
    }
    while (more() && (peek() == '\n' || peek() == '\r')) pos_++;
  }
};

/* ------------------------------------------------------------------ 2. stacks and frontiers */
struct VecHash {
  size_t operator()(const std::vector<int32_t> &v) const {
    uint64_t h = 0xcbf29ce484222325ull ^ v.size();
    for (int32_t x : v) h = (h ^ (uint32_t)x) * 0x100000001b3ull;
    return (size_t)h;
  }
};

class StackMachine {
 public:
  explicit StackMachine(const GbnfReader &g) : g_(g) {}

  /* frontier of `seeds` (each a stack, top last); sorted unique stack ids; throws on the guard */
  std::vector<int32_t> expand(const std::vector<std::vector<Sym>> &seeds) {
    std::vector<std::vector<Sym>> work;
    std::unordered_map<std::vector<Sym>, char, VecHash> seen;
    for (const auto &s : seeds)
      if (seen.emplace(s, 1).second) work.push_back(s);
    std::vector<int32_t> out;
    for (size_t i = 0; i < work.size(); i++) {
      if (work.size() >= kStackGuard)
        throw GrammarError(BL_EGRAMMAR_AMBIG, "grammar is left-recursive or too ambiguous to match");
      std::vector<Sym> st = work[i];
      if (st.empty() || st.back() >= 0) {
        out.push_back(intern(st));
        continue;
      }
      int r = sym_rule(st.back());
      st.pop_back();
      for (const auto &alt : g_.rules[r]) {
        std::vector<Sym> nx = st;
        nx.insert(nx.end(), alt.rbegin(), alt.rend());
        if (seen.emplace(nx, 1).second) work.push_back(nx);
      }
    }
    std::sort(out.begin(), out.end());
    out.erase(std::unique(out.begin(), out.end()), out.end());
    return out;
  }

  std::vector<int32_t> start() {
    std::vector<std::vector<Sym>> seeds;
    for (const auto &alt : g_.rules[g_.root]) seeds.emplace_back(alt.rbegin(), alt.rend());
    return expand(seeds);
  }

  /* stacks whose top set matches a code point of class-representative `cp`, popped, then expanded */
  std::vector<int32_t> step(const std::vector<int32_t> &front, uint32_t cp) {
    std::vector<std::vector<Sym>> next;
    for (int32_t id : front) {
      const auto &st = stacks_[id];
      if (!st.empty() && g_.sets[st.back()].matches(cp)) next.emplace_back(st.begin(), st.end() - 1);
    }
    return expand(next);
  }

  uint8_t flags(const std::vector<int32_t> &front) const {
    uint8_t f = 0;
    for (int32_t id : front) {
      const auto &st = stacks_[id];
      if (st.empty()) {
        f |= BL_GS_COMPLETE;
        continue;
      }
      f |= BL_GS_CONTINUE;
      const CharSet &cs = g_.sets[st.back()];
      bool wide = cs.negated;
      for (size_t k = 1; k < cs.ranges.size(); k += 2) wide |= cs.ranges[k] >= 128;
      if (wide) f |= BL_GS_NONASCII;
    }
    return f;
  }

 private:
  const GbnfReader &g_;
  std::vector<std::vector<Sym>> stacks_;
  std::unordered_map<std::vector<Sym>, int32_t, VecHash> stack_ids_;

  int32_t intern(const std::vector<Sym> &st) {
    auto it = stack_ids_.find(st);
    if (it != stack_ids_.end()) return it->second;
    int32_t id = (int32_t)stacks_.size();
    stacks_.push_back(st);
    stack_ids_.emplace(st, id);
    return id;
  }
};

}  // namespace

/* ------------------------------------------------------------------ lossy UTF-8 (src/io.br:70-115) */
void bl_utf8_decode(const uint8_t *b, size_t n, std::vector<uint32_t> &out) {
  out.clear();
  size_t i = 0;
  auto cont = [&](size_t k) { return k < n && (b[k] & 0xC0) == 0x80; };
  while (i < n) {
    uint32_t b0 = b[i];
    uint32_t cp = 0xFFFD;
    size_t len = 1;
    if (b0 < 0x80) {
      cp = b0;
    } else if (b0 >= 0xC2 && b0 <= 0xDF) {
      if (cont(i + 1)) {
        cp = ((b0 & 0x1F) << 6) | (b[i + 1] & 0x3F);
        len = 2;
      }
    } else if (b0 >= 0xE0 && b0 <= 0xEF) {
      if (cont(i + 1) && cont(i + 2)) {
        uint32_t c = ((b0 & 0x0F) << 12) | ((uint32_t)(b[i + 1] & 0x3F) << 6) | (b[i + 2] & 0x3F);
        if (c >= 0x800 && !(c >= 0xD800 && c <= 0xDFFF)) {
          cp = c;
          len = 3;
        }
      }
    } else if (b0 >= 0xF0 && b0 <= 0xF4) {
      if (cont(i + 1) && cont(i + 2) && cont(i + 3)) {
        uint32_t c = ((b0 & 0x07) << 18) | ((uint32_t)(b[i + 1] & 0x3F) << 12) | ((uint32_t)(b[i + 2] & 0x3F) << 6) |
                     (b[i + 3] & 0x3F);
        if (c >= 0x10000 && c <= 0x10FFFF) {
          cp = c;
          len = 4;
        }
      }
    }
    out.push_back(cp);
    i += len;
  }
}

int32_t bl_gram_class(const bl_gram_tables &g, uint32_t cp) {
  if (cp < 128) return g.ascii[cp];
  size_t lo = 0, hi = g.ivl_lo.size();
  while (hi - lo > 1) {
    size_t mid = (lo + hi) / 2;
    if (g.ivl_lo[mid] <= cp) lo = mid;
    else hi = mid;
  }
  return g.ivl_cls[lo];
}

/* ------------------------------------------------------------------ 3. the automaton */
int bl_gram_compile(const std::string &gbnf, int max_states, bl_gram_tables &out, std::string &err) {
  out = bl_gram_tables();
  try {
    GbnfReader g(gbnf);
    /* code-point classes: cut the axis at every range edge, then merge intervals with equal signatures */
    std::vector<uint32_t> cuts = {0, 128, 0x110000};
    for (const CharSet &cs : g.sets)
      for (size_t k = 0; k + 1 < cs.ranges.size(); k += 2) {
        int64_t lo = cs.ranges[k], hi = cs.ranges[k + 1];
        if (lo >= 0 && lo < 0x110000) cuts.push_back((uint32_t)lo);
        if (hi + 1 >= 0 && hi + 1 < 0x110000) cuts.push_back((uint32_t)(hi + 1));
      }
    std::sort(cuts.begin(), cuts.end());
    cuts.erase(std::unique(cuts.begin(), cuts.end()), cuts.end());
    std::map<std::vector<bool>, int> sig_class;
    std::vector<uint32_t> rep; /* a code point of each class */
    std::vector<std::pair<uint32_t, int>> ivl;
    for (size_t k = 0; k + 1 < cuts.size(); k++) {
      uint32_t lo = cuts[k];
      std::vector<bool> sig(g.sets.size());
      for (size_t s = 0; s < g.sets.size(); s++) sig[s] = g.sets[s].matches(lo);
      auto it = sig_class.find(sig);
      int cls;
      if (it == sig_class.end()) {
        cls = (int)rep.size();
        sig_class.emplace(sig, cls);
        rep.push_back(lo);
      } else {
        cls = it->second;
      }
      ivl.emplace_back(lo, cls);
    }
    if (rep.size() > 65535) {
      err = "grammar: too many character classes for the device tables";
      return BL_EUNSUPPORTED;
    }
    out.n_classes = (int32_t)rep.size();
    out.ascii.assign(128, 0);
    for (size_t k = 0; k < ivl.size(); k++) {
      uint32_t lo = ivl[k].first, hi = k + 1 < ivl.size() ? ivl[k + 1].first : 0x110000;
      for (uint32_t c = lo; c < hi && c < 128; c++) out.ascii[c] = (uint16_t)ivl[k].second;
      if (hi > 128) {
        uint32_t a = std::max(lo, 128u);
        if (out.ivl_cls.empty() || out.ivl_cls.back() != ivl[k].second) {
          out.ivl_lo.push_back(a);
          out.ivl_cls.push_back((uint16_t)ivl[k].second);
        }
      }
    }

    StackMachine m(g);
    std::map<std::vector<int32_t>, int32_t> ids;
    std::vector<std::vector<int32_t>> fronts;
    std::vector<int32_t> s0;
    try {
      s0 = m.start();
    } catch (const GrammarError &e) {
      if (e.code != BL_EGRAMMAR_AMBIG) throw;
      err = e.what();
      out.start_error = 1;
      return BL_EGRAMMAR_AMBIG;
    }
    if (s0.empty()) {
      /* no stack at all: every text is rejected (the reference reports a dead reply) */
      out.n_states = 1;
      out.start = 0;
      out.trans.assign(out.n_classes, BL_GT_DEAD);
      out.flags.assign(1, 0);
      return BL_OK;
    }
    ids[s0] = 0;
    fronts.push_back(s0);
    for (size_t q = 0; q < fronts.size(); q++) {
      out.flags.push_back(m.flags(fronts[q]));
      for (int c = 0; c < out.n_classes; c++) {
        int32_t target;
        try {
          std::vector<int32_t> nx = m.step(fronts[q], rep[c]);
          if (nx.empty()) {
            target = BL_GT_DEAD;
          } else {
            auto it = ids.find(nx);
            if (it != ids.end()) {
              target = it->second;
            } else {
              if ((int)fronts.size() >= max_states) {
                err = "grammar: the automaton of this grammar exceeds " + std::to_string(max_states) +
                      " states (a recursive grammar reachable from root is not supported on the device)";
                return BL_EUNSUPPORTED;
              }
              target = (int32_t)fronts.size();
              ids.emplace(nx, target);
              fronts.push_back(nx);
            }
          }
        } catch (const GrammarError &e) {
          if (e.code != BL_EGRAMMAR_AMBIG) throw;
          target = BL_GT_AMBIG;
        }
        out.trans.push_back(target);
      }
    }
    out.n_states = (int32_t)fronts.size();
    out.start = 0;
    return BL_OK;
  } catch (const GrammarError &e) {
    err = e.what();
    return e.code;
  }
}
