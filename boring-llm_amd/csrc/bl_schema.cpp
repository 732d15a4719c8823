/*
 * bl_schema.cpp — JSON Schema -> GBNF text for libbl_select (host C++).
 *
 * A request's `response_format` JSON schema (src/server.br:733-745) becomes the GBNF grammar that
 * json_schema_to_gbnf (src/schema_grammar.br:313-337) generates for it, which the slot's grammar is then
 * compiled from. The JSON text is parsed as src/json.br's json_parse does (its grammar, nesting limit,
 * duplicate keys, `null` read as an absent value and its error messages, whose positions count code
 * points); const/enum values are printed as src/jinja.br's jv_to_json prints them.
 *
 * The parser works on the UTF-8 bytes (no code-point array): positions in messages are converted to
 * code-point counts only when an error is raised. Parsed values live in one arena of nodes.
 */
#include "bl_schema.h"

#include <charconv>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

namespace {

struct Node {
  enum Kind : uint8_t { Absent, Bool, Int, Float, Str, List, Dict } kind = Absent;
  bool b = false;
  int64_t i = 0;
  double f = 0.0;
  std::string s;
  std::vector<int32_t> kids;      /* list items, or dict values (parallel to keys) */
  std::vector<std::string> keys;  /* dict keys in first-occurrence order */
};

struct Fail : std::runtime_error {
  using std::runtime_error::runtime_error;
};

/* Length of the UTF-8 sequence starting with byte c (the input is validated first). */
inline int seq_len(uint8_t c) { return c < 0x80 ? 1 : c < 0xE0 ? 2 : c < 0xF0 ? 3 : 4; }

bool valid_utf8(const uint8_t *p, size_t n) {
  size_t i = 0;
  while (i < n) {
    uint8_t c = p[i];
    if (c < 0x80) { i++; continue; }
    int len;
    uint32_t cp, min;
    if (c >= 0xC2 && c <= 0xDF) { len = 2; cp = c & 0x1F; min = 0x80; }
    else if (c >= 0xE0 && c <= 0xEF) { len = 3; cp = c & 0x0F; min = 0x800; }
    else if (c >= 0xF0 && c <= 0xF4) { len = 4; cp = c & 0x07; min = 0x10000; }
    else return false;
    if (i + len > n) return false;
    for (int k = 1; k < len; k++) {
      if ((p[i + k] & 0xC0) != 0x80) return false;
      cp = cp << 6 | (p[i + k] & 0x3F);
    }
    if (cp < min || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return false;
    i += len;
  }
  return true;
}

void put_utf8(std::string &o, uint32_t cp) {
  if (cp < 0x80) o += (char)cp;
  else if (cp < 0x800) { o += (char)(0xC0 | cp >> 6); o += (char)(0x80 | (cp & 63)); }
  else if (cp < 0x10000) {
    o += (char)(0xE0 | cp >> 12); o += (char)(0x80 | (cp >> 6 & 63)); o += (char)(0x80 | (cp & 63));
  } else {
    o += (char)(0xF0 | cp >> 18); o += (char)(0x80 | (cp >> 12 & 63)); o += (char)(0x80 | (cp >> 6 & 63));
    o += (char)(0x80 | (cp & 63));
  }
}

/* ------------------------------------------------------------------ JSON text -> arena */
class Parser {
 public:
  Parser(const char *text, size_t n, std::vector<Node> &arena) : t_((const uint8_t *)text), n_(n), a_(arena) {}

  int32_t parse_document() {
    size_t end;
    int32_t v = value(0, 0, end);
    size_t tail = ws(end);
    if (tail != n_) throw Fail("json: trailing characters at " + at(tail));
    return v;
  }

 private:
  const uint8_t *t_;
  size_t n_;
  std::vector<Node> &a_;
  static constexpr int kMaxDepth = 128; /* src/json.br nesting limit */

  /* A byte offset as the code-point index the reference reports. */
  std::string at(size_t byte) const {
    size_t cps = 0;
    for (size_t k = 0; k < byte && k < n_; k++) cps += (t_[k] & 0xC0) != 0x80;
    return std::to_string(cps);
  }
  std::string char_at(size_t p) const { return std::string((const char *)t_ + p, seq_len(t_[p])); }
  size_t ws(size_t p) const {
    while (p < n_ && (t_[p] == ' ' || t_[p] == '\n' || t_[p] == '\t' || t_[p] == '\r')) p++;
    return p;
  }
  bool digit(size_t p) const { return p < n_ && t_[p] >= '0' && t_[p] <= '9'; }
  int32_t make(Node::Kind k) {
    a_.emplace_back();
    a_.back().kind = k;
    return (int32_t)a_.size() - 1;
  }

  /* Four hex digits at byte p (code-point-counted truncation, as the reference's char array has it). */
  uint32_t hex4(size_t p) const {
    size_t q = p;
    for (int k = 0; k < 4; k++) {
      if (q >= n_) throw Fail("json: truncated \\u escape");
      q += seq_len(t_[q]);
    }
    uint32_t v = 0;
    for (int k = 0; k < 4; k++) {
      uint8_t c = t_[p];
      uint32_t d;
      if (c >= '0' && c <= '9') d = c - '0';
      else if (c >= 'a' && c <= 'f') d = c - 'a' + 10;
      else if (c >= 'A' && c <= 'F') d = c - 'A' + 10;
      else throw Fail("json: invalid hex digit '" + char_at(p) + "' in \\u escape");
      v = v * 16 + d;
      p++;
    }
    return v;
  }

  std::string string_at(size_t p, size_t &end) const {
    std::string out;
    p++; /* opening quote */
    for (;;) {
      if (p >= n_) throw Fail("json: unterminated string");
      uint8_t c = t_[p];
      if (c == '"') { end = p + 1; return out; }
      if (c != '\\') {
        if (c < 0x20) throw Fail("json: unescaped control character in string");
        int len = seq_len(c);
        out.append((const char *)t_ + p, len);
        p += len;
        continue;
      }
      if (p + 1 >= n_) throw Fail("json: truncated escape");
      uint8_t e = t_[p + 1];
      switch (e) {
        case 'n': out += '\n'; p += 2; break;
        case 't': out += '\t'; p += 2; break;
        case 'r': out += '\r'; p += 2; break;
        case 'b': out += '\b'; p += 2; break;
        case 'f': out += '\f'; p += 2; break;
        case '"': case '\\': case '/': out += (char)e; p += 2; break;
        case 'u': {
          uint32_t cp = hex4(p + 2);
          p += 6;
          if (cp >= 0xD800 && cp <= 0xDBFF) {
            if (!(p + 1 < n_ && t_[p] == '\\' && t_[p + 1] == 'u'))
              throw Fail("json: high surrogate without a low surrogate");
            uint32_t lo = hex4(p + 2);
            if (lo < 0xDC00 || lo > 0xDFFF) throw Fail("json: invalid low surrogate");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
            p += 6;
          } else if (cp >= 0xDC00 && cp <= 0xDFFF) {
            throw Fail("json: low surrogate without a high surrogate");
          }
          put_utf8(out, cp);
          break;
        }
        default: throw Fail("json: invalid escape '\\" + char_at(p + 1) + "'");
      }
    }
  }

  int32_t number_at(size_t start, size_t &end) {
    size_t p = start;
    bool frac = false;
    if (p < n_ && t_[p] == '-') p++;
    if (p >= n_) throw Fail("json: truncated number");
    if (t_[p] == '0') p++;
    else if (t_[p] >= '1' && t_[p] <= '9') { while (digit(p)) p++; }
    else throw Fail("json: invalid number at " + at(start));
    if (p < n_ && t_[p] == '.') {
      frac = true;
      if (!digit(++p)) throw Fail("json: expected digit after decimal point");
      while (digit(p)) p++;
    }
    if (p < n_ && (t_[p] == 'e' || t_[p] == 'E')) {
      frac = true;
      p++;
      if (p < n_ && (t_[p] == '+' || t_[p] == '-')) p++;
      if (!digit(p)) throw Fail("json: expected exponent digits");
      while (digit(p)) p++;
    }
    end = p;
    const char *b = (const char *)t_ + start, *e = (const char *)t_ + p;
    if (!frac) { /* an integer literal that fits i64 stays an integer; a larger one is read as a float */
      int64_t x;
      auto r = std::from_chars(b, e, x);
      if (r.ec == std::errc() && r.ptr == e) {
        int32_t v = make(Node::Int);
        a_[v].i = x;
        return v;
      }
    }
    int32_t v = make(Node::Float);
    a_[v].f = std::strtod(std::string(b, e).c_str(), nullptr);
    return v;
  }

  bool literal(size_t p, const char *lit) const {
    size_t L = std::strlen(lit);
    return p + L <= n_ && std::memcmp(t_ + p, lit, L) == 0;
  }

  int32_t value(size_t pos, int depth, size_t &end) {
    if (depth > kMaxDepth) throw Fail("json: nesting is deeper than " + std::to_string(kMaxDepth) + " levels");
    size_t p = ws(pos);
    if (p >= n_) throw Fail("json: unexpected end of input");
    uint8_t c = t_[p];
    if (c == '{') return object(p, depth, end);
    if (c == '[') return array(p, depth, end);
    if (c == '"') {
      int32_t v = make(Node::Str);
      std::string s = string_at(p, end);
      a_[v].s = std::move(s);
      return v;
    }
    if (literal(p, "true")) { int32_t v = make(Node::Bool); a_[v].b = true; end = p + 4; return v; }
    if (literal(p, "false")) { int32_t v = make(Node::Bool); end = p + 5; return v; }
    if (literal(p, "null")) { end = p + 4; return make(Node::Absent); }
    return number_at(p, end);
  }

  int32_t object(size_t p, int depth, size_t &end) {
    int32_t v = make(Node::Dict);
    size_t q = ws(p + 1);
    if (q < n_ && t_[q] == '}') { end = q + 1; return v; }
    for (;;) {
      q = ws(q);
      if (!(q < n_ && t_[q] == '"')) throw Fail("json: expected object key at " + at(q));
      size_t after;
      std::string key = string_at(q, after);
      q = ws(after);
      if (!(q < n_ && t_[q] == ':')) throw Fail("json: expected ':' after key '" + key + "'");
      int32_t child = value(q + 1, depth + 1, after);
      Node &d = a_[v];
      size_t k = 0;
      while (k < d.keys.size() && d.keys[k] != key) k++;
      if (k == d.keys.size()) { d.keys.push_back(std::move(key)); d.kids.push_back(child); }
      else d.kids[k] = child; /* a repeated key keeps its first position and its last value */
      q = ws(after);
      if (q >= n_) throw Fail("json: unterminated object");
      if (t_[q] == ',') { q++; continue; }
      if (t_[q] == '}') { end = q + 1; return v; }
      throw Fail("json: expected ',' or '}' at " + at(q));
    }
  }

  int32_t array(size_t p, int depth, size_t &end) {
    int32_t v = make(Node::List);
    size_t q = ws(p + 1);
    if (q < n_ && t_[q] == ']') { end = q + 1; return v; }
    for (;;) {
      size_t after;
      int32_t item = value(q, depth + 1, after);
      a_[v].kids.push_back(item);
      q = ws(after);
      if (q >= n_) throw Fail("json: unterminated array");
      if (t_[q] == ',') { q++; continue; }
      if (t_[q] == ']') { end = q + 1; return v; }
      throw Fail("json: expected ',' or ']' at " + at(q));
    }
  }
};

/* ------------------------------------------------------------------ value -> JSON text (jv_to_json) */
/* Rust's `{}` for f64: the shortest digits that read back to the same value, in positional notation. */
std::string rust_display(double f) {
  if (std::isnan(f)) return "NaN";
  if (std::isinf(f)) return f < 0 ? "-inf" : "inf";
  char buf[64];
  auto r = std::to_chars(buf, buf + sizeof buf, f, std::chars_format::scientific);
  std::string sci(buf, r.ptr); /* [-]d[.ddd]e(+|-)xx */
  std::string out;
  size_t k = 0;
  if (sci[0] == '-') { out += '-'; k = 1; }
  size_t e = sci.find('e');
  std::string digits;
  for (size_t j = k; j < e; j++)
    if (sci[j] != '.') digits += sci[j];
  int exp10 = std::atoi(sci.c_str() + e + 1);
  while (digits.size() > 1 && digits.back() == '0') digits.pop_back();
  int point = exp10 + 1; /* digits before the decimal point */
  if (point <= 0) out += "0." + std::string(-point, '0') + digits;
  else if ((size_t)point >= digits.size()) out += digits + std::string(point - digits.size(), '0');
  else out += digits.substr(0, point) + "." + digits.substr(point);
  return out;
}

void json_quote(std::string &o, const std::string &s) {
  static const char hexd[] = "0123456789abcdef";
  o += '"';
  for (unsigned char c : s) {
    switch (c) {
      case '"': o += "\\\""; break;
      case '\\': o += "\\\\"; break;
      case '\n': o += "\\n"; break;
      case '\r': o += "\\r"; break;
      case '\t': o += "\\t"; break;
      default:
        if (c < 0x20) { o += "\\u00"; o += hexd[c >> 4]; o += hexd[c & 15]; }
        else o += (char)c;
    }
  }
  o += '"';
}

void to_json(const std::vector<Node> &a, int32_t v, std::string &o) {
  const Node &x = a[v];
  switch (x.kind) {
    case Node::Absent: o += "null"; break;
    case Node::Bool: o += x.b ? "true" : "false"; break;
    case Node::Int: o += std::to_string(x.i); break;
    case Node::Float: o += rust_display(x.f); break;
    case Node::Str: json_quote(o, x.s); break;
    case Node::List:
      o += '[';
      for (size_t k = 0; k < x.kids.size(); k++) {
        if (k) o += ", ";
        to_json(a, x.kids[k], o);
      }
      o += ']';
      break;
    case Node::Dict:
      o += '{';
      for (size_t k = 0; k < x.keys.size(); k++) {
        if (k) o += ", ";
        json_quote(o, x.keys[k]);
        o += ": ";
        to_json(a, x.kids[k], o);
      }
      o += '}';
      break;
  }
}

/* GBNF string literal of a text (gbnf_literal, src/schema_grammar.br:48-63). */
std::string gbnf_quote(const std::string &s) {
  std::string o = "\"";
  for (char c : s) {
    switch (c) {
      case '"': o += "\\\""; break;
      case '\\': o += "\\\\"; break;
      case '\n': o += "\\n"; break;
      case '\r': o += "\\r"; break;
      case '\t': o += "\\t"; break;
      default: o += c;
    }
  }
  return o + "\"";
}

/* ------------------------------------------------------------------ schema -> rules */
/* The primitive rules every generated grammar ends with (src/schema_grammar.br:21, :324-337). */
const char kPrimitives[] =
    "space ::= | \" \" | \"\\n\"{1,2} [ \\t]{0,20}\n"
    "boolean ::= (\"true\" | \"false\") space\n"
    "decimal-part ::= [0-9]{1,16}\n"
    "integral-part ::= [0] | [1-9] [0-9]{0,15}\n"
    "number ::= (\"-\"? integral-part) (\".\" decimal-part)? ([eE] [-+]? integral-part)? space\n"
    "integer ::= (\"-\"? integral-part) space\n"
    "null ::= \"null\" space\n"
    "char ::= [^\"\\\\\\x7F\\x00-\\x1F] | [\\\\] ([\"\\\\bfnrt] | \"u\" [0-9a-fA-F]{4})\n"
    "string ::= \"\\\"\" char* \"\\\"\" space\n"
    "value ::= object | array | string | number | boolean | null\n"
    "object ::= \"{\" space ( string \":\" space value (\",\" space string \":\" space value)* )? \"}\" space\n"
    "array ::= \"[\" space ( value (\",\" space value)* )? \"]\" space\n";

class Compiler {
 public:
  Compiler(const std::vector<Node> &a, int32_t root) : a_(a), root_(root) {}

  std::string run() {
    std::string top = visit(root_, "root");
    std::string out = "root ::= ";
    if (top == "root") {
      std::string body = rules_["root"];
      static const char tail[] = " space";
      if (body.size() >= 6 && body.compare(body.size() - 6, 6, tail) == 0) body.resize(body.size() - 6);
      out += body;
    } else {
      out += top;
    }
    out += '\n';
    for (const std::string &name : order_) {
      if (name == "root") continue;
      out += name;
      out += " ::= ";
      out += rules_[name];
      out += '\n';
    }
    return out + kPrimitives;
  }

 private:
  const std::vector<Node> &a_;
  int32_t root_;
  std::unordered_map<std::string, std::string> rules_, refs_;
  std::vector<std::string> order_;

  /* ---- value helpers (json_get and friends of src/json.br, list/dict accessors of schema_grammar.br) */
  int32_t get(int32_t v, const char *key) const {
    if (v < 0 || a_[v].kind != Node::Dict) return -1;
    const Node &d = a_[v];
    for (size_t k = 0; k < d.keys.size(); k++)
      if (d.keys[k] == key) return a_[d.kids[k]].kind == Node::Absent ? -1 : d.kids[k];
    return -1;
  }
  Node::Kind kind(int32_t v) const { return v < 0 ? Node::Absent : a_[v].kind; }
  bool is(int32_t v, Node::Kind k) const { return kind(v) == k; }
  std::vector<std::string> strings(int32_t list) const { /* non-strings read as "" */
    std::vector<std::string> out;
    if (!is(list, Node::List)) return out;
    for (int32_t it : a_[list].kids) out.push_back(is(it, Node::Str) ? a_[it].s : std::string());
    return out;
  }
  int64_t as_int(int32_t v, int64_t fallback, bool floats) const {
    if (is(v, Node::Int)) return a_[v].i;
    if (floats && is(v, Node::Float)) { /* Rust `as`: saturating, NaN -> 0 */
      double f = a_[v].f;
      if (std::isnan(f)) return 0;
      if (f >= 9223372036854775807.0) return INT64_MAX;
      if (f <= -9223372036854775808.0) return INT64_MIN;
      return (int64_t)f;
    }
    return fallback;
  }

  static std::string sanitize(const std::string &raw) {
    std::string out;
    for (size_t k = 0; k < raw.size();) {
      unsigned char c = raw[k];
      bool alnum = (c >= '0' && c <= '9') || (c >= 'A' && c <= 'Z') || (c >= 'a' && c <= 'z');
      out += alnum ? (char)c : '-';
      k += seq_len(c); /* one '-' per code point */
    }
    return out.empty() ? "x" : out;
  }

  /* add_rule (src/schema_grammar.br:36-45): the hint's name, or the first free numbered variant. */
  std::string add(const std::string &hint, const std::string &body) {
    const std::string base = sanitize(hint);
    std::string name = base;
    for (int n = 1;; n++) {
      auto it = rules_.find(name);
      if (it == rules_.end()) {
        rules_.emplace(name, body);
        order_.push_back(name);
        return name;
      }
      if (it->second == body) return name;
      name = base + "-" + std::to_string(n);
    }
  }

  std::string literal_of(int32_t v) const {
    std::string j;
    to_json(a_, v, j);
    return gbnf_quote(j);
  }

  int32_t resolve(const std::string &ref) const {
    if (ref[0] != '#') throw Fail("only local $ref values are supported (got '" + ref + "')");
    if (ref.size() == 1) return root_;
    if (ref[1] != '/') throw Fail("unsupported $ref '" + ref + "'");
    int32_t node = root_;
    size_t p = 2;
    for (;;) {
      size_t slash = ref.find('/', p);
      std::string part = ref.substr(p, slash == std::string::npos ? std::string::npos : slash - p);
      node = get(node, part.c_str());
      if (node < 0) throw Fail("$ref '" + ref + "' does not resolve");
      if (slash == std::string::npos) return node;
      p = slash + 1;
    }
  }

  std::string visit(int32_t s, const std::string &name) {
    if (!is(s, Node::Dict)) {
      if (is(s, Node::Bool)) return "value";
      throw Fail("a schema must be an object or a boolean");
    }
    int32_t ref = get(s, "$ref");
    if (is(ref, Node::Str) && !a_[ref].s.empty()) {
      const std::string &text = a_[ref].s;
      auto hit = refs_.find(text);
      if (hit != refs_.end()) return hit->second;
      std::string rname = sanitize("ref-" + text);
      refs_[text] = rname;
      rules_[rname] = "value"; /* reserved first: a recursive schema refers to it */
      order_.push_back(rname);
      std::string target = visit(resolve(text), rname);
      rules_[rname] = target;
      return rname;
    }
    int32_t c = get(s, "const");
    if (c >= 0) return add(name, literal_of(c));
    int32_t en = get(s, "enum");
    if (is(en, Node::List)) {
      if (a_[en].kids.empty()) throw Fail("enum must not be empty");
      std::string body = "(";
      for (size_t k = 0; k < a_[en].kids.size(); k++) {
        if (k) body += " | ";
        body += literal_of(a_[en].kids[k]);
      }
      return add(name, body + ") space");
    }
    std::vector<std::string> alts; /* anyOf then oneOf alternatives, each list numbered from 0 */
    bool combined = false;
    for (const char *key : {"anyOf", "oneOf"}) {
      int32_t l = get(s, key);
      if (!is(l, Node::List)) continue;
      combined = true;
      for (size_t k = 0; k < a_[l].kids.size(); k++) alts.push_back(visit(a_[l].kids[k], name + "-" + std::to_string(k)));
    }
    if (combined) {
      std::string body;
      for (size_t k = 0; k < alts.size(); k++) body += (k ? " | " : "") + alts[k];
      return add(name, body);
    }
    std::vector<std::string> types;
    int32_t ty = get(s, "type");
    if (is(ty, Node::Str)) types.push_back(a_[ty].s);
    else types = strings(ty);
    if (types.empty()) {
      if (!is(get(s, "properties"), Node::Dict)) return "value";
      types.push_back("object");
    }
    if (types.size() > 1) {
      std::string body;
      for (size_t k = 0; k < types.size(); k++) {
        if (k) body += " | ";
        body += typed(s, types[k], name + "-" + types[k]);
      }
      return add(name, body);
    }
    return typed(s, types[0], name);
  }

  std::string typed(int32_t s, const std::string &t, const std::string &name) {
    if (t == "object") return add(name, object(s, name));
    if (t == "array") return add(name, array(s, name));
    if (t == "string") {
      int64_t lo = as_int(get(s, "minLength"), 0, true), hi = as_int(get(s, "maxLength"), -1, false);
      if (lo == 0 && hi < 0) return "string";
      return add(name, "\"\\\"\" char{" + std::to_string(lo) + "," + (hi < 0 ? "" : std::to_string(hi)) +
                           "} \"\\\"\" space");
    }
    if (t == "integer" || t == "number" || t == "boolean" || t == "null") return t;
    throw Fail("unsupported schema type '" + t + "'");
  }

  std::string object(int32_t s, const std::string &name) {
    std::vector<std::string> req, opt;
    const std::vector<std::string> required = strings(get(s, "required"));
    int32_t props = get(s, "properties");
    const std::vector<std::string> *keys = is(props, Node::Dict) ? &a_[props].keys : nullptr;
    auto listed = [&](const std::string &k) {
      for (const std::string &r : required)
        if (r == k) return true;
      return false;
    };
    for (int pass = 0; pass < 2 && keys; pass++) {
      for (const std::string &k : *keys) {
        if (listed(k) != (pass == 0)) continue;
        std::string child = visit(get(props, k.c_str()), name + "-" + k);
        std::string key_json;
        json_quote(key_json, k);
        std::string kv = add(name + "-" + k + "-kv", gbnf_quote(key_json) + " space \":\" space " + child);
        (pass == 0 ? req : opt).push_back(kv);
      }
    }
    int32_t extra_v = get(s, "additionalProperties");
    bool extra = is(extra_v, Node::Dict) || (is(extra_v, Node::Bool) && a_[extra_v].b);
    std::string extra_kv;
    if (extra) {
      std::string child = is(extra_v, Node::Dict) ? visit(extra_v, name + "-additional") : "value";
      extra_kv = add(name + "-additional-kv", "string \":\" space " + child);
    }
    std::string body = "\"{\" space ";
    if (!req.empty()) {
      std::string inner = req[0];
      for (size_t k = 1; k < req.size(); k++) inner += " \",\" space " + req[k];
      for (const std::string &o : opt) inner += " (\",\" space " + o + ")?";
      if (extra) inner += " (\",\" space " + extra_kv + ")*";
      body += inner + " ";
    } else if (!opt.empty() || extra) {
      if (opt.size() > 128)
        throw Fail("an object with more than 128 optional properties and no required one is not supported");
      std::string alts;
      for (size_t k = 0; k < opt.size(); k++) {
        if (k) alts += " | ";
        alts += opt[k];
        for (size_t j = k + 1; j < opt.size(); j++) alts += " (\",\" space " + opt[j] + ")?";
        if (extra) alts += " (\",\" space " + extra_kv + ")*";
      }
      if (extra) {
        if (!opt.empty()) alts += " | ";
        alts += extra_kv + " (\",\" space " + extra_kv + ")*";
      }
      body += "(" + alts + ")? ";
    }
    return body + "\"}\" space";
  }

  std::string array(int32_t s, const std::string &name) {
    int32_t items = get(s, "items");
    std::string item = is(items, Node::Dict) ? visit(items, name + "-item") : "value";
    int64_t lo = as_int(get(s, "minItems"), 0, true), hi = as_int(get(s, "maxItems"), -1, false);
    if (hi >= 0 && hi < lo) throw Fail("maxItems is smaller than minItems");
    if (hi == 0) return "\"[\" space \"]\" space";
    std::string inner = item;
    if (lo > 1 || hi > 1 || hi < 0) {
      inner += " (\",\" space " + item + "){" + std::to_string(lo > 1 ? lo - 1 : 0) + "," +
               (hi < 0 ? "" : std::to_string(hi - 1)) + "}";
    }
    return lo == 0 ? "\"[\" space (" + inner + ")? \"]\" space" : "\"[\" space " + inner + " \"]\" space";
  }
};

}  // namespace

int bl_schema_to_gbnf(const char *text, size_t len, std::string &gbnf, std::string &err) {
  if (!valid_utf8((const uint8_t *)text, len)) {
    err = "json: the schema text is not valid UTF-8";
    return -1;
  }
  try {
    std::vector<Node> arena;
    arena.reserve(64);
    Parser p(text, len, arena);
    int32_t root = p.parse_document();
    gbnf = Compiler(arena, root).run();
    return 0;
  } catch (const Fail &e) {
    err = e.what();
    return -1;
  }
}
