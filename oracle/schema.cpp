/*
 * schema.cpp — restatement of the reference's src/schema_grammar.br (JSON Schema -> GBNF text), with
 * the pieces it depends on: src/json.br json_parse / json_get*, src/jinja.br jv_to_json /
 * json_escape. TEST INFRASTRUCTURE ONLY (see oracle.h).
 */
#include <errno.h>
#include <stdio.h>
#include <string.h>
#include <algorithm>
#include <stdlib.h>

#include <memory>
#include <stdexcept>
#include <string>

#include "oracle.h"

namespace orc {
namespace {

/* src/jinja.br:49-57 JValue (JSON null parses to JUndefined) */
struct JValue;
typedef std::shared_ptr<JValue> JPtr;
struct JValue {
  enum Kind { Str, Int, Bool, Float, List, Dict, Undefined } kind = Undefined;
  std::string s;
  int64_t n = 0;
  bool b = false;
  double f = 0.0;
  std::vector<JPtr> items;
  std::map<std::string, JPtr> fields;
  std::vector<std::string> keys;
};

JPtr undefined() { return std::make_shared<JValue>(); }

typedef std::vector<uint32_t> Chars;

std::string utf8(uint32_t cp) { return cps_to_utf8(std::vector<uint32_t>{cp}); }
std::string utf8(const Chars &cs, int64_t a, int64_t b) {
  return cps_to_utf8(std::vector<uint32_t>(cs.begin() + a, cs.begin() + b));
}
Chars chars_of(const std::string &s) { return bytes_to_cps((const uint8_t *)s.data(), s.size()); }

/* ---------- src/json.br ---------- */
bool is_json_ws(uint32_t c) { return c == ' ' || c == '\n' || c == '\t' || c == '\r'; }
int64_t json_skip_ws(const Chars &cs, int64_t p) {
  while (p < (int64_t)cs.size() && is_json_ws(cs[p])) p++;
  return p;
}
int64_t json_hex_val(uint32_t c) {
  if (c >= '0' && c <= '9') return c - '0';
  if (c >= 'a' && c <= 'f') return c - 'a' + 10;
  if (c >= 'A' && c <= 'F') return c - 'A' + 10;
  throw std::runtime_error("json: invalid hex digit '" + utf8(c) + "' in \\u escape");
}
int64_t json_hex4(const Chars &cs, int64_t pos) {
  if (!(pos + 4 <= (int64_t)cs.size())) throw std::runtime_error("json: truncated \\u escape");
  int64_t v = 0;
  for (int i = 0; i < 4; i++) v = v * 16 + json_hex_val(cs[pos + i]);
  return v;
}
std::string json_parse_string(const Chars &cs, int64_t pos, int64_t &end) {
  std::string out;
  int64_t p = pos + 1, n = (int64_t)cs.size();
  while (true) {
    if (!(p < n)) throw std::runtime_error("json: unterminated string");
    uint32_t ch = cs[p];
    if (ch == '"') {
      end = p + 1;
      return out;
    } else if (ch == '\\') {
      if (!(p + 1 < n)) throw std::runtime_error("json: truncated escape");
      uint32_t e = cs[p + 1];
      if (e == 'n') { out += "\n"; p += 2; }
      else if (e == 't') { out += "\t"; p += 2; }
      else if (e == 'r') { out += "\r"; p += 2; }
      else if (e == 'b') { out += utf8(8); p += 2; }
      else if (e == 'f') { out += utf8(12); p += 2; }
      else if (e == 'u') {
        int64_t cp = json_hex4(cs, p + 2);
        p += 6;
        if (cp >= 0xD800 && cp <= 0xDBFF) {
          if (!(p + 1 < n && cs[p] == '\\' && cs[p + 1] == 'u'))
            throw std::runtime_error("json: high surrogate without a low surrogate");
          int64_t lo = json_hex4(cs, p + 2);
          if (!(lo >= 0xDC00 && lo <= 0xDFFF)) throw std::runtime_error("json: invalid low surrogate");
          cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          p += 6;
        } else if (cp >= 0xDC00 && cp <= 0xDFFF) {
          throw std::runtime_error("json: low surrogate without a high surrogate");
        }
        out += utf8((uint32_t)cp);
      } else if (e == '"' || e == '\\' || e == '/') {
        out += utf8(e);
        p += 2;
      } else {
        throw std::runtime_error("json: invalid escape '\\" + utf8(e) + "'");
      }
    } else {
      if (!(ch >= 0x20)) throw std::runtime_error("json: unescaped control character in string");
      out += utf8(ch);
      p += 1;
    }
  }
}
JPtr json_parse_number(const Chars &cs, int64_t pos, int64_t &end) {
  bool is_float = false;
  int64_t p = pos, n = (int64_t)cs.size();
  auto digit = [&](int64_t q) { return q < n && cs[q] >= '0' && cs[q] <= '9'; };
  if (p < n && cs[p] == '-') p++;
  if (!(p < n)) throw std::runtime_error("json: truncated number");
  if (cs[p] == '0') p++;
  else if (cs[p] >= '1' && cs[p] <= '9') {
    p++;
    while (digit(p)) p++;
  } else throw std::runtime_error("json: invalid number at " + std::to_string(pos));
  if (p < n && cs[p] == '.') {
    is_float = true;
    p++;
    if (!digit(p)) throw std::runtime_error("json: expected digit after decimal point");
    while (digit(p)) p++;
  }
  if (p < n && (cs[p] == 'e' || cs[p] == 'E')) {
    is_float = true;
    p++;
    if (p < n && (cs[p] == '+' || cs[p] == '-')) p++;
    if (!digit(p)) throw std::runtime_error("json: expected exponent digits");
    while (digit(p)) p++;
  }
  std::string text = utf8(cs, pos, p);
  end = p;
  auto v = std::make_shared<JValue>();
  if (!is_float) {
    /* `text as int`: i64 parse; overflow falls through to float */
    errno = 0;
    char *e = nullptr;
    long long x = strtoll(text.c_str(), &e, 10);
    if (errno == 0 && e && *e == 0) {
      v->kind = JValue::Int;
      v->n = x;
      return v;
    }
  }
  v->kind = JValue::Float;
  v->f = strtod(text.c_str(), nullptr);
  return v;
}
bool json_has_literal(const Chars &cs, int64_t pos, const char *lit) {
  Chars lc = chars_of(lit);
  if (pos + (int64_t)lc.size() > (int64_t)cs.size()) return false;
  for (size_t i = 0; i < lc.size(); i++)
    if (cs[pos + i] != lc[i]) return false;
  return true;
}
const int JSON_MAX_DEPTH = 128;
JPtr json_parse_value(const Chars &cs, int64_t pos, int depth, int64_t &end) {
  if (!(depth <= JSON_MAX_DEPTH))
    throw std::runtime_error("json: nesting is deeper than " + std::to_string(JSON_MAX_DEPTH) + " levels");
  int64_t p = json_skip_ws(cs, pos), n = (int64_t)cs.size();
  if (!(p < n)) throw std::runtime_error("json: unexpected end of input");
  uint32_t ch = cs[p];
  auto v = std::make_shared<JValue>();
  if (ch == '{') {
    v->kind = JValue::Dict;
    int64_t q = json_skip_ws(cs, p + 1);
    if (q < n && cs[q] == '}') {
      end = q + 1;
      return v;
    }
    while (true) {
      q = json_skip_ws(cs, q);
      if (!(q < n && cs[q] == '"')) throw std::runtime_error("json: expected object key at " + std::to_string(q));
      int64_t after_key;
      std::string key = json_parse_string(cs, q, after_key);
      q = json_skip_ws(cs, after_key);
      if (!(q < n && cs[q] == ':')) throw std::runtime_error("json: expected ':' after key '" + key + "'");
      int64_t after_val;
      JPtr child = json_parse_value(cs, q + 1, depth + 1, after_val);
      if (!v->fields.count(key)) v->keys.push_back(key);
      v->fields[key] = child;
      q = json_skip_ws(cs, after_val);
      if (!(q < n)) throw std::runtime_error("json: unterminated object");
      if (cs[q] == ',') q += 1;
      else if (cs[q] == '}') {
        end = q + 1;
        return v;
      } else throw std::runtime_error("json: expected ',' or '}' at " + std::to_string(q));
    }
  } else if (ch == '[') {
    v->kind = JValue::List;
    int64_t q = json_skip_ws(cs, p + 1);
    if (q < n && cs[q] == ']') {
      end = q + 1;
      return v;
    }
    while (true) {
      int64_t after_val;
      v->items.push_back(json_parse_value(cs, q, depth + 1, after_val));
      q = json_skip_ws(cs, after_val);
      if (!(q < n)) throw std::runtime_error("json: unterminated array");
      if (cs[q] == ',') q += 1;
      else if (cs[q] == ']') {
        end = q + 1;
        return v;
      } else throw std::runtime_error("json: expected ',' or ']' at " + std::to_string(q));
    }
  } else if (ch == '"') {
    v->kind = JValue::Str;
    v->s = json_parse_string(cs, p, end);
    return v;
  } else if (json_has_literal(cs, p, "true")) {
    v->kind = JValue::Bool;
    v->b = true;
    end = p + 4;
    return v;
  } else if (json_has_literal(cs, p, "false")) {
    v->kind = JValue::Bool;
    end = p + 5;
    return v;
  } else if (json_has_literal(cs, p, "null")) {
    end = p + 4;
    return v; /* JUndefined */
  }
  return json_parse_number(cs, p, end);
}
JPtr json_parse(const std::string &src) {
  Chars cs = chars_of(src);
  int64_t end;
  JPtr v = json_parse_value(cs, 0, 0, end);
  int64_t tail = json_skip_ws(cs, end);
  if (tail != (int64_t)cs.size()) throw std::runtime_error("json: trailing characters at " + std::to_string(tail));
  return v;
}
JPtr json_get(const JPtr &v, const std::string &key) {
  if (v->kind != JValue::Dict) return undefined();
  auto it = v->fields.find(key);
  return it == v->fields.end() ? undefined() : it->second;
}
std::string json_get_str(const JPtr &v, const std::string &key, const std::string &fallback) {
  JPtr x = json_get(v, key);
  return x->kind == JValue::Str ? x->s : fallback;
}
int64_t json_get_int(const JPtr &v, const std::string &key, int64_t fallback) {
  JPtr x = json_get(v, key);
  if (x->kind == JValue::Int) return x->n;
  if (x->kind == JValue::Float) return (int64_t)x->f; /* Rust `as int` */
  return fallback;
}

/* ---------- src/jinja.br:196-248 ---------- */
std::string hex4(int64_t n) {
  const char *d = "0123456789abcdef";
  std::string s;
  s += d[(n >> 12) & 15];
  s += d[(n >> 8) & 15];
  s += d[(n >> 4) & 15];
  s += d[n & 15];
  return s;
}
std::string json_escape(const std::string &s) {
  std::string out;
  for (uint32_t ch : chars_of(s)) {
    if (ch == '"') out += "\\\"";
    else if (ch == '\\') out += "\\\\";
    else if (ch == '\n') out += "\\n";
    else if (ch == '\r') out += "\\r";
    else if (ch == '\t') out += "\\t";
    else if (ch < 32) out += "\\u" + hex4(ch);
    else out += utf8(ch);
  }
  return out;
}
/* Rust `{}` Display of f64: shortest round-trip digits, plain decimal notation */
std::string rust_f64(double f) {
  if (f != f) return "NaN";
  if (f == 1.0 / 0.0) return "inf";
  if (f == -1.0 / 0.0) return "-inf";
  char buf[64];
  int prec = 0;
  for (; prec < 17; prec++) {
    snprintf(buf, sizeof buf, "%.*e", prec, f);
    if (strtod(buf, nullptr) == f) break;
  }
  /* buf = [-]d.ddde[+-]xx */
  std::string s(buf);
  bool neg = s[0] == '-';
  if (neg) s = s.substr(1);
  size_t epos = s.find('e');
  int exp10 = atoi(s.c_str() + epos + 1);
  std::string digits;
  for (size_t i = 0; i < epos; i++)
    if (s[i] != '.') digits += s[i];
  int point = 1 + exp10; /* position of decimal point within digits */
  std::string out;
  if (point <= 0) out = "0." + std::string(-point, '0') + digits;
  else if (point >= (int)digits.size()) out = digits + std::string(point - digits.size(), '0');
  else out = digits.substr(0, point) + "." + digits.substr(point);
  while (out.find('.') != std::string::npos && (out.back() == '0')) out.pop_back();
  if (!out.empty() && out.back() == '.') out.pop_back();
  return (neg ? "-" : "") + out;
}
std::string jv_to_json(const JPtr &v) {
  switch (v->kind) {
    case JValue::Str: return "\"" + json_escape(v->s) + "\"";
    case JValue::Int: return std::to_string(v->n);
    case JValue::Float: return rust_f64(v->f);
    case JValue::Bool: return v->b ? "true" : "false";
    case JValue::Undefined: return "null";
    case JValue::List: {
      std::string out = "[";
      for (size_t i = 0; i < v->items.size(); i++) {
        if (i > 0) out += ", ";
        out += jv_to_json(v->items[i]);
      }
      return out + "]";
    }
    case JValue::Dict: {
      std::string out = "{";
      for (size_t i = 0; i < v->keys.size(); i++) {
        if (i > 0) out += ", ";
        const std::string &k = v->keys[i];
        auto it = v->fields.find(k);
        JPtr child = it == v->fields.end() ? undefined() : it->second;
        out += "\"" + json_escape(k) + "\": " + jv_to_json(child);
      }
      return out + "}";
    }
  }
  return "null";
}

/* ---------- src/schema_grammar.br ---------- */
struct SchemaGrammar {
  JPtr root;
  std::map<std::string, std::string> rules;
  std::vector<std::string> order;
  std::map<std::string, std::string> ref_rules;
};

/* :21 */
const char *SPACE_RULE = "| \" \" | \"\\n\"{1,2} [ \\t]{0,20}";

/* :23-34 */
std::string sanitize_name(const std::string &raw) {
  std::string out;
  for (uint32_t c : chars_of(raw)) {
    if ((c >= 48 && c <= 57) || (c >= 65 && c <= 90) || (c >= 97 && c <= 122)) out += (char)c;
    else out += "-";
  }
  return out.empty() ? "x" : out;
}
/* :36-46 */
std::string add_rule(SchemaGrammar &g, const std::string &hint, const std::string &body) {
  std::string base = sanitize_name(hint);
  std::string name = base;
  int64_t n = 0;
  while (g.rules.count(name) && g.rules[name] != body) {
    n += 1;
    name = base + "-" + std::to_string(n);
  }
  if (!g.rules.count(name)) {
    g.rules[name] = body;
    g.order.push_back(name);
  }
  return name;
}
/* :49-65 */
std::string gbnf_literal(const std::string &text) {
  std::string out = "\"";
  for (uint32_t c : chars_of(text)) {
    if (c == 34) out += "\\\"";
    else if (c == 92) out += "\\\\";
    else if (c == 10) out += "\\n";
    else if (c == 13) out += "\\r";
    else if (c == 9) out += "\\t";
    else out += utf8(c);
  }
  return out + "\"";
}
/* :68-69 */
std::string json_value_literal(const JPtr &v) { return gbnf_literal(jv_to_json(v)); }
/* :71-78 */
std::string drop_prefix(const std::string &text, size_t n) {
  Chars cs = chars_of(text);
  if (n >= cs.size()) return "";
  return utf8(cs, (int64_t)n, (int64_t)cs.size());
}
bool is_defined(const JPtr &v) { return v->kind != JValue::Undefined; }
bool is_list(const JPtr &v) { return v->kind == JValue::List; }
bool is_dict(const JPtr &v) { return v->kind == JValue::Dict; }
std::vector<std::string> string_items(const JPtr &v) {
  std::vector<std::string> out;
  if (v->kind == JValue::List)
    for (auto &it : v->items) out.push_back(it->kind == JValue::Str ? it->s : "");
  return out;
}
std::vector<std::string> dict_keys(const JPtr &v) { return v->kind == JValue::Dict ? v->keys : std::vector<std::string>{}; }
int64_t int_or(const JPtr &v, int64_t fallback) { return v->kind == JValue::Int ? v->n : fallback; }

std::vector<std::string> split(const std::string &s, char sep) {
  std::vector<std::string> out;
  size_t a = 0;
  while (true) {
    size_t b = s.find(sep, a);
    if (b == std::string::npos) {
      out.push_back(s.substr(a));
      return out;
    }
    out.push_back(s.substr(a, b - a));
    a = b + 1;
  }
}
/* :80-92 */
JPtr resolve_ref(const JPtr &root, const std::string &ref_text) {
  if (ref_text.rfind("#", 0) != 0) throw std::runtime_error("only local $ref values are supported (got '" + ref_text + "')");
  JPtr node = root;
  std::string path = drop_prefix(ref_text, 1);
  if (path.empty()) return node;
  if (path.rfind("/", 0) != 0) throw std::runtime_error("unsupported $ref '" + ref_text + "'");
  for (const std::string &part : split(drop_prefix(path, 1), '/')) {
    JPtr next = json_get(node, part);
    if (!is_defined(next)) throw std::runtime_error("$ref '" + ref_text + "' does not resolve");
    node = next;
  }
  return node;
}
/* :132-137 */
bool schema_allows_extra(const JPtr &schema) {
  JPtr extra = json_get(schema, "additionalProperties");
  if (extra->kind == JValue::Bool) return extra->b;
  return extra->kind == JValue::Dict;
}
std::string join(const std::vector<std::string> &v, const std::string &sep) {
  std::string out;
  for (size_t i = 0; i < v.size(); i++) {
    if (i) out += sep;
    out += v[i];
  }
  return out;
}

std::string visit(SchemaGrammar &g, const JPtr &schema, const std::string &name);

/* :139-144 */
std::string extra_value_rule(SchemaGrammar &g, const JPtr &schema, const std::string &name) {
  JPtr extra = json_get(schema, "additionalProperties");
  if (is_dict(extra)) return visit(g, extra, name + "-additional");
  return "value";
}

/* :146-196 */
std::string object_rule(SchemaGrammar &g, const JPtr &schema, const std::string &name) {
  std::vector<std::string> req_kv, opt_kv;
  std::vector<std::string> required = string_items(json_get(schema, "required"));
  std::vector<std::string> keys = dict_keys(json_get(schema, "properties"));
  JPtr props = json_get(schema, "properties");
  for (bool want_required : {true, false}) {
    for (const std::string &k : keys) {
      bool is_req = std::find(required.begin(), required.end(), k) != required.end();
      if (is_req == want_required) {
        std::string child = visit(g, json_get(props, k), name + "-" + k);
        auto ks = std::make_shared<JValue>();
        ks->kind = JValue::Str;
        ks->s = k;
        std::string kv = add_rule(g, name + "-" + k + "-kv", gbnf_literal(jv_to_json(ks)) + " space \":\" space " + child);
        if (want_required) req_kv.push_back(kv);
        else opt_kv.push_back(kv);
      }
    }
  }
  bool extra = schema_allows_extra(schema);
  std::string extra_kv;
  if (extra) {
    std::string extra_child = extra_value_rule(g, schema, name);
    extra_kv = add_rule(g, name + "-additional-kv", "string \":\" space " + extra_child);
  }
  std::string body = "\"{\" space ";
  if (!req_kv.empty()) {
    std::string inner = req_kv[0];
    for (size_t i = 1; i < req_kv.size(); i++) inner += " \",\" space " + req_kv[i];
    for (const std::string &o : opt_kv) inner += " (\",\" space " + o + ")?";
    if (extra) inner += " (\",\" space " + extra_kv + ")*";
    body += inner + " ";
  } else if (!opt_kv.empty() || extra) {
    if (!(opt_kv.size() <= 128))
      throw std::runtime_error("an object with more than 128 optional properties and no required one is not supported");
    std::vector<std::string> alts;
    for (size_t i = 0; i < opt_kv.size(); i++) {
      std::string alt = opt_kv[i];
      for (size_t j = i + 1; j < opt_kv.size(); j++) alt += " (\",\" space " + opt_kv[j] + ")?";
      if (extra) alt += " (\",\" space " + extra_kv + ")*";
      alts.push_back(alt);
    }
    if (extra) alts.push_back(extra_kv + " (\",\" space " + extra_kv + ")*");
    body += "(" + join(alts, " | ") + ")? ";
  }
  return body + "\"}\" space";
}

/* :198-216 */
std::string array_rule(SchemaGrammar &g, const JPtr &schema, const std::string &name) {
  JPtr items = json_get(schema, "items");
  std::string item = is_dict(items) ? visit(g, items, name + "-item") : "value";
  int64_t min = json_get_int(schema, "minItems", 0);
  int64_t max = int_or(json_get(schema, "maxItems"), -1);
  if (!(max < 0 || max >= min)) throw std::runtime_error("maxItems is smaller than minItems");
  if (max == 0) return "\"[\" space \"]\" space";
  std::string inner = item;
  if (min > 1 || max > 1 || max < 0) {
    int64_t more_min = min > 1 ? min - 1 : 0;
    if (max < 0) inner = item + " (\",\" space " + item + "){" + std::to_string(more_min) + ",}";
    else inner = item + " (\",\" space " + item + "){" + std::to_string(more_min) + "," + std::to_string(max - 1) + "}";
  }
  if (min == 0) return "\"[\" space (" + inner + ")? \"]\" space";
  return "\"[\" space " + inner + " \"]\" space";
}

std::string visit_type(SchemaGrammar &g, const JPtr &schema, const std::string &type_name, const std::string &name);

/* :218-270 */
std::string visit(SchemaGrammar &g, const JPtr &schema, const std::string &name) {
  if (!is_dict(schema)) {
    if (schema->kind == JValue::Bool) return "value";
    throw std::runtime_error("a schema must be an object or a boolean");
  }
  std::string ref_text = json_get_str(schema, "$ref", "");
  if (!ref_text.empty()) {
    auto it = g.ref_rules.find(ref_text);
    if (it != g.ref_rules.end()) return it->second;
    std::string ref_name = sanitize_name("ref-" + ref_text);
    g.ref_rules[ref_text] = ref_name;
    g.rules[ref_name] = "value";
    g.order.push_back(ref_name);
    std::string target = visit(g, resolve_ref(g.root, ref_text), ref_name);
    g.rules[ref_name] = target;
    return ref_name;
  }
  JPtr const_value = json_get(schema, "const");
  if (is_defined(const_value)) return add_rule(g, name, json_value_literal(const_value));
  JPtr en = json_get(schema, "enum");
  if (is_list(en)) {
    if (en->items.empty()) throw std::runtime_error("enum must not be empty");
    std::vector<std::string> lits;
    for (auto &o : en->items) lits.push_back(json_value_literal(o));
    return add_rule(g, name, "(" + join(lits, " | ") + ") space");
  }
  std::vector<std::string> alt_rules;
  bool combined = false;
  for (const char *key : {"anyOf", "oneOf"}) {
    JPtr lst = json_get(schema, key);
    if (is_list(lst)) {
      int64_t i = 0;
      for (auto &a : lst->items) {
        alt_rules.push_back(visit(g, a, name + "-" + std::to_string(i)));
        i += 1;
      }
      combined = true;
    }
  }
  if (combined) return add_rule(g, name, join(alt_rules, " | "));
  std::vector<std::string> types;
  JPtr t = json_get(schema, "type");
  if (t->kind == JValue::Str) types.push_back(t->s);
  else types = string_items(t);
  if (types.empty()) {
    if (is_dict(json_get(schema, "properties"))) types.push_back("object");
    else return "value";
  }
  if (types.size() > 1) {
    std::vector<std::string> parts;
    for (const std::string &ty : types) parts.push_back(visit_type(g, schema, ty, name + "-" + ty));
    return add_rule(g, name, join(parts, " | "));
  }
  return visit_type(g, schema, types[0], name);
}

/* :272-296 */
std::string visit_type(SchemaGrammar &g, const JPtr &schema, const std::string &type_name, const std::string &name) {
  if (type_name == "object") return add_rule(g, name, object_rule(g, schema, name));
  if (type_name == "array") return add_rule(g, name, array_rule(g, schema, name));
  if (type_name == "string") {
    int64_t min = json_get_int(schema, "minLength", 0);
    int64_t max = int_or(json_get(schema, "maxLength"), -1);
    if (min == 0 && max < 0) return "string";
    std::string upper = max < 0 ? "" : std::to_string(max);
    return add_rule(g, name, "\"\\\"\" char{" + std::to_string(min) + "," + upper + "} \"\\\"\" space");
  }
  if (type_name == "integer") return "integer";
  if (type_name == "number") return "number";
  if (type_name == "boolean") return "boolean";
  if (type_name == "null") return "null";
  throw std::runtime_error("unsupported schema type '" + type_name + "'");
}

/* :300-310 */
std::string without_trailing_space(const std::string &body) {
  const std::string suf = " space";
  if (body.size() < suf.size() || body.compare(body.size() - suf.size(), suf.size(), suf) != 0) return body;
  return body.substr(0, body.size() - suf.size());
}

}  // namespace

/* :313-337 */
std::string json_schema_to_gbnf(const std::string &schema_json) {
  SchemaGrammar g;
  g.root = json_parse(schema_json);
  std::string top = visit(g, g.root, "root");
  std::string out;
  if (top == "root") out = "root ::= " + without_trailing_space(g.rules["root"]) + "\n";
  else out = "root ::= " + top + "\n";
  for (const std::string &name : g.order)
    if (name != "root") out += name + " ::= " + g.rules[name] + "\n";
  std::string prims = std::string("space ::= ") + SPACE_RULE + "\n";
  prims += "boolean ::= (\"true\" | \"false\") space\n";
  prims += "decimal-part ::= [0-9]{1,16}\n";
  prims += "integral-part ::= [0] | [1-9] [0-9]{0,15}\n";
  prims += "number ::= (\"-\"? integral-part) (\".\" decimal-part)? ([eE] [-+]? integral-part)? space\n";
  prims += "integer ::= (\"-\"? integral-part) space\n";
  prims += "null ::= \"null\" space\n";
  prims += "char ::= [^\"\\\\\\x7F\\x00-\\x1F] | [\\\\] ([\"\\\\bfnrt] | \"u\" [0-9a-fA-F]{4})\n";
  prims += "string ::= \"\\\"\" char* \"\\\"\" space\n";
  prims += "value ::= object | array | string | number | boolean | null\n";
  prims += "object ::= \"{\" space ( string \":\" space value (\",\" space string \":\" space value)* )? \"}\" space\n";
  prims += "array ::= \"[\" space ( value (\",\" space value)* )? \"]\" space\n";
  return out + prims;
}

} /* namespace orc */
