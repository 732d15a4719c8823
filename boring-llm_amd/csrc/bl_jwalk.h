/*
 * bl_jwalk.h — the reference's incremental JSON classifier (json_prefix_state / json_object_prefix_state,
 * src/json.br:227-406) as a pushdown automaton over code points, for `response_format: json_object`
 * (sample_json_token, src/server.br:261-304). Shared by the device kernels and the host (one definition:
 * the host sets a slot's position up from its reply).
 *
 * The reference re-scans the whole decoded reply for every candidate; the classifier is deterministic and
 * left to right, so a slot keeps instead the state after the code points before the reply's unfinished
 * trailing UTF-8 sequence (the carry, as for grammars) and the candidate T is allowed when the state after
 * decode(carry ++ T) is viable. State: the stack of container states (the reference's `states`: 0 root
 * value, 1 object key/end, 2 colon, 3 object value, 4 object comma/end, 5 array value/end, 6 array
 * comma/end, 7 root done) and the lexer's position inside a string, literal or number, whose scanning the
 * reference does in inner loops (a text that ends inside one is viable; a number ends at the first code
 * point that cannot continue it, which is then read as structure).
 */
#ifndef BL_JWALK_H
#define BL_JWALK_H

#include <stdint.h>

#include "bl_gwalk.h"

#define BL_JSON_DEPTH 1024 /* container stack capacity per slot */
#if defined(__HIPCC__)
#define BL_JM __host__ __device__ __forceinline__ /* member functions */
#else
#define BL_JM inline
#endif
#define BL_JLOC 32         /* stack entries a candidate's walk pushes past the slot's stack */

/* lexer modes */
#define BL_JL_NONE 0
#define BL_JL_KSTR 1 /* inside an object key */
#define BL_JL_VSTR 2 /* inside a string value */
#define BL_JL_LIT 3  /* inside true / false / null: sub = word * 8 + next index */
#define BL_JL_NUM 4  /* inside a number: sub = BL_JN_* */
/* number positions */
#define BL_JN_MINUS 0
#define BL_JN_ZERO 1
#define BL_JN_INT 2
#define BL_JN_DOT 3
#define BL_JN_FRAC 4
#define BL_JN_E 5
#define BL_JN_ESIGN 6
#define BL_JN_EXP 7

/* a slot's classifier position; the stack's entries [0, depth) live in the slot's array */
struct bl_json_pos {
  int32_t depth;
  int32_t lex, sub;
  int32_t dead;     /* 1: not viable (-1); 2: the stack outgrew BL_JSON_DEPTH */
  uint32_t carry;   /* the reply's unfinished trailing UTF-8 sequence, bytes little-endian */
  int32_t ncarry;
};

BL_SD bool bl_js_ws(uint32_t c) { return c == ' ' || c == '\n' || c == '\t' || c == '\r'; }
BL_SD bool bl_js_dig(uint32_t c) { return c >= '0' && c <= '9'; }
BL_SD bool bl_js_hex(uint32_t c) { return bl_js_dig(c) || (c >= 'a' && c <= 'f') || (c >= 'A' && c <= 'F'); }
/* the literal words; index 0 is their first letter */
BL_SD uint32_t bl_js_word(int w, int i) {
  const char *s = w == 0 ? "true" : (w == 1 ? "false" : "null");
  return (uint32_t)(unsigned char)s[i];
}

/* a stack read from `base` (entries [0, nbase)) with the entries pushed past it in `loc` */
struct bl_jstack_overlay {
  const uint8_t *base;
  int nbase;
  uint8_t loc[BL_JLOC];
  int nloc;
  bool over;
  BL_JM int size() const { return nbase + nloc; }
  BL_JM int top() const { return nloc > 0 ? loc[nloc - 1] : (nbase > 0 ? base[nbase - 1] : -1); }
  BL_JM void push(int v) {
    if (nloc == BL_JLOC) over = true;
    else loc[nloc++] = (uint8_t)v;
  }
  BL_JM void pop() {
    if (nloc > 0) nloc--;
    else if (nbase > 0) nbase--;
  }
  BL_JM void set_top(int v) {
    if (nloc > 0) {
      loc[nloc - 1] = (uint8_t)v;
    } else {
      pop();
      push(v);
    }
  }
};

/* the slot's own stack (the commit writes it) */
struct bl_jstack_own {
  uint8_t *s;
  int n;
  bool over;
  BL_JM int size() const { return n; }
  BL_JM int top() const { return n > 0 ? s[n - 1] : -1; }
  BL_JM void push(int v) {
    if (n == BL_JSON_DEPTH) over = true;
    else s[n++] = (uint8_t)v;
  }
  BL_JM void pop() {
    if (n > 0) n--;
  }
  BL_JM void set_top(int v) {
    if (n > 0) s[n - 1] = (uint8_t)v;
  }
};

/* one code point of json_prefix_state (src/json.br:233-390); `object`: the root value must be an object
 * (json_object_prefix_state, :394-406). Returns false when the text is no longer viable */
template <class Stk>
BL_SD bool bl_js_step(int &lex, int &sub, Stk &st, uint32_t ch, bool object) {
  if (lex == BL_JL_NUM) {
    const bool dig = bl_js_dig(ch), ex = ch == 'e' || ch == 'E';
    switch (sub) {
    case BL_JN_MINUS:
      if (ch == '0') sub = BL_JN_ZERO;
      else if (ch >= '1' && ch <= '9') sub = BL_JN_INT;
      else return false;
      return true;
    case BL_JN_DOT:
      if (!dig) return false;
      sub = BL_JN_FRAC;
      return true;
    case BL_JN_E:
      if (ch == '+' || ch == '-') sub = BL_JN_ESIGN;
      else if (dig) sub = BL_JN_EXP;
      else return false;
      return true;
    case BL_JN_ESIGN:
      if (!dig) return false;
      sub = BL_JN_EXP;
      return true;
    case BL_JN_ZERO:
      if (ch == '.') {
        sub = BL_JN_DOT;
        return true;
      }
      if (ex) {
        sub = BL_JN_E;
        return true;
      }
      break;
    case BL_JN_INT:
      if (dig) return true;
      if (ch == '.') {
        sub = BL_JN_DOT;
        return true;
      }
      if (ex) {
        sub = BL_JN_E;
        return true;
      }
      break;
    case BL_JN_FRAC:
      if (dig) return true;
      if (ex) {
        sub = BL_JN_E;
        return true;
      }
      break;
    default: /* BL_JN_EXP */
      if (dig) return true;
      break;
    }
    lex = BL_JL_NONE; /* the number ended: the code point is structure */
  } else if (lex == BL_JL_KSTR || lex == BL_JL_VSTR) {
    if (sub == 0) {
      if (ch == '"') {
        if (lex == BL_JL_KSTR) st.set_top(2);
        lex = BL_JL_NONE;
      } else if (ch == '\\') {
        sub = 1;
      } else if (ch < 0x20u) {
        return false;
      }
    } else if (sub == 1) {
      if (ch == 'u') sub = 2;
      else if (ch == '"' || ch == '\\' || ch == '/' || ch == 'b' || ch == 'f' || ch == 'n' || ch == 'r' || ch == 't')
        sub = 0;
      else return false;
    } else {
      if (!bl_js_hex(ch)) return false;
      sub = sub == 5 ? 0 : sub + 1;
    }
    return true;
  } else if (lex == BL_JL_LIT) {
    const int w = sub >> 3, i = sub & 7;
    if (ch != bl_js_word(w, i)) return false;
    if (bl_js_word(w, i + 1) == 0u) lex = BL_JL_NONE;
    else sub = w * 8 + i + 1;
    return true;
  }
  if (bl_js_ws(ch)) return true;
  const int state = st.top();
  if (state == 7 || state < 0) return false;
  if (state == 2) {
    if (ch != ':') return false;
    st.set_top(3);
  } else if (state == 4 || state == 6) {
    if (ch == ',') st.set_top(state == 4 ? 1 : 5);
    else if (ch == (state == 4 ? (uint32_t)'}' : (uint32_t)']')) st.pop();
    else return false;
  } else if (state == 1) {
    if (ch == '}') st.pop();
    else if (ch == '"') {
      lex = BL_JL_KSTR;
      sub = 0;
    } else return false;
  } else if (ch == ']' && state == 5) {
    st.pop();
  } else {
    if (object && state == 0 && ch != '{') return false;
    st.set_top(state == 0 ? 7 : (state == 3 ? 4 : 6));
    if (ch == '{') st.push(1);
    else if (ch == '[') st.push(5);
    else if (ch == '"') {
      lex = BL_JL_VSTR;
      sub = 0;
    } else if (ch == 't' || ch == 'f' || ch == 'n') {
      lex = BL_JL_LIT;
      sub = (ch == 't' ? 0 : (ch == 'f' ? 1 : 2)) * 8 + 1;
    } else if (ch == '-') {
      lex = BL_JL_NUM;
      sub = BL_JN_MINUS;
    } else if (ch == '0') {
      lex = BL_JL_NUM;
      sub = BL_JN_ZERO;
    } else if (ch >= '1' && ch <= '9') {
      lex = BL_JL_NUM;
      sub = BL_JN_INT;
    } else return false;
  }
  if (st.size() == 0) st.push(7); /* a closed top-level container is a complete root value */
  return true;
}

/* the decoded reply is a complete object (json_object_prefix_state == 1): nothing unfinished */
BL_SD bool bl_js_complete(const bl_json_pos &p, int top) {
  return p.dead == 0 && p.ncarry == 0 && p.depth == 1 && top == 7 && p.lex == BL_JL_NONE;
}

/* json_object_decoded_candidate_allowed for token bytes tb[0..nt) (src/json.br:420-426): the state after
 * decode(carry ++ T) is viable. *over: the walk outgrew its overlay (undecided) */
template <class TokByte>
BL_SD bool bl_js_walk(const bl_json_pos &p, const uint8_t *stack, TokByte tb, int nt, bool *over) {
  *over = false;
  if (p.dead) return false;
  bl_jstack_overlay st;
  st.base = stack;
  st.nbase = p.depth;
  st.nloc = 0;
  st.over = false;
  int lex = p.lex, sub = p.sub;
  const int nc = p.ncarry, n = nc + nt;
  auto get = [&](int i) -> uint32_t { return i < nc ? (p.carry >> (8 * i)) & 0xFFu : (uint32_t)tb(i - nc); };
  int i = 0;
  while (i < n) {
    const uint32_t cp = bl_gw_decode(get, n, i);
    if (!bl_js_step(lex, sub, st, cp, true)) return false;
    if (st.over) {
      *over = true;
      return false;
    }
  }
  return true;
}

/* reply_tokens.push(T) (src/server.br:1037): the code points before the new carry advance the position */
template <class TokByte>
BL_SD void bl_js_commit(bl_json_pos &p, uint8_t *stack, TokByte tb, int nt) {
  const bl_json_pos old = p;
  const int nc = old.ncarry, n = nc + nt;
  auto get = [&](int i) -> uint32_t { return i < nc ? (old.carry >> (8 * i)) & 0xFFu : (uint32_t)tb(i - nc); };
  int cstart = n;
  for (int q = n - 1; q >= 0 && q >= n - 4; q--) {
    const uint32_t b = get(q);
    if (bl_gw_cont(b)) continue;
    if (b >= 0xC2u && b <= 0xF4u && n - q < bl_gw_need(b)) cstart = q;
    break;
  }
  bl_jstack_own st;
  st.s = stack;
  st.n = old.depth;
  st.over = false;
  int lex = old.lex, sub = old.sub, dead = old.dead;
  int i = 0;
  while (i < cstart && dead == 0) {
    const uint32_t cp = bl_gw_decode(get, cstart, i);
    if (!bl_js_step(lex, sub, st, cp, true)) dead = 1;
    else if (st.over) dead = 2;
  }
  uint32_t carry = 0;
  for (int q = cstart; q < n; q++) carry |= get(q) << (8 * (q - cstart));
  p.depth = st.n;
  p.lex = lex;
  p.sub = sub;
  p.dead = dead;
  p.carry = carry;
  p.ncarry = n - cstart;
}

/* the position of an empty reply */
BL_SD void bl_js_start(bl_json_pos &p, uint8_t *stack) {
  stack[0] = 0;
  p.depth = 1;
  p.lex = BL_JL_NONE;
  p.sub = 0;
  p.dead = 0;
  p.carry = 0u;
  p.ncarry = 0;
}

#endif /* BL_JWALK_H */
