/*
 * bl_gwalk.h — walks of the grammar automaton, shared by the device kernels and the host (one
 * definition: the host uses it to set up a slot's state from its reply).
 *
 * The reference re-decodes the whole reply every step (src/server.br:312-351): the frontier is
 * grammar_advance_text(start, chars) with chars = bytes_to_str(reply) minus one trailing U+FFFD, and a
 * candidate T is allowed when grammar_advance_text(frontier, piece) is not empty, piece being what
 * bytes_to_str(reply ++ T) adds after those chars. A slot keeps instead:
 *   carry  the reply's last bytes that a following token can still re-decode: from the last lead byte
 *          C2..F4 that has fewer continuation bytes than it needs, or else the last byte when the decoded
 *          reply ends in U+FFFD (at most 3 bytes);
 *   zk     the frontier after plainly consuming every code point before the carry's (the carry's m =
 *          |carry| code points are all U+FFFD);
 *   zk1, last  the frontier before the last of those code points, and that code point (none at start).
 * Then frontier = (m >= 2) ? trail(zk advanced by m-2 U+FFFD) : (no code point ? start :
 * last == U+FFFD ? trail(zk1) : zk), and piece(T) = decode(carry ++ T) without its first m-1 code
 * points. Committing T decodes carry ++ T, finds the new carry, and plainly advances zk over the code
 * points that leave the carry region. "plainly" = grammar_advance per code point (src/grammar.br:394-404);
 * trail(s) = the trailing-U+FFFD rule of grammar_advance_text (:425-437).
 */
#ifndef BL_GWALK_H
#define BL_GWALK_H

#include <stdint.h>

#include "bl_exact.h" /* BL_SD */

#define BL_GW_NONE 0xFFFFFFFFu /* no code point before the carry */
#define BL_GW_FFFD 0xFFFDu

/* one compiled grammar: device or host pointers */
struct bl_gram_view {
  const int32_t *trans;   /* [n_states][n_classes]; < 0: dead (-1) / guard hit (-2) */
  const uint8_t *flags;   /* [n_states] BL_GS_* */
  const uint16_t *ascii;  /* [128] */
  const uint32_t *ivl_lo; /* [n_ivl], first = 128 */
  const uint16_t *ivl_cls;
  int32_t n_ivl, n_classes, start, pad;
};

/* a slot's grammar position (see above) */
struct bl_gram_pos {
  int32_t zk, zk1;
  uint32_t last;
  uint32_t carry; /* bytes little-endian */
  int32_t ncarry;
};

/* state flags */
#define BL_GS_COMPLETE 1u /* a stack of the frontier is empty (grammar_complete, src/grammar.br:439-445) */
#define BL_GS_CONTINUE 2u /* a stack is non-empty (grammar_can_continue, :447-451) */
#define BL_GS_NONASCII 4u /* the frontier accepts a trailing U+FFFD (grammar_allows_non_ascii, :408-420) */
/* transition targets below 0 */
#define BL_GT_DEAD (-1)   /* empty frontier */
#define BL_GT_AMBIG (-2)  /* the expansion hit the reference's 20,000-stack guard */

BL_SD int32_t bl_gw_class(const bl_gram_view &g, uint32_t cp) {
  if (cp < 128) return g.ascii[cp];
  int lo = 0, hi = g.n_ivl;
  while (hi - lo > 1) {
    int mid = (lo + hi) >> 1;
    if (g.ivl_lo[mid] <= cp) lo = mid;
    else hi = mid;
  }
  return g.ivl_cls[lo];
}

/* grammar_advance: s < 0 stays */
BL_SD int32_t bl_gw_step(const bl_gram_view &g, int32_t s, uint32_t cp) {
  if (s < 0) return s;
  return g.trans[(int64_t)s * g.n_classes + bl_gw_class(g, cp)];
}

/* trailing U+FFFD of grammar_advance_text: kept when the frontier allows non-ASCII, else empty */
BL_SD int32_t bl_gw_trail(const bl_gram_view &g, int32_t s) {
  if (s < 0) return s;
  return (g.flags[s] & BL_GS_NONASCII) ? s : -1;
}

BL_SD bool bl_gw_cont(uint32_t b) { return (b & 0xC0u) == 0x80u; }

/* one code point of bytes_to_str (src/io.br:70-115) starting at byte i of the n bytes get(0..n-1);
 * advances i */
template <class Get>
BL_SD uint32_t bl_gw_decode(Get get, int n, int &i) {
  uint32_t b0 = get(i);
  if (b0 < 0x80u) {
    i += 1;
    return b0;
  }
  if (b0 >= 0xC2u && b0 <= 0xDFu) {
    if (i + 1 < n) {
      uint32_t b1 = get(i + 1);
      if (bl_gw_cont(b1)) {
        i += 2;
        return ((b0 & 0x1Fu) << 6) | (b1 & 0x3Fu);
      }
    }
  } else if (b0 >= 0xE0u && b0 <= 0xEFu) {
    if (i + 2 < n) {
      uint32_t b1 = get(i + 1), b2 = get(i + 2);
      if (bl_gw_cont(b1) && bl_gw_cont(b2)) {
        uint32_t c = ((b0 & 0x0Fu) << 12) | ((b1 & 0x3Fu) << 6) | (b2 & 0x3Fu);
        if (c >= 0x800u && !(c >= 0xD800u && c <= 0xDFFFu)) {
          i += 3;
          return c;
        }
      }
    }
  } else if (b0 >= 0xF0u && b0 <= 0xF4u) {
    if (i + 3 < n) {
      uint32_t b1 = get(i + 1), b2 = get(i + 2), b3 = get(i + 3);
      if (bl_gw_cont(b1) && bl_gw_cont(b2) && bl_gw_cont(b3)) {
        uint32_t c = ((b0 & 0x07u) << 18) | ((b1 & 0x3Fu) << 12) | ((b2 & 0x3Fu) << 6) | (b3 & 0x3Fu);
        if (c >= 0x10000u && c <= 0x10FFFFu) {
          i += 4;
          return c;
        }
      }
    }
  }
  i += 1;
  return BL_GW_FFFD;
}

BL_SD uint32_t bl_gw_carry_byte(const bl_gram_pos &p, int k) { return (p.carry >> (8 * k)) & 0xFFu; }

/* the frontier candidates are walked from (grammar_ctx, src/server.br:312-320) */
BL_SD int32_t bl_gw_frontier(const bl_gram_view &g, const bl_gram_pos &p) {
  const int m = p.ncarry;
  if (m >= 2) {
    int32_t s = p.zk;
    for (int k = 0; k < m - 2; k++) s = bl_gw_step(g, s, BL_GW_FFFD);
    return bl_gw_trail(g, s);
  }
  if (p.last == BL_GW_NONE) return g.start;
  if (p.last == BL_GW_FFFD) return bl_gw_trail(g, p.zk1);
  return p.zk;
}

/* grammar_advance_text(frontier, piece(T)) for the token bytes tb[0..nt): returns the final frontier
 * (< 0 when rejected: -1 empty, -2 guard hit) */
template <class TokByte>
BL_SD int32_t bl_gw_walk(const bl_gram_view &g, const bl_gram_pos &p, int32_t frontier, TokByte tb, int nt) {
  const int nc = p.ncarry;
  const int n = nc + nt;
  auto get = [&](int i) -> uint32_t { return i < nc ? bl_gw_carry_byte(p, i) : (uint32_t)tb(i - nc); };
  int skip = nc > 1 ? nc - 1 : 0;
  int32_t s = frontier;
  int i = 0;
  while (i < n && s >= 0) {
    uint32_t cp = bl_gw_decode(get, n, i);
    if (skip > 0) {
      skip--;
      continue;
    }
    if (cp == BL_GW_FFFD && i >= n) s = bl_gw_trail(g, s); /* last code point of the piece */
    else s = bl_gw_step(g, s, cp);
  }
  return s;
}

BL_SD int bl_gw_need(uint32_t b) { return b >= 0xF0u ? 4 : (b >= 0xE0u ? 3 : 2); }

/* reply_tokens.push(T) for a non-EOG token: the new position from carry ++ T */
template <class TokByte>
BL_SD void bl_gw_commit(const bl_gram_view &g, bl_gram_pos &p, TokByte tb, int nt) {
  const bl_gram_pos old = p;
  const int nc = old.ncarry;
  const int n = nc + nt;
  auto get = [&](int i) -> uint32_t { return i < nc ? bl_gw_carry_byte(old, i) : (uint32_t)tb(i - nc); };
  /* an unfinished sequence at the end (a lead byte with fewer continuation bytes than it needs, within
   * the last four bytes) starts the new carry; the bytes before it decode on their own */
  int cstart = n;
  for (int q = n - 1; q >= 0 && q >= n - 4; q--) {
    uint32_t b = get(q);
    if (bl_gw_cont(b)) continue;
    if (b >= 0xC2u && b <= 0xF4u && n - q < bl_gw_need(b)) cstart = q;
    break;
  }
  /* advance over the code points before the carry; each is applied when the next one is known, so the
   * last can stay with the carry when the text ends in U+FFFD */
  int32_t zk = old.zk, zk1 = old.zk1;
  uint32_t last = old.last, pend = BL_GW_NONE;
  int i = 0;
  while (i < cstart) {
    uint32_t cp = bl_gw_decode(get, cstart, i);
    if (pend != BL_GW_NONE) {
      zk1 = zk;
      zk = bl_gw_step(g, zk, pend);
      last = pend;
    }
    pend = cp;
  }
  if (pend != BL_GW_NONE) {
    if (cstart == n && pend == BL_GW_FFFD) {
      cstart = n - 1; /* the text ends in U+FFFD: its last byte is the carry */
    } else {
      zk1 = zk;
      zk = bl_gw_step(g, zk, pend);
      last = pend;
    }
  }
  uint32_t carry = 0;
  for (int q = cstart; q < n; q++) carry |= get(q) << (8 * (q - cstart));
  p.zk = zk;
  p.zk1 = zk1;
  p.last = last;
  p.carry = carry;
  p.ncarry = n - cstart;
}

#endif /* BL_GWALK_H */
