/*
 * bl_grammar.h — host-side GBNF compiler of libbl_select: grammar text -> the stack-set automaton whose
 * tables the mask and commit kernels walk on the device.
 *
 * Language and errors are those of the reference's src/grammar.br: the GBNF syntax and its limits
 * (:39-41, :57-323), the stack-machine frontier (expand_stacks :343-376, with its 20,000-stack guard
 * :354), advance by one code point (:384-404) and the trailing-U+FFFD rule of grammar_advance_text
 * (:406-437). The automaton's states are the distinct frontiers reachable from `root`; its alphabet is
 * the partition of the code points into classes that no character set of the grammar tells apart.
 */
#ifndef BL_GRAMMAR_H
#define BL_GRAMMAR_H

#include <stdint.h>

#include <string>
#include <vector>

#include "bl_gwalk.h"


struct bl_gram_tables {
  int32_t n_states = 0, n_classes = 0, start = 0;
  std::vector<int32_t> trans;     /* [n_states][n_classes] */
  std::vector<uint8_t> flags;     /* [n_states] */
  std::vector<uint16_t> ascii;    /* class of code points 0..127 */
  std::vector<uint32_t> ivl_lo;   /* classes of code points >= 128: interval starts, ascending (first = 128) */
  std::vector<uint16_t> ivl_cls;
  int32_t start_error = 0;        /* the start frontier itself hit the guard */
};

/* Compiles `gbnf`. Returns 0, or a negative BL_* code with `err` set to the reference's message
 * (BL_EGRAMMAR for parse errors, BL_EGRAMMAR_AMBIG, BL_EUNSUPPORTED when the automaton exceeds
 * `max_states` states, which only a recursive grammar reachable from root does). */
int bl_gram_compile(const std::string &gbnf, int max_states, bl_gram_tables &out, std::string &err);

/* Host walks over the tables (the device kernels implement the same functions). */
int32_t bl_gram_class(const bl_gram_tables &g, uint32_t cp);
/* lossy UTF-8 decoding of src/io.br:70-115 */
void bl_utf8_decode(const uint8_t *b, size_t n, std::vector<uint32_t> &out);

#endif /* BL_GRAMMAR_H */
