/* Host build of boring-llm_amd/csrc/bl_jwalk.h for tests/test_jwalk.py: the reply's position after
 * committing tokens one at a time, and the allowed predicate of a candidate after them. */
#include <stdint.h>
#include <string.h>

#include "../../boring-llm_amd/csrc/bl_jwalk.h"

extern "C" {
/* tokens: n tokens of lens[i] bytes concatenated in `bytes`. Commits tokens [0, n-1) and walks token
 * n-1 from there: returns 1 allowed, 0 not, -1 the walk outgrew its overlay; *complete = the committed
 * reply is a complete object; *dead = the committed position's dead flag */
int jw_check(const uint8_t *bytes, const int32_t *lens, int n, int *complete, int *dead) {
  static uint8_t stack[BL_JSON_DEPTH];
  bl_json_pos p;
  bl_js_start(p, stack);
  int at = 0;
  for (int k = 0; k + 1 < n; k++) {
    const uint8_t *tb = bytes + at;
    bl_js_commit(p, stack, [&](int i) { return (uint32_t)tb[i]; }, lens[k]);
    at += lens[k];
  }
  *complete = bl_js_complete(p, p.depth > 0 ? stack[p.depth - 1] : -1) ? 1 : 0;
  *dead = p.dead;
  const uint8_t *tb = bytes + at;
  bool over = false;
  const bool ok = bl_js_walk(p, stack, [&](int i) { return (uint32_t)tb[i]; }, lens[n - 1], &over);
  return over ? -1 : (ok ? 1 : 0);
}
}
