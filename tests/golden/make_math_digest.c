/* Writes tests/golden/math_digest.bin: per 2^20-input block digests of the host glibc expf, tanhf and
 * logf over all 2^32 float bit patterns (4096 uint64 for each, in that order, little endian).
 * Digest of a block = wrapping sum over its inputs u of splitmix64(u << 32 | bits(f(u))), NaN results
 * canonicalised to 0x7fc00000.
 * Build: gcc -O2 -ffp-contract=off -fopenmp make_math_digest.c -lm -o /tmp/mmd && /tmp/mmd out.bin */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
static uint64_t splitmix(uint64_t x) {
  x += 0x9e3779b97f4a7c15ull;
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}
/* NaN results are canonicalised (payload propagation is not part of the path) */
static uint32_t bits(float f) { uint32_t u; memcpy(&u, &f, 4); return f != f ? 0x7fc00000u : u; }
static float fl(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
int main(int argc, char **argv) {
  static uint64_t dig[3][4096];
  for (int fn = 0; fn < 3; fn++) {
    #pragma omp parallel for schedule(dynamic, 16)
    for (int b = 0; b < 4096; b++) {
      uint64_t h = 0;
      for (uint32_t k = 0; k < (1u << 20); k++) {
        uint32_t u = ((uint32_t)b << 20) | k;
        float y = fn == 0 ? expf(fl(u)) : fn == 1 ? tanhf(fl(u)) : logf(fl(u));
        h += splitmix(((uint64_t)u << 32) | bits(y));
      }
      dig[fn][b] = h;
    }
  }
  FILE *f = fopen(argc > 1 ? argv[1] : "math_digest.bin", "wb");
  fwrite(dig, sizeof dig, 1, f);
  fclose(f);
  return 0;
}
