/* Writes tests/golden/math_digest.bin: per 2^20-input block digests of the host glibc expf, tanhf, logf,
 * powf(x, 0.7f), powf(2, x) and powf(x, y(u)) over all 2^32 float bit patterns u (4096 uint64 for each, in
 * that order, little endian); y(u) = ((splitmix64(u) >> 40) % 8193 - 4096) / 512, a multiple of 1/512 in
 * [-8, 8] (integers among them, so negative x takes the integer-exponent path).
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
  static uint64_t dig[6][4096];
  for (int fn = 0; fn < 6; fn++) {
    #pragma omp parallel for schedule(dynamic, 16)
    for (int b = 0; b < 4096; b++) {
      uint64_t h = 0;
      for (uint32_t k = 0; k < (1u << 20); k++) {
        uint32_t u = ((uint32_t)b << 20) | k;
        const float x = fl(u);
        float y;
        if (fn == 0) y = expf(x);
        else if (fn == 1) y = tanhf(x);
        else if (fn == 2) y = logf(x);
        else if (fn == 3) y = powf(x, 0.7f);
        else if (fn == 4) y = powf(2.0f, x);
        else y = powf(x, (float)((int)((splitmix(u) >> 40) % 8193u) - 4096) * 0x1p-9f);
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
