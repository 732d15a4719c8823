/*
 * bl_workload.h — host-side generators for the sparse per-slot inputs of the five workloads:
 * uniform and Zipf(1.1) histories, logit_bias lists, the +8 "bump" ids of workload 1, speculative
 * drafts and the synthetic byte vocabulary of workload 3. Header-only C++; deterministic given the
 * seed. Used by the benchmark, the tests and the oracle harness to build identical inputs.
 */
#ifndef BL_WORKLOAD_H
#define BL_WORKLOAD_H

#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "bl_synth.h"

namespace blw {

/* Workload 1: +8.0 on 20 distinct uniform ids per step (drawn in order, duplicates skipped). */
inline std::vector<int32_t> c1_bump_ids(int64_t seed, int64_t step, int vocab) {
  uint64_t s = bl_stream(1, seed, step, 0, BL_P_BUMP);
  std::vector<int32_t> ids;
  for (uint64_t i = 0; ids.size() < 20; i++) {
    int32_t id = (int32_t)bl_below(bl_draw(s, i), (uint64_t)vocab);
    if (std::find(ids.begin(), ids.end(), id) == ids.end()) ids.push_back(id);
  }
  return ids;
}

/* n uniform ids (workload 1 prompt history). */
inline std::vector<int32_t> uniform_ids(int cfg, int64_t seed, int64_t row, int n, int vocab) {
  uint64_t s = bl_stream((uint32_t)cfg, seed, 0, row, BL_P_HIST);
  std::vector<int32_t> ids(n);
  for (int i = 0; i < n; i++) ids[i] = (int32_t)bl_below(bl_draw(s, (uint64_t)i), (uint64_t)vocab);
  return ids;
}

/* n Zipf(exponent)-distributed ids over [0, vocab): rank r has weight (r+1)^-exponent and id r.
 * Inverse-CDF sampling on a host-libm table (host only). */
inline std::vector<int32_t> zipf_ids(int cfg, int64_t seed, int64_t row, int n, int vocab, double exponent) {
  std::vector<double> cdf(vocab);
  double acc = 0.0;
  for (int r = 0; r < vocab; r++) {
    acc += pow((double)(r + 1), -exponent);
    cdf[r] = acc;
  }
  uint64_t s = bl_stream((uint32_t)cfg, seed, 0, row, BL_P_ZIPF);
  std::vector<int32_t> ids(n);
  for (int i = 0; i < n; i++) {
    double u = (double)(bl_draw(s, (uint64_t)i) >> 11) * (1.0 / 9007199254740992.0) * acc;
    ids[i] = (int32_t)(std::upper_bound(cdf.begin(), cdf.end(), u) - cdf.begin());
    if (ids[i] >= vocab) ids[i] = vocab - 1;
  }
  return ids;
}

/* logit_bias: n distinct uniform ids with values uniform in [lo, hi). */
inline void bias_list(int cfg, int64_t seed, int64_t row, int n, int vocab, double lo, double hi,
                      std::vector<int32_t> &ids, std::vector<float> &vals) {
  uint64_t si = bl_stream((uint32_t)cfg, seed, 0, row, BL_P_BIAS_ID);
  uint64_t sv = bl_stream((uint32_t)cfg, seed, 0, row, BL_P_BIAS_VAL);
  ids.clear();
  vals.clear();
  for (uint64_t i = 0; (int)ids.size() < n; i++) {
    int32_t id = (int32_t)bl_below(bl_draw(si, i), (uint64_t)vocab);
    if (std::find(ids.begin(), ids.end(), id) != ids.end()) continue;
    ids.push_back(id);
    vals.push_back(bl_uniform_f(bl_draw(sv, (uint64_t)ids.size()), lo, hi));
  }
}

/* Workload 5 drafts: position i of sequence b equals the row's argmax with probability 0.7, else a
 * uniform id. `argmax` holds the greedy id of each of the k target rows of the sequence. */
inline std::vector<int32_t> c5_drafts(int64_t seed, int64_t step, int64_t seq, const int32_t *argmax, int k,
                                      int vocab) {
  uint64_t s = bl_stream(5, seed, step, seq, BL_P_DRAFT);
  std::vector<int32_t> d(k);
  for (int i = 0; i < k; i++) {
    uint64_t h = bl_draw(s, (uint64_t)(2 * i));
    bool match = bl_below(h, 10) < 7;
    d[i] = match ? argmax[i] : (int32_t)bl_below(bl_draw(s, (uint64_t)(2 * i + 1)), (uint64_t)vocab);
  }
  return d;
}

/*
 * Workload 3 vocabulary: ids 0..255 are the single bytes; ids 256..V-2 are byte strings whose length
 * L in 1..16 is Zipf(1.1)-distributed, 70% of them printable ASCII (0x20..0x7E) and 30% random valid
 * UTF-8 (code points drawn from the 2-, 3- and 4-byte ranges, excluding surrogates, cut to fit L);
 * id V-1 is the end-of-sequence token, written as the special text "<|eos|>".
 */
inline void c3_vocab(int64_t seed, int vocab, std::vector<uint8_t> &blob, std::vector<uint32_t> &offsets,
                     int32_t &eos_id) {
  blob.clear();
  offsets.assign(1, 0);
  double w[16], acc = 0.0;
  for (int l = 0; l < 16; l++) { acc += pow((double)(l + 1), -1.1); w[l] = acc; }
  uint64_t s = bl_stream(3, seed, 0, 0, BL_P_VOCAB);
  uint64_t ctr = 0;
  auto next = [&]() { return bl_draw(s, ctr++); };
  auto put_cp = [&](uint32_t cp) {
    if (cp < 0x80) blob.push_back((uint8_t)cp);
    else if (cp < 0x800) { blob.push_back((uint8_t)(0xC0 | (cp >> 6))); blob.push_back((uint8_t)(0x80 | (cp & 0x3F))); }
    else if (cp < 0x10000) {
      blob.push_back((uint8_t)(0xE0 | (cp >> 12)));
      blob.push_back((uint8_t)(0x80 | ((cp >> 6) & 0x3F)));
      blob.push_back((uint8_t)(0x80 | (cp & 0x3F)));
    } else {
      blob.push_back((uint8_t)(0xF0 | (cp >> 18)));
      blob.push_back((uint8_t)(0x80 | ((cp >> 12) & 0x3F)));
      blob.push_back((uint8_t)(0x80 | ((cp >> 6) & 0x3F)));
      blob.push_back((uint8_t)(0x80 | (cp & 0x3F)));
    }
  };
  for (int id = 0; id < vocab; id++) {
    if (id < 256) {
      blob.push_back((uint8_t)id);
    } else if (id == vocab - 1) {
      const char *eos = "<|eos|>";
      blob.insert(blob.end(), eos, eos + strlen(eos));
    } else {
      double u = (double)(next() >> 11) * (1.0 / 9007199254740992.0) * acc;
      int len = (int)(std::upper_bound(w, w + 16, u) - w) + 1;
      if (len > 16) len = 16;
      bool ascii = bl_below(next(), 10) < 7;
      int have = 0;
      while (have < len) {
        int room = len - have;
        if (ascii) {
          blob.push_back((uint8_t)(0x20 + bl_below(next(), 95)));
          have += 1;
          continue;
        }
        /* pick a UTF-8 length that fits */
        int nb = 1 + (int)bl_below(next(), 4);
        if (nb > room) nb = room;
        uint32_t cp;
        if (nb == 1) cp = (uint32_t)(0x20 + bl_below(next(), 95));
        else if (nb == 2) cp = (uint32_t)(0x80 + bl_below(next(), 0x800 - 0x80));
        else if (nb == 3) {
          cp = (uint32_t)(0x800 + bl_below(next(), 0x10000 - 0x800 - 0x800));
          if (cp >= 0xD800) cp += 0x800; /* skip surrogates */
        } else cp = (uint32_t)(0x10000 + bl_below(next(), 0x110000 - 0x10000));
        put_cp(cp);
        have += nb;
      }
    }
    offsets.push_back((uint32_t)blob.size());
  }
  eos_id = vocab - 1;
}

/* The JSON Schema of workload 3 (all three fields required). */
inline const char *c3_schema() {
  return "{\"type\":\"object\",\"properties\":{\"name\":{\"type\":\"string\",\"pattern\":\"^[a-z_]+$\"},"
         "\"count\":{\"type\":\"integer\"},\"tags\":{\"type\":\"array\",\"items\":{\"type\":\"string\"}}},"
         "\"required\":[\"name\",\"count\",\"tags\"]}";
}

} /* namespace blw */

#endif /* BL_WORKLOAD_H */
