/*
 * bl_api.hip — host side of libbl_select: contexts, per-slot state upload, the C ABI of
 * include/bl_select.h, and the launch sequence of a step.
 */
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <chrono>
#include <mutex>
#include <string>
#include <type_traits>
#include <unordered_map>
#include <vector>

#include "../../include/bl_select.h"
#include "bl_grammar.h"
#include "bl_internal.h"
#include "bl_math.h"
#include "bl_schema.h"
#include "bl_workload.h"

void bl_launch_step(const bl_dev &d, const float *logits, int64_t ld, const bl_rows &rows, int B, bool need_pass2,
                    bool need_gram, hipStream_t s, hipEvent_t *ev);
void bl_launch_gmask(const bl_dev &d, const bl_rows &rows, hipStream_t s);
void bl_launch_synth(float *out, int64_t ld, int cfg, int64_t seed, int64_t step, int rows, int V, hipStream_t s);
void bl_launch_math_digest(int fn, uint32_t first_block, int n_blocks, unsigned long long *out, hipStream_t s);
void bl_launch_dry_prime(const bl_dev &d, int slot, hipStream_t s);

static thread_local std::string g_err;

/* Waits for the stream's work. hipStreamSynchronize spins on the completion signal before it blocks; on
 * MI355X it returns 9.4 us after the launch of an empty kernel, where a loop of hipStreamQuery calls
 * (each one a runtime round trip) takes 28 us (median of 500, ROCm 7.2). */
static hipError_t wait_stream(hipStream_t s) { return hipStreamSynchronize(s); }

static int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

#define HIPCHK(x)                                                                   \
  do {                                                                              \
    hipError_t e_ = (x);                                                            \
    if (e_ != hipSuccess) return fail(BL_EDEVICE, "%s: %s", #x, hipGetErrorString(e_)); \
  } while (0)

struct bl_ctx {
  int device = 0;
  hipStream_t own = nullptr, stream = nullptr;
  bl_dev d{};
  std::vector<bl_slot_dev> host_slots;
  std::vector<bool> slot_ready;
  /* row table + outputs */
  int32_t *d_slot = nullptr, *d_skip = nullptr, *d_tok = nullptr, *d_status = nullptr, *d_top_ids = nullptr;
  float *d_lp = nullptr, *d_top_lp = nullptr;
  int32_t *h_slot = nullptr, *h_tok = nullptr, *h_status = nullptr, *h_top_ids = nullptr, *h_skip = nullptr;
  /* the rows of bl_bind_rows: read only by the asynchronous step and graphs, written only by bl_bind_rows
   * (the synchronous step and speculative verification build their own row table in d_slot/h_slot) */
  int32_t *d_bound = nullptr, *h_bound = nullptr;
  float *h_lp = nullptr, *h_top_lp = nullptr;
  /* the synchronous step's outputs packed in one block per side: tokens, statuses, logprobs, top ids, top
   * logprobs of the call's B rows back to back, so one copy brings them to the host */
  int32_t *d_out = nullptr, *h_out = nullptr;
  int32_t *d_commit_toks = nullptr;
  int32_t *d_mslot = nullptr; /* row table of bl_grammar_mask */
  /* speculative verification's inputs (row slots, RNG skips, drafts, sequence slots) and outputs (tokens,
   * statuses, accepted lengths), each packed in one block per side: one copy each way */
  int32_t *d_spec_in = nullptr, *h_spec_in = nullptr, *d_spec_out = nullptr, *h_spec_out = nullptr;
  bl_sdelta *d_delta = nullptr; /* speculative rows' count corrections [rows][BL_SPEC_DCAP] */
  int32_t *d_delta_n = nullptr;
  int bound_B = 0;
  std::vector<void *> allocs;
  bool timing = false;
  hipEvent_t ev[6] = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr}; /* kernel timing: start, end of each */
  double kernel_ms[3] = {0.0, 0.0, 0.0};
  int64_t timed_steps = 0;
  /* grammar: host copies of the vocabulary and of each slot's reply, compiled grammars by text */
  std::vector<uint8_t> vblob;
  std::vector<uint32_t> voff;
  uint8_t *d_vblob = nullptr;
  uint32_t *d_voff = nullptr;
  std::vector<std::vector<int32_t>> reply;
  struct gram_entry {
    bl_gram_tables tab;
    bl_gram_view dev{}, host{};
    std::vector<void *> mem;
  };
  std::unordered_map<std::string, gram_entry *> grammars;
  std::vector<char> stepped; /* the slot took part in a step since its reset */
  std::vector<void *> dry_mem; /* [slots] the slot's DRY breakers on the device (bl_slot_dry_breakers) */
  std::vector<int32_t> eog_ids; /* host copy of the end-of-generation registry */
};

template <class T>
static hipError_t dalloc(bl_ctx *c, T **p, size_t n) {
  hipError_t e = hipMalloc((void **)p, n * sizeof(T) + 16);
  if (e == hipSuccess) c->allocs.push_back(*p);
  return e;
}

/* ------------------------------------------------------------------ commit kernels */
/* tokens.push / reply_tokens.push of one token (src/server.br:1004, :1037): repeat window, reply counts,
 * grammar position; one thread */
__device__ void commit_one(const bl_dev &d, bl_slot_dev &sp, int slot, int32_t tok) {
  const int V = d.vocab;
  if (tok < 0 || tok >= V) return;
  bool is_eog = false;
  for (int k = 0; k < d.n_eog; k++) is_eog |= d.eog[k] == tok;
  sp.n_tokens += 1;
  bl_dry_push(d, sp, slot, tok);
  if (sp.rep_on) {
    int rl = sp.repeat_last_n;
    if (rl > 0) {
      int32_t *ring = d.ring + (int64_t)slot * BL_WCAP;
      if (sp.win_len == rl) {
        int32_t old = ring[sp.win_head];
        bl_rec_get(d, slot, old)->wf -= 1u;
        ring[sp.win_head] = tok;
        sp.win_head = (sp.win_head + 1) % rl;
      } else {
        ring[(sp.win_head + sp.win_len) % rl] = tok;
        sp.win_len += 1;
      }
    }
    bl_rec_get(d, slot, tok)->wf += 1u;
  }
  if (!is_eog) {
    sp.n_reply += 1;
    if (sp.fp_on) bl_rec_get(d, slot, tok)->cnt += 1;
    if (sp.g_on) grammar_commit(d, sp, d.gram[slot], tok, slot);
  }
}

/* tokens chosen outside the library (one thread: a handful of writes) */
__global__ void bl_k_commit(bl_dev d, int slot, const int32_t *toks, int n, int rng_draws) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  bl_slot_dev &sp = d.slots[slot];
  for (int i = 0; i < n; i++) commit_one(d, sp, slot, toks[i]);
  for (int k = 0; k < rng_draws; k++) sp.rng = bl_xorshift(sp.rng);
}

/*
 * Speculative verification after the selection, one workgroup per sequence (src/server.br:1173-1216):
 * the accepted prefix (leading rows whose token equals the draft and is not end-of-generation), then the
 * accepted drafts and the next row's token are pushed and the RNG advances by the draws a sequential
 * decode makes (accepted + 1 for a sampled slot). Nothing is committed when any row of the call reported
 * a status (the call then fails as a whole).
 */
__global__ void bl_k_spec_commit(bl_dev d, const int32_t *slots, const int32_t *drafts, int k, const int32_t *tok,
                                 const int32_t *status, int R, int32_t *accepted) {
  const int b = blockIdx.x;
  __shared__ int bad;
  if (threadIdx.x == 0) bad = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < R; i += blockDim.x)
    if (status[i]) bad = 1;
  __syncthreads();
  if (threadIdx.x != 0) return;
  const int32_t *tb = tok + (int64_t)b * (k + 1), *db = drafts + (int64_t)b * k;
  int a = 0;
  while (a < k && tb[a] == db[a]) {
    bool eog = false;
    for (int q = 0; q < d.n_eog; q++) eog |= d.eog[q] == tb[a];
    if (eog) break;
    a++;
  }
  accepted[b] = a;
  if (bad) return;
  const int slot = slots[b];
  bl_slot_dev &sp = d.slots[slot];
  for (int i = 0; i < a; i++) commit_one(d, sp, slot, db[i]);
  commit_one(d, sp, slot, tb[a]);
  if (sp.temperature > 0.0f)
    for (int q = 0; q <= a; q++) sp.rng = bl_xorshift(sp.rng);
}

/*
 * Count corrections of speculative rows: row i of sequence b is sampled as if drafts[0..i) had been pushed
 * to tokens and reply_tokens (src/server.br:1173-1216), as commit_one would push them: each draft adds one
 * to its reply count and, while it is still in the repeat window, to its window count; once the window holds
 * repeat_last_n tokens each push evicts the oldest ring entry. One thread per row.
 */
__global__ void bl_k_spec_delta(bl_dev d, const int32_t *slots, const int32_t *drafts, int k, bl_sdelta *delta,
                                int32_t *delta_n) {
  const int b = blockIdx.x, i = threadIdx.x;
  if (i > k) return;
  const int slot = slots[b];
  const bl_slot_dev &sp = d.slots[slot];
  const int32_t *db = drafts + (int64_t)b * k;
  bl_sdelta *out = delta + ((int64_t)b * (k + 1) + i) * BL_SPEC_DCAP;
  const int rl = sp.repeat_last_n;
  int n = 0;
  for (int j = 0; j < i; j++) {
    const int dc = sp.fp_on ? 1 : 0;
    const int dw = sp.rep_on && (rl < 0 || j >= i - rl) ? 1 : 0;
    if (dc || dw) out[n++] = bl_sdelta{db[j], (int16_t)dc, (int16_t)dw};
  }
  if (sp.rep_on && rl > 0) {
    const int leave = min(max(sp.win_len + i - rl, 0), sp.win_len);
    const int32_t *ring = d.ring + (int64_t)slot * BL_WCAP;
    for (int m = 0; m < leave; m++) out[n++] = bl_sdelta{ring[(sp.win_head + m) % rl], 0, -1};
  }
  delta_n[(int64_t)b * (k + 1) + i] = n;
}

__global__ void bl_k_bump(float *out, const int32_t *ids, int n, float add) {
  int i = threadIdx.x;
  if (i < n) out[ids[i]] = out[ids[i]] + add;
}

/* The device buffers of a step (bl_dev) for S slots, R rows and a vocabulary of V tokens, in this order, each
 * from take(pointer, element count); false when one could not be had. A context takes them from hipMalloc,
 * the allocation-free step from its fixed array. */
template <class Take>
static bool dev_layout(bl_dev &d, size_t S, size_t R, int vocab, Take take) {
  const size_t V = (size_t)vocab, G = V / 64 + 64;
  d.vocab = vocab;
  d.nc = (vocab + BL_CH - 1) / BL_CH;
  d.nb = (vocab + BL_EB - 1) / BL_EB;
  d.gm_blocks = (vocab + BL_GM_THREADS - 1) / BL_GM_THREADS;
  d.max_slots = (int)S;
  d.max_rows = (int)R;
  d.eos_id = -1;
  d.n_eog = 0;
  char *grec = nullptr, *brec = nullptr;
  const bool ok = take(d.slots, S) && take(d.rec, S * d.nb * BL_EB) && take(d.rcnt, S * d.nb) && take(d.ridx, S * V) &&
                  take(d.ring, S * BL_WCAP) && take(d.dring, S * BL_DRY_WCAP) && take(d.dlist, S * BL_DRY_WCAP) &&
                  take(d.eog, 1024) && take(d.eff, R * V) && take(d.c_max, R * d.nc) && take(d.c_arg, R * d.nc) &&
                  take(d.c_bsum, R * d.nc * BL_SUBS) && take(d.c_tns, R * d.nc * BL_TNS_W) && take(d.cand_v, R * d.nc * BL_KSEL_MAX) &&
                  take(d.cand_i, R * d.nc * BL_KSEL_MAX) && take(grec, R * 2 * G * 32) && take(d.full_v, R * d.nb * BL_EB) &&
                  take(d.full_i, R * d.nb * BL_EB) && take(d.full_cnt, R * d.nb) && take(d.full_s, R * d.nb) &&
                  take(d.sortk, R * 2 * V) && take(d.gsum, R * G) && take(d.crit, R * BL_CRIT_MAX) && take(d.ncrit, R) &&
                  take(d.mkeys, R * BL_KSEL_MAX) && take(d.mstat, R) && take(d.rmax, R) && take(d.rarg, R) &&
                  take(brec, R * d.nb * 16) && take(d.bcrit, R * d.nb) && take(d.gram, S) && take(d.jstack, S * BL_JSON_DEPTH) &&
                  take(d.gmask, R * 2 * ((V + 63) / 64)) && take(d.gstat, R) && take(d.gamb, R) &&
                  take(d.gm_max, R * d.gm_blocks) && take(d.gm_arg, R * d.gm_blocks) && take(d.gm_eq, R * d.gm_blocks);
  d.grec = grec;
  d.brec = brec;
  return ok;
}

extern "C" {

const char *bl_last_error(void) { return g_err.c_str(); }

int64_t bl_resolve_seed(int64_t requested, uint64_t entropy, int64_t request_counter) {
  if (requested >= 0) return requested;
  const uint64_t c = (uint64_t)request_counter;
  uint64_t x = entropy ^ (c << 32) ^ c;
  x ^= x << 13;
  x ^= x >> 7;
  x ^= x << 17;
  const int64_t chosen = (int64_t)(x & 0x7fffffffull);
  return chosen ? chosen : 1;
}

uint64_t bl_seed_rng(int64_t seed) {
  const uint64_t fold = 88172645463325252ull; /* keeps the state off xorshift's fixed point 0 */
  return seed == 0 ? fold : ((uint64_t)seed ^ fold);
}

void bl_params_default(bl_params *p) {
  memset(p, 0, sizeof *p);
  p->temperature = 0.0f;
  p->dynatemp_range = 0.0f;
  p->dynatemp_exponent = 1.0f;
  p->top_n_sigma = -1.0f;
  p->top_k = 0;
  p->typical_p = 1.0f;
  p->top_p = 1.0f;
  p->min_p = 0.0f;
  p->xtc_probability = 0.0f;
  p->xtc_threshold = 0.1f;
  p->mirostat = 0;
  p->mirostat_tau = 5.0f;
  p->mirostat_eta = 0.1f;
  p->min_keep = 0;
  p->repeat_penalty = 1.0f;
  p->repeat_last_n = 64;
  p->adaptive_target = -1.0f;
  p->adaptive_decay = 0.9f;
  p->dry_multiplier = 0.0f;
  p->dry_base = 1.75f;
  p->dry_allowed_length = 2;
  p->dry_penalty_last_n = 64;
  p->final_softcap = 0.0f;
  p->logit_mul = 1.0f;
}

int bl_create(int device, int max_slots, int max_rows, int vocab, bl_ctx **out) {
  if (!out || max_slots <= 0 || max_slots > 32767 || max_rows <= 0 || vocab <= 0 || vocab > BL_MAX_CHUNKS * BL_CH)
    return fail(BL_EPARAM, "bl_create: invalid sizes (slots %d, rows %d, vocab %d)", max_slots, max_rows, vocab);
  bl_ctx *c = new bl_ctx;
  c->device = device;
  hipError_t e = hipSetDevice(device);
  if (e != hipSuccess) {
    delete c;
    return fail(BL_EDEVICE, "hipSetDevice(%d): %s", device, hipGetErrorString(e));
  }
  bl_dev &d = c->d;
  const size_t R = (size_t)max_rows;
#define ALLOC(p, n)                                   \
  do {                                                \
    if (dalloc(c, &(p), (n)) != hipSuccess) {         \
      bl_destroy(c);                                  \
      return fail(BL_EDEVICE, "hipMalloc failed (%s)", #p); \
    }                                                 \
  } while (0)
  if (!dev_layout(d, max_slots, max_rows, vocab, [&](auto *&p, size_t n) { return dalloc(c, &p, n) == hipSuccess; })) {
    bl_destroy(c);
    return fail(BL_EDEVICE, "hipMalloc failed (step workspace)");
  }
  ALLOC(c->d_slot, R);
  ALLOC(c->d_bound, R);
  ALLOC(c->d_skip, R);
  ALLOC(c->d_tok, R);
  ALLOC(c->d_status, R);
  ALLOC(c->d_lp, R);
  ALLOC(c->d_top_ids, R * 256);
  ALLOC(c->d_top_lp, R * 256);
  ALLOC(c->d_commit_toks, 4096);
  ALLOC(c->d_mslot, 1);
  ALLOC(c->d_out, R * (3 + 2 * 256));
  ALLOC(c->d_delta, R * BL_SPEC_DCAP);
  ALLOC(c->d_delta_n, R);
  ALLOC(c->d_spec_in, 3 * (size_t)R + 4096);
  ALLOC(c->d_spec_out, 3 * (size_t)R);
#undef ALLOC
  /* slot records and grammar views start zeroed: a slot is only stepped or committed after bl_slot_reset, and
   * nothing reads uninitialised state even when a caller breaks that rule */
  if (hipMemset(d.slots, 0, max_slots * sizeof(bl_slot_dev)) != hipSuccess ||
      hipMemset(d.gram, 0, max_slots * sizeof(bl_gram_view)) != hipSuccess ||
      hipDeviceSynchronize() != hipSuccess) {
    bl_destroy(c);
    return fail(BL_EDEVICE, "hipMemset failed");
  }
  if (hipHostMalloc((void **)&c->h_slot, R * sizeof(int32_t)) != hipSuccess ||
      hipHostMalloc((void **)&c->h_bound, R * sizeof(int32_t)) != hipSuccess ||
      hipHostMalloc((void **)&c->h_skip, R * sizeof(int32_t)) != hipSuccess ||
      hipHostMalloc((void **)&c->h_tok, R * sizeof(int32_t)) != hipSuccess ||
      hipHostMalloc((void **)&c->h_status, R * sizeof(int32_t)) != hipSuccess ||
      hipHostMalloc((void **)&c->h_lp, R * sizeof(float)) != hipSuccess ||
      hipHostMalloc((void **)&c->h_top_ids, R * 256 * sizeof(int32_t)) != hipSuccess ||
      hipHostMalloc((void **)&c->h_top_lp, R * 256 * sizeof(float)) != hipSuccess ||
      hipHostMalloc((void **)&c->h_spec_in, (3 * (size_t)R + 4096) * sizeof(int32_t)) != hipSuccess ||
      hipHostMalloc((void **)&c->h_spec_out, 3 * (size_t)R * sizeof(int32_t)) != hipSuccess ||
      hipHostMalloc((void **)&c->h_out, R * (3 + 2 * 256) * sizeof(int32_t)) != hipSuccess) {
    bl_destroy(c);
    return fail(BL_EDEVICE, "hipHostMalloc failed");
  }
  if (hipStreamCreateWithFlags(&c->own, hipStreamNonBlocking) != hipSuccess) {
    bl_destroy(c);
    return fail(BL_EDEVICE, "hipStreamCreate failed");
  }
  c->stream = c->own;
  c->host_slots.assign(max_slots, bl_slot_dev{});
  c->slot_ready.assign(max_slots, false);
  c->reply.assign(max_slots, {});
  c->stepped.assign(max_slots, 0);
  c->dry_mem.assign(max_slots, nullptr);
  *out = c;
  return BL_OK;
}

void bl_destroy(bl_ctx *c) {
  if (!c) return;
  hipSetDevice(c->device);
  if (c->stream) hipStreamSynchronize(c->stream);
  for (void *p : c->allocs) hipFree(p);
  for (auto &kv : c->grammars) {
    for (void *p : kv.second->mem) hipFree(p);
    delete kv.second;
  }
  if (c->d_vblob) hipFree(c->d_vblob);
  if (c->d_voff) hipFree(c->d_voff);
  for (void *p : c->dry_mem)
    if (p) hipFree(p);
  void *hp[] = {c->h_slot, c->h_bound, c->h_skip, c->h_tok, c->h_status, c->h_lp, c->h_top_ids, c->h_top_lp, c->h_out,
                c->h_spec_in, c->h_spec_out};
  for (void *p : hp)
    if (p) hipHostFree(p);
  for (hipEvent_t e : c->ev)
    if (e) hipEventDestroy(e);
  if (c->own) hipStreamDestroy(c->own);
  delete c;
}

int bl_set_stream(bl_ctx *c, void *stream) {
  if (!c) return fail(BL_EPARAM, "null context");
  c->stream = stream ? (hipStream_t)stream : c->own;
  return BL_OK;
}

int bl_set_eog(bl_ctx *c, int32_t eos_id, const int32_t *eog_ids, int n_eog) {
  if (!c || n_eog < 0 || n_eog > 1000) return fail(BL_EPARAM, "bl_set_eog: invalid arguments");
  std::vector<int32_t> ids;
  if (eos_id >= 0) ids.push_back(eos_id);
  for (int i = 0; i < n_eog; i++) ids.push_back(eog_ids[i]);
  hipSetDevice(c->device);
  if (!ids.empty()) HIPCHK(hipMemcpy(c->d.eog, ids.data(), ids.size() * sizeof(int32_t), hipMemcpyHostToDevice));
  c->d.n_eog = (int32_t)ids.size();
  c->d.eos_id = eos_id;
  c->eog_ids = ids;
  return BL_OK;
}

/* mode and unsupported-stage checks for one slot's parameters */
static int configure(int V, const bl_params *p, bl_slot_dev &s) {
  if (p->temperature != p->temperature || p->top_p != p->top_p) return fail(BL_EPARAM, "NaN sampling parameter");
  if (p->n_probs < 0 || p->n_probs > 256) return fail(BL_EPARAM, "n_probs must be in 0..256 (got %d)", p->n_probs);
  s.temperature = p->temperature;
  s.dynatemp_range = p->dynatemp_range;
  s.dynatemp_exponent = p->dynatemp_exponent;
  s.top_n_sigma = p->top_n_sigma;
  s.typical_p = p->typical_p;
  s.top_p = p->top_p;
  s.min_p = p->min_p;
  s.xtc_probability = p->xtc_probability;
  s.xtc_threshold = p->xtc_threshold;
  s.repeat_penalty = p->repeat_penalty;
  s.frequency_penalty = p->frequency_penalty;
  s.presence_penalty = p->presence_penalty;
  s.final_softcap = p->final_softcap;
  s.logit_mul = p->logit_mul;
  s.top_k = p->top_k;
  s.min_keep = p->min_keep;
  s.repeat_last_n = p->repeat_last_n;
  s.n_probs = p->logprobs ? p->n_probs : 0;
  s.ignore_eos = p->ignore_eos;
  s.post_sampling_probs = p->post_sampling_probs;
  s.fp_on = !(p->frequency_penalty == 0.0f && p->presence_penalty == 0.0f);
  s.rep_on = !(p->repeat_penalty == 1.0f || p->repeat_last_n == 0);
  int mode = 0;
  if (p->temperature <= 0.0f) mode |= BL_M_GREEDY;
  else if (p->top_k > 0 && p->top_k < V) mode |= BL_M_TOPK;
  else mode |= BL_M_FULL;
  /* logprobs: the effective logits' normaliser and top n_probs, or the draw's own probabilities */
  if (p->logprobs) mode |= p->post_sampling_probs ? BL_M_PSP : BL_M_LOGPROBS;
  /* mirostat replaces the sampler chain (src/server.br:964-976); a greedy row stays greedy */
  if (p->mirostat < 0 || p->mirostat > 2 || !(p->mirostat_tau >= 0.0f) || !(p->mirostat_eta >= 0.0f))
    return fail(BL_EPARAM, "`mirostat` must be 0, 1, or 2 with non-negative tau and eta");
  if (p->mirostat != 0 && p->post_sampling_probs && p->logprobs)
    return fail(BL_EPARAM, "post_sampling_probs require the standard unconstrained sampling chain");
  s.mirostat = p->mirostat;
  s.mirostat_tau = p->mirostat_tau;
  s.mirostat_eta = p->mirostat_eta;
  s.mu = 2.0f * p->mirostat_tau;
  if (p->mirostat != 0 && p->temperature > 0.0f) mode = (mode & ~(BL_M_TOPK | BL_M_FULL)) | BL_M_FULL | BL_M_MIRO;
  /* adaptive-p takes the step before mirostat and the chain (src/server.br:953-963), at any temperature */
  if (p->adaptive_target >= 0.0f) {
    if (p->post_sampling_probs && p->logprobs)
      return fail(BL_EPARAM, "post_sampling_probs require the standard unconstrained sampling chain");
    mode = (mode & BL_M_LOGPROBS) | BL_M_ADAPT;
    s.adapt_target = p->adaptive_target;
    s.adapt_decay = p->adaptive_decay;
    const float one_minus = 1.0f - p->adaptive_decay;
    s.adapt_ws = p->adaptive_target / one_minus;
    s.adapt_tw = 1.0f / one_minus;
  }
  s.mode = mode;
  int k = 0;
  if (mode & BL_M_TOPK) k = p->top_k;
  if ((mode & BL_M_LOGPROBS) && p->n_probs > k) k = p->n_probs;
  /* mirostat v1 fits the first min(V, 100) ranked probabilities: the merged top-K list supplies them */
  if ((mode & BL_M_MIRO) && p->mirostat == 1 && k < (V < 100 ? V : 100)) k = V < 100 ? V : 100;
  s.k_sel = k;
  /* top-n-sigma filters the candidates of a sampled row (src/sampling.br:752-753); mirostat replaces that chain */
  if (p->temperature > 0.0f && p->top_n_sigma > 0.0f && !(mode & (BL_M_MIRO | BL_M_ADAPT))) mode |= BL_M_TNS;
  s.mode = mode;
  /* DRY (src/sampling.br:114-171): off at multiplier 0, base below 1 or a window of 0; a negative window
   * leaves the logits unchanged as well */
  s.dry_on = (p->dry_multiplier != 0.0f && p->dry_base >= 1.0f && p->dry_penalty_last_n > 0) ? 1 : 0;
  s.dry_mult = p->dry_multiplier;
  s.dry_base = p->dry_base;
  s.dry_allowed = p->dry_allowed_length;
  s.dry_n = p->dry_penalty_last_n;
  s.dry_maxexp = 0x7fffffff;
  if (s.dry_on) {
    if (p->dry_penalty_last_n > BL_DRY_WCAP)
      return fail(BL_EUNSUPPORTED, "dry_penalty_last_n above %d", BL_DRY_WCAP);
    if (p->dry_allowed_length < 0) return fail(BL_EUNSUPPORTED, "a negative dry_allowed_length");
    /* llama.cpp's overflow guard, `(88.7228391 / base.ln()) as int` (truncating, saturating) */
    if (p->dry_base > 1.000001f) {
      const float q = 88.7228391f / bl_logf(p->dry_base);
      s.dry_maxexp = q >= 2147483647.0f ? 0x7fffffff : (int)q;
    }
  }
  if (k > BL_KSEL_MAX)
    return fail(BL_EUNSUPPORTED, "top_k/n_probs of %d exceeds the device selection limit", k);
  if (p->repeat_last_n > BL_WCAP) return fail(BL_EUNSUPPORTED, "repeat_last_n above %d", BL_WCAP);
  return BL_OK;
}

int bl_slot_reset(bl_ctx *c, int slot, const bl_params *p, uint64_t rng_state, const int32_t *history, int n_hist,
                  const int32_t *reply, int n_reply, const int32_t *bias_ids, const float *bias_vals, int n_bias) {
  if (!c || !p || slot < 0 || slot >= c->d.max_slots || n_hist < 0 || n_reply < 0 || n_bias < 0)
    return fail(BL_EPARAM, "bl_slot_reset: invalid arguments");
  const int V = c->d.vocab;
  bl_slot_dev s{};
  int rc = configure(V, p, s);
  if (rc) return rc;
  for (int i = 0; i < n_hist; i++)
    if (history[i] < 0 || history[i] >= V) return fail(BL_EPARAM, "history token %d outside the vocabulary", history[i]);
  for (int i = 0; i < n_reply; i++)
    if (reply[i] < 0 || reply[i] >= V) return fail(BL_EPARAM, "reply token %d outside the vocabulary", reply[i]);
  for (int i = 0; i < n_bias; i++)
    if (bias_ids[i] < 0 || bias_ids[i] >= V)
      return fail(BL_EPARAM, "logit_bias token id %d is outside the vocabulary", bias_ids[i]);
  /* the slot's records: one per modified token, packed per bucket in first-touch order */
  const int NB = c->d.nb;
  std::vector<bl_rec> rec((size_t)NB * BL_EB, bl_rec{0, 0.0f, 0, 0u});
  std::vector<int32_t> rcnt(NB, 0);
  std::vector<int16_t> ridx(V, (int16_t)-1);
  std::vector<int32_t> ring(BL_WCAP, 0);
  auto rec_of = [&](int32_t id) -> bl_rec & {
    const int b = id / BL_EB;
    if (ridx[id] < 0) {
      ridx[id] = (int16_t)rcnt[b];
      rec[(size_t)b * BL_EB + rcnt[b]++] = bl_rec{id, 0.0f, 0, 0u};
    }
    return rec[(size_t)b * BL_EB + ridx[id]];
  };
  for (int i = 0; i < n_bias; i++) {
    bl_rec &r = rec_of(bias_ids[i]);
    r.wf |= BL_TF_BIAS << BL_WF_SHIFT;
    r.bias = bias_vals[i]; /* a repeated id keeps the last value, as a JSON object would */
  }
  if (s.fp_on)
    for (int i = 0; i < n_reply; i++) rec_of(reply[i]).cnt += 1;
  if (s.rep_on) {
    int rl = p->repeat_last_n;
    int win = (rl > 0 && n_hist > rl) ? rl : n_hist;
    for (int i = n_hist - win; i < n_hist; i++) rec_of(history[i]).wf += 1u;
    if (rl > 0) {
      for (int i = 0; i < win; i++) ring[i] = history[n_hist - win + i];
      s.win_len = win;
      s.win_head = 0;
    }
  }
  /* DRY's window: the last dry_penalty_last_n history tokens, each with a record; the breakers are set by
   * bl_slot_dry_breakers (none until then) */
  std::vector<int32_t> dwin;
  if (s.dry_on) {
    const int w = n_hist < s.dry_n ? n_hist : s.dry_n;
    dwin.assign(history + (n_hist - w), history + n_hist);
    for (int32_t id : dwin) rec_of(id);
    s.dh_len = w;
    s.dh_head = 0;
  }
  s.dry_cnt = 0;
  s.n_bsingle = s.n_bmulti = 0;
  s.bsingle = nullptr;
  s.bmulti = nullptr;
  s.rng = rng_state;
  s.n_tokens = n_hist;
  s.n_reply = n_reply;
  s.g_on = 0; /* a grammar is attached by bl_slot_grammar */
  c->reply[slot].assign(reply, reply + n_reply);
  c->stepped[slot] = 0;
  hipSetDevice(c->device);
  HIPCHK(hipStreamSynchronize(c->stream));
  HIPCHK(hipMemcpy(c->d.rec + (size_t)slot * NB * BL_EB, rec.data(), rec.size() * sizeof(bl_rec), hipMemcpyHostToDevice));
  HIPCHK(hipMemcpy(c->d.rcnt + (size_t)slot * NB, rcnt.data(), NB * sizeof(int32_t), hipMemcpyHostToDevice));
  HIPCHK(hipMemcpy(c->d.ridx + (size_t)slot * V, ridx.data(), (size_t)V * sizeof(int16_t), hipMemcpyHostToDevice));
  HIPCHK(hipMemcpy(c->d.ring + (size_t)slot * BL_WCAP, ring.data(), BL_WCAP * 4, hipMemcpyHostToDevice));
  if (!dwin.empty())
    HIPCHK(hipMemcpy(c->d.dring + (size_t)slot * BL_DRY_WCAP, dwin.data(), dwin.size() * 4, hipMemcpyHostToDevice));
  HIPCHK(hipMemcpy(c->d.slots + slot, &s, sizeof s, hipMemcpyHostToDevice));
  if (c->dry_mem[slot]) {
    HIPCHK(hipFree(c->dry_mem[slot]));
    c->dry_mem[slot] = nullptr;
  }
  if (s.dry_on) {
    bl_launch_dry_prime(c->d, slot, c->stream);
    HIPCHK(hipGetLastError());
    HIPCHK(hipStreamSynchronize(c->stream));
  }
  c->host_slots[slot] = s;
  c->slot_ready[slot] = true;
  return BL_OK;
}

int bl_slot_dry_breakers(bl_ctx *c, int slot, const int32_t *tokens, const int32_t *lens, int n) {
  if (!c || slot < 0 || slot >= c->d.max_slots || n < 0 || (n > 0 && (!tokens || !lens)))
    return fail(BL_EPARAM, "bl_slot_dry_breakers: invalid arguments");
  if (!c->slot_ready[slot]) return fail(BL_EPARAM, "slot %d is not set up", slot);
  const int V = c->d.vocab;
  /* singles: first occurrence, with the count of longer breakers before it; longer ones in list order */
  std::unordered_map<int32_t, int32_t> first;
  std::vector<int32_t> multi;
  int nm = 0;
  size_t at = 0;
  for (int i = 0; i < n; i++) {
    const int L = lens[i];
    if (L < 0) return fail(BL_EPARAM, "bl_slot_dry_breakers: negative length");
    for (int q = 0; q < L; q++)
      if (tokens[at + q] < 0 || tokens[at + q] >= V)
        return fail(BL_EPARAM, "DRY breaker token %d is outside the vocabulary", tokens[at + q]);
    if (L == 1) {
      first.emplace(tokens[at], nm);
    } else if (L > 1) {
      if (L > BL_DRY_MLEN || nm >= BL_DRY_MMAX)
        return fail(BL_EUNSUPPORTED, "DRY breakers: at most %d of 2 to %d tokens", BL_DRY_MMAX, BL_DRY_MLEN);
      multi.push_back(L);
      for (int q = 0; q < BL_DRY_MLEN; q++) multi.push_back(q < L ? tokens[at + q] : -1);
      nm++;
    }
    at += (size_t)L;
  }
  std::vector<uint64_t> single;
  single.reserve(first.size());
  for (auto &kv : first) single.push_back((uint64_t)(uint32_t)kv.first << 32 | (uint32_t)kv.second);
  std::sort(single.begin(), single.end());
  hipSetDevice(c->device);
  HIPCHK(hipStreamSynchronize(c->stream));
  if (c->dry_mem[slot]) HIPCHK(hipFree(c->dry_mem[slot]));
  c->dry_mem[slot] = nullptr;
  const size_t sb = single.size() * 8, mb = multi.size() * 4;
  if (sb + mb) {
    HIPCHK(hipMalloc(&c->dry_mem[slot], sb + mb + 16));
    if (sb) HIPCHK(hipMemcpy(c->dry_mem[slot], single.data(), sb, hipMemcpyHostToDevice));
    if (mb) HIPCHK(hipMemcpy((char *)c->dry_mem[slot] + sb, multi.data(), mb, hipMemcpyHostToDevice));
  }
  /* the device slot has advanced since its reset: only the breaker fields change */
  bl_slot_dev s;
  HIPCHK(hipMemcpy(&s, c->d.slots + slot, sizeof s, hipMemcpyDeviceToHost));
  s.n_bsingle = (int32_t)single.size();
  s.n_bmulti = nm;
  s.bsingle = sb ? (const uint64_t *)c->dry_mem[slot] : nullptr;
  s.bmulti = mb ? (const int32_t *)((char *)c->dry_mem[slot] + sb) : nullptr;
  HIPCHK(hipMemcpy(c->d.slots + slot, &s, sizeof s, hipMemcpyHostToDevice));
  c->host_slots[slot].n_bsingle = s.n_bsingle;
  c->host_slots[slot].n_bmulti = s.n_bmulti;
  c->host_slots[slot].bsingle = s.bsingle;
  c->host_slots[slot].bmulti = s.bmulti;
  if (s.dry_on) {
    bl_launch_dry_prime(c->d, slot, c->stream);
    HIPCHK(hipGetLastError());
    HIPCHK(hipStreamSynchronize(c->stream));
  }
  return BL_OK;
}

int bl_slot_rng(bl_ctx *c, int slot, uint64_t *state) {
  if (!c || slot < 0 || slot >= c->d.max_slots || !state) return fail(BL_EPARAM, "bl_slot_rng: invalid arguments");
  if (!c->slot_ready[slot]) return fail(BL_EPARAM, "slot %d is not set up", slot);
  hipSetDevice(c->device);
  bl_slot_dev s;
  HIPCHK(hipStreamSynchronize(c->stream));
  HIPCHK(hipMemcpy(&s, c->d.slots + slot, sizeof s, hipMemcpyDeviceToHost));
  *state = s.rng;
  return BL_OK;
}

int bl_slot_commit(bl_ctx *c, int slot, const int32_t *toks, int n) {
  if (!c || slot < 0 || slot >= c->d.max_slots || n < 0 || n > 4096 || (n > 0 && !toks))
    return fail(BL_EPARAM, "bl_slot_commit: invalid arguments");
  if (!c->slot_ready[slot]) return fail(BL_EPARAM, "slot %d is not set up", slot);
  if (n == 0) return BL_OK;
  for (int i = 0; i < n; i++)
    if (toks[i] >= 0 && toks[i] < c->d.vocab) {
      bool eog = false;
      for (int32_t e : c->eog_ids) eog |= e == toks[i];
      if (!eog) c->reply[slot].push_back(toks[i]);
    }
  hipSetDevice(c->device);
  HIPCHK(hipMemcpyAsync(c->d_commit_toks, toks, n * sizeof(int32_t), hipMemcpyHostToDevice, c->stream));
  hipLaunchKernelGGL(bl_k_commit, dim3(1), dim3(64), 0, c->stream, c->d, slot, c->d_commit_toks, n, 0);
  HIPCHK(hipGetLastError());
  if (c->host_slots[slot].dry_on) {
    bl_launch_dry_prime(c->d, slot, c->stream);
    HIPCHK(hipGetLastError());
  }
  HIPCHK(hipStreamSynchronize(c->stream));
  return BL_OK;
}

/* ------------------------------------------------------------------ grammar-constrained slots */
int bl_set_vocab(bl_ctx *c, const uint8_t *blob, const uint32_t *offsets, int n_tokens) {
  if (!c || !blob || !offsets || n_tokens != c->d.vocab)
    return fail(BL_EPARAM, "bl_set_vocab: expected %d token pieces", c ? c->d.vocab : 0);
  for (int i = 0; i < n_tokens; i++)
    if (offsets[i + 1] < offsets[i]) return fail(BL_EPARAM, "bl_set_vocab: offsets must not decrease");
  const size_t nb = offsets[n_tokens];
  hipSetDevice(c->device);
  HIPCHK(hipStreamSynchronize(c->stream));
  if (c->d_vblob) HIPCHK(hipFree(c->d_vblob));
  if (c->d_voff) HIPCHK(hipFree(c->d_voff));
  c->d_vblob = nullptr;
  c->d_voff = nullptr;
  HIPCHK(hipMalloc((void **)&c->d_vblob, nb + 16));
  HIPCHK(hipMalloc((void **)&c->d_voff, ((size_t)n_tokens + 1) * sizeof(uint32_t)));
  if (nb) HIPCHK(hipMemcpy(c->d_vblob, blob, nb, hipMemcpyHostToDevice));
  HIPCHK(hipMemcpy(c->d_voff, offsets, ((size_t)n_tokens + 1) * sizeof(uint32_t), hipMemcpyHostToDevice));
  c->vblob.assign(blob, blob + nb);
  c->voff.assign(offsets, offsets + n_tokens + 1);
  c->d.vblob = c->d_vblob;
  c->d.voff = c->d_voff;
  return BL_OK;
}

static const int kMaxGrammarStates = 1 << 16;

/* compiled tables of `text`, uploaded once per context */
static int grammar_tables(bl_ctx *c, const std::string &text, bl_ctx::gram_entry **out) {
  auto it = c->grammars.find(text);
  if (it != c->grammars.end()) {
    *out = it->second;
    return BL_OK;
  }
  bl_ctx::gram_entry *e = new bl_ctx::gram_entry;
  std::string err;
  int rc = bl_gram_compile(text, kMaxGrammarStates, e->tab, err);
  if (rc) {
    delete e;
    return fail(rc, "%s", err.c_str());
  }
  const bl_gram_tables &t = e->tab;
  auto up = [&](const void *src, size_t bytes, void **dst) -> hipError_t {
    hipError_t r = hipMalloc(dst, bytes + 16);
    if (r != hipSuccess) return r;
    e->mem.push_back(*dst);
    return bytes ? hipMemcpy(*dst, src, bytes, hipMemcpyHostToDevice) : hipSuccess;
  };
  void *tr, *fl, *as, *il, *ic;
  hipError_t r = up(t.trans.data(), t.trans.size() * 4, &tr);
  if (r == hipSuccess) r = up(t.flags.data(), t.flags.size(), &fl);
  if (r == hipSuccess) r = up(t.ascii.data(), t.ascii.size() * 2, &as);
  if (r == hipSuccess) r = up(t.ivl_lo.data(), t.ivl_lo.size() * 4, &il);
  if (r == hipSuccess) r = up(t.ivl_cls.data(), t.ivl_cls.size() * 2, &ic);
  if (r != hipSuccess) {
    for (void *p : e->mem) hipFree(p);
    delete e;
    return fail(BL_EDEVICE, "grammar tables: %s", hipGetErrorString(r));
  }
  e->dev = bl_gram_view{(const int32_t *)tr, (const uint8_t *)fl, (const uint16_t *)as, (const uint32_t *)il,
                        (const uint16_t *)ic, (int32_t)t.ivl_lo.size(), t.n_classes, t.start, 0};
  e->host = bl_gram_view{t.trans.data(), t.flags.data(), t.ascii.data(), t.ivl_lo.data(), t.ivl_cls.data(),
                         (int32_t)t.ivl_lo.size(), t.n_classes, t.start, 0};
  c->grammars[text] = e;
  *out = e;
  return BL_OK;
}

int bl_slot_grammar(bl_ctx *c, int slot, const char *gbnf, size_t len) {
  if (!c || slot < 0 || slot >= c->d.max_slots || !c->slot_ready[slot])
    return fail(BL_EPARAM, "bl_slot_grammar: slot %d is not set up", slot);
  if (c->stepped[slot]) return fail(BL_EPARAM, "bl_slot_grammar: attach the grammar before the slot's first step");
  bl_slot_dev s = c->host_slots[slot];
  s.g_kind = 0;
  if (!gbnf || len == 0) {
    s.g_on = 0;
    s.mode &= ~(BL_M_GRAMMAR | BL_M_GFULL);
  } else {
    if (c->voff.empty()) return fail(BL_EPARAM, "bl_slot_grammar: the vocabulary pieces are not set (bl_set_vocab)");
    if (s.mirostat != 0 || (s.mode & BL_M_ADAPT))
      return fail(BL_EPARAM, "stateful adaptive sampling cannot be combined with constrained decoding");
    if (s.temperature > 0.0f && s.top_n_sigma > 0.0f)
      return fail(BL_EUNSUPPORTED, "grammar-constrained sampling with top_n_sigma is not supported on the device");
    bl_ctx::gram_entry *e = nullptr;
    int rc = grammar_tables(c, std::string(gbnf, len), &e);
    if (rc) return rc;
    /* the slot's position after its reply (the reference re-decodes it every step) */
    bl_gram_pos pos{e->tab.start, e->tab.start, BL_GW_NONE, 0u, 0};
    for (int32_t id : c->reply[slot]) {
      const uint8_t *b = c->vblob.data() + c->voff[id];
      bl_gw_commit(e->host, pos, [&](int i) { return (uint32_t)b[i]; }, (int)(c->voff[id + 1] - c->voff[id]));
    }
    s.gpos = pos;
    s.g_on = 1;
    s.mode |= BL_M_GRAMMAR;
    /* a sampled top-k row widens k 4-fold while no allowed token ranks within it: the merged list keeps the
     * first BL_KSEL_MAX ranks for those levels */
    if (s.temperature > 0.0f && (s.mode & BL_M_TOPK)) {
      s.k_sel = BL_KSEL_MAX < c->d.vocab ? BL_KSEL_MAX : c->d.vocab;
      s.mode |= BL_M_GFULL;
    }
    hipSetDevice(c->device);
    HIPCHK(hipStreamSynchronize(c->stream));
    HIPCHK(hipMemcpy(c->d.gram + slot, &e->dev, sizeof(bl_gram_view), hipMemcpyHostToDevice));
  }
  hipSetDevice(c->device);
  HIPCHK(hipStreamSynchronize(c->stream));
  HIPCHK(hipMemcpy(c->d.slots + slot, &s, sizeof s, hipMemcpyHostToDevice));
  c->host_slots[slot] = s;
  return BL_OK;
}

int bl_slot_json_object(bl_ctx *c, int slot, int on) {
  if (!c || slot < 0 || slot >= c->d.max_slots || !c->slot_ready[slot])
    return fail(BL_EPARAM, "bl_slot_json_object: slot %d is not set up", slot);
  if (c->stepped[slot]) return fail(BL_EPARAM, "bl_slot_json_object: constrain the slot before its first step");
  bl_slot_dev s = c->host_slots[slot];
  if (!on) {
    s.g_on = 0;
    s.g_kind = 0;
    s.mode &= ~(BL_M_GRAMMAR | BL_M_GFULL);
  } else {
    if (c->voff.empty()) return fail(BL_EPARAM, "bl_slot_json_object: the vocabulary pieces are not set (bl_set_vocab)");
    if (s.mirostat != 0 || (s.mode & BL_M_ADAPT))
      return fail(BL_EPARAM, "stateful adaptive sampling cannot be combined with constrained decoding");
    if (s.temperature > 0.0f && s.top_n_sigma > 0.0f)
      return fail(BL_EUNSUPPORTED, "JSON-object sampling with top_n_sigma is not supported on the device");
    /* the classifier's position after the reply (the reference re-decodes it every step) */
    std::vector<uint8_t> stack(BL_JSON_DEPTH, 0);
    bl_json_pos p;
    bl_js_start(p, stack.data());
    for (int32_t id : c->reply[slot]) {
      const uint8_t *b = c->vblob.data() + c->voff[id];
      bl_js_commit(p, stack.data(), [&](int i) { return (uint32_t)b[i]; }, (int)(c->voff[id + 1] - c->voff[id]));
    }
    s.jpos = p;
    s.g_on = 1;
    s.g_kind = 1;
    s.mode |= BL_M_GRAMMAR;
    if (s.temperature > 0.0f && (s.mode & BL_M_TOPK)) {
      s.k_sel = BL_KSEL_MAX < c->d.vocab ? BL_KSEL_MAX : c->d.vocab;
      s.mode |= BL_M_GFULL;
    }
    hipSetDevice(c->device);
    HIPCHK(hipStreamSynchronize(c->stream));
    HIPCHK(hipMemcpy(c->d.jstack + (size_t)slot * BL_JSON_DEPTH, stack.data(), BL_JSON_DEPTH, hipMemcpyHostToDevice));
  }
  hipSetDevice(c->device);
  HIPCHK(hipStreamSynchronize(c->stream));
  HIPCHK(hipMemcpy(c->d.slots + slot, &s, sizeof s, hipMemcpyHostToDevice));
  c->host_slots[slot] = s;
  return BL_OK;
}

int bl_json_schema_to_gbnf(const char *schema, size_t len, char *out, size_t cap, size_t *out_len) {
  if (!schema) return fail(BL_EPARAM, "bl_json_schema_to_gbnf: no schema text");
  std::string gbnf, err;
  if (bl_schema_to_gbnf(schema, len, gbnf, err)) {
    g_err = err;
    return BL_ESCHEMA;
  }
  if (out_len) *out_len = gbnf.size();
  if (out) {
    if (cap < gbnf.size() + 1)
      return fail(BL_EPARAM, "bl_json_schema_to_gbnf: the grammar needs %zu bytes, the buffer holds %zu",
                  gbnf.size() + 1, cap);
    memcpy(out, gbnf.c_str(), gbnf.size() + 1);
  }
  return BL_OK;
}

int bl_slot_schema(bl_ctx *c, int slot, const char *schema, size_t len) {
  if (!schema) return bl_slot_grammar(c, slot, nullptr, 0);
  std::string gbnf, err;
  if (bl_schema_to_gbnf(schema, len, gbnf, err)) {
    g_err = "the JSON schema is not supported: " + err; /* the 400 body of src/server.br:738-741 */
    return BL_ESCHEMA;
  }
  return bl_slot_grammar(c, slot, gbnf.data(), gbnf.size());
}

int bl_grammar_mask(bl_ctx *c, int slot, uint32_t *d_mask_out, int32_t *forced_eos) {
  if (!c || slot < 0 || slot >= c->d.max_slots || !c->slot_ready[slot] || !c->host_slots[slot].g_on || !d_mask_out)
    return fail(BL_EPARAM, "bl_grammar_mask: slot %d has no grammar", slot);
  hipSetDevice(c->device);
  HIPCHK(hipStreamSynchronize(c->stream));
  HIPCHK(hipMemcpy(c->d_mslot, &slot, sizeof(int32_t), hipMemcpyHostToDevice));
  bl_rows rows{};
  rows.slot = c->d_mslot; /* its own row table: the bound rows of the asynchronous step stay intact */
  rows.slot_inline[0] = (int16_t)slot;
  bl_launch_gmask(c->d, rows, c->stream);
  HIPCHK(hipGetLastError());
  const size_t words = ((size_t)c->d.vocab + 31) / 32;
  HIPCHK(hipMemcpyAsync(d_mask_out, c->d.gmask, words * 4, hipMemcpyDeviceToDevice, c->stream));
  int32_t st[2] = {0, 0};
  HIPCHK(hipMemcpyAsync(&st[0], c->d.gstat, 4, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(hipMemcpyAsync(&st[1], c->d.gamb, 4, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(hipStreamSynchronize(c->stream));
  if (forced_eos) *forced_eos = (st[0] & BL_GR_FORCED) ? 1 : 0;
  if (st[1] & 2) return fail(BL_EUNSUPPORTED, "a JSON reply nested past the device's stack capacity");
  if ((st[0] & BL_GR_FAMBIG) || st[1]) return fail(BL_EGRAMMAR_AMBIG, "grammar is left-recursive or too ambiguous to match");
  if (st[0] & BL_GR_DEAD) return fail(BL_EGRAMMAR_DEAD, "the reply no longer matches the grammar");
  return BL_OK;
}

static int check_rows(bl_ctx *c, const int32_t *slots, int B) {
  if (!c || !slots || B <= 0 || B > c->d.max_rows) return fail(BL_EPARAM, "invalid row count %d", B);
  std::vector<char> seen(c->d.max_slots, 0);
  for (int i = 0; i < B; i++) {
    int s = slots[i];
    if (s < 0 || s >= c->d.max_slots || !c->slot_ready[s]) return fail(BL_EPARAM, "slot %d is not set up", s);
    if (seen[s]) return fail(BL_EPARAM, "slot %d appears twice in one step", s);
    seen[s] = 1;
  }
  return BL_OK;
}

static bool needs_gram(bl_ctx *c, const int32_t *slots, int B) {
  for (int i = 0; i < B; i++)
    if (c->host_slots[slots[i]].g_on) return true;
  return false;
}

static void mark_stepped(bl_ctx *c, const int32_t *slots, int B) {
  for (int i = 0; i < B; i++) c->stepped[slots[i]] = 1;
}

/* the exponent pass runs when a row has logprobs or a full-vocabulary rank */
static bool needs_pass2(bl_ctx *c, const int32_t *slots, int B) {
  for (int i = 0; i < B; i++) {
    const bl_slot_dev &s = c->host_slots[slots[i]];
    if (s.mode & (BL_M_LOGPROBS | BL_M_FULL | BL_M_GFULL | BL_M_ADAPT)) return true;
  }
  return false;
}

static int status_error(int st) {
  if (st & BL_SE_UNSUPPORTED) return fail(BL_EUNSUPPORTED, "a sampler stage outside the device path was reached");
  if (st & BL_SE_TIE)
    return fail(BL_ETIE, "the draw landed on equal logits past the device's heap-order simulation");
  if (st & BL_SE_SIGMA)
    return fail(BL_ETIE, "top_n_sigma: the standard deviation lies within the reference's float64 rounding error of a "
                         "float32 rounding boundary");
  if (st & BL_SE_CAND_FULL) return fail(BL_EDEVICE, "candidate buffer overflow");
  if (st & BL_SE_EMPTY) return fail(BL_EEMPTY, "sample_candidates: empty or mismatched candidates");
  if (st & BL_SE_GDEAD) return fail(BL_EGRAMMAR_DEAD, "the reply no longer matches the grammar");
  if (st & BL_SE_GAMBIG) return fail(BL_EGRAMMAR_AMBIG, "grammar is left-recursive or too ambiguous to match");
  if (st & BL_SE_GREJECT) return fail(BL_EGRAMMAR_REJECT, "the grammar rejected every vocabulary token");
  if (st & BL_SE_JREJECT) return fail(BL_EGRAMMAR_REJECT, "JSON response grammar rejected every vocabulary token");
  return BL_OK;
}

int bl_slot_status(bl_ctx *c, int slot) {
  if (!c || slot < 0 || slot >= c->d.max_slots) return fail(BL_EPARAM, "bl_slot_status: invalid arguments");
  if (!c->slot_ready[slot]) return fail(BL_EPARAM, "slot %d is not set up", slot);
  hipSetDevice(c->device);
  int32_t err = 0;
  const int32_t zero = 0;
  int32_t *dp = &c->d.slots[slot].err;
  HIPCHK(hipStreamSynchronize(c->stream));
  HIPCHK(hipMemcpy(&err, dp, sizeof err, hipMemcpyDeviceToHost));
  HIPCHK(hipMemcpy(dp, &zero, sizeof zero, hipMemcpyHostToDevice));
  return status_error(err);
}

static bl_rows make_rows(bl_ctx *c, bool with_skip, int commit, int top_stride, bool bound = false) {
  bl_rows r{};
  const int32_t *h = bound ? c->h_bound : c->h_slot;
  r.slot = bound ? c->d_bound : c->d_slot;
  for (int i = 0; i < BL_ROWS_INLINE && i < c->d.max_rows; i++) r.slot_inline[i] = (int16_t)h[i];
  r.rng_skip = with_skip ? c->d_skip : nullptr;
  r.commit = commit;
  r.tok = c->d_tok;
  r.lp = c->d_lp;
  r.top_ids = c->d_top_ids;
  r.top_lp = c->d_top_lp;
  r.top_stride = top_stride;
  r.status = c->d_status;
  return r;
}

int bl_sample_step(bl_ctx *c, const int32_t *slots, int B, const float *d_logits, int64_t ld, int32_t *tokens,
                   float *logprobs, int32_t *top_ids, float *top_logprobs, int top_stride) {
  int rc = check_rows(c, slots, B);
  if (rc) return rc;
  if (!tokens || !d_logits || ld < c->d.vocab) return fail(BL_EPARAM, "bl_sample_step: invalid buffers");
  if (top_stride < 0 || top_stride > 256) return fail(BL_EPARAM, "top_stride must be in 0..256");
  hipSetDevice(c->device);
  memcpy(c->h_slot, slots, B * sizeof(int32_t));
  /* rows past the inline slot indices read the device table */
  if (B > BL_ROWS_INLINE)
    HIPCHK(hipMemcpyAsync(c->d_slot, c->h_slot, B * sizeof(int32_t), hipMemcpyHostToDevice, c->stream));
  bl_rows rows = make_rows(c, false, 1, top_stride > 0 ? top_stride : 1);
  const int ts = top_stride;
  rows.tok = c->d_out;
  rows.status = c->d_out + B;
  rows.lp = reinterpret_cast<float *>(c->d_out + 2 * B);
  if (ts > 0) {
    rows.top_ids = c->d_out + 3 * B;
    rows.top_lp = reinterpret_cast<float *>(c->d_out + 3 * B + B * ts);
  }
  mark_stepped(c, slots, B);
  bl_launch_step(c->d, d_logits, ld, rows, B, needs_pass2(c, slots, B), needs_gram(c, slots, B), c->stream, nullptr);
  HIPCHK(hipGetLastError());
  HIPCHK(hipMemcpyAsync(c->h_out, c->d_out, (size_t)(3 * B + 2 * B * ts) * 4, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(wait_stream(c->stream));
  const int32_t *h = c->h_out;
  int st = 0;
  for (int i = 0; i < B; i++) st |= h[B + i];
  memcpy(tokens, h, B * sizeof(int32_t));
  if (logprobs) memcpy(logprobs, h + 2 * B, B * sizeof(float));
  if (top_ids && ts > 0) memcpy(top_ids, h + 3 * B, (size_t)B * ts * 4);
  if (top_logprobs && ts > 0) memcpy(top_logprobs, h + 3 * B + B * ts, (size_t)B * ts * 4);
  return status_error(st);
}

/* ------------------------------------------------------------------ allocation-free step */
/* The allocation-free step's slot state and workspace. Each device that runs the call holds its own copy
 * for the life of the process; host code takes its device address from hipGetSymbolAddress, once per
 * device, and never passes the name itself to a kernel or a copy. */
static __device__ __align__(256) unsigned char scratch[BL_NOALLOC_BYTES];
#define BL_MAX_DEVICES 64
static std::mutex g_scratch_mu;
static unsigned char *g_scratch[BL_MAX_DEVICES];

/* the device address of `scratch` on the current device `dev` */
static int scratch_of(int dev, unsigned char **out) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch[dev]) {
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(BL_EDEVICE, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    g_scratch[dev] = (unsigned char *)p;
  }
  *out = g_scratch[dev];
  return BL_OK;
}

int bl_sample_rows_noalloc(int device, void *stream, const bl_params *params, uint64_t *rng_states, int B,
                           const float *d_logits, int64_t ld, int vocab, int32_t *tokens, float *logprobs,
                           int32_t *top_ids, float *top_logprobs, int top_stride) {
  if (device < 0 || device >= BL_MAX_DEVICES || !params || !rng_states || !d_logits || !tokens)
    return fail(BL_EPARAM, "bl_sample_rows_noalloc: invalid arguments");
  if (B <= 0 || B > BL_NOALLOC_ROWS)
    return fail(BL_EPARAM, "bl_sample_rows_noalloc: %d rows (1..%d)", B, BL_NOALLOC_ROWS);
  if (vocab <= 0 || vocab > BL_MAX_CHUNKS * BL_CH || ld < vocab)
    return fail(BL_EPARAM, "bl_sample_rows_noalloc: invalid vocabulary %d (ld %lld)", vocab, (long long)ld);
  if (top_stride < 0 || top_stride > 256) return fail(BL_EPARAM, "top_stride must be in 0..256");
  bl_slot_dev hs[BL_NOALLOC_ROWS];
  int32_t tbl[BL_NOALLOC_ROWS];
  for (int i = 0; i < B; i++) {
    hs[i] = bl_slot_dev{};
    int rc = configure(vocab, params + i, hs[i]);
    if (rc) return rc;
    hs[i].rng = rng_states[i];
    tbl[i] = i;
  }
  HIPCHK(hipSetDevice(device));
  unsigned char *base = nullptr;
  int rc = scratch_of(device, &base);
  if (rc) return rc;
  /* carve a context's buffers for B slots and rows out of the array, then the row table and outputs */
  size_t off = 0;
  auto take = [&](auto *&p, size_t n) {
    using T = std::remove_reference_t<decltype(*p)>;
    off = (off + 255) & ~(size_t)255;
    const size_t bytes = n * sizeof(T) + 16;
    if (off + bytes > BL_NOALLOC_BYTES) return false;
    p = reinterpret_cast<T *>(base + off);
    off += bytes;
    return true;
  };
  bl_dev d{};
  int32_t *d_tbl = nullptr, *d_out = nullptr;
  const int ts = top_stride, tsa = ts > 0 ? ts : 1; /* rows with logprobs write one alternative at stride 0 */
  if (!dev_layout(d, B, B, vocab, take) || !take(d_tbl, B) || !take(d_out, (size_t)B * (3 + 2 * tsa)))
    return fail(BL_EPARAM, "bl_sample_rows_noalloc: %d rows of %d tokens need more than the %u bytes of its array", B,
                vocab, (unsigned)BL_NOALLOC_BYTES);
  hipStream_t st = (hipStream_t)stream;
  /* the array keeps the previous call's contents: slot state and records start afresh (no records, no
   * token has one, an empty window) */
  HIPCHK(hipMemcpyAsync(d.slots, hs, B * sizeof(bl_slot_dev), hipMemcpyHostToDevice, st));
  HIPCHK(hipMemcpyAsync(d_tbl, tbl, B * sizeof(int32_t), hipMemcpyHostToDevice, st));
  HIPCHK(hipMemsetAsync(d.rcnt, 0, (size_t)B * d.nb * sizeof(int32_t), st));
  HIPCHK(hipMemsetAsync(d.ridx, 0xFF, (size_t)B * vocab * sizeof(int16_t), st));
  bl_rows rows{};
  rows.slot = d_tbl;
  for (int i = 0; i < B; i++) rows.slot_inline[i] = (int16_t)i;
  rows.commit = 1; /* the commit is what stores the advanced RNG state */
  rows.tok = d_out;
  rows.status = d_out + B;
  rows.lp = reinterpret_cast<float *>(d_out + 2 * B);
  rows.top_stride = tsa;
  rows.top_ids = d_out + 3 * B;
  rows.top_lp = reinterpret_cast<float *>(d_out + 3 * B + B * tsa);
  bool pass2 = false;
  for (int i = 0; i < B; i++) pass2 |= (hs[i].mode & (BL_M_LOGPROBS | BL_M_FULL | BL_M_GFULL | BL_M_ADAPT)) != 0;
  bl_launch_step(d, d_logits, ld, rows, B, pass2, false, st, nullptr);
  HIPCHK(hipGetLastError());
  int32_t status[BL_NOALLOC_ROWS];
  HIPCHK(hipMemcpyAsync(tokens, d_out, B * sizeof(int32_t), hipMemcpyDeviceToHost, st));
  HIPCHK(hipMemcpyAsync(status, d_out + B, B * sizeof(int32_t), hipMemcpyDeviceToHost, st));
  if (logprobs) HIPCHK(hipMemcpyAsync(logprobs, d_out + 2 * B, B * sizeof(float), hipMemcpyDeviceToHost, st));
  if (top_ids && ts > 0)
    HIPCHK(hipMemcpyAsync(top_ids, d_out + 3 * B, (size_t)B * ts * 4, hipMemcpyDeviceToHost, st));
  if (top_logprobs && ts > 0)
    HIPCHK(hipMemcpyAsync(top_logprobs, d_out + 3 * B + B * ts, (size_t)B * ts * 4, hipMemcpyDeviceToHost, st));
  HIPCHK(hipMemcpyAsync(hs, d.slots, B * sizeof(bl_slot_dev), hipMemcpyDeviceToHost, st));
  HIPCHK(wait_stream(st));
  int err = 0;
  for (int i = 0; i < B; i++) {
    err |= status[i];
    rng_states[i] = hs[i].rng;
  }
  return status_error(err);
}

int bl_bind_rows(bl_ctx *c, const int32_t *slots, int B) {
  int rc = check_rows(c, slots, B);
  if (rc) return rc;
  hipSetDevice(c->device);
  HIPCHK(hipStreamSynchronize(c->stream)); /* a step in flight may still read the previous table */
  HIPCHK(hipMemcpy(c->d_bound, slots, B * sizeof(int32_t), hipMemcpyHostToDevice));
  memcpy(c->h_bound, slots, B * sizeof(int32_t));
  c->bound_B = B;
  mark_stepped(c, slots, B);
  return BL_OK;
}

int bl_sample_step_async(bl_ctx *c, int B, const float *d_logits, int64_t ld, int32_t *d_tokens, float *d_logprobs,
                         int32_t *d_top_ids, float *d_top_logprobs, int top_stride) {
  if (!c || B != c->bound_B || B <= 0) return fail(BL_EPARAM, "bl_sample_step_async: rows not bound (bl_bind_rows)");
  if (!d_logits || !d_tokens || ld < c->d.vocab || top_stride < 0 || top_stride > 256)
    return fail(BL_EPARAM, "bl_sample_step_async: invalid buffers");
  bl_rows rows = make_rows(c, false, 1, top_stride > 0 ? top_stride : 1, true);
  rows.tok = d_tokens;
  rows.lp = d_logprobs;
  rows.top_ids = d_top_ids ? d_top_ids : c->d_top_ids;
  rows.top_lp = d_top_logprobs ? d_top_logprobs : c->d_top_lp;
  hipEvent_t *ev = nullptr;
  if (c->timing) {
    if (!c->ev[0])
      for (int k = 0; k < 6; k++) HIPCHK(hipEventCreate(&c->ev[k]));
    ev = c->ev;
  }
  const bool pass2 = needs_pass2(c, c->h_bound, B);
  bl_launch_step(c->d, d_logits, ld, rows, B, pass2, needs_gram(c, c->h_bound, B), c->stream, ev);
  HIPCHK(hipGetLastError());
  if (ev) {
    /* each kernel's own duration in this step, accumulated (the caller asked for timing: synchronous) */
    HIPCHK(hipEventSynchronize(ev[5]));
    for (int k = 0; k < 3; k++) {
      if (k == 1 && !pass2) continue;
      float ms = 0.0f;
      HIPCHK(hipEventElapsedTime(&ms, ev[2 * k], ev[2 * k + 1]));
      c->kernel_ms[k] += ms;
    }
    c->timed_steps += 1;
  }
  return BL_OK;
}

int bl_step_graph_create(bl_ctx *c, int B, const float *d_logits, int64_t ld, int32_t *d_tokens, float *d_logprobs,
                         int32_t *d_top_ids, float *d_top_logprobs, int top_stride, void **graph_out) {
  if (!c || !graph_out) return fail(BL_EPARAM, "bl_step_graph_create: invalid arguments");
  if (c->timing) return fail(BL_EPARAM, "bl_step_graph_create: kernel timing is enabled");
  hipSetDevice(c->device);
  hipGraph_t g = nullptr;
  hipGraphExec_t ge = nullptr;
  HIPCHK(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
  const int rc = bl_sample_step_async(c, B, d_logits, ld, d_tokens, d_logprobs, d_top_ids, d_top_logprobs, top_stride);
  const std::string msg = g_err;
  hipError_t e = hipStreamEndCapture(c->stream, &g);
  if (rc != BL_OK) {
    if (e == hipSuccess && g) hipGraphDestroy(g);
    g_err = msg;
    return rc;
  }
  if (e != hipSuccess) return fail(BL_EDEVICE, "hipStreamEndCapture: %s", hipGetErrorString(e));
  e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
  hipGraphDestroy(g);
  if (e != hipSuccess) return fail(BL_EDEVICE, "hipGraphInstantiate: %s", hipGetErrorString(e));
  *graph_out = (void *)ge;
  return BL_OK;
}

int bl_step_graph_launch(bl_ctx *c, void *graph) {
  if (!c || !graph) return fail(BL_EPARAM, "bl_step_graph_launch: invalid arguments");
  HIPCHK(hipGraphLaunch((hipGraphExec_t)graph, c->stream));
  return BL_OK;
}

int bl_step_graph_destroy(void *graph) {
  if (graph) HIPCHK(hipGraphExecDestroy((hipGraphExec_t)graph));
  return BL_OK;
}

int bl_stream_sync(bl_ctx *c) {
  if (!c) return fail(BL_EPARAM, "null context");
  HIPCHK(wait_stream(c->stream));
  return BL_OK;
}

int bl_set_timing(bl_ctx *c, int enable) {
  if (!c) return fail(BL_EPARAM, "null context");
  c->timing = enable != 0;
  for (int k = 0; k < 3; k++) c->kernel_ms[k] = 0.0;
  c->timed_steps = 0;
  return BL_OK;
}

int bl_get_timing(bl_ctx *c, double *ms_total3, int64_t *steps) {
  if (!c || !ms_total3 || !steps) return fail(BL_EPARAM, "bl_get_timing: invalid arguments");
  for (int k = 0; k < 3; k++) ms_total3[k] = c->kernel_ms[k];
  *steps = c->timed_steps;
  return BL_OK;
}

int bl_spec_verify(bl_ctx *c, const int32_t *slots, int B, int k, const float *d_rows, int64_t ld,
                   const int32_t *drafts, int32_t *tokens, int32_t *accepted) {
  int rc = check_rows(c, slots, B);
  if (rc) return rc;
  const int R = B * (k + 1);
  if (k < 0 || R > c->d.max_rows || !d_rows || !tokens || !accepted || ld < c->d.vocab || (k > 0 && !drafts) ||
      (int64_t)B * k > 4096)
    return fail(BL_EPARAM, "bl_spec_verify: invalid arguments (B %d, k %d)", B, k);
  bool pen = false; /* a sequence whose rows' penalties depend on the drafts before them */
  for (int b = 0; b < B; b++) {
    const bl_slot_dev &s = c->host_slots[slots[b]];
    if (k > 0 && (s.fp_on || s.rep_on)) {
      if (2 * k > BL_SPEC_DCAP)
        return fail(BL_EUNSUPPORTED, "speculative rows with history-dependent penalties take at most %d drafts",
                    BL_SPEC_DCAP / 2);
      for (int i = 0; i < k; i++)
        if (drafts[b * k + i] < 0 || drafts[b * k + i] >= c->d.vocab)
          return fail(BL_EPARAM, "bl_spec_verify: draft token %d is outside the vocabulary", drafts[b * k + i]);
      pen = true;
    }
    if (s.g_on) return fail(BL_EUNSUPPORTED, "speculative rows of a grammar-constrained slot are not supported on the device");
    /* each row's draw starts at its position in the RNG chain; an XTC chance draw would shift the rest */
    if (k > 0 && s.temperature > 0.0f && s.xtc_probability > 0.0f && s.xtc_threshold <= 0.5f)
      return fail(BL_EUNSUPPORTED, "speculative rows with XTC are not supported on the device");
    if (k > 0 && (s.mode & (BL_M_MIRO | BL_M_ADAPT)))
      return fail(BL_EUNSUPPORTED, "speculative rows with mirostat or adaptive-p are not supported on the device");
    /* row i's DRY window would hold drafts[0..i) */
    if (k > 0 && s.dry_on) return fail(BL_EUNSUPPORTED, "speculative rows with DRY are not supported on the device");
    /* with dynatemp_range >= temperature the effective temperature can reach 0, and such a row makes no draw
     * (src/sampling.br:576-582): the rows after it would start one draw early in the RNG chain */
    if (k > 0 && s.temperature > 0.0f && s.dynatemp_range > 0.0f && s.dynatemp_range >= s.temperature)
      return fail(BL_EUNSUPPORTED, "speculative rows with dynatemp_range >= temperature are not supported on the device");
  }
  hipSetDevice(c->device);
  /* one block in: row slots [0, R), RNG skips [R, 2R), drafts [2R, 2R + Bk), sequence slots [2R + Bk, 2R + Bk + B) */
  const int nd = B * k;
  int32_t *hin = c->h_spec_in;
  for (int b = 0; b < B; b++)
    for (int i = 0; i <= k; i++) {
      hin[b * (k + 1) + i] = slots[b];
      hin[R + b * (k + 1) + i] = i;
      c->h_slot[b * (k + 1) + i] = slots[b];
    }
  if (nd > 0) memcpy(hin + 2 * R, drafts, (size_t)nd * 4);
  memcpy(hin + 2 * R + nd, slots, B * sizeof(int32_t));
  HIPCHK(hipMemcpyAsync(c->d_spec_in, hin, ((size_t)2 * R + nd + B) * sizeof(int32_t), hipMemcpyHostToDevice,
                        c->stream));
  const int32_t *d_rslot = c->d_spec_in, *d_rskip = c->d_spec_in + R, *d_drafts = c->d_spec_in + 2 * R,
                *d_sslot = c->d_spec_in + 2 * R + nd;
  /* one block out: tokens [0, R), statuses [R, 2R), accepted lengths [2R, 2R + B) */
  int32_t *d_tok = c->d_spec_out, *d_stat = c->d_spec_out + R, *d_acc = c->d_spec_out + 2 * R;
  bl_rows rows = make_rows(c, true, 0, 1);
  rows.slot = d_rslot;
  rows.rng_skip = d_rskip;
  rows.tok = d_tok;
  rows.status = d_stat;
  rows.lp = nullptr; /* no logprobs are returned for speculative rows */
  if (pen) {
    hipLaunchKernelGGL(bl_k_spec_delta, dim3(B), dim3(BL_SPEC_DCAP / 2 + 64), 0, c->stream, c->d, d_sslot, d_drafts, k,
                       c->d_delta, c->d_delta_n);
    HIPCHK(hipGetLastError());
    rows.delta = c->d_delta;
    rows.delta_n = c->d_delta_n;
  }
  mark_stepped(c, slots, B);
  bl_launch_step(c->d, d_rows, ld, rows, R, needs_pass2(c, slots, B), false, c->stream, nullptr);
  hipLaunchKernelGGL(bl_k_spec_commit, dim3(B), dim3(64), 0, c->stream, c->d, d_sslot, d_drafts, k, d_tok, d_stat, R,
                     d_acc);
  HIPCHK(hipGetLastError());
  HIPCHK(hipMemcpyAsync(c->h_spec_out, c->d_spec_out, ((size_t)2 * R + B) * sizeof(int32_t), hipMemcpyDeviceToHost,
                        c->stream));
  HIPCHK(wait_stream(c->stream));
  const int32_t *hout = c->h_spec_out;
  int st = 0;
  for (int i = 0; i < R; i++) st |= hout[R + i];
  memcpy(tokens, hout, R * sizeof(int32_t));
  if ((rc = status_error(st))) return rc;
  memcpy(accepted, hout + 2 * R, B * sizeof(int32_t));
  return BL_OK;
}

int bl_synth_logits(bl_ctx *c, float *d_out, int64_t ld, int cfg, int64_t seed, int64_t step, int rows, int vocab) {
  if (!c || !d_out || rows <= 0 || vocab <= 0 || ld < vocab) return fail(BL_EPARAM, "bl_synth_logits: invalid arguments");
  hipSetDevice(c->device);
  bl_launch_synth(d_out, ld, cfg, seed, step, rows, vocab, c->stream);
  HIPCHK(hipGetLastError());
  if (cfg == 1) {
    std::vector<int32_t> ids = blw::c1_bump_ids(seed, step, vocab);
    for (int r = 0; r < rows; r++) {
      HIPCHK(hipMemcpyAsync(c->d_commit_toks, ids.data(), ids.size() * 4, hipMemcpyHostToDevice, c->stream));
      hipLaunchKernelGGL(bl_k_bump, dim3(1), dim3(64), 0, c->stream, d_out + (int64_t)r * ld, c->d_commit_toks,
                         (int)ids.size(), 8.0f);
      HIPCHK(hipStreamSynchronize(c->stream));
    }
  }
  HIPCHK(hipStreamSynchronize(c->stream));
  return BL_OK;
}

int bl_workload_ids(int kind, int cfg, int64_t seed, int row, int n, int vocab, int32_t *out) {
  if (n < 0 || vocab <= 0 || !out || (kind != 0 && kind != 1)) return fail(BL_EPARAM, "bl_workload_ids: invalid arguments");
  std::vector<int32_t> v = kind == 0 ? blw::uniform_ids(cfg, seed, row, n, vocab) : blw::zipf_ids(cfg, seed, row, n, vocab, 1.1);
  memcpy(out, v.data(), v.size() * sizeof(int32_t));
  return BL_OK;
}

int bl_workload_bias(int cfg, int64_t seed, int row, int n, int vocab, float lo, float hi, int32_t *ids, float *vals) {
  if (n < 0 || n > vocab || !ids || !vals) return fail(BL_EPARAM, "bl_workload_bias: invalid arguments");
  std::vector<int32_t> i;
  std::vector<float> v;
  blw::bias_list(cfg, seed, row, n, vocab, lo, hi, i, v);
  memcpy(ids, i.data(), i.size() * sizeof(int32_t));
  memcpy(vals, v.data(), v.size() * sizeof(float));
  return BL_OK;
}

int bl_workload_c3_vocab(int64_t seed, int vocab, uint8_t *blob, size_t blob_cap, uint32_t *offsets, int32_t *eos_id) {
  if (vocab <= 257 || !offsets || !eos_id) return fail(BL_EPARAM, "bl_workload_c3_vocab: invalid arguments");
  std::vector<uint8_t> b;
  std::vector<uint32_t> off;
  int32_t eos = -1;
  blw::c3_vocab(seed, vocab, b, off, eos);
  if (!blob || b.size() > blob_cap) return fail(BL_EPARAM, "bl_workload_c3_vocab: blob needs %zu bytes", b.size());
  memcpy(blob, b.data(), b.size());
  memcpy(offsets, off.data(), off.size() * sizeof(uint32_t));
  *eos_id = eos;
  return (int)b.size();
}

int bl_workload_drafts(int64_t seed, int64_t step, int seq, const int32_t *argmax, int k, int vocab, int32_t *out) {
  if (k < 0 || !argmax || !out) return fail(BL_EPARAM, "bl_workload_drafts: invalid arguments");
  std::vector<int32_t> d = blw::c5_drafts(seed, step, seq, argmax, k, vocab);
  memcpy(out, d.data(), d.size() * sizeof(int32_t));
  return BL_OK;
}

int bl_math_digest(bl_ctx *c, int fn, uint32_t first_block, int n_blocks, uint64_t *out) {
  if (!c || fn < 0 || fn > 5 || n_blocks <= 0 || (uint64_t)first_block + n_blocks > 4096 || !out)
    return fail(BL_EPARAM, "bl_math_digest: invalid arguments");
  hipSetDevice(c->device);
  unsigned long long *d = nullptr;
  HIPCHK(hipMalloc((void **)&d, n_blocks * sizeof(unsigned long long)));
  bl_launch_math_digest(fn, first_block, n_blocks, d, c->stream);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = hipMemcpyAsync(out, d, n_blocks * sizeof(uint64_t), hipMemcpyDeviceToHost, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  (void)hipFree(d);
  if (e != hipSuccess) return fail(BL_EDEVICE, "bl_math_digest: %s", hipGetErrorString(e));
  return BL_OK;
}

} /* extern "C" */
