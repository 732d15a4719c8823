/*
 * bl_select.h — C ABI of boring-llm's per-step token selection on MI355X (libbl_select.so).
 *
 * The reference runs this path as Boring functions on host rows (src/sampling.br, src/grammar.br,
 * src/server.br:939-1231); its generated Rust target would declare these functions in an
 * `extern "C"` block and keep the Boring-level API unchanged. Every entry point below names the
 * reference function(s) it replaces. Plain C types only; logits are borrowed device pointers.
 *
 * Threading: a context is used by one host thread at a time; contexts are independent. Calls are
 * ordered on the context's stream; the synchronous entry points return once results are in host
 * memory. Errors: a negative BL_E* code, with the reference's message from bl_last_error().
 */
#ifndef BL_SELECT_H
#define BL_SELECT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct bl_ctx bl_ctx;

enum {
  BL_OK = 0,
  BL_EPARAM = -1,          /* a value outside the request validation ranges (src/openai.br:1652-1890) */
  BL_EDEVICE = -2,         /* HIP runtime failure */
  BL_EEMPTY = -3,          /* "sample_candidates: empty or mismatched candidates" (src/sampling.br:495) */
  BL_EGRAMMAR = -4,        /* GBNF parse error (src/grammar.br:57-323) */
  BL_EGRAMMAR_DEAD = -5,   /* "the reply no longer matches the grammar" (src/server.br:320) */
  BL_EGRAMMAR_REJECT = -6, /* "the grammar rejected every vocabulary token" (src/server.br:361) */
  BL_EGRAMMAR_AMBIG = -7,  /* "grammar is left-recursive or too ambiguous to match" (src/grammar.br:354) */
  BL_EUNSUPPORTED = -8,    /* a sampler stage this library does not run on the device yet: DRY windows above
                              2048 tokens or a negative dry_allowed_length (rejected by bl_slot_reset); XTC,
                              mirostat, adaptive-p, DRY or a grammar on speculative rows, or more than 128
                              drafts with history-dependent penalties; typical_p over a list that is neither
                              complete nor a full-vocabulary rank; a mirostat draw that falls through to a prefix end past
                              the candidates within 17.6 T of the maximum */
  BL_ETIE = -9,            /* a draw on equal logits whose heap order is past the device simulation (more than
                              8192 values at or above the tied one), equal allowed values of a grammar row
                              (the greedy maxima, or a draw) where the heap's order applies with more than 4096
                              values at or above them (or, greedy, with top_n_sigma), post-sampling
                              alternatives of a full-vocabulary rank that meet equal values, or a
                              top_n_sigma whose float32 sigma the reference's float64 rounding error leaves
                              undecided (the sigma within ~1e-11 relative of a float32 rounding boundary) */
  BL_ESCHEMA = -10         /* a JSON schema that does not parse (src/json.br json_parse messages) or that
                              json_schema_to_gbnf rejects (src/schema_grammar.br messages) */
};

/* SamplingParams (src/model.br:1565-1584) + the per-request server fields (src/server.br:665-760).
 * Defaults are greedy_params() (src/model.br:1586-1589). */
typedef struct {
  float temperature;       /* <= 0: greedy */
  float dynatemp_range;
  float dynatemp_exponent;
  float top_n_sigma;       /* <= 0: off; with temperature > 0, keep values >= max - n * sigma (population sigma
                              of the values above -1e29, src/sampling.br:376-407) */
  int32_t top_k;           /* <= 0 or >= vocab: full-vocabulary rank */
  float typical_p;
  float top_p;
  float min_p;
  float xtc_probability;   /* XTC (src/sampling.br:552-572): on when > 0 and xtc_threshold <= 0.5 */
  float xtc_threshold;
  int32_t min_keep;
  float repeat_penalty;    /* 1: off */
  int32_t repeat_last_n;   /* 0: off, -1: whole history */
  float dry_multiplier;    /* 0: off */
  float dry_base;
  int32_t dry_allowed_length;
  int32_t dry_penalty_last_n;
  float frequency_penalty; /* server extras */
  float presence_penalty;
  int32_t logprobs;        /* 1: return the chosen token's logprob (wants_logprobs) */
  int32_t n_probs;         /* alternatives returned with logprobs (0..256) */
  int32_t post_sampling_probs; /* with logprobs: the draw's probabilities instead (src/server.br:1015-1025): the
                                  chosen token's probability and those of the first n_probs candidates of the
                                  drawn range; alternatives past the range read id -1, probability 0 */
  int32_t ignore_eos;
  float final_softcap;     /* model tail (src/model.br:973-984): 0 = off */
  float logit_mul;         /* model tail: 1 = off */
  int32_t mirostat;        /* server extras (src/server.br:684-686): 0 off, 1 = sample_mirostat_v1
                              (src/sampling.br:676-700), 2 = sample_mirostat_v2 (:663-674) */
  float mirostat_tau;      /* target surprise; the slot's mu starts at 2 tau (src/server.br:936) */
  float mirostat_eta;
  float adaptive_target;   /* adaptive-p (src/sampling.br:705-740, src/server.br:953-963): on when >= 0 (it then
                              replaces the sampler chain, at any temperature); default -1 */
  float adaptive_decay;    /* the running average's decay; default 0.9 */
} bl_params;

void bl_params_default(bl_params *p);

/* Context on `device` for up to `max_slots` (<= 32767) concurrent requests and `max_rows` rows per call,
 * over a vocabulary of `vocab` tokens (<= 4,194,304). Replaces nothing in the reference (it holds no
 * device state). Device memory: about 20 * vocab bytes per slot (a 16-byte record slot and a 4-byte index
 * per token: 3 MB at V = 151936, 5.2 MB at V = 262144), plus windows and per-row buffers; BL_EDEVICE
 * when an allocation fails. */
int bl_create(int device, int max_slots, int max_rows, int vocab, bl_ctx **out);
void bl_destroy(bl_ctx *ctx);
const char *bl_last_error(void);
/* The HIP stream the context's work is ordered on (hipStream_t); NULL selects the context's own. */
int bl_set_stream(bl_ctx *ctx, void *stream);

/* End-of-generation registry: src/sampling.br:200-237 (set_eog_tokens / is_eog_token). Every step reads the
 * current registry (ignore_eos suppression, the grammar's end of sequence); a step graph captured before
 * a change holds the old registry's length: create a new graph after bl_set_eog. */
int bl_set_eog(bl_ctx *ctx, int32_t eos_id, const int32_t *eog_ids, int n_eog);

/* Request seeds (host arithmetic, no device work; callable without a GPU):
 * bl_resolve_seed replaces resolve_seed (src/sampling.br:21-33): a non-negative request seed is kept; a
 * negative one is chosen from `entropy` (the caller's wall-clock bits) and the server's request counter by
 * one xorshift round, masked to 31 bits, 0 mapped to 1.
 * bl_seed_rng replaces seed_rng (:35-40): the initial xorshift state of a seed, the value bl_slot_reset
 * takes as rng_state. */
int64_t bl_resolve_seed(int64_t requested, uint64_t entropy, int64_t request_counter);
uint64_t bl_seed_rng(int64_t seed);

/* A new request on `slot`: seed_rng (src/sampling.br:35-40) is the caller's rng_state; history =
 * prompt + reply tokens (repeat penalty / DRY, src/sampling.br:65-85), reply = reply tokens
 * (frequency / presence, :91-107), logit_bias as parallel arrays (src/server.br:150-185, :940). */
int bl_slot_reset(bl_ctx *ctx, int slot, const bl_params *p, uint64_t rng_state, const int32_t *history, int n_hist,
                  const int32_t *reply, int n_reply, const int32_t *bias_ids, const float *bias_vals, int n_bias);

/* The request's DRY sequence breakers, already tokenised (request_dry_breakers, src/server.br:187-232):
 * n breakers of lens[i] tokens each, concatenated in `tokens`, in the request's order (the order decides where
 * the repeated suffix may start, src/sampling.br:121-134). bl_slot_reset clears them; call this after it and
 * before the slot's first step. One-token breakers are unlimited; at most 512 longer ones of up to 24 tokens
 * (BL_EUNSUPPORTED past that). */
int bl_slot_dry_breakers(bl_ctx *ctx, int slot, const int32_t *tokens, const int32_t *lens, int n);
/* The slot's current xorshift64 state (Rng.state, src/sampling.br:18-19). */
int bl_slot_rng(bl_ctx *ctx, int slot, uint64_t *state);
/* Append tokens chosen elsewhere to the slot history (tokens.push / reply_tokens.push,
 * src/server.br:1004, :1037). BL_EPARAM for a slot that bl_slot_reset has not set up. */
int bl_slot_commit(bl_ctx *ctx, int slot, const int32_t *toks, int n);
/* The failures of the slot's rows since the previous call or its reset (the error a synchronous step would
 * have returned for them, with its message), cleared by the call: how a caller of bl_sample_step_async or
 * of a step graph learns why a row's token came back as -1. Replaces the `throws` of the reference's
 * sampler calls (src/sampling.br:495, src/server.br:318-361) for steps that do not return to the host. */
int bl_slot_status(bl_ctx *ctx, int slot);

/* Vocabulary pieces for grammar-constrained slots: token t's bytes are blob[offsets[t] .. offsets[t+1]),
 * n_tokens = the context's vocabulary (Tokenizer.decode / piece_bytes, src/tokenizer.br:122-151,
 * :227-240; special tokens as their literal UTF-8). The grammar's end-of-sequence token is the
 * eos_id of bl_set_eog. */
int bl_set_vocab(bl_ctx *ctx, const uint8_t *blob, const uint32_t *offsets, int n_tokens);

/* Attach a GBNF grammar to a slot set up by bl_slot_reset, before its first step (the request's
 * `grammar` field; parse_gbnf src/grammar.br:309-323). The slot's steps then follow
 * sample_grammar_token (src/server.br:308-361): forced EOS when the reply is complete and cannot
 * continue, otherwise the allowed candidates in rank order: the first (temperature <= 0), or a draw of
 * sample_candidates over them (temperature > 0: the allowed entries of top_k_select(k), k widened 4-fold
 * while none is allowed; of the whole ranking without top_k). gbnf = NULL detaches. Errors: BL_EGRAMMAR
 * (parse, with the reference's message), BL_EGRAMMAR_AMBIG, BL_EUNSUPPORTED (top_n_sigma with
 * temperature > 0, or a grammar whose reachable automaton exceeds 65536 states: a recursive one). A
 * sampled step returns BL_EUNSUPPORTED when the widening reaches a level whose ranks go past the values
 * within the candidate span of the row maximum, and BL_ETIE when a whole-vocabulary draw lands on equal
 * allowed values with more than 4096 values at or above them. */
int bl_slot_grammar(bl_ctx *ctx, int slot, const char *gbnf, size_t len);

/* `response_format: {type: json_object}` on a slot set up by bl_slot_reset, before its first step (on = 0
 * lifts it): the steps follow sample_json_token (src/server.br:261-304) with the classifier
 * json_object_prefix_state (src/json.br:394-426): end of sequence once the reply is a complete object,
 * otherwise the candidates whose piece keeps the reply a viable object prefix, in rank order (greedy or
 * sampled, with the K×4 widening of bl_slot_grammar). Needs bl_set_vocab. Errors: BL_EPARAM (mirostat),
 * BL_EUNSUPPORTED (top_n_sigma with temperature > 0). A step returns BL_EGRAMMAR_REJECT ("JSON response
 * grammar rejected every vocabulary token") when no token is allowed, and BL_EUNSUPPORTED past 1024 nested
 * containers or for a token that opens more than 32. */
int bl_slot_json_object(bl_ctx *ctx, int slot, int on);

/* JSON Schema -> GBNF (json_schema_to_gbnf, src/schema_grammar.br:313-337, over the schema text parsed as
 * src/json.br's json_parse does; the text must be UTF-8). Writes the NUL-terminated grammar into `out`
 * (`cap` bytes) and its length into *out_len (either may be NULL: out = NULL only reports the length).
 * BL_ESCHEMA with the reference's message; BL_EPARAM when `cap` is too small. */
int bl_json_schema_to_gbnf(const char *schema, size_t len, char *out, size_t cap, size_t *out_len);

/* Attach the grammar of a JSON schema to a slot: a request's response_format json_schema (src/server.br:733-745:
 * the schema is compiled to GBNF, then parsed as the slot's grammar), with bl_slot_grammar's rules and errors.
 * BL_ESCHEMA reads "the JSON schema is not supported: <message>" (src/server.br:738-741). schema = NULL
 * detaches. */
int bl_slot_schema(bl_ctx *ctx, int slot, const char *schema, size_t len);

/* The slot's allow-bitmask for the next token (the `allowed` predicate of src/server.br:334-350 over
 * every vocabulary id, including the EOG rule): ceil(vocab/32) words into device memory, bit t of
 * word t/32 set when token t is allowed; *forced_eos = the step would return EOS without sampling.
 * BL_EGRAMMAR_DEAD when the reply no longer matches (src/server.br:318). */
int bl_grammar_mask(bl_ctx *ctx, int slot, uint32_t *d_mask_out, int32_t *forced_eos);

/* One decode-loop sampling block for B slots (src/server.br:940-1037: logit_bias, ignore_eos,
 * frequency/presence, then sample() = sampling_logits + greedy | rank + sample_candidates, then
 * logprob_normalizer + top_k_select for logprobs). `d_logits` is a device pointer to B rows of
 * `ld` floats. The chosen tokens are appended to each slot's history. Host outputs; `logprobs`,
 * `top_ids`, `top_logprobs` may be NULL; `top_stride` entries per row. A row without logprobs reads
 * logprob 0; alternatives past a row's n_probs (all of them without logprobs) read id -1, logprob 0. */
int bl_sample_step(bl_ctx *ctx, const int32_t *slots, int B, const float *d_logits, int64_t ld, int32_t *tokens,
                   float *logprobs, int32_t *top_ids, float *top_logprobs, int top_stride);

/* The same step with device-memory outputs and no host synchronisation, on the context stream
 * (capturable in a HIP graph once bl_bind_rows has fixed the row table). A row that fails (an error the
 * synchronous step would return) gets token -1 and commits nothing; bl_slot_status reports the error.
 * bl_bind_rows keeps its own row table: synchronous steps and speculative verification on other slots
 * in between do not change the bound rows. */
int bl_bind_rows(bl_ctx *ctx, const int32_t *slots, int B);
int bl_sample_step_async(bl_ctx *ctx, int B, const float *d_logits, int64_t ld, int32_t *d_tokens, float *d_logprobs,
                         int32_t *d_top_ids, float *d_top_logprobs, int top_stride);

/* Allocation-free step: no counterpart in the reference; for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Row i of d_logits
 * (B rows of `ld` floats, `vocab` tokens, on `device`) is sampled as bl_sample_step samples a slot reset with
 * params[i], RNG state rng_states[i] and no history, reply or logit_bias, in a context without
 * end-of-generation ids; rng_states (host) are advanced in place and the outputs are bl_sample_step's. The
 * slot state and step workspace live in one fixed device array of BL_NOALLOC_BYTES, which each device that
 * runs the call holds until the process ends; no device memory is allocated or freed. Limits: B up to
 * BL_NOALLOC_ROWS, and the workspace (about 48.5 bytes per row and vocabulary entry, e.g. B = 8 at V = 151936)
 * within the array, else BL_EPARAM. Work is ordered on `stream` (a hipStream_t; NULL: the null stream) and
 * the call returns when results are in host memory. Calls that overlap on one device (threads or streams)
 * race on the array. */
#define BL_NOALLOC_BYTES (64u << 20)
#define BL_NOALLOC_ROWS 16
int bl_sample_rows_noalloc(int device, void *stream, const bl_params *params, uint64_t *rng_states, int B,
                           const float *d_logits, int64_t ld, int vocab, int32_t *tokens, float *logprobs,
                           int32_t *top_ids, float *top_logprobs, int top_stride);

/* A serving loop's step without host work (no reference counterpart; the reference samples on the host):
 * bl_step_graph_create captures one bl_sample_step_async of the bound rows, with these buffers, into an
 * instantiated HIP graph (*graph_out, a hipGraphExec_t); bl_step_graph_launch replays it on the context
 * stream; bl_stream_sync waits for the stream. A replay reads the slots' current state and parameters,
 * so it follows later bl_slot_commit calls and resets that keep each row's kind; rebinding rows,
 * changing buffers, or a reset that changes which passes a row needs (logprobs, top-k / n_probs, a
 * grammar, full-vocabulary sampling) needs a new graph, as does bl_set_eog. BL_EPARAM while kernel timing is
 * enabled (it synchronises). */
int bl_step_graph_create(bl_ctx *ctx, int B, const float *d_logits, int64_t ld, int32_t *d_tokens, float *d_logprobs,
                         int32_t *d_top_ids, float *d_top_logprobs, int top_stride, void **graph_out);
int bl_step_graph_launch(bl_ctx *ctx, void *graph);
int bl_step_graph_destroy(void *graph);
int bl_stream_sync(bl_ctx *ctx);

/* Kernel timing for measurement (no reference counterpart): while enabled, bl_sample_step_async records
 * HIP events around its three kernels (row pass, exponent pass, selection) on the context stream,
 * waits for them, and accumulates the durations; bl_get_timing returns the totals in ms and the
 * number of timed steps. Enabling resets the totals. */
int bl_set_timing(bl_ctx *ctx, int enable);
int bl_get_timing(bl_ctx *ctx, double *ms_total3, int64_t *steps);

/* Speculative verification (src/server.br:1173-1216): for each of the B slots, rows
 * d_rows[b*(k+1) + i] (i = 0..k) are the target logits after feeding drafts[b*k .. b*k+i). Row i is
 * sampled with the slot's RNG advanced by i draws; accepted[b] = number of leading rows whose token
 * equals its draft; the slot commits drafts[0..accepted) and tokens[b*(k+1)+accepted]. With frequency,
 * presence or repeat penalties, row i counts drafts[0..i) in the reply and the repeat window (and drops the
 * window entries they evict), as the reference's loop does after pushing them; drafts must then be
 * vocabulary ids and k at most 32.
 * `tokens` receives every row's token (row i as if drafts[0..i) were accepted). */
int bl_spec_verify(bl_ctx *ctx, const int32_t *slots, int B, int k, const float *d_rows, int64_t ld,
                   const int32_t *drafts, int32_t *tokens, int32_t *accepted);

/* Benchmark/test input generation (no reference counterpart): fills `rows` rows of `ld` floats with
 * the synthetic logits of workload `cfg` (integer-only generator, identical on host and device). */
int bl_synth_logits(bl_ctx *ctx, float *d_out, int64_t ld, int cfg, int64_t seed, int64_t step, int rows, int vocab);

/* Sparse inputs of the benchmark workloads (no reference counterpart; host only): kind 0 = uniform
 * ids, kind 1 = Zipf(1.1) ids; logit_bias lists of n distinct ids with values in [lo, hi); the
 * workload-3 vocabulary (256 single-byte tokens, byte strings of Zipf lengths 1..16, 70% printable
 * ASCII / 30% valid UTF-8, EOS "<|eos|>" = vocab-1; returns the blob size, BL_EPARAM when blob_cap is
 * too small); speculative drafts (argmax with probability 0.7, else uniform). Deterministic in
 * (cfg, seed, row/step). */
int bl_workload_ids(int kind, int cfg, int64_t seed, int row, int n, int vocab, int32_t *out);
int bl_workload_bias(int cfg, int64_t seed, int row, int n, int vocab, float lo, float hi, int32_t *ids, float *vals);
int bl_workload_c3_vocab(int64_t seed, int vocab, uint8_t *blob, size_t blob_cap, uint32_t *offsets, int32_t *eos_id);
int bl_workload_drafts(int64_t seed, int64_t step, int seq, const int32_t *argmax, int k, int vocab, int32_t *out);

/* Self-test (no reference counterpart): digests of the device expf (fn 0) / tanhf (fn 1) / logf (fn 2) /
 * powf(x, 0.7f) (fn 3) / powf(2, x) (fn 4) / powf(x, y(u)) (fn 5, y(u) = ((splitmix64(u) >> 40) % 8193 - 4096)
 * / 512) over input bit-pattern blocks [b*2^20, (b+1)*2^20), b = first_block .. first_block+n_blocks-1; each digest
 * is the wrapping sum of splitmix64(u << 32 | bits(f(u))) with NaN results canonicalised to 0x7fc00000.
 * Compared with host-glibc fixtures. */
int bl_math_digest(bl_ctx *ctx, int fn, uint32_t first_block, int n_blocks, uint64_t *out);

#ifdef __cplusplus
}
#endif

#endif /* BL_SELECT_H */
