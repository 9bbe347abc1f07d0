/* C ABI of the MI355X qwen4_exp engine.
 *
 * This is the drop-in boundary for the reference's engine API: each entry
 * point restates a public method of `Gpu` (/root/reference/src/qwen4_exp/
 * gpu.rs and gpu/*.rs) with the same argument meaning and the same error
 * conditions.  Conventions:
 *   - every call returns 0 on success or -1 with a message retrievable by
 *     chk_last_error() (thread-local), standing in for anyhow::Result;
 *   - one handle is driven by one thread at a time (`&mut self`);
 *   - host pointers returned by the engine (logits rows) stay valid until
 *     the next mutating call on the same handle (gpu.rs:601-607);
 *   - tokens are u32 ids, rows are at most chk_trunk_rows() per step.
 * The weights are the seeded synthetic weights of synth.h, generated in HBM
 * at load time (chk_engine_load), or a packed store's (chk_engine_load_store).
 */
#ifndef CHERENKOV_ENGINE_H
#define CHERENKOV_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#include "cherenkov/types.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ChkEngine ChkEngine;
typedef struct ChkPrefixState ChkPrefixState;

/* "no token" for optional token arguments (Option<u32>::None). */
#define CHK_NO_TOKEN 0xffffffffu

/* Last error message of this thread ("" if none). */
const char* chk_last_error(void);

/* Gpu::load / load_bounded (gpu/load.rs:8-19): builds the HBM-resident
 * store (dense tensors + every routed-expert record, Q4 and, when
 * opt->experts is 3 or 2, the low-bit store repacked from it), state, KV
 * and scratch for contexts of opt->max_t tokens and 1 + opt->drafts rows. */
int chk_engine_load(const ChkConfig* cfg, const ChkOptions* opt, ChkEngine** out);
void chk_engine_free(ChkEngine* e);

/* Gpu::load over a packed store (gpu/load.rs:8-19 with Packed::open,
 * packed.rs:66-100): `dir` holds manifest.json, dense.bin and experts.bin
 * (or a packed/ subdirectory does) and config.json (beside them or in
 * `dir`), in the reference's formats (manifest.rs:7-110, config.rs:93-122,
 * pack.rs:351-393).  Every weight is read from the store into the same HBM
 * layout chk_engine_load generates; a low-bit expert store (opt->experts 3
 * or 2) is repacked on the device from the Q4 records.  Errors name the
 * missing or mismatched tensor. */
int chk_engine_load_store(const char* dir, const ChkOptions* opt, ChkEngine** out);

/* Gpu::load_bounded (gpu/load.rs:12-63; src/server.rs:90-97): the loads
 * above under a server memory budget of memory_bytes - reserve (memory_bytes
 * 0: no budget, as load passes None; reserve above memory_bytes: "cache
 * exceeds memory budget").  Every device buffer the engine allocates then,
 * and later (prefill scratch), counts against it ("allocation would exceed
 * the server memory budget; reduce pool or prefill chunk size"); the load
 * fails unless the prefill scratch of prefill_rows rows (at most max_t, at
 * least 1) still fits beside the resident store (budget.rs:14-40), and
 * chk_prefill_rows_fit answers within the budget.  Checkpoints
 * (chk_save_prefix / chk_save_into) are the caller's objects and are not
 * counted. */
int chk_engine_load_bounded(const ChkConfig* cfg, const ChkOptions* opt, uint64_t reserve, uint64_t memory_bytes,
                            uint32_t prefill_rows, ChkEngine** out);
int chk_engine_load_store_bounded(const char* dir, const ChkOptions* opt, uint64_t reserve, uint64_t memory_bytes,
                                  uint32_t prefill_rows, ChkEngine** out);

/* The ChkConfig of a packed store's config.json after the manifest checks
 * of chk_engine_load_store (file reads only, no device work). */
int chk_store_config(const char* dir, ChkConfig* out);

/* Gpu::step_rows (gpu/decode.rs:13-58): run tokens[0..n) at positions
 * pos.. as one batch, write the greedy argmax after each row to out[0..n).
 * Nothing is committed until chk_commit.  `snap` keeps rollback snapshots
 * after each row but the last; `fold_mtp` runs the MTP head's first pass
 * over the same rows (requires an MTP head). */
int chk_step_rows(ChkEngine* e, const uint32_t* tokens, uint32_t n, int snap, int fold_mtp, uint32_t* out);

/* Gpu::step (gpu/decode.rs:335-341): one token, committed. */
int chk_step(ChkEngine* e, uint32_t token, uint32_t* out);

/* Gpu::commit (gpu/state.rs:10-56): keep the first n rows of the last
 * step; rolls DeltaNet state and conv history back when n < rows. */
int chk_commit(ChkEngine* e, uint32_t n);

/* Gpu::reset (gpu/state.rs:61-82): forget the sequence. */
int chk_reset(ChkEngine* e);

/* Gpu::mtp_draft (gpu/mtp.rs:11-78): after a commit of n rows, row r pairs
 * the trunk residual at batch_pos + r with next[r]; returns `chain` greedy
 * drafts in drafts[0..*n_drafts). */
int chk_mtp_draft(ChkEngine* e, const uint32_t* next, uint32_t n, uint32_t chain, uint32_t* drafts,
                  uint32_t* n_drafts);

/* Gpu::mtp_chain (gpu/mtp.rs:248-252): one more draft chained on the MTP
 * residual left by the last draft pass. */
int chk_mtp_chain(ChkEngine* e, uint32_t draft, uint32_t* out);

/* Gpu::prefill_chunk (gpu/prefill.rs:190-464): process tokens[0..n) as
 * prompt rows, commit them, and write the greedy next token (and, with an
 * MTP head, its first draft, else CHK_NO_TOKEN).  `next_after` is the token
 * that follows the chunk when the caller knows it (the next chunk's first
 * token, runner.rs:124): the MTP head pairs it with the chunk's last row,
 * else the trunk's greedy token (CHK_NO_TOKEN).  With all_logits every
 * row's logits are kept for chk_pf_logits_row.  Afterwards no step is in
 * flight (commit has nothing to keep) and logits_row(0) is the last row's. */
int chk_prefill_chunk(ChkEngine* e, const uint32_t* tokens, uint32_t n, uint32_t next_after, int all_logits,
                      uint32_t* next, uint32_t* draft);

/* Gpu::prefill_release (gpu/prefill.rs:467-469): free the prefill scratch
 * (reallocated by the next chunk). */
void chk_prefill_release(ChkEngine* e);

/* Gpu::prefill_rows_fit (prefill/allocation.rs:150-169): the largest chunk,
 * at most min(max_t, 4096) rows, whose prefill scratch fits the device
 * memory free now (errors when not even one row fits). */
int chk_prefill_rows_fit(const ChkEngine* e, int all_logits, uint32_t* rows);
/* Gpu::debug_engine_blocks (gpu/prefill.rs:471-484): the QSA blocks
 * selected for row r of the last prefill chunk at its latest attention
 * layer (rows within the budget, which attend densely, select none); and
 * Gpu::debug_row_vis (gpu/prefill.rs:486-494): the tokens row r of the last
 * row step attended to at its latest attention layer, ascending.  Up to cap
 * ids go to out, n receives the count. */
int chk_debug_engine_blocks(const ChkEngine* e, uint32_t r, uint32_t* out, uint32_t cap, uint32_t* n);
int chk_debug_row_vis(const ChkEngine* e, uint32_t r, uint32_t* out, uint32_t cap, uint32_t* n);

/* Gpu::pf_logits_row (gpu/prefill.rs:496-507): row r of the last prefill
 * chunk's logits (all-logits mode only; NULL + error otherwise). */
const float* chk_pf_logits_row(ChkEngine* e, uint32_t r);

/* Gpu::logits_row / logits / last_logits_row / mtp_logits_row
 * (gpu.rs:601-624): host copy of the logits of row r of the last step
 * (vocab_size floats); chk_logits is row 0; chk_last_logits_row is the row
 * that holds the latest token's logits (rows - 1; 0 after a prefill). */
const float* chk_logits_row(ChkEngine* e, uint32_t r);
const float* chk_logits(ChkEngine* e);
uint32_t chk_last_logits_row(const ChkEngine* e);
const float* chk_mtp_logits_row(ChkEngine* e, uint32_t r);

uint32_t chk_pos(const ChkEngine* e);
uint32_t chk_eos_token(const ChkEngine* e);
uint32_t chk_vocab_size(const ChkEngine* e);
uint32_t chk_max_t(const ChkEngine* e);
uint32_t chk_trunk_rows(const ChkEngine* e);
int chk_has_mtp(const ChkEngine* e);

/* Gpu::memory_stats (gpu/memory.rs:10-60), bytes. */
typedef struct ChkMemoryStats {
    uint64_t dense;
    uint64_t experts;
    uint64_t experts_low_bit;
    uint64_t state;
    uint64_t kv_cache;
    uint64_t scratch;
    uint64_t total;
} ChkMemoryStats;
int chk_memory_stats(const ChkEngine* e, ChkMemoryStats* out);

/* Gpu::allocated_gb (gpu.rs:626-628): device memory this engine holds, in
 * decimal GB (units.rs:7). */
double chk_allocated_gb(const ChkEngine* e);

/* KV-cache occupancy (gpu.rs:630-690): bytes of the positional caches in
 * use (trunk attention layers at pos, the MTP layer at its own length),
 * their capacity at max_t, the ratio, and pos / max_t. */
uint64_t chk_kv_cache_bytes(const ChkEngine* e);
uint64_t chk_kv_cache_capacity(const ChkEngine* e);
double chk_kv_cache_fullness(const ChkEngine* e);
double chk_context_fullness(const ChkEngine* e);

/* Gpu::reset_request / clear_profile (gpu/state.rs:232-263): reset the
 * sequence and drop the profiling counters; the weights stay loaded. */
int chk_reset_request(ChkEngine* e);
int chk_clear_profile(ChkEngine* e);

/* Sequence checkpoints (gpu/state.rs:85-230).  A checkpoint holds the
 * position, the MTP cache length, the token history and a copy of every
 * prefix region (DeltaNet state and conv history, q8 K/V rows and scales,
 * index and block keys up to the length; the MTP layer's at its own
 * length).  Copies stay in device memory.
 *   chk_prefix_state_bytes  prefix_state_bytes (bytes a checkpoint now takes)
 *   chk_state_bytes_at      state_bytes_at(pos, mtp_len)
 *   chk_save_prefix         save_prefix: a new checkpoint (free it with chk_prefix_free)
 *   chk_save_into           save_into: reuse *checkpoint's buffers (created when NULL)
 *   chk_restore_prefix      restore_prefix: errors "prefix exceeds context" /
 *                           "prefix state layout mismatch" / "prefix region mismatch" */
uint64_t chk_prefix_state_bytes(const ChkEngine* e);
uint64_t chk_state_bytes_at(const ChkEngine* e, uint32_t pos, uint32_t mtp_len);
int chk_save_prefix(ChkEngine* e, ChkPrefixState** out);
int chk_save_into(ChkEngine* e, ChkPrefixState** checkpoint);
int chk_restore_prefix(ChkEngine* e, const ChkPrefixState* state);
void chk_prefix_free(ChkPrefixState* state);
uint32_t chk_prefix_pos(const ChkPrefixState* state);
uint32_t chk_prefix_mtp_len(const ChkPrefixState* state);
/* Copies min(cap, length) token ids; returns the history's length. */
uint32_t chk_prefix_tokens(const ChkPrefixState* state, uint32_t* out, uint32_t cap);

/* Expert-cache interface (residency::Pool, gpu/residency.rs:255-460) over
 * the all-resident HBM store: every record is a member from load on, so
 * acquire(rids, step) never needs a read (n_need = 0), plan_reads plans no
 * read (warm = n) and finish waits for nothing.  Each record has a kind
 * (Pool::kind / set_kind, residency.rs:290-306): 0 (4-bit) or, when a
 * low-bit store is attached (ChkOptions.experts 3 or 2, which is also every
 * record's starting kind), that store's kind (1 = Q3, 2 = Q2); set_kind
 * switches one record between the two, refuses any other kind, and the
 * next step or prefill decodes the record from the store of its kind (one
 * launch mixes both).  addr(rid) = that store's base + rid * stride with
 * the kind tag in bits 62-63 (residency.rs:437-451); buf(rid) = (store
 * base, byte offset); bytes = the records' bytes in the stores of their
 * kinds; chk_pool_store gives the device store behind a kind (store_file,
 * residency.rs:300-311). */
uint32_t chk_pool_slots(const ChkEngine* e);
uint32_t chk_pool_budget(const ChkEngine* e);
uint32_t chk_pool_resident(const ChkEngine* e);
int chk_pool_is_member(const ChkEngine* e, uint32_t rid);
int chk_pool_acquire(ChkEngine* e, const uint32_t* rids, uint32_t n, uint64_t step, uint32_t* need,
                     uint32_t* n_need);
int chk_pool_plan_reads(const ChkEngine* e, const uint32_t* need, uint32_t n, uint32_t* n_reads, uint32_t* warm);
int chk_pool_finish(ChkEngine* e, const uint32_t* rids, uint32_t n);
uint64_t chk_pool_addr(const ChkEngine* e, uint32_t rid);
int chk_pool_buf(const ChkEngine* e, uint32_t rid, void** base, uint64_t* offset);
uint32_t chk_pool_kind(const ChkEngine* e, uint32_t rid);
int chk_pool_set_kind(ChkEngine* e, uint32_t rid, uint32_t kind);
int chk_pool_store(const ChkEngine* e, uint32_t kind, void** base, uint64_t* stride);
uint64_t chk_pool_bytes(const ChkEngine* e);

/* Gpu::throttle_ms (gpu.rs:596-599): milliseconds of a fixed dependent-FMA
 * probe (higher = lower clocks). */
int chk_throttle_ms(ChkEngine* e, double* ms);
/* Gpu::working_set_limit_gb (gpu.rs:690-694): device memory, decimal GB. */
double chk_working_set_limit_gb(const ChkEngine* e);

/* Gpu::expert_activity (gpu/activity.rs:11-89, 110): cumulative counters per
 * expert record since load (n = record layers x num_experts, main layers
 * then the MTP layer), fields as ExpertCounters; verification and draft
 * rows count even when rolled back; every record is resident, so each
 * lookup is a cache hit and no read is requested. */
typedef struct ChkExpertCounters {
    uint64_t selected_rows;
    uint64_t cache_hits;
    uint64_t cache_misses;
    uint64_t prefetch_requests;
    uint64_t read_requests;
    uint64_t read_bytes_requested;
} ChkExpertCounters;
int chk_expert_activity(const ChkEngine* e, ChkExpertCounters* records, uint32_t n, double* elapsed_seconds);

/* Per-step expert activity (gpu/activity.rs:110): routed ids of row r of
 * the last step for layer l (num_experts_per_tok entries). */
int chk_last_routes(const ChkEngine* e, uint32_t layer, uint32_t r, uint32_t* ids, float* weights);
/* Router softmax (num_experts entries) behind those routes, for row r of
 * the last row-path step at layer l: the margin of the top-k cut is what
 * the parity bar exempts near-ties on (diagnostic; no reference
 * counterpart beyond activity.rs, whose per-expert counts come from it). */
int chk_last_probs(const ChkEngine* e, uint32_t layer, uint32_t r, float* probs);

/* ---- request sampling ----
 * Sampling / Sampler (src/sampling.rs:8-226): the request's options and
 * its host sampler over one row of logits (f64 penalties, temperature,
 * top-k, nucleus, then a draw from the seeded stream).  The stream is
 * rand 0.9's StdRng (ChaCha12, seed_from_u64); has_seed = 0 seeds from
 * the OS.  Errors carry the reference's messages (chk_last_error). */
typedef struct ChkSampling {
    double temperature;       /* 0..2; 0 = greedy (argmax) */
    double top_p;             /* (0, 1] */
    uint32_t top_k;           /* 0 = whole vocabulary, else <= 1000000 */
    uint32_t has_seed;
    uint64_t seed;
    double presence_penalty;  /* -2..2 */
    double frequency_penalty; /* -2..2 */
} ChkSampling;
/* Sampling::validate (sampling.rs:46-68). */
int chk_sampling_validate(const ChkSampling* s);
/* Sampling::greedy (sampling.rs:71-73): 1 when argmax MTP verification
 * applies (temperature and both penalties zero). */
int chk_sampling_greedy(const ChkSampling* s);
typedef struct ChkSampler ChkSampler;
/* Sampler::new (sampling.rs:114-134): counts start from the prompt. */
int chk_sampler_new(const ChkSampling* s, const uint32_t* prompt, uint32_t n, uint32_t vocab, ChkSampler** out);
void chk_sampler_free(ChkSampler* s);
/* Sampler::accept (sampling.rs:136-144). */
int chk_sampler_accept(ChkSampler* s, uint32_t token);
/* Sampler::sample (sampling.rs:146-209) over logits[0..n), n = vocab. */
int chk_sampler_sample(ChkSampler* s, const float* logits, uint32_t n, uint32_t* token);
/* The sampler's stream alone: n next_u64 draws of StdRng::from_seed(seed32)
 * or, with seed32 NULL, of seed_from_u64(seed) (no reference counterpart;
 * pins the ChaCha12 restatement in tests). */
int chk_rng_u64(const uint8_t* seed32, uint64_t seed, uint64_t* out, uint32_t n);
/* PCG32 as its reference generator seeds and runs it (pcg32_srandom_r /
 * pcg32_random_r) on the step and output the seeding uses (no reference
 * counterpart; pins seed_from_u64's generator in tests). */
void chk_pcg32(uint64_t init_state, uint64_t init_seq, uint32_t* out, uint32_t n);
/* The ChaCha block function, `rounds` rounds over a 16-word input state
 * (no reference counterpart; RFC 8439 vectors pin it in tests). */
void chk_chacha_block(const uint32_t* in, int rounds, uint32_t* out);

/* ---- prefix cache: bounded LRU checkpoints of prompt prefixes ----
 * PrefixCache / Prefill (src/prefix_cache.rs:12-335) over this ABI.
 *   chk_prefix_matches        matches (prefix_cache.rs:35-45): may an entry of
 *                             tokens (made while drafting: `following`
 *                             pinned) serve this request?
 *   chk_prefill_chunk_len     chunk_len (prefix_cache.rs:256-266)
 *   chk_prefill_pacing_sample pacing_sample (prefix_cache.rs:251-253)
 *   chk_prefix_cache_new      PrefixCache::new(capacity bytes, max entries,
 *                             idle seconds; 0 = never)
 *   chk_prefix_cache_begin    PrefixCache::begin: restore the longest
 *                             matching entry into the engine and plan the
 *                             prompt's boundaries (stable ones kept when
 *                             the cache can hold entries)
 *   chk_prefill_advance       Prefill::advance: one chunk toward the next
 *                             boundary (engine prefill from
 *                             CHERENKOV_PREFILL_MIN rows, else row steps),
 *                             storing an entry at boundaries and after
 *                             engine chunks; *done when the prompt is in
 *   chk_prefill_next / drafts / logits  the resume point for decode
 * An entry's bytes are its checkpoint, its tokens, its drafts and logits
 * and the host record. */
typedef struct ChkPrefixCache ChkPrefixCache;
typedef struct ChkPrefill ChkPrefill;
int chk_prefix_matches(const uint32_t* tokens, uint32_t n_tokens, int has_following, uint32_t following,
                       int complete, const uint32_t* request, uint32_t n_request);
int chk_prefill_chunk_len(uint32_t remaining, uint32_t capacity, uint32_t quantum, uint32_t* out);
int chk_prefill_pacing_sample(uint32_t remaining, uint32_t capacity, uint32_t quantum, int engine);
int chk_prefix_cache_new(uint64_t capacity, uint64_t max_entries, uint64_t idle_seconds, ChkPrefixCache** out);
void chk_prefix_cache_free(ChkPrefixCache* c);
void chk_prefix_cache_expire(ChkPrefixCache* c);
void chk_prefix_cache_stats(const ChkPrefixCache* c, uint64_t* entries, uint64_t* used, uint64_t* evictions);
int chk_prefix_cache_begin(ChkPrefixCache* c, ChkEngine* e, const uint32_t* ids, uint32_t n,
                           const uint32_t* stable_boundaries, uint32_t n_boundaries, uint32_t effective_drafts,
                           ChkPrefill** out);
void chk_prefill_free(ChkPrefill* p);
uint32_t chk_prefill_cached(const ChkPrefill* p);
int chk_prefill_advance(ChkPrefill* p, ChkPrefixCache* c, ChkEngine* e, const uint32_t* ids, uint32_t n,
                        uint32_t effective_drafts, uint32_t quantum, int* done, uint32_t* pacing_tokens);
uint32_t chk_prefill_next(const ChkPrefill* p);
uint32_t chk_prefill_drafts(const ChkPrefill* p, uint32_t* out, uint32_t cap);
const float* chk_prefill_logits(const ChkPrefill* p);

/* ---- runner: the greedy speculative decode loop ----
 * Decode::new / Decode::step (src/runner/decode.rs:28-171) for the greedy
 * sampler.  `next` and drafts[0..n_drafts) come from the prompt's prefill;
 * n_draft is the effective draft count (0..3); generation stops after
 * `limit` tokens or at EOS (the config's eos_token_id) unless no_eos. */
typedef struct ChkDecode ChkDecode;
int chk_decode_new(ChkEngine* e, uint32_t next, const uint32_t* drafts, uint32_t n_drafts, uint32_t n_draft,
                   uint32_t limit, uint32_t no_eos, ChkDecode** out);
/* Decode::new (decode.rs:28-71) with the request's sampling options.
 * Greedy options behave as chk_decode_new.  Otherwise the sampler starts
 * from prompt[0..n_prompt), the first token is sampled from
 * final_logits (the prompt's last-row logits, vocab_size floats), and no
 * drafts are used (Options::effective_drafts, options.rs:165-171): each
 * step runs one row and samples from its logits. */
int chk_decode_new_sampling(ChkEngine* e, const ChkSampling* sampling, const uint32_t* prompt, uint32_t n_prompt,
                            const float* final_logits, uint32_t next, const uint32_t* drafts, uint32_t n_drafts,
                            uint32_t n_draft, uint32_t limit, uint32_t no_eos, ChkDecode** out);
void chk_decode_free(ChkDecode* d);
/* The ids that end generation (Decode.eos = [tok.im_end, tok.endoftext],
 * src/runner/decode.rs:64): the caller that owns the tokenizer passes them
 * (1..=16 ids); until then the config's eos_token_id alone. */
int chk_decode_set_eos(ChkDecode* d, const uint32_t* ids, uint32_t n);
/* One step: the tokens it emits (1 + accepted drafts, <= 4) go to emitted. */
int chk_decode_step(ChkDecode* d, uint32_t* emitted, uint32_t* n_emitted);
/* 0 running, 1 stopped at EOS, 2 length limit reached. */
int chk_decode_finished(ChkDecode* d);
int chk_decode_stats(ChkDecode* d, uint32_t* steps, uint32_t* accepted);
const char* chk_decode_error(void);

#ifdef __cplusplus
}
#endif

#endif
