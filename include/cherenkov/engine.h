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
 * at load time (the reference mmaps a packed checkpoint instead; see
 * INTEGRATION.md for how a packed-store loader plugs in).
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

/* Last error message of this thread ("" if none). */
const char* chk_last_error(void);

/* Gpu::load / load_bounded (gpu/load.rs:8-19): builds the HBM-resident
 * store (dense tensors + every routed-expert record, Q4 and, when
 * opt->experts is 3 or 2, the low-bit store repacked from it), state, KV
 * and scratch for contexts of opt->max_t tokens and 1 + opt->drafts rows. */
int chk_engine_load(const ChkConfig* cfg, const ChkOptions* opt, ChkEngine** out);
void chk_engine_free(ChkEngine* e);

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

/* Gpu::prefill_chunk (gpu/prefill.rs:196-464): process tokens[0..n) as
 * prompt rows, commit them, and write the greedy next token (and, with an
 * MTP head, its first draft, else UINT32_MAX). */
int chk_prefill_chunk(ChkEngine* e, const uint32_t* tokens, uint32_t n, uint32_t* next, uint32_t* draft);

/* Gpu::logits_row / last_logits_row / mtp_logits_row (gpu.rs:601-624):
 * host copy of the logits of row r of the last step (vocab_size floats). */
const float* chk_logits_row(ChkEngine* e, uint32_t r);
const float* chk_mtp_logits_row(ChkEngine* e, uint32_t r);

uint32_t chk_pos(const ChkEngine* e);
uint32_t chk_eos_token(const ChkEngine* e);
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

/* Expert-cache interface (residency::Pool, gpu/residency.rs:255-460) over
 * the all-resident HBM store: every record is a member, acquire never
 * needs a read, addr(rid) = base + rid * stride with the kind tag in bits
 * 62-63 (1 = Q3, 2 = Q2; residency.rs:437-451). */
uint32_t chk_pool_slots(const ChkEngine* e);
uint32_t chk_pool_resident(const ChkEngine* e);
int chk_pool_is_member(const ChkEngine* e, uint32_t rid);
uint32_t chk_pool_acquire(ChkEngine* e, const uint32_t* rids, uint32_t n, uint32_t* need);
uint64_t chk_pool_addr(const ChkEngine* e, uint32_t rid);
uint32_t chk_pool_kind(const ChkEngine* e, uint32_t rid);
uint64_t chk_pool_bytes(const ChkEngine* e);

/* Per-step expert activity (gpu/activity.rs:110): routed ids of row r of
 * the last step for layer l (num_experts_per_tok entries). */
int chk_last_routes(const ChkEngine* e, uint32_t layer, uint32_t r, uint32_t* ids, float* weights);
/* Router softmax (num_experts entries) behind those routes, for row r of
 * the last row-path step at layer l: the margin of the top-k cut is what
 * the parity bar exempts near-ties on (diagnostic; no reference
 * counterpart beyond activity.rs, whose per-expert counts come from it). */
int chk_last_probs(const ChkEngine* e, uint32_t layer, uint32_t r, float* probs);

/* ---- runner: the greedy speculative decode loop ----
 * Decode::new / Decode::step (src/runner/decode.rs:28-171) for the greedy
 * sampler.  `next` and drafts[0..n_drafts) come from the prompt's prefill;
 * n_draft is the effective draft count (0..3); generation stops after
 * `limit` tokens or at EOS (the config's eos_token_id) unless no_eos. */
typedef struct ChkDecode ChkDecode;
int chk_decode_new(ChkEngine* e, uint32_t next, const uint32_t* drafts, uint32_t n_drafts, uint32_t n_draft,
                   uint32_t limit, uint32_t no_eos, ChkDecode** out);
void chk_decode_free(ChkDecode* d);
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
