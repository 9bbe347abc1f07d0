/* Kernel-level test ABI: the engine's blocks and primitives one at a time,
 * on device buffers the caller owns.  These have no single counterpart in
 * the reference's public API; they expose, for parity tests and block
 * benchmarks, the pieces the reference engine dispatches inside
 * `Gpu::step_rows` (gpu/decode.rs:13-294):
 *   chk_q4_matvec         qmv_multi_h / fn_qmv_small_b (quant.rs:49-88 semantics)
 *   chk_moe_block         router_b + experts_b (gpu/experts.rs:8-187)
 *   chk_deltanet_block    deltanet_b (gpu/deltanet.rs:8-113)
 *   chk_attention_block   attention_b (gpu/attention.rs:10-273)
 *   chk_hc_read           hc_read_b (gpu/hyperconnection.rs:59-152)
 * Device pointers are plain addresses (e.g. torch's data_ptr()); `stream`
 * is a hipStream_t (0 = the engine's stream).  Calls are stream-ordered and
 * synchronous on return.
 */
#ifndef CHERENKOV_KERNELS_H
#define CHERENKOV_KERNELS_H

#include <stdint.h>

#include "cherenkov/engine.h"

#ifdef __cplusplus
extern "C" {
#endif

/* y[b][r] = sum_g s[r,g] sum_j q x_b + b[r,g] sum_j x_b for b < nb <= 4.
 * w u32 [out][in/8], s/b bf16 [out][in/64], x f32 [nb][in], y f32 [nb][out]. */
int chk_q4_matvec(const void* w, const void* s, const void* b, uint32_t out, uint32_t in, const float* x,
                  float* y, uint32_t nb, void* stream);

/* The prefill GEMM: y [T][out] = x [T][in] W^T for a Q4 g64 W [out][in]
 * (the prefill qmm, gpu/prefill/projection.rs:8-108): MFMA on the integer
 * codes, each group's scale and bias applied to its partial sums in f32,
 * activations split into two fp16 parts.  in a multiple of 64. */
int chk_q4_gemm(const void* w, const void* s, const void* b, uint32_t out, uint32_t in, const float* x, uint32_t T,
                float* y, void* stream);

/* The decode LM head: logits [nb][out] = W x as chk_q4_matvec, and ids[nb]
 * (device u32) = the greedy token of each row, lowest index on exact ties,
 * 0 when every logit is -inf (argmax_partial/argmax_final,
 * kernels/common/sampling.metal:10-84; head_b, gpu/sampling.rs:10-63).
 * out must be a multiple of 8. */
int chk_lm_head_argmax(const void* w, const void* s, const void* b, uint32_t out, uint32_t in, const float* x,
                       uint32_t nb, float* logits, uint32_t* ids, void* stream);

/* chk_lm_head_argmax without any allocation: no counterpart in the
 * reference; for callers that cannot allocate device memory (code under
 * graph capture, serving loops that forbid hipMalloc).  Same arguments and
 * results; the argmax partials live in a 32 KiB file-scope device array of
 * the library (nb <= 4 rows of 1024 workgroup partials), one per device,
 * shared by every call on that device: calls that overlap on one device
 * race.  It never waits on the stream, so it can be captured into a graph;
 * the first call on each device (which looks the array's address up) must
 * be made outside capture and is refused under it. */
int chk_lm_head_argmax_noalloc(const void* w, const void* s, const void* b, uint32_t out, uint32_t in,
                               const float* x, uint32_t nb, float* logits, uint32_t* ids, void* stream);

/* Flash-decode core over a q8 KV cache of T tokens (no projections, norms
 * or RoPE): q f32 [nh][2 hd] holds each head's [q | gate] (the q_proj row
 * order, cpu.rs:577-582); k, v int8 [T][nkv hd]; ks, vs fp16 [T][nkv hd/32];
 * out f32 [nh][hd] = softmax(q.k / sqrt(hd)) . v * sigmoid(gate), each
 * value dequantised as q8 * fp16 scale (attn_part2_q8 + attn_combine,
 * kernels/common/attention.metal:138-185,236-310).  hd is 128 or 256 and
 * nh / nkv one of 1, 2, 4, 8, 12. */
int chk_attn_decode_q8(const float* q, const void* k, const void* v, const void* ks, const void* vs, uint32_t T,
                       uint32_t nh, uint32_t nkv, uint32_t hd, float* out, void* stream);

/* QSA block selection (select_tokens' sparse branch, cpu.rs:701-716; the
 * Metal index_select kernel of kernels/qwen4_exp/qsa.metal): of the
 * t_len / ratio complete blocks' scores (device f32, >= 0), keep the kblk
 * largest, ties to the lowest block; vmask (device u32, one bit per block,
 * ceil((t_len / ratio + 1) / 32) words) receives the selection.  Writes
 * nothing while t_len / ratio <= kblk (the dense case). */
int chk_qsa_select(const float* scores, uint32_t t_len, uint32_t kblk, uint32_t ratio, uint32_t* vmask, void* stream);

/* The prefill's gated delta rule over T rows (linear_attention's recurrence,
 * cpu.rs:745-812; the reference prefill scan, gpu/prefill/deltanet.rs:80-95):
 * conv f32 [T][2 nk dk + nv dv] holds each row's q (normed, scaled), k
 * (normed) and v as the conv stage leaves them; decay, beta f32 [T][nv];
 * state f32 [nv][dv][dk] is read and left updated; y f32 [T][nv dv].
 * chunked = 0 runs the recurrence row by row, 1 the chunked form (64 rows
 * per chunk, MFMA products; key and value head dims 128).  dk is 128. */
int chk_dn_scan(const float* conv, const float* decay, const float* beta, float* state, float* y, uint32_t T,
                uint32_t nk, uint32_t nv, uint32_t dk, uint32_t dv, int chunked, void* stream);

/* MoE block of decoder layer `layer` (num_hidden_layers = the MTP layer) on
 * normalised inputs x [nb][H]: out [nb][H] = routed experts (per the
 * engine's expert precision) + sigmoid-gated shared expert; top_ids
 * [nb][k] u32 and top_w [nb][k] f32 receive the routing; probs [nb][E]
 * (optional) the router softmax. */
int chk_moe_block(ChkEngine* e, uint32_t layer, const float* x, uint32_t nb, float* out, uint32_t* top_ids,
                  float* top_w, float* probs);

/* DeltaNet mixer of decoder layer `layer` on x [nb][H] -> out [nb][H],
 * advancing that layer's recurrent state and conv history (snapshots
 * after each row but the last when `snap`). */
int chk_deltanet_block(ChkEngine* e, uint32_t layer, const float* x, uint32_t nb, int snap, float* out);

/* Copy a DeltaNet layer's state [nv][dk][dv] (the reference's CPU order)
 * and conv history [conv_dim][k-1] to host buffers. */
int chk_deltanet_state(ChkEngine* e, uint32_t layer, float* s_host, float* conv_host);

/* Restore snapshot plane `plane` of a DeltaNet layer into its live state
 * (the commit rollback, gpu/state.rs:20-47). */
int chk_deltanet_rollback(ChkEngine* e, uint32_t layer, uint32_t plane);

/* Attention mixer of decoder layer `layer` on x [nb][H] for the engine's
 * sequence at positions pos.. (rows see positions <= their own) ->
 * out [nb][H]; appends K/V (q8) and index keys at those positions. */
int chk_attention_block(ChkEngine* e, uint32_t layer, const float* x, uint32_t nb, uint32_t pos, float* out);

/* Fill positions [0, T) of attention layer `layer`'s q8 KV cache by
 * quantising k, v f32 [T][nkv * hd] with the engine's q8 rule.
 * `seq` selects the engine's sequence (0) or a second sequence slot (1)
 * used by the batch-2 attention decode below. */
int chk_kv_fill(ChkEngine* e, uint32_t layer, uint32_t seq, const float* k, const float* v, uint32_t T);

/* Batch-2 attention decode over two independent sequences (two interleaved
 * requests): row b uses sequence slot b at position pos[b]. */
int chk_attention_block2(ChkEngine* e, uint32_t layer, const float* x, const uint32_t* pos, float* out);

/* Hyper-connection read `which` (0 attn, 1 mlp, 2 final mixer, 3 MTP
 * mixer) of layer `layer` on hyper [nb][hc H] -> mixed [nb][H] and the
 * injection weights inj [nb][hc] (absent for the mixers). */
int chk_hc_read(ChkEngine* e, uint32_t layer, uint32_t which, const float* hyper, uint32_t nb, float* mixed,
                float* inj);

/* Copy `n` bytes of the routed-expert store record (layer, expert) in the
 * Q4 layout (bits = 4) or the engine's low-bit layout (bits = 3 or 2). */
int chk_expert_record(ChkEngine* e, uint32_t layer, uint32_t expert, uint32_t bits, void* host, uint64_t n);
uint64_t chk_record_stride(const ChkEngine* e, uint32_t bits);

/* Per-layer trace of the trunk residual: when enabled, each step keeps
 * hyper after every layer; chk_layer_hyper copies layer l, row r. */
int chk_trace_enable(ChkEngine* e, int on);
int chk_layer_hyper(ChkEngine* e, uint32_t layer, uint32_t r, float* host);

/* Live kernel profiler: bracket every launch of one kernel class with HIP
 * events on the engine's stream (1 = MoE experts gate/up,
 * 2 = DeltaNet input projections, 3 = LM head + argmax; 0 = off) and
 * accumulate its algorithmic HBM bytes; chk_profile_read returns the
 * summed event time, launch count and bytes since chk_profile_kernel. */
int chk_profile_kernel(ChkEngine* e, int kind);
int chk_profile_read(ChkEngine* e, double* ms_total, uint64_t* launches, uint64_t* bytes);

/* The device ranges of the prefix regions at (pos, mtp_len), in the order
 * a checkpoint stores them: count receives their number, ptrs/bytes the
 * first `cap`.  Test support for the checkpoint round trip (the reference
 * test writes the regions directly, tests/unit/qwen4_exp/gpu/state.rs). */
int chk_prefix_regions(const ChkEngine* e, uint32_t pos, uint32_t mtp_len, uint64_t* ptrs, uint64_t* bytes,
                       uint32_t cap, uint32_t* count);
/* Copy the first n bytes of a checkpoint's region i to host memory. */
int chk_prefix_read(const ChkPrefixState* state, uint32_t i, void* host, uint64_t n);
/* dst[i] = value for i < n bytes of device memory. */
int chk_fill_u8(void* dst, uint32_t value, uint64_t n, void* stream);

/* dst[i] = src[i], i < n (f32 device buffers): the library's plain copy
 * kernel, used to calibrate HBM byte counters (rocprofv3 FETCH_SIZE /
 * WRITE_SIZE) against a transfer of known size.  Profiling support, no
 * reference counterpart. */
int chk_copy_f32(float* dst, const float* src, uint64_t n, void* stream);

/* Times one kernel class alone (kind 1: MoE gate/up, 3: LM head): a
 * captured HIP graph of `reps` rounds of its batch-1 launches over every
 * decoder layer, with the step's own arguments and current inputs,
 * replayed once between two HIP events on the engine stream.  Returns the
 * elapsed time, the launch count and their algorithmic HBM bytes.  Only
 * scratch buffers are written.  Profiling support, no reference
 * counterpart. */
int chk_profile_graph(ChkEngine* e, int kind, uint32_t reps, double* ms_total, uint64_t* launches,
                      uint64_t* bytes);

/* Phase-cost microbenchmarks (profiling support, no reference
 * counterpart; csrc/phasebench.hip).  One dependent phase of `wgs`
 * workgroups of 256 threads, `phases` times:
 *   mode 0  captured graph of empty dependent launches;
 *   mode 1  graph of launches that each read the previous one's output and
 *           stream bytes_per_phase of weights;
 *   mode 2  one cooperative kernel, a grid barrier per phase (per-workgroup
 *           flags, relaxed system-scope atomics) and data exchanged at
 *           system scope;
 *   mode 3  mode 2 + each phase streams its weights after the barrier;
 *   mode 4  mode 2 + the next phase's weights issued before the wait;
 *           (modes 3-4 stream a phase's slice in rounds of 16 uint4 per
 *           thread; under mode 4 only the first round precedes the wait)
 *   mode 5  float atomicAdd without return: wgs workgroups x
 *           bytes_per_phase / 4 adds over a window of `phases` addresses;
 *           us_per_phase = microseconds per launch.
 *   mode 6  XCD-local barrier: wgs (a multiple of 8) workgroups, those of
 *           one XCD meeting at a counter in that XCD's L2 each phase and
 *           reading two others' values (errors: +1000 per workgroup not on
 *           XCD id % 8).
 * us_per_phase receives the time per phase (modes 2-4: the slope between
 * a quarter-length and a full-length run); errors counts values read back
 * wrong across workgroups (+1e6 if a barrier gave up: every spin is
 * bounded). */
int chk_phase_bench(int mode, uint32_t wgs, uint32_t phases, uint64_t bytes_per_phase, double* us_per_phase,
                    uint32_t* errors);

/* Time blocks as the decode step runs them (profiling support, no
 * reference counterpart): one captured graph runs the block of `kind`
 * (2 MoE, 3 DeltaNet, 4 attention) once per layer of layers[0..n_layers),
 * block i on input rows x + (i % nx) * nb * H (device f32), and is
 * replayed `reps` times between HIP events; us_per_block = elapsed /
 * (reps * n_layers).  Attention rows sit at positions pos[0..nb) of the
 * engine's sequence (nb 1) or of its two sequence slots (nb 2); DeltaNet
 * blocks with nb > 1 take the verify form.  The blocks advance recurrent
 * state and write K/V at those positions, like the block entry points. */
int chk_time_blocks(ChkEngine* e, int kind, uint32_t nb, const uint32_t* layers, uint32_t n_layers, const float* x,
                    uint32_t nx, const uint32_t* pos, uint32_t reps, float* us_per_block);

/* The prefill attention's work plan for T dense rows at pos0 over max_wg
 * workgroups per kv head (host code, no device call; a test entry point,
 * no reference counterpart): *W workgroups, each with up to FA_MAXSEG (6)
 * segments of 4 u32 (row block, first tile, end tile, partial slot or
 * 0xffffffff for a whole row block; row block 0xffffffff ends the list),
 * written to seg[W * 6 * 4] (seg_cap u32); merge entries (row block, first
 * slot, pieces, 0) to merge (merge_cap u32), *nmerge of them; *nslots
 * partial slots. */
int chk_pf_flash_plan(uint32_t T, uint32_t pos0, uint32_t max_wg, uint32_t* W, uint32_t* nslots, uint32_t* seg,
                      uint64_t seg_cap, uint32_t* merge, uint64_t merge_cap, uint32_t* nmerge);

/* Time the decode step on the engine's stream: runs `steps` step_rows(1)
 * + commit pairs, returns milliseconds per step (HIP events). */
int chk_time_decode(ChkEngine* e, uint32_t first_token, uint32_t steps, float* ms_per_step, uint32_t* last_token);

#ifdef __cplusplus
}
#endif

#endif
