// The qwen4_exp engine on one MI355X: HBM-resident store, state, step
// orchestration, and the C ABI of include/cherenkov/{engine,kernels}.h.
//
// Restates the reference engine's behaviour (src/qwen4_exp/gpu.rs and
// gpu/{load,decode,state,mtp,experts,deltanet,attention}.rs) without its
// Metal structure: no command-buffer encoding, no CPU<->GPU handshake per
// MoE block (every expert record is resident, so expert addresses are
// computed on the device from the router's ids), no expert streaming.
#include <hip/hip_runtime.h>

#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include <fcntl.h>
#include <unistd.h>

#include "cherenkov/engine.h"
#include "cherenkov/kernels.h"
#include "kernels_internal.h"
#include "store.h"

namespace chk {

thread_local std::string g_err;

struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

#define HIPCHK(x)                                                                                   \
    do {                                                                                            \
        hipError_t e_ = (x);                                                                        \
        if (e_ != hipSuccess)                                                                       \
            throw Error(std::string("HIP error ") + hipGetErrorString(e_) + " at " #x);             \
    } while (0)

static void ensure(bool ok, const std::string& msg) {
    if (!ok) throw Error(msg);
}

RecordLayout record_layout(uint32_t bits, uint32_t hidden, uint32_t inter) {
    RecordLayout L{};
    const uint64_t page = 16384;
    uint64_t codes = (uint64_t)inter * hidden;
    L.bits = bits;
    L.scale_up = (uint64_t)inter * (hidden / 64) * 2;
    L.scale_down = (uint64_t)hidden * (inter / 64) * 2;
    if (bits == 4) {
        uint64_t off = 0;
        auto take = [&](uint64_t n) { uint64_t o = off; off += n; return o; };
        L.mat = codes / 2;
        L.gate_w = take(codes / 2); L.up_w = take(codes / 2); L.down_w = take(codes / 2);
        L.gate_s = take(L.scale_up); L.gate_b = take(L.scale_up);
        L.up_s = take(L.scale_up); L.up_b = take(L.scale_up);
        L.down_s = take(L.scale_down); L.down_b = take(L.scale_down);
        L.bytes = off;
    } else {
        // lowbit::Layout::new (lowbit.rs:81-115): 3 matrices then 6
        // scale/bias blocks of scale_bytes each.
        uint64_t mat = codes * bits / 8, sb = L.scale_up;
        L.mat = mat;
        L.gate_w = 0; L.up_w = mat; L.down_w = 2 * mat;
        L.gate_s = 3 * mat; L.gate_b = 3 * mat + sb; L.up_s = 3 * mat + 2 * sb; L.up_b = 3 * mat + 3 * sb;
        L.down_s = 3 * mat + 4 * sb; L.down_b = 3 * mat + 5 * sb;
        L.bytes = 3 * mat + 6 * sb;
    }
    L.stride = (L.bytes + page - 1) / page * page;
    return L;
}

// Bump allocator over one HBM block; a dry run (base == 0) sizes it.
struct Bump {
    uint8_t* base = nullptr;
    uint64_t off = 0;
    bool gen = false;
    template <class T>
    T* take(uint64_t n) {
        off = (off + 255) & ~(uint64_t)255;
        T* p = reinterpret_cast<T*>(base + off);
        off += n * sizeof(T);
        return p;
    }
};

// The PLE block's weights (PleWeights, cpu.rs:62-75): key / value
// projections of the n-gram embedding, three grouped-norm weights and the
// depthwise conv [hc * H][kernel].
struct PleDev {
    Q4Mat key{}, value{};
    const uint16_t *norm_key = nullptr, *norm_query = nullptr, *norm_conv = nullptr, *conv = nullptr;
};

struct LayerDev {
    bool linear = false;
    int dn_idx = -1, at_idx = -1;
    HcDev attn_hc{}, mlp_hc{};
    DnDev dn{};
    AtDev at{};
    MoeDev moe{};
    bool has_ple = false;
    PleDev ple{};
};

enum { PROF_NONE = 0, PROF_MOE = 1, PROF_DN_PROJ = 2, PROF_LM_HEAD = 3 };

struct Scratch {
    uint32_t* tokens;
    float *hyper, *hc_d, *hc_inv, *inj_a, *inj_m, *mixed;
    float *dn_conv, *dn_z, *dn_decay, *dn_beta, *dn_y, *dn_ssq;
    XqChunk *dn_y_xq, *act_xq;
    float *q_raw, *k_raw, *v_raw, *idx_raw, *q_ready, *attn_out, *part;
    float *iq_ready, *bscore;  // QSA (allocated when some context can pass the budget)
    uint32_t* vmask;
    float *router_logits, *router_probs, *sg, *route_w, *act, *mix_out;
    uint32_t *route_ids, *counter;
    float *logits, *pv;
    uint32_t *pi, *out_tok;
    uint32_t *rowpos, *rowpos_aux;  // device row positions: trunk rows / other callers
    StepIn* h_in;                   // pinned host, device-mapped
    StepIn* d_in;
    uint32_t* h_out;                // pinned host, device-mapped argmax output
    uint32_t* d_out;
    // MTP
    float *mtp_hyper, *mtp_hn, *mtp_fe, *mtp_fh, *mtp_src, *mtp_logits;
    uint32_t* mtp_out;
    float* trace;  // [L][MAX_NB][hh] when tracing
    // PLE: n-gram embedding, key, value, gated value and its norm per row
    float *ple_e, *ple_key, *ple_value, *ple_gated, *ple_gvn;
};

// Chunk buffers of the GEMM prefill (allocated on its first use), `cap`
// rows per chunk.  The DeltaNet and attention blocks share one arena.
struct PfBufs {
    uint32_t cap = 0;
    uint32_t *tokens, *pos;
    float* hyper;
    uint4 *hi, *lo, *bhi, *bmid, *blo;
    float* xs;
    float *inv, *d, *inj_a, *inj_m, *mixed, *hc_part;
    uint4 *dhi, *dlo;  // d staged as the hyper-connection up GEMM's operands
    float* dxs;
    uint4 *ahi, *alo;  // the expert activations staged as the down GEMM's operands
    float* axs;
    float *raw, *z, *a, *b, *conv, *decay, *beta, *y;
    uint32_t ab_split = 1;  // K chunks of the a / b projections
    // the block's out-projection, left as K-chunk partials (in yd) for the
    // next hyper-connection read to inject
    const float* pend = nullptr;
    uint32_t pend_split = 0;
    // the expert block's combine and inject, left (in yd) for the next
    // hyper-connection read: the streams it goes into, and the rows
    float* moe_pend = nullptr;
    uint32_t moe_pend_T = 0;
    float* dcw;  // chunked-scan workspace (null: sequential scan)
    float *q_raw, *k_raw, *v_raw, *idx_raw, *q_ready, *attn_out;
    float *logits, *sg, *wts;
    uint32_t *ids, *list, *count, *tiles, *ntiles;
    uint32_t* gcnt;  // [E][PF_GCNT_STRIDE] per-expert entry counts, zero between layers
    uint2* tinfo;   // per tile of both lists: (group's first grouped row, group's rows)
    uint32_t* goff;  // [E + 1] each group's first grouped row of act / yd
    uint32_t* gpos;  // [T][k + 1] each entry's group << 22 | place in the group
    float *act, *yd;
    float* act_sh;  // [T][SI] the shared expert's activations when SI != I (else null)
    // MTP head over a chunk: the tokens after each row, rms_norm_shift(e),
    // the normed trunk streams, fc_e / fc_h outputs and the head's residual
    uint32_t* mtp_tok;
    float *mtp_en, *mtp_hn, *mtp_fe, *mtp_fh, *mtp_hyper;
    // the flash attention plan (pf_flash_plan) for the chunk's dense rows,
    // uploaded for the (rows, first position) key it was made for
    uint4 *fa_seg, *fa_merge;
    float* fa_part;
    uint64_t fa_key = ~0ull;
    uint32_t fa_W = 0, fa_nslots = 0, fa_nmerge = 0;
    // QSA past the budget: every row's index queries; scores, selections
    // and attention partials of qsa_rows rows at a time
    float *iq_ready, *qsa_bscore, *qsa_part;
    uint32_t* qsa_vmask;
    uint32_t qsa_rows;
    // every row's block mask of the chunk's latest attention layer (rows
    // that attend densely: no bits), for the debug_engine_blocks view;
    // rows of the latest chunk
    uint32_t* qsa_rows_mask;
    uint32_t last_rows, last_pos0;
    // PLE over a chunk: table rows of each row's token, then as Scratch
    uint32_t* ple_ids;
    float *ple_e, *ple_key, *ple_value, *ple_gated, *ple_gvn;
};

}  // namespace chk

using namespace chk;

struct ChkEngine {
    ChkConfig c{};
    ChkOptions o{};
    Dims D{};
    hipStream_t st = nullptr;
    std::vector<void*> allocs;
    uint8_t* dense = nullptr;
    uint64_t dense_bytes = 0;
    RecordLayout rl4{}, rllo{};
    uint8_t* experts4 = nullptr;
    uint8_t* experts_lo = nullptr;
    // per-record precision (residency.rs:290-310): kind of record rid (0
    // 4-bit, else the low-bit store's kind), on the device for the expert
    // kernels and in pinned host memory, from which each change is copied
    uint8_t* rec_kind = nullptr;
    uint8_t* rec_kind_host = nullptr;
    // records of a low-bit store switched to their 4-bit copy: while none
    // is, the expert kernels take the kind table as absent (their pure
    // low-bit form); the step graphs are recaptured when that changes
    uint32_t kinds_q4 = 0;
    uint32_t record_layers = 0;
    uint32_t ncu = 256;  // compute units of the device (flash attention plans)
    uint64_t state_bytes = 0, kv_bytes = 0, scratch_bytes = 0;
    Q4Mat embed{}, lm_head{};
    std::vector<LayerDev> layers;
    HcDev final_mixer{};
    bool has_mtp = false;
    LayerDev mtp_layer{};
    HcDev mtp_mixer{};
    const uint16_t* mtp_enorm = nullptr;
    const uint16_t* mtp_hnorm = nullptr;
    Q4Mat fc_e{}, fc_h{};
    // PLE n-gram block: its decoder layer (-1: none), the n-gram table
    // (ngram.bin rows in HBM), the hash metadata the host computes row ids
    // with, the gvn ring [span][hh] and the ring rows a verify step may
    // roll back [MAX_NB][hh]
    int ple_l = -1;
    uint8_t* ngram = nullptr;
    uint64_t ngram_rows = 0, ngram_row_bytes = 0;
    uint32_t ngram_dim = 0, ngram_group = 0, ngram_heads = 0, ple_span = 0;
    std::vector<int64_t> ngram_mult;
    std::vector<uint64_t> ngram_offs, ngram_sizes;
    float* ple_ring = nullptr;
    float* ple_backup = nullptr;
    // cumulative routed-expert activity (activity.rs:11-89): per record
    // (record layer, expert) the rows that chose it and its lookups
    uint64_t* act = nullptr;
    std::chrono::steady_clock::time_point act_started;
    // state
    std::vector<float*> dn_state, dn_hist, dn_snap_state, dn_snap_hist;
    std::vector<KvDev> kv, kv2;
    KvDev mtp_kv{};
    Scratch s{};
    PfBufs pf{};
    // all-logits mode of prefill_chunk: every row's logits of the last call
    float* pf_all = nullptr;
    uint64_t pf_all_cap = 0;  // rows the buffer holds
    uint32_t pf_all_rows = 0; // rows of the last call kept (0: not kept)
    std::vector<float> host_pf_row;
    // rows of s.logits valid for logits_row (the last step's rows; 1 after
    // a prefill, which writes its final row only)
    uint32_t logit_rows = 0;
    uint32_t max_chunks = 1, lm_parts = 1024;
    // sequence
    uint32_t pos = 0, batch_pos = 0, batch_nb = 0, max_t = 0, trunk_rows = 1;
    bool batch_snap = false;
    uint32_t mtp_len = 0;
    std::vector<uint32_t> tokens;
    std::vector<float> host_logits, host_mtp_logits;
    uint32_t last_mtp_rows = 0;
    bool tracing = false;
    // captured decode steps, keyed by (rows * 2 + snap) * 4 + profiled
    // kernel class; a profiled graph holds HIP event pairs around each
    // launch of that class (graph-owned events [ev0, ev1) of graph_events)
    struct StepGraph {
        hipGraphExec_t exec;
        size_t ev0, ev1;
    };
    std::map<int, StepGraph> graphs;
    bool use_graphs = true;
    bool capturing = false;
    struct EvPair {
        hipEvent_t a, b;
        uint64_t bytes;
    };
    std::vector<EvPair> graph_events;
    // folded MTP pass results of the last step (one draft per row)
    bool folded_valid = false;
    std::vector<uint32_t> folded;
    // live profiler: HIP events around one kernel class on the engine stream
    int prof_kind = 0;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> prof_events;
    size_t prof_used = 0;
    uint64_t prof_bytes = 0, prof_launches = 0;
    double prof_ms = 0.0;

    // the next unused eager event pair (created on first use)
    std::pair<hipEvent_t, hipEvent_t> prof_pair() {
        if (prof_used == prof_events.size()) {
            hipEvent_t a, b;
            HIPCHK(hipEventCreate(&a));
            HIPCHK(hipEventCreate(&b));
            prof_events.push_back({a, b});
        }
        return prof_events[prof_used];
    }
    void prof_begin(int kind) {
        if (prof_kind != kind) return;
        if (capturing) {
            EvPair ev{};
            HIPCHK(hipEventCreate(&ev.a));
            HIPCHK(hipEventCreate(&ev.b));
            graph_events.push_back(ev);
            HIPCHK(hipEventRecord(ev.a, st));
            return;
        }
        if (prof_used == prof_events.size()) {
            hipEvent_t a, b;
            HIPCHK(hipEventCreate(&a));
            HIPCHK(hipEventCreate(&b));
            prof_events.push_back({a, b});
        }
        HIPCHK(hipEventRecord(prof_events[prof_used].first, st));
    }
    void prof_end(int kind, uint64_t bytes) {
        if (prof_kind != kind) return;
        if (capturing) {
            graph_events.back().bytes = bytes;
            HIPCHK(hipEventRecord(graph_events.back().b, st));
            return;
        }
        HIPCHK(hipEventRecord(prof_events[prof_used].second, st));
        ++prof_used;
        prof_bytes += bytes;
        ++prof_launches;
    }
    void prof_collect() {
        if (!prof_used) return;
        HIPCHK(hipStreamSynchronize(st));
        for (size_t i = 0; i < prof_used; ++i) {
            float ms = 0;
            HIPCHK(hipEventElapsedTime(&ms, prof_events[i].first, prof_events[i].second));
            prof_ms += ms;
        }
        prof_used = 0;
    }
    // after a replay of a profiled graph has finished: its event pairs
    void prof_collect_graph(const StepGraph& g) {
        for (size_t i = g.ev0; i < g.ev1; ++i) {
            float ms = 0;
            HIPCHK(hipEventElapsedTime(&ms, graph_events[i].a, graph_events[i].b));
            prof_ms += ms;
            prof_bytes += graph_events[i].bytes;
            ++prof_launches;
        }
    }
    uint64_t q4_bytes(const Q4Mat& m) const { return (uint64_t)m.out * m.in / 2 + 4ull * (m.out * (m.in / 64)); }
    uint64_t expert_mat_bytes() const {
        uint64_t codes = (uint64_t)D.I * D.H;
        if (o.experts == 4) return codes / 2 + 4 * (codes / 64);
        return codes * o.experts / 8 + 4 * (codes / 64);
    }

    // drops the captured step graphs (recaptured on their next use)
    void drop_graphs() {
        HIPCHK(hipStreamSynchronize(st));
        for (auto& kv : graphs) HIPCHK(hipGraphExecDestroy(kv.second.exec));
        graphs.clear();
    }

    ~ChkEngine() {
        if (st) hipStreamSynchronize(st);
        for (auto& kv : graphs) hipGraphExecDestroy(kv.second.exec);
        for (auto& ev : graph_events) {
            hipEventDestroy(ev.a);
            hipEventDestroy(ev.b);
        }
        if (staging) hipHostFree(staging);
        if (dense_fd >= 0) close(dense_fd);
        if (experts_fd >= 0) close(experts_fd);
        if (ngram_fd >= 0) close(ngram_fd);
        if (rec_kind_host) hipHostFree(rec_kind_host);
        if (s.h_in) hipHostFree(s.h_in);
        if (s.h_out) hipHostFree(s.h_out);
        for (void* p : allocs) hipFree(p);
        for (void* p : pf_allocs) hipFree(p);
        if (st) hipStreamDestroy(st);
    }

    // Device allocations: engine lifetime (`allocs`) or prefill scratch
    // (`pf_allocs`, dropped by prefill_release); `alloc_bytes` counts both.
    std::vector<void*> pf_allocs;
    uint64_t alloc_bytes = 0, pf_alloc_bytes = 0;
    // Gpu::load_bounded (gpu/load.rs:12-63): the server's memory budget
    // (memory_bytes - reserve) every device buffer of the engine counts
    // against (0: no budget), and the prefill rows whose scratch the load
    // keeps room for
    uint64_t mem_limit = 0;
    uint32_t budget_prefill_rows = 0;
    template <class T>
    T* dalloc(uint64_t n, bool prefill_scratch = false) {
        void* p = nullptr;
        const uint64_t bytes = std::max<uint64_t>(n * sizeof(T), 256);
        // MetalContext::check_allocation (metal.rs:145-156)
        ensure(!mem_limit || alloc_bytes + bytes <= mem_limit,
               "allocation would exceed the server memory budget; reduce pool or prefill chunk size");
        HIPCHK(hipMalloc(&p, bytes));
        (prefill_scratch ? pf_allocs : allocs).push_back(p);
        alloc_bytes += bytes;
        if (prefill_scratch) pf_alloc_bytes += bytes;
        return reinterpret_cast<T*>(p);
    }
    template <class T>
    T* pfalloc(uint64_t n) { return dalloc<T>(n, true); }
    void prefill_release() {
        if (st) hipStreamSynchronize(st);
        for (void* p : pf_allocs) hipFree(p);
        pf_allocs.clear();
        alloc_bytes -= pf_alloc_bytes;
        pf_alloc_bytes = 0;
        pf = PfBufs{};
        pf_all = nullptr;
        pf_all_rows = 0;
        pf_all_cap = 0;
    }

    bool is_linear(uint32_t l) const { return (l + 1) % c.full_attention_interval != 0; }

    // ------------------------------------------------------ store build
    // Weights come from the seeded generator (synth.h), or, for an engine
    // loaded from a packed store, from its dense.bin / experts.bin.
    const Store* src = nullptr;
    int dense_fd = -1, experts_fd = -1, ngram_fd = -1;
    uint8_t* staging = nullptr;  // pinned host buffer for store uploads
    static constexpr uint64_t STAGING = 64ull << 20;

    // copy `n` bytes at `off` of an open store file to device memory
    void upload(int fd, uint64_t off, uint64_t n, void* dst) {
        uint8_t* d = static_cast<uint8_t*>(dst);
        for (uint64_t done = 0; done < n;) {
            const uint64_t m = std::min<uint64_t>(STAGING, n - done);
            HIPCHK(hipStreamSynchronize(st));  // the staging buffer is free again
            uint64_t got = 0;
            while (got < m) {
                const ssize_t r = pread(fd, staging + got, m - got, (off_t)(off + done + got));
                ensure(r > 0, "short read of the packed store");
                got += (uint64_t)r;
            }
            HIPCHK(hipMemcpyAsync(d + done, staging, m, hipMemcpyHostToDevice, st));
            done += m;
        }
    }
    const DenseEntry& store_entry(const std::string& name, const char* dtype, std::vector<uint64_t> shape) {
        const DenseEntry& e = src->entry(name);
        ensure(e.dtype == dtype, name + ": expected " + dtype + ", got " + e.dtype);
        ensure(e.shape == shape, name + ": shape does not match the config");
        uint64_t n = e.dtype == "U32" ? 4 : e.dtype == "I64" ? 8 : 2;
        for (uint64_t x : shape) n *= x;
        ensure(e.nbytes == n, name + ": byte count does not match its shape");
        return e;
    }

    std::vector<int64_t> store_i64(const std::string& name, uint64_t n) {
        const DenseEntry& e = store_entry(name, "I64", {n});
        std::vector<int64_t> v(n);
        for (uint64_t done = 0; done < e.nbytes;) {
            const ssize_t r = pread(dense_fd, reinterpret_cast<uint8_t*>(v.data()) + done, e.nbytes - done,
                                    (off_t)(e.offset + done));
            ensure(r > 0, "short read of the packed store");
            done += (uint64_t)r;
        }
        return v;
    }
    Q4Mat q4(Bump& B, uint32_t kind, uint32_t slot, uint32_t part, uint32_t out, uint32_t in) {
        Q4Mat m{};
        m.out = out;
        m.in = in;
        uint32_t* w = B.take<uint32_t>((uint64_t)out * in / 8);
        uint16_t* s = B.take<uint16_t>((uint64_t)out * in / 64);
        uint16_t* b = B.take<uint16_t>((uint64_t)out * in / 64);
        m.w = w; m.s = s; m.b = b;
        if (B.gen && src) {
            // Packed::qlinear (packed.rs:154-179): {prefix}.weight U32
            // [out, in/8], .scales / .biases BF16 [out, in/64]
            const std::string p = tensor_name(c, kind, slot, part);
            const DenseEntry& ew = store_entry(p + ".weight", "U32", {out, in / 8});
            const DenseEntry& es = store_entry(p + ".scales", "BF16", {out, in / 64});
            const DenseEntry& eb = store_entry(p + ".biases", "BF16", {out, in / 64});
            upload(dense_fd, ew.offset, ew.nbytes, w);
            upload(dense_fd, es.offset, es.nbytes, s);
            upload(dense_fd, eb.offset, eb.nbytes, b);
        } else if (B.gen) {
            gen_q4(w, s, b, out, in, c.seed, chk_tensor_id(kind, slot, 0, part), st);
        }
        return m;
    }
    const uint16_t* bf(Bump& B, uint32_t kind, uint32_t slot, uint32_t part, uint64_t n) {
        uint16_t* p = B.take<uint16_t>(n);
        if (B.gen && src) {
            const std::string name = tensor_name(c, kind, slot, part);
            const DenseEntry& e = src->entry(name);
            ensure(e.dtype == "BF16", name + ": expected BF16, got " + e.dtype);
            ensure(e.nbytes == n * 2, name + ": element count does not match the config");
            upload(dense_fd, e.offset, e.nbytes, p);
        } else if (B.gen) {
            gen_bf16(p, n, c.seed, chk_tensor_id(kind, slot, 0, part), kind, st);
        }
        return p;
    }
    // experts.bin: record layer rl of this engine is the store's record
    // layer of the same prefix (main layers in order, then the MTP layer,
    // pack.rs:351-393); a record's fields move to this engine's layout
    void upload_records() {
        const StoreExperts& X = src->experts;
        const bool same = X.record_stride == rl4.stride && X.gate_w == rl4.gate_w && X.up_w == rl4.up_w &&
                          X.down_w == rl4.down_w && X.gate_s == rl4.gate_s && X.gate_b == rl4.gate_b &&
                          X.up_s == rl4.up_s && X.up_b == rl4.up_b && X.down_s == rl4.down_s &&
                          X.down_b == rl4.down_b;
        for (uint32_t rl = 0; rl < record_layers; ++rl) {
            const std::string want = rl < c.num_hidden_layers
                                         ? "language_model.model.layers." + std::to_string(rl) + ".mlp.switch_mlp"
                                         : std::string("mtp.layers.0.mlp.switch_mlp");
            uint64_t idx = X.layers;
            for (uint64_t i = 0; i < X.layers; ++i)
                if (X.layer_prefixes[i] == want) idx = i;
            ensure(idx < X.layers, "no expert records for " + want);
            uint8_t* dst = experts4 + (uint64_t)rl * D.E * rl4.stride;
            if (same) {
                upload(experts_fd, idx * X.experts * X.record_stride, (uint64_t)D.E * rl4.stride, dst);
                continue;
            }
            const uint64_t codes = (uint64_t)D.I * D.H / 2;
            const uint64_t src_off[9] = {X.gate_w, X.up_w, X.down_w, X.gate_s, X.gate_b, X.up_s, X.up_b, X.down_s, X.down_b};
            const uint64_t dst_off[9] = {rl4.gate_w, rl4.up_w, rl4.down_w, rl4.gate_s, rl4.gate_b,
                                         rl4.up_s, rl4.up_b, rl4.down_s, rl4.down_b};
            const uint64_t len[9] = {codes, codes, codes, rl4.scale_up, rl4.scale_up, rl4.scale_up, rl4.scale_up,
                                     rl4.scale_down, rl4.scale_down};
            for (uint32_t e = 0; e < D.E; ++e) {
                const uint64_t rec = (idx * X.experts + e) * X.record_stride;
                for (int k = 0; k < 9; ++k) upload(experts_fd, rec + src_off[k], len[k], dst + e * rl4.stride + dst_off[k]);
            }
        }
        HIPCHK(hipStreamSynchronize(st));
    }
    HcDev hc(Bump& B, uint32_t slot, uint32_t part, bool inject) {
        HcDev w{};
        uint32_t hh = D.hh;
        w.norm = bf(B, CHK_T_HC_NORM, slot, part, hh);
        w.down = q4(B, CHK_T_HC_DOWN, slot, part, c.hc_lowrank, hh);
        w.up = q4(B, CHK_T_HC_UP, slot, part, hh, c.hc_lowrank);
        w.has_inject = inject;
        if (inject) w.inject = q4(B, CHK_T_HC_INJECT, slot, part, c.hc_count, hh);
        return w;
    }
    void layer(Bump& B, LayerDev& L, uint32_t slot, bool linear, uint32_t record_layer) {
        uint32_t H = D.H;
        L.linear = linear;
        L.attn_hc = hc(B, slot, CHK_HC_ATTN, true);
        L.mlp_hc = hc(B, slot, CHK_HC_MLP, true);
        if (linear) {
            L.dn.qkv = q4(B, CHK_T_DN_QKV, slot, 0, D.conv_dim, H);
            L.dn.z = q4(B, CHK_T_DN_Z, slot, 0, D.v_dim, H);
            L.dn.a = q4(B, CHK_T_DN_A, slot, 0, D.nv, H);
            L.dn.b = q4(B, CHK_T_DN_B, slot, 0, D.nv, H);
            L.dn.out = q4(B, CHK_T_DN_OUT, slot, 0, H, D.v_dim);
            L.dn.conv = bf(B, CHK_T_DN_CONV, slot, 0, (uint64_t)D.conv_dim * D.ck);
            L.dn.a_log = bf(B, CHK_T_DN_ALOG, slot, 0, D.nv);
            L.dn.dt_bias = bf(B, CHK_T_DN_DTBIAS, slot, 0, D.nv);
            L.dn.norm = bf(B, CHK_T_DN_NORM, slot, 0, D.dv);
        } else {
            L.at.q = q4(B, CHK_T_AT_Q, slot, 0, 2 * D.nh * D.hd, H);
            L.at.k = q4(B, CHK_T_AT_K, slot, 0, D.nkv * D.hd, H);
            L.at.v = q4(B, CHK_T_AT_V, slot, 0, D.nkv * D.hd, H);
            L.at.o = q4(B, CHK_T_AT_O, slot, 0, H, D.nh * D.hd);
            L.at.idx = q4(B, CHK_T_AT_IDX, slot, 0, D.idx_out, H);
            L.at.q_norm = bf(B, CHK_T_AT_QNORM, slot, 0, D.hd);
            L.at.k_norm = bf(B, CHK_T_AT_KNORM, slot, 0, D.hd);
            L.at.idx_q_norm = bf(B, CHK_T_AT_IDX_QNORM, slot, 0, D.ihd);
            L.at.idx_k_norm = bf(B, CHK_T_AT_IDX_KNORM, slot, 0, D.ihd);
        }
        L.moe.router = bf(B, CHK_T_MOE_ROUTER, slot, 0, (uint64_t)D.E * H);
        L.moe.shared_gate = bf(B, CHK_T_MOE_SHARED_GATE, slot, 0, H);
        L.moe.sh_gate = q4(B, CHK_T_MOE_SH_GATE_PROJ, slot, 0, D.SI, H);
        L.moe.sh_up = q4(B, CHK_T_MOE_SH_UP, slot, 0, D.SI, H);
        L.moe.sh_down = q4(B, CHK_T_MOE_SH_DOWN, slot, 0, H, D.SI);
        L.moe.record_layer = record_layer;
        if ((int)slot == ple_l) {
            const uint32_t E = c.ple_embed_dim;
            L.has_ple = true;
            L.ple.key = q4(B, CHK_T_PLE_KEY, slot, 0, D.hh, E);
            L.ple.value = q4(B, CHK_T_PLE_VALUE, slot, 0, H, E);
            L.ple.norm_key = bf(B, CHK_T_PLE_NORM_KEY, slot, 0, D.hh);
            L.ple.norm_query = bf(B, CHK_T_PLE_NORM_QUERY, slot, 0, D.hh);
            L.ple.norm_conv = bf(B, CHK_T_PLE_NORM_CONV, slot, 0, D.hh);
            L.ple.conv = bf(B, CHK_T_PLE_CONV, slot, 0, (uint64_t)D.hh * c.ple_conv_kernel_size);
        }
    }
    // The n-gram table and its hash metadata: a store's ngram.bin and
    // {layer}.ple.ple_embedding.* tensors (packed.rs:134-148), else the
    // synthetic table of synth.h.
    void build_ngram() {
        const uint32_t heads = ngram_heads;
        if (src) {
            const StoreNgram& N = src->ngram;
            const std::string pre = tensor_name(c, CHK_T_NGRAM_MULT, (uint32_t)ple_l, 0);
            ngram_mult = store_i64(pre + ".layer_multipliers", c.ngram_size);
            const std::vector<int64_t> offs = store_i64(pre + ".ngram_heads_offsets", heads);
            const std::vector<int64_t> sizes = store_i64(pre + ".ngram_heads_vocab_sizes", heads);
            for (uint32_t h = 0; h < heads; ++h)
                ensure(offs[h] >= 0 && sizes[h] >= 0, "n-gram heads exceed the table");
            ngram_offs.assign(offs.begin(), offs.end());
            ngram_sizes.assign(sizes.begin(), sizes.end());
            ensure(N.dim * heads == c.ple_embed_dim, "n-gram head layout mismatch");
            ngram_rows = N.rows;
            ngram_row_bytes = N.row_bytes;
        } else {
            ngram_mult.resize(c.ngram_size);
            for (uint32_t k = 0; k < c.ngram_size; ++k) ngram_mult[k] = chk_ngram_multiplier(c.seed, k);
            ngram_offs.resize(heads);
            ngram_sizes.resize(heads);
            uint64_t off = 0;
            for (uint32_t h = 0; h < heads; ++h) {
                ngram_sizes[h] = chk_ngram_head_size(c.ngram_head_rows, h);
                ngram_offs[h] = off;
                off += ngram_sizes[h];
            }
            ngram_rows = off;
            ngram_row_bytes = chk_ngram_row_bytes(ngram_dim, ngram_group);
        }
        for (uint32_t h = 0; h < heads; ++h)
            ensure(ngram_sizes[h] >= 1 && ngram_offs[h] <= ngram_rows && ngram_sizes[h] <= ngram_rows - ngram_offs[h],
                   "n-gram heads exceed the table");
        ensure(ngram_rows < (1ull << 32), "n-gram table above 2^32 rows");
        ngram = dalloc<uint8_t>(ngram_rows * ngram_row_bytes);
        if (src) upload(ngram_fd, 0, ngram_rows * ngram_row_bytes, ngram);
        else gen_ngram_table(ngram, ngram_rows, ngram_dim, ngram_group, c.seed, st);
    }
    void build_dense(Bump& B) {
        uint32_t H = D.H, L = c.num_hidden_layers;
        embed = q4(B, CHK_T_EMBED, 0, 0, D.V, H);
        lm_head = q4(B, CHK_T_LM_HEAD, 0, 0, D.V, H);
        layers.assign(L, LayerDev{});
        int dn_i = 0, at_i = 0;
        for (uint32_t l = 0; l < L; ++l) {
            layer(B, layers[l], l, is_linear(l), l);
            if (layers[l].linear) layers[l].dn_idx = dn_i++;
            else layers[l].at_idx = at_i++;
        }
        final_mixer = hc(B, 0, CHK_HC_FINAL, false);
        if (has_mtp) {
            mtp_enorm = bf(B, CHK_T_MTP_ENORM, L, 0, H);
            mtp_hnorm = bf(B, CHK_T_MTP_HNORM, L, 0, D.hh);
            fc_e = q4(B, CHK_T_MTP_FC_E, L, 0, H, H);
            fc_h = q4(B, CHK_T_MTP_FC_H, L, 0, H, H);
            layer(B, mtp_layer, L, false, L);
            mtp_mixer = hc(B, L, CHK_HC_MTP, false);
        }
    }

    // the store the expert kernels decode at its precision (bits 4: the
    // 4-bit store; 3 / 2: the low-bit store, whose records of kind 0 come
    // from the 4-bit one)
    ExpertsDev experts_dev(bool q4 = false) const {
        ExpertsDev X{};
        q4 = q4 || o.experts == 4;
        const RecordLayout& R = q4 ? rl4 : rllo;
        X.base = q4 ? experts4 : experts_lo;
        X.stride = R.stride;
        X.bits = q4 ? 4 : o.experts;
        X.experts = D.E;
        X.gate_w = R.gate_w; X.up_w = R.up_w; X.down_w = R.down_w;
        X.gate_s = R.gate_s; X.gate_b = R.gate_b; X.up_s = R.up_s; X.up_b = R.up_b;
        X.down_s = R.down_s; X.down_b = R.down_b;
        return X;
    }

    KvDev alloc_kv() {
        KvDev k{};
        k.k = dalloc<int8_t>((uint64_t)max_t * D.kv_row);
        k.v = dalloc<int8_t>((uint64_t)max_t * D.kv_row);
        k.ks = dalloc<uint16_t>((uint64_t)max_t * D.kv_row / 32);
        k.vs = dalloc<uint16_t>((uint64_t)max_t * D.kv_row / 32);
        k.index_k = dalloc<float>((uint64_t)max_t * D.ihd);
        kv_bytes += (uint64_t)max_t * (2 * D.kv_row + D.kv_row / 8 + 4 * D.ihd);
        if (D.qsa) {
            k.block_k = dalloc<float>((uint64_t)D.max_blocks * D.ihd);
            kv_bytes += (uint64_t)D.max_blocks * D.ihd * 4;
        }
        return k;
    }

    void load(const ChkConfig* cfg, const ChkOptions* opt) {
        c = *cfg;
        o = *opt;
        ensure(o.experts == 4 || o.experts == 3 || o.experts == 2, "expert precision must be 4, 3 or 2 bits");
        ensure(o.drafts <= 3, "drafts must be 0..=3");
        ensure(o.max_t >= 1, "max_t must be positive");
        ensure(c.full_attention_interval >= 1 && c.num_hidden_layers >= 1, "layer pattern");
        ensure(c.hc_count >= 2 && c.hc_count <= 4, "hc_count must be 2..=4 (one hyper-connection stream per wave)");
        ensure(c.hidden_size % 256 == 0, "hidden % 256 == 0 (gpu/load.rs:25-28)");
        // the batch-1 kernels hold one or two 32-input chunks per lane of a
        // wave (64 lanes)
        ensure(c.hidden_size <= 4096, "hidden size must be at most 4096 (two 32-input chunks per lane)");
        // the up + mix kernel keeps one row slot per stream in a wave's 64
        // lanes (<= 16 lanes a slot at hc 4), each lane one 32-input chunk
        ensure(c.hc_lowrank % 32 == 0 && c.hc_lowrank <= 512, "hc_lowrank must be a multiple of 32 up to 512");
        ensure(c.moe_intermediate_size % 64 == 0, "expert width must be a multiple of 64 (gpu/load.rs:37-40)");
        ensure(c.shared_expert_intermediate_size % 64 == 0 && c.shared_expert_intermediate_size >= 64 &&
                   c.shared_expert_intermediate_size <= 1024,
               "shared expert width must be a multiple of 64 up to 1024");
        ensure(c.linear_key_head_dim == 128, "DeltaNet key head dim must be 128");
        ensure(c.linear_value_head_dim * 4 <= 1024, "DeltaNet value head dim too wide");
        ensure(c.linear_num_value_heads % c.linear_num_key_heads == 0, "value heads must group key heads");
        ensure(c.head_dim <= 256 && c.head_dim % 64 == 0, "head_dim must be 64..256");
        ensure(c.indexer_head_dim <= 256 && c.indexer_head_dim % 32 == 0,
               "indexer head dim must be a multiple of 32 up to 256 (gpu/load.rs:29-32)");
        ensure(c.indexer_budget % c.indexer_compress_ratio == 0,
               "indexer budget must be a multiple of the block size (gpu/load.rs:33-36)");
        ensure(c.num_experts <= 512 && c.num_experts_per_tok <= 64 && c.num_experts_per_tok <= c.num_experts,
               "at most 512 experts and 64 per token");
        ensure(c.ple_layer <= c.num_hidden_layers, "ple_layer_ids beyond the decoder layers");
        if (c.ple_layer) {
            ple_l = (int)c.ple_layer - 1;
            ensure(c.ngram_size >= 2 && c.ngram_size <= 16 && c.heads_per_ngram >= 1,
                   "n-gram orders 2..=ngram_size (at most 16) need heads");
            ngram_heads = (c.ngram_size - 1) * c.heads_per_ngram;
            ensure(ngram_heads <= MAX_NGRAM_IDS, "at most 32 n-gram heads");
            ensure(c.ple_embed_dim % 64 == 0 && c.ple_embed_dim % ngram_heads == 0,
                   "ple_embed_dim must be a multiple of 64 and of the n-gram heads");
            ngram_dim = c.ple_embed_dim / ngram_heads;
            ngram_group = src ? (uint32_t)src->ngram.group : c.ngram_group;
            ensure(ngram_group >= 1 && ngram_dim % 8 == 0 && ngram_dim % ngram_group == 0,
                   "n-gram rows must be whole words and groups");
            ensure(c.ple_conv_kernel_size >= 2 && c.ple_conv_kernel_size <= 16, "PLE conv kernel 2..=16");
            ple_span = (c.ple_conv_kernel_size - 1) * c.ngram_size;
            ensure(ple_span >= MAX_NB, "PLE ring shorter than a verify step");
            ensure(src || c.ngram_head_rows > ngram_heads, "synthetic n-gram heads need rows");
        }
        ensure(c.linear_conv_kernel_dim >= 2 && c.linear_conv_kernel_dim <= 9, "conv kernel 2..=9");
        ensure(c.indexer_compress_ratio >= 1 && c.indexer_budget >= c.indexer_compress_ratio,
               "indexer budget must hold at least one block");
        D.H = c.hidden_size;
        D.hc = c.hc_count;
        D.hh = D.H * D.hc;
        D.lowrank = c.hc_lowrank;
        D.nk = c.linear_num_key_heads;
        D.nv = c.linear_num_value_heads;
        D.dk = c.linear_key_head_dim;
        D.dv = c.linear_value_head_dim;
        D.qk_dim = D.nk * D.dk;
        D.v_dim = D.nv * D.dv;
        D.conv_dim = 2 * D.qk_dim + D.v_dim;
        D.ck = c.linear_conv_kernel_dim;
        D.nh = c.num_attention_heads;
        D.nkv = c.num_key_value_heads;
        D.hd = c.head_dim;
        D.rot = (uint32_t)((double)D.hd * c.partial_rotary_factor);
        D.kv_row = D.nkv * D.hd;
        D.inh = c.indexer_n_heads;
        D.ihd = c.indexer_head_dim;
        D.idx_out = (D.inh + 1) * D.ihd;
        D.ratio = c.indexer_compress_ratio;
        D.kblk = c.indexer_budget / D.ratio;
        D.max_blocks = o.max_t / D.ratio + 1;
        D.mask_words = (D.max_blocks + 31) / 32;
        D.qsa = o.max_t / D.ratio > D.kblk;
        D.E = c.num_experts;
        D.topk = c.num_experts_per_tok;
        D.I = c.moe_intermediate_size;
        D.SI = c.shared_expert_intermediate_size;
        D.V = c.vocab_size;
        D.eps = (float)c.rms_norm_eps;
        D.theta = (float)c.rope_theta;
        D.attn_scale = powf((float)D.hd, -0.5f);
        D.qscale = powf((float)D.dk, -0.5f);
        D.norm_topk = c.norm_topk_prob != 0;
        // the decode kernels walk row blocks of 4 (R) rows
        for (uint32_t rows : {D.conv_dim, D.v_dim, D.nv, 2 * D.nh * D.hd, D.kv_row, D.idx_out, D.H, D.V, D.I})
            ensure(rows % 8 == 0 || (rows % 4 == 0 && rows != D.V), "matrix heights must be multiples of 4 (8 for vocab)");
        ensure(D.dv % 64 == 0 && D.dv <= 512, "DeltaNet value head dim must be a multiple of 64");
        ensure(D.E % 8 == 0 && D.E <= 512 && D.topk < 64, "experts must be a multiple of 8, at most 512, top-k below 64");
        ensure(D.I % 64 == 0, "expert width must be a multiple of 64");
        ensure(attn_shape_ok(D.nh, D.nkv, D.hd),
               "attention needs head_dim 128 or 256 and 1, 2, 4, 8 or 12 query heads per kv head");
        has_mtp = c.mtp_num_hidden_layers > 0;
        ensure(o.drafts == 0 || has_mtp, "drafts need an MTP head");
        max_t = o.max_t;
        trunk_rows = 1 + o.drafts;
        HIPCHK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
        {
            int dev = 0, n = 0;
            HIPCHK(hipGetDevice(&dev));
            HIPCHK(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
            ncu = n > 0 ? (uint32_t)n : 256u;
        }

        // dense store: dry run for the size, then allocate and generate
        Bump dry;
        build_dense(dry);
        dense_bytes = dry.off;
        dense = dalloc<uint8_t>(dense_bytes);
        if (src) HIPCHK(hipHostMalloc((void**)&staging, STAGING, hipHostMallocDefault));
        Bump B;
        B.base = dense;
        B.gen = true;
        build_dense(B);
        if (ple_l >= 0) build_ngram();

        // routed-expert store: all records resident, main layers then MTP
        record_layers = c.num_hidden_layers + (has_mtp ? 1 : 0);
        rl4 = record_layout(4, D.H, D.I);
        uint64_t n_rec = (uint64_t)record_layers * D.E;
        experts4 = dalloc<uint8_t>(n_rec * rl4.stride);
        // page padding between records stays zero whichever way the
        // records are filled (generated, uploaded whole, or field by field)
        HIPCHK(hipMemsetAsync(experts4, 0, n_rec * rl4.stride, st));
        if (src) upload_records();
        else gen_records(experts4, rl4, c.seed, D.E, 0, record_layers, D.H, D.I, st);
        if (o.experts != 4) {
            rllo = record_layout(o.experts, D.H, D.I);
            experts_lo = dalloc<uint8_t>(n_rec * rllo.stride);
            HIPCHK(hipMemsetAsync(experts_lo, 0, n_rec * rllo.stride, st));
            repack_lowbit(experts4, rl4, experts_lo, rllo, (uint32_t)n_rec, (uint64_t)D.I * D.H, st);
            // every record starts at the low-bit store's kind (8 bytes of
            // slack: the kernels read a layer's kinds 8 at a time)
            const uint8_t kind0 = o.experts == 3 ? 1 : 2;
            rec_kind = dalloc<uint8_t>(n_rec + 8);
            HIPCHK(hipHostMalloc((void**)&rec_kind_host, n_rec + 8, hipHostMallocDefault));
            memset(rec_kind_host, kind0, n_rec + 8);
            HIPCHK(hipMemcpyAsync(rec_kind, rec_kind_host, n_rec + 8, hipMemcpyHostToDevice, st));
        }

        // recurrent state, snapshots, KV
        for (uint32_t l = 0; l < c.num_hidden_layers; ++l) {
            if (layers[l].linear) {
                uint64_t sn = (uint64_t)D.nv * D.dv * D.dk, hn = (uint64_t)D.conv_dim * (D.ck - 1);
                dn_state.push_back(dalloc<float>(sn));
                dn_hist.push_back(dalloc<float>(hn));
                dn_snap_state.push_back(dalloc<float>(sn * MAX_SNAP));
                dn_snap_hist.push_back(dalloc<float>(hn * MAX_SNAP));
                state_bytes += (sn + hn) * 4 * (1 + MAX_SNAP);
            } else {
                kv.push_back(alloc_kv());
            }
        }
        if (has_mtp) mtp_kv = alloc_kv();
        if (ple_l >= 0) {
            ple_ring = dalloc<float>((uint64_t)ple_span * D.hh);
            ple_backup = dalloc<float>((uint64_t)MAX_NB * D.hh);
            state_bytes += (uint64_t)(ple_span + MAX_NB) * D.hh * 4;
        }
        max_chunks = (max_t + ATTN_CHUNK - 1) / ATTN_CHUNK;
        ensure(max_chunks <= (uint32_t)MAX_ATTN_CHUNKS, "context capacity above 262144 tokens");

        // scratch
        const uint32_t NB = MAX_NB;
        s.tokens = dalloc<uint32_t>(NB);
        s.hyper = dalloc<float>(NB * D.hh);
        s.hc_d = dalloc<float>(NB * D.lowrank);
        s.hc_inv = dalloc<float>(NB * D.hc);
        s.inj_a = dalloc<float>(NB * D.hc);
        s.inj_m = dalloc<float>(NB * D.hc);
        s.mixed = dalloc<float>(NB * D.H);
        s.dn_conv = dalloc<float>(NB * D.conv_dim);
        s.dn_z = dalloc<float>(NB * D.v_dim);
        s.dn_decay = dalloc<float>(NB * D.nv);
        s.dn_beta = dalloc<float>(NB * D.nv);
        s.dn_y = dalloc<float>(NB * D.v_dim);
        s.dn_y_xq = dalloc<XqChunk>(NB * D.v_dim / 32);
        s.dn_ssq = dalloc<float>((uint64_t)NB * D.nv * (D.dv / 16));
        s.q_raw = dalloc<float>(NB * 2 * D.nh * D.hd);
        s.k_raw = dalloc<float>(NB * D.kv_row);
        s.v_raw = dalloc<float>(NB * D.kv_row);
        s.idx_raw = dalloc<float>(NB * D.idx_out);
        s.q_ready = dalloc<float>(NB * D.nh * D.hd);
        s.attn_out = dalloc<float>(NB * D.nh * D.hd);
        s.part = dalloc<float>((uint64_t)NB * D.nh * max_chunks * (D.hd + 2));
        if (D.qsa) {
            s.iq_ready = dalloc<float>(NB * D.inh * D.ihd);
            s.bscore = dalloc<float>((uint64_t)NB * D.max_blocks);
            s.vmask = dalloc<uint32_t>((uint64_t)NB * D.mask_words);
        }
        s.router_logits = dalloc<float>(NB * D.E);
        uint32_t LR = record_layers;
        s.router_probs = dalloc<float>((uint64_t)LR * NB * D.E);
        s.route_ids = dalloc<uint32_t>((uint64_t)LR * NB * D.topk);
        s.route_w = dalloc<float>((uint64_t)LR * NB * D.topk);
        s.sg = dalloc<float>(NB);
        // a row: topk routed slots of I activations, then the shared expert's SI
        s.act = dalloc<float>((uint64_t)NB * (D.topk * D.I + D.SI));
        s.act_xq = dalloc<XqChunk>((uint64_t)NB * (D.topk * D.I + D.SI) / 32);
        s.mix_out = dalloc<float>(NB * D.H);
        act = dalloc<uint64_t>((uint64_t)LR * D.E * 2);
        HIPCHK(hipMemsetAsync(act, 0, (uint64_t)LR * D.E * 2 * 8, st));
        act_started = std::chrono::steady_clock::now();
        s.counter = dalloc<uint32_t>(64);
        HIPCHK(hipMemsetAsync(s.counter, 0, 256, st));
        s.logits = dalloc<float>((uint64_t)NB * D.V);
        s.pv = dalloc<float>((uint64_t)NB * lm_parts);
        s.pi = dalloc<uint32_t>((uint64_t)NB * lm_parts);
        s.out_tok = dalloc<uint32_t>(NB);
        s.rowpos = dalloc<uint32_t>(NB);
        s.rowpos_aux = dalloc<uint32_t>(NB);
        HIPCHK(hipHostMalloc((void**)&s.h_in, sizeof(StepIn), hipHostMallocMapped));
        HIPCHK(hipHostGetDevicePointer((void**)&s.d_in, s.h_in, 0));
        HIPCHK(hipHostMalloc((void**)&s.h_out, 64, hipHostMallocMapped));
        HIPCHK(hipHostGetDevicePointer((void**)&s.d_out, s.h_out, 0));
        memset(s.h_in, 0, sizeof(StepIn));
        s.mtp_hyper = dalloc<float>(NB * D.hh);
        s.mtp_hn = dalloc<float>((uint64_t)NB * (D.H + D.hh));
        s.mtp_src = dalloc<float>((uint64_t)D.hh);
        s.mtp_fe = dalloc<float>(NB * D.H);
        s.mtp_fh = dalloc<float>((uint64_t)NB * D.hh);
        s.mtp_logits = dalloc<float>((uint64_t)NB * D.V);
        s.mtp_out = dalloc<uint32_t>(NB);
        s.trace = nullptr;
        if (ple_l >= 0) {
            s.ple_e = dalloc<float>((uint64_t)NB * c.ple_embed_dim);
            s.ple_key = dalloc<float>((uint64_t)NB * D.hh);
            s.ple_value = dalloc<float>((uint64_t)NB * D.H);
            s.ple_gated = dalloc<float>((uint64_t)NB * D.hh);
            s.ple_gvn = dalloc<float>((uint64_t)NB * D.hh);
        }
        scratch_bytes = 4ull * (NB * (3 * D.hh + 4 * D.H + D.conv_dim + 3 * D.v_dim + 4 * D.nh * D.hd) +
                                 (uint64_t)NB * D.nh * max_chunks * (D.hd + 2) + 2ull * NB * D.V);
        host_logits.resize((size_t)NB * D.V);
        host_mtp_logits.resize((size_t)NB * D.V);
        reset_state();
        HIPCHK(hipStreamSynchronize(st));
        HIPCHK(hipGetLastError());
        // PoolMemory::bytes (budget.rs:14-40): with every record resident the
        // pool is the whole store, an explicit size that must leave room for
        // the prefill scratch of budget_prefill_rows rows
        if (mem_limit) {
            const uint64_t rows = std::max<uint32_t>(1, std::min(budget_prefill_rows, max_t));
            ensure(alloc_bytes + prefill_scratch_bytes(rows, false) <= mem_limit,
                   "explicit expert pool exceeds server memory budget after fixed buffers and prefill scratch");
        }
    }

    // Gpu::load_bounded (gpu/load.rs:12-63): the budget is memory_bytes -
    // reserve (memory_bytes 0: no budget, as load's None).
    void set_budget(uint64_t reserve, uint64_t memory_bytes, uint32_t prefill_rows) {
        if (!memory_bytes) return;
        ensure(reserve <= memory_bytes, "cache exceeds memory budget");
        mem_limit = memory_bytes - reserve;
        budget_prefill_rows = prefill_rows;
    }

    // Gpu::load over a packed store (gpu/load.rs:8-19 with Packed::open):
    // the config comes from the store's config.json, every weight from its
    // dense.bin and experts.bin
    void load_store(const std::string& dir, const ChkOptions* opt) {
        std::unique_ptr<Store> S = open_store(dir);
        dense_fd = open((S->dir + "/dense.bin").c_str(), O_RDONLY);
        ensure(dense_fd >= 0, "opening " + S->dir + "/dense.bin");
        experts_fd = open((S->dir + "/experts.bin").c_str(), O_RDONLY);
        ensure(experts_fd >= 0, "opening " + S->dir + "/experts.bin");
        if (S->cfg.ple_layer) {
            ngram_fd = open((S->dir + "/ngram.bin").c_str(), O_RDONLY);
            ensure(ngram_fd >= 0, "opening " + S->dir + "/ngram.bin");
        }
        src = S.get();
        const ChkConfig cfg = S->cfg;
        try {
            load(&cfg, opt);
        } catch (...) {
            src = nullptr;
            throw;
        }
        src = nullptr;
        hipHostFree(staging);
        staging = nullptr;
        close(dense_fd);
        close(experts_fd);
        if (ngram_fd >= 0) close(ngram_fd);
        dense_fd = experts_fd = ngram_fd = -1;
    }

    void reset_state() {
        for (size_t i = 0; i < dn_state.size(); ++i) {
            launch_zero_f32(dn_state[i], (uint64_t)D.nv * D.dv * D.dk, st);
            launch_zero_f32(dn_hist[i], (uint64_t)D.conv_dim * (D.ck - 1), st);
        }
        if (ple_ring) launch_zero_f32(ple_ring, (uint64_t)ple_span * D.hh, st);
        pos = 0;
        batch_pos = 0;
        batch_nb = 0;
        mtp_len = 0;
        tokens.clear();
        folded_valid = false;
        logit_rows = 0;
    }

    // ----------------------------------------------------------- blocks
    void hc_read(const HcDev& w, const float* hyper, float* inj, int nb, const ActivityArgs* activity = nullptr) {
        launch_hc_down(w, hyper, s.hc_d, inj, s.hc_inv, D.H, D.hc, D.eps, nb, st, activity);
        launch_hc_up_mix(w, hyper, s.hc_inv, s.hc_d, s.mixed, D.H, D.hc, nb, st);
    }

    void deltanet(const LayerDev& L, const float* x, int nb, bool snap, float* hyper, const float* inj,
                  float* raw_out) {
        const int di = L.dn_idx;
        SegArgs a{};
        a.nseg = 4;
        uint32_t r0 = 0;
        a.seg[0] = Seg{L.dn.qkv, x, s.dn_conv, D.H, D.conv_dim, r0, EPI_DN_CONV};
        r0 += D.conv_dim;
        a.seg[1] = Seg{L.dn.z, x, s.dn_z, D.H, D.v_dim, r0, EPI_RAW};
        r0 += D.v_dim;
        a.seg[2] = Seg{L.dn.a, x, s.dn_decay, D.H, D.nv, r0, EPI_DN_DECAY};
        r0 += D.nv;
        a.seg[3] = Seg{L.dn.b, x, s.dn_beta, D.H, D.nv, r0, EPI_DN_BETA};
        r0 += D.nv;
        a.total = r0;
        a.conv_w = L.dn.conv;
        a.hist = dn_hist[di];
        a.snap_hist = dn_snap_hist[di];
        a.ck = D.ck;
        a.conv_dim = D.conv_dim;
        a.snap = snap;
        a.a_log = L.dn.a_log;
        a.dt_bias = L.dn.dt_bias;
        uint64_t bytes = q4_bytes(L.dn.qkv) + q4_bytes(L.dn.z) + q4_bytes(L.dn.a) + q4_bytes(L.dn.b) +
                         (uint64_t)D.conv_dim * D.ck * 2 + 2ull * D.conv_dim * (D.ck - 1) * 4 +
                         (uint64_t)nb * (D.H * 4 + (D.conv_dim + D.v_dim + 2 * D.nv) * 4);
        prof_begin(PROF_DN_PROJ);
        launch_qmv(a, nb, st);
        prof_end(PROF_DN_PROJ, bytes);
        DnScanArgs sa{};
        sa.state = dn_state[di];
        sa.snap_state = dn_snap_state[di];
        sa.conv_out = s.dn_conv;
        sa.decay = s.dn_decay;
        sa.beta = s.dn_beta;
        sa.z = s.dn_z;
        sa.norm = L.dn.norm;
        sa.y = s.dn_y;
        sa.y_xq = s.dn_y_xq;
        sa.ssq = s.dn_ssq;
        sa.nk = D.nk;
        sa.nv = D.nv;
        sa.dv = D.dv;
        sa.qk_dim = D.qk_dim;
        sa.conv_dim = D.conv_dim;
        sa.qscale = D.qscale;
        sa.snap = snap;
        launch_dn_scan(sa, nb, st);
        InjArgs ia{};
        ia.m = L.dn.out;
        ia.x = s.dn_y;
        ia.xs = D.v_dim;
        ia.xmode = XM_DN_GATED;
        ia.z = s.dn_z;
        ia.norm = L.dn.norm;
        ia.ssq = s.dn_ssq;
        ia.x_xq = sa.y_xq;
        ia.dv = D.dv;
        ia.nheads = D.nv;
        ia.ssq_blocks = D.dv / 16;
        ia.hyper = hyper;
        ia.inj = inj;
        ia.hc = D.hc;
        ia.raw_out = raw_out;
        launch_qmv_inject(ia, nb, st);
    }

    void attention(const LayerDev& L, const float* x, int nb, const KvDev* kvs, const uint32_t* d_rowpos,
                   float* hyper, const float* inj, float* raw_out) {
        SegArgs a{};
        a.nseg = 4;
        uint32_t r0 = 0;
        a.seg[0] = Seg{L.at.q, x, s.q_raw, D.H, 2 * D.nh * D.hd, r0, EPI_RAW};
        r0 += 2 * D.nh * D.hd;
        a.seg[1] = Seg{L.at.k, x, s.k_raw, D.H, D.kv_row, r0, EPI_RAW};
        r0 += D.kv_row;
        a.seg[2] = Seg{L.at.v, x, s.v_raw, D.H, D.kv_row, r0, EPI_RAW};
        r0 += D.kv_row;
        a.seg[3] = Seg{L.at.idx, x, s.idx_raw, D.H, D.idx_out, r0, EPI_RAW};
        r0 += D.idx_out;
        a.total = r0;
        launch_qmv(a, nb, st);
        AttnArgs aa{};
        aa.q_raw = s.q_raw;
        aa.k_raw = s.k_raw;
        aa.v_raw = s.v_raw;
        aa.idx_raw = s.idx_raw;
        aa.q_norm = L.at.q_norm;
        aa.k_norm = L.at.k_norm;
        aa.q_ready = s.q_ready;
        for (int b = 0; b < nb; ++b) aa.kv[b] = kvs[b];
        aa.pos = d_rowpos;
        aa.part = s.part;
        aa.out = s.attn_out;
        aa.nh = D.nh;
        aa.nkv = D.nkv;
        aa.hd = D.hd;
        aa.rot = D.rot;
        aa.inh = D.inh;
        aa.ihd = D.ihd;
        aa.max_chunks = max_chunks;
        aa.eps = D.eps;
        aa.theta = D.theta;
        aa.scale = D.attn_scale;
        set_qsa(aa, L);
        launch_attn(aa, nb, st);
        InjArgs ia{};
        ia.m = L.at.o;
        ia.x = s.attn_out;
        ia.xs = D.nh * D.hd;
        ia.xmode = XM_PLAIN;
        ia.hyper = hyper;
        ia.inj = inj;
        ia.hc = D.hc;
        ia.raw_out = raw_out;
        launch_qmv_inject(ia, nb, st);
    }

    // the QSA indexer's fields of an attention launch (dense: qsa = 0)
    void set_qsa(AttnArgs& aa, const LayerDev& L) const {
        aa.qsa = D.qsa;
        aa.iq_norm = L.at.idx_q_norm;
        aa.ik_norm = L.at.idx_k_norm;
        aa.iq_ready = s.iq_ready;
        aa.bscore = s.bscore;
        aa.vmask = s.vmask;
        aa.ratio = D.ratio;
        aa.kblk = D.kblk;
        aa.max_blocks = D.max_blocks;
        aa.mask_words = D.mask_words;
    }

    MoeArgs moe_args(const LayerDev& L, uint32_t route_slot, const float* x, int nb, float* hyper, const float* inj,
                     float* raw_out) {
        MoeArgs m{};
        m.X = experts_dev();
        m.X4 = experts_dev(true);
        m.kinds = o.experts == 4 || kinds_q4 == 0 ? nullptr : rec_kind;
        m.record_layer = L.moe.record_layer;
        m.sh_gate = L.moe.sh_gate;
        m.sh_up = L.moe.sh_up;
        m.sh_down = L.moe.sh_down;
        m.x = x;
        m.logits = s.router_logits;
        m.probs = s.router_probs + (uint64_t)route_slot * MAX_NB * D.E;
        m.E = D.E;
        m.norm_topk = D.norm_topk;
        m.ids_out = s.route_ids + (uint64_t)route_slot * MAX_NB * D.topk;
        m.w_out = s.route_w + (uint64_t)route_slot * MAX_NB * D.topk;
        m.ids = m.ids_out;
        m.w = m.w_out;
        m.sg = s.sg;
        m.act = s.act;
        m.act_xq = s.act_xq;
        m.hyper = hyper;
        m.inj = inj;
        m.raw_out = raw_out;
        m.nb = nb;
        m.H = D.H;
        m.I = D.I;
        m.SI = D.SI;
        m.topk = D.topk;
        m.hc = D.hc;
        return m;
    }

    // algorithmic bytes of the gate/up kernel: each routed row-slot's gate
    // and up matrices + the shared expert's, the router logits, the input
    // rows and the activations written
    // (routed and shared gate/up matrices; logits, x and the act rows out,
    // in f32 and as nibble-plane chunks)
    uint64_t gate_up_bytes(const LayerDev& L, int nb) const {
        return (uint64_t)nb * D.topk * 2 * expert_mat_bytes() + 2 * q4_bytes(L.moe.sh_gate) +
               (uint64_t)nb * (D.E * 4 + D.H * 4 + (D.topk * D.I + D.SI) * 4 +
                               (uint64_t)((D.topk * D.I + D.SI) / 32) * sizeof(XqChunk));
    }

    void moe(const LayerDev& L, uint32_t route_slot, const float* x, int nb, float* hyper, const float* inj,
             float* raw_out) {
        RouterArgs r{};
        r.router = L.moe.router;
        r.shared_gate = L.moe.shared_gate;
        r.x = x;
        r.logits = s.router_logits;
        r.sg = s.sg;
        r.E = D.E;
        r.H = D.H;
        launch_router(r, nb, st);
        const MoeArgs m = moe_args(L, route_slot, x, nb, hyper, inj, raw_out);
        if (prof_kind == PROF_MOE && !capturing) {
            // timed by events its own dispatch records (start and end of the kernel)
            std::pair<hipEvent_t, hipEvent_t> ev = prof_pair();
            launch_moe_gate_up(m, st, ev.first, ev.second);
            ++prof_used;
            prof_bytes += gate_up_bytes(L, nb);
            ++prof_launches;
        } else {
            launch_moe_gate_up(m, st);
        }
        launch_moe_down(m, st);
    }

    // Time one kernel class alone: a captured graph of `reps` rounds of its
    // launches over every decoder layer (the arguments the decode step
    // passes at batch 1, on the current router logits and mixer output),
    // replayed on the engine stream between two HIP events.  The kernels
    // only write scratch (activations, routing of the profiled layers, LM
    // head logits), never the sequence state.
    double profile_graph(int kind, uint32_t reps, uint64_t& bytes, uint64_t& launches) {
        ensure(kind == PROF_MOE || kind == PROF_LM_HEAD, "graph timing covers the MoE gate/up and LM head kernels");
        ensure(reps >= 1 && reps <= 64, "reps must be 1..=64");
        HIPCHK(hipStreamSynchronize(st));
        bytes = 0;
        launches = 0;
        hipGraph_t g;
        HIPCHK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        for (uint32_t r = 0; r < reps; ++r) {
            if (kind == PROF_MOE) {
                for (uint32_t l = 0; l < c.num_hidden_layers; ++l) {
                    const LayerDev& L = layers[l];
                    launch_moe_gate_up(moe_args(L, l, s.mixed, 1, nullptr, nullptr, nullptr), st);
                    bytes += gate_up_bytes(L, 1);
                    ++launches;
                }
            } else {
                launch_lm_head(lm_head, s.mixed, s.logits, s.pv, s.pi, lm_parts, s.d_out, 1, st);
                bytes += q4_bytes(lm_head) + (uint64_t)(D.H + D.V) * 4;
                ++launches;
            }
        }
        HIPCHK(hipStreamEndCapture(st, &g));
        hipGraphExec_t ge;
        HIPCHK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
        hipEvent_t a, b;
        HIPCHK(hipEventCreate(&a));
        HIPCHK(hipEventCreate(&b));
        HIPCHK(hipGraphLaunch(ge, st));  // warm
        HIPCHK(hipEventRecord(a, st));
        HIPCHK(hipGraphLaunch(ge, st));
        HIPCHK(hipEventRecord(b, st));
        HIPCHK(hipEventSynchronize(b));
        float ms = 0.0f;
        HIPCHK(hipEventElapsedTime(&ms, a, b));
        HIPCHK(hipEventDestroy(a));
        HIPCHK(hipEventDestroy(b));
        HIPCHK(hipGraphExecDestroy(ge));
        HIPCHK(hipGraphDestroy(g));
        return ms;
    }

    // ------------------------------------------------------------ PLE
    // the table rows of tokens[t0 .. t0 + n) into out[i * stride ..]
    void ple_ids(size_t t0, uint32_t n, uint32_t* out, uint32_t stride) const {
        for (uint32_t i = 0; i < n; ++i) ngram_rows_at(t0 + i, out + (size_t)i * stride);
    }
    // CpuModel::ngram_ids_from (cpu.rs:848-887) for the token at index t of
    // `tokens`: bigram heads, then trigram heads, each hashing the token
    // and the ones before it (EOS when the window [t - k, t) holds an EOS
    // or reaches before the start) with wrapping i64 products, XOR, and the
    // Euclidean remainder by the head's size; the host computes these for
    // the gather kernel, as the reference's GPU path does (gpu/ple.rs:7-15).
    void ngram_rows_at(size_t t, uint32_t* out) const {
        const uint32_t eos = c.eos_token_id;
        int64_t shifted[16];
        for (uint32_t k = 0; k < c.ngram_size; ++k) {
            if (k == 0) {
                shifted[0] = (int64_t)tokens[t];
                continue;
            }
            bool before = t < k;
            for (size_t j = before ? t : t - k; j < t && !before; ++j) before = tokens[j] == eos;
            shifted[k] = before ? (int64_t)eos : (int64_t)tokens[t - k];
        }
        uint32_t n = 0;
        for (uint32_t ng = 2; ng <= c.ngram_size; ++ng) {
            uint64_t mixed = (uint64_t)shifted[0] * (uint64_t)ngram_mult[0];
            for (uint32_t p = 1; p < ng; ++p) mixed ^= (uint64_t)shifted[p] * (uint64_t)ngram_mult[p];
            const int64_t mx = (int64_t)mixed;
            for (uint32_t h = (ng - 2) * c.heads_per_ngram; h < (ng - 1) * c.heads_per_ngram; ++h) {
                const int64_t size = (int64_t)ngram_sizes[h];
                int64_t r = mx % size;
                if (r < 0) r += size;
                out[n++] = (uint32_t)((uint64_t)r + ngram_offs[h]);
            }
        }
    }

    // The PLE block over `rows` rows whose n-gram table rows are `ids`
    // ([rows][heads], device-visible), hyper rows `hyper` at positions
    // `rowpos`; `backup`: where the ring rows go that a rollback restores.
    void ple_rows(const PleDev& P, const uint32_t* ids, uint32_t ids_stride, float* hyper, const uint32_t* rowpos,
                  uint32_t rows, float* e, float* key, float* value, float* gated, float* gvn, float* backup,
                  bool gemm) {
        const uint32_t E = c.ple_embed_dim;
        launch_ple_gather(ids, ids_stride, ngram_heads, ngram, ngram_row_bytes, ngram_dim, ngram_group, e, rows, st);
        if (gemm) {
            launch_pf_xprep(e, E, rows, E, pf.hi, pf.lo, pf.xs, st);
            launch_pf_gemm(P.key, pf.hi, pf.lo, pf.xs, key, rows, D.hh, st);
            launch_pf_gemm(P.value, pf.hi, pf.lo, pf.xs, value, rows, D.H, st);
        } else {
            SegArgs a{};
            a.nseg = 2;
            a.seg[0] = Seg{P.key, e, key, E, D.hh, 0, EPI_RAW};
            a.seg[1] = Seg{P.value, e, value, E, D.H, D.hh, EPI_RAW};
            a.total = D.hh + D.H;
            launch_qmv(a, (int)rows, st);
        }
        launch_ple_gate(key, hyper, D.hh, value, P.norm_key, P.norm_query, P.norm_conv, gated, gvn, D.H, D.hc, D.eps,
                        rows, st);
        launch_ple_conv(gated, gvn, P.conv, ple_ring, hyper, D.hh, rowpos, D.hh, c.ple_conv_kernel_size,
                        c.ngram_size, ple_span, rows, st);
        launch_ple_ring(gvn, ple_ring, backup, rowpos, D.hh, ple_span, rows, st);
    }

    // ---------------------------------------------------------- step
    void run_rows(int nb, bool snap) {
        launch_embed(s.d_in, s.tokens, s.rowpos, embed, s.hyper, D.H, D.hc, nb, st);
        KvDev kvs[MAX_NB];
        for (uint32_t l = 0; l < c.num_hidden_layers; ++l) {
            const LayerDev& L = layers[l];
            if (L.has_ple)
                ple_rows(L.ple, &s.d_in->ngram[0][0], MAX_NGRAM_IDS, s.hyper, s.rowpos, (uint32_t)nb, s.ple_e, s.ple_key,
                         s.ple_value, s.ple_gated, s.ple_gvn, snap ? ple_backup : nullptr, false);
            hc_read(L.attn_hc, s.hyper, s.inj_a, nb);
            if (L.linear) {
                deltanet(L, s.mixed, nb, snap, s.hyper, s.inj_a, nullptr);
            } else {
                for (int b = 0; b < nb; ++b) kvs[b] = kv[L.at_idx];
                attention(L, s.mixed, nb, kvs, s.rowpos, s.hyper, s.inj_a, nullptr);
            }
            hc_read(L.mlp_hc, s.hyper, s.inj_m, nb);
            moe(L, l, s.mixed, nb, s.hyper, s.inj_m, nullptr);
            if (tracing && s.trace)
                HIPCHK(hipMemcpyAsync(s.trace + (uint64_t)l * MAX_NB * D.hh, s.hyper, (uint64_t)nb * D.hh * 4,
                                      hipMemcpyDeviceToDevice, st));
        }
        // the step's expert activity rides on the final read's launch
        const ActivityArgs aa{s.route_ids, (uint64_t)MAX_NB * D.topk, c.num_hidden_layers, (uint32_t)nb, D.topk, D.E, 0,
                              reinterpret_cast<unsigned long long*>(act)};
        hc_read(final_mixer, s.hyper, nullptr, nb, &aa);
        prof_begin(PROF_LM_HEAD);
        launch_lm_head(lm_head, s.mixed, s.logits, s.pv, s.pi, lm_parts, s.d_out, nb, st);
        prof_end(PROF_LM_HEAD, q4_bytes(lm_head) + (uint64_t)nb * (D.H + D.V) * 4);
    }

    void step_rows(const uint32_t* toks, uint32_t n, bool snap, bool fold, uint32_t* out) {
        ensure(!fold || has_mtp, "folding the MTP pass needs the MTP head");
        ensure(n >= 1 && n <= trunk_rows,
               "rows per step must be 1..=" + std::to_string(trunk_rows) + " (set --drafts to raise it)");
        ensure(pos + n <= max_t, "context capacity exceeded");
        ensure(!snap || n - 1 <= (uint32_t)MAX_SNAP, "at most 3 draft rows per verify step");
        for (uint32_t i = 0; i < n; ++i) ensure(toks[i] < D.V, "token id out of range");
        folded_valid = false;
        tokens.resize(pos);
        tokens.insert(tokens.end(), toks, toks + n);
        batch_pos = pos;
        batch_nb = n;
        batch_snap = snap;
        logit_rows = n;
        for (uint32_t i = 0; i < n; ++i) s.h_in->tokens[i] = toks[i];
        s.h_in->pos = pos;
        if (ple_l >= 0) ple_ids(pos, n, &s.h_in->ngram[0][0], MAX_NGRAM_IDS);
        std::atomic_thread_fence(std::memory_order_seq_cst);
        const StepGraph* replayed = nullptr;
        if (use_graphs && !tracing && prof_kind == PROF_NONE) {
            const int key = ((int)n * 2 + (snap ? 1 : 0)) * 4 + prof_kind;
            auto it = graphs.find(key);
            if (it == graphs.end()) {
                hipGraph_t g;
                StepGraph sg{};
                sg.ev0 = graph_events.size();
                HIPCHK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
                capturing = true;
                try {
                    run_rows((int)n, snap);
                } catch (...) {
                    capturing = false;
                    hipGraph_t dead;
                    (void)hipStreamEndCapture(st, &dead);
                    throw;
                }
                capturing = false;
                HIPCHK(hipStreamEndCapture(st, &g));
                sg.ev1 = graph_events.size();
                HIPCHK(hipGraphInstantiate(&sg.exec, g, nullptr, nullptr, 0));
                HIPCHK(hipGraphDestroy(g));
                it = graphs.emplace(key, sg).first;
            }
            HIPCHK(hipGraphLaunch(it->second.exec, st));
            replayed = &it->second;
        } else {
            run_rows((int)n, snap);
        }
        if (fold) {
            // pair row b's residual with the trunk's own prediction for it
            HIPCHK(hipMemcpyAsync(s.out_tok, s.d_out, n * 4, hipMemcpyDeviceToDevice, st));
            mtp_pass_trunk((int)n, batch_pos, s.out_tok);
        }
        if (fold) {
            folded.assign(n, 0);
            HIPCHK(hipMemcpyAsync(folded.data(), s.mtp_out, n * 4, hipMemcpyDeviceToHost, st));
        }
        HIPCHK(hipStreamSynchronize(st));
        HIPCHK(hipGetLastError());
        for (uint32_t i = 0; i < n; ++i) out[i] = s.h_out[i];
        prof_collect();
        if (replayed && replayed->ev1 > replayed->ev0) prof_collect_graph(*replayed);
        if (fold) {
            folded_valid = true;
            last_mtp_rows = n;
        }
        logits_fresh = false;
        mtp_logits_fresh = false;
    }

    bool logits_fresh = false, mtp_logits_fresh = false;

    void commit(uint32_t n) {
        ensure(n >= 1 && n <= batch_nb, "commit " + std::to_string(n) + " of " + std::to_string(batch_nb) + " rows");
        if (n < batch_nb) {
            ensure(batch_snap, "rollback needs a snapshotting step");
            uint32_t plane = n - 1;
            uint64_t sn = (uint64_t)D.nv * D.dv * D.dk, hn = (uint64_t)D.conv_dim * (D.ck - 1);
            for (size_t i = 0; i < dn_state.size(); ++i) {
                launch_copy_f32(dn_state[i], dn_snap_state[i] + plane * sn, sn, st);
                launch_copy_f32(dn_hist[i], dn_snap_hist[i] + plane * hn, hn, st);
            }
            // the ring slots the rejected rows overwrote get their old rows
            // back: the oldest tap (back = span) of a later position reads
            // exactly the slot its own row writes, so positional overwrite
            // alone would leave a rejected row's gvn there
            for (uint32_t j = n; ple_ring && j < batch_nb; ++j)
                launch_copy_f32(ple_ring + (uint64_t)((batch_pos + j) % ple_span) * D.hh,
                                ple_backup + (uint64_t)j * D.hh, D.hh, st);
            HIPCHK(hipStreamSynchronize(st));
        }
        pos = batch_pos + n;
        tokens.resize(pos);
    }

    // ------------------------------------------------ prefix checkpoints
    // Gpu::prefix_regions (gpu/state.rs:85-124): the device ranges that hold
    // a sequence's state at trunk length `n` and MTP length `mtp_n`: every
    // DeltaNet layer's recurrent state and conv history (whole), every
    // attention layer's q8 K and V rows and their fp16 scale rows, its
    // index keys and (past the QSA budget) its pooled block keys up to the
    // length, then the MTP layer's at its own length.
    struct Region {
        void* ptr;
        uint64_t bytes;
    };
    std::vector<Region> prefix_regions(uint32_t n, uint32_t mtp_n) const {
        std::vector<Region> r;
        const uint64_t sn = (uint64_t)D.nv * D.dv * D.dk * 4, hn = (uint64_t)D.conv_dim * (D.ck - 1) * 4;
        auto attn = [&](const KvDev& k, uint32_t len) {
            r.push_back({k.k, (uint64_t)len * D.kv_row});
            r.push_back({k.ks, (uint64_t)len * (D.kv_row / 32) * 2});
            r.push_back({k.v, (uint64_t)len * D.kv_row});
            r.push_back({k.vs, (uint64_t)len * (D.kv_row / 32) * 2});
            r.push_back({k.index_k, (uint64_t)len * D.ihd * 4});
            if (k.block_k) r.push_back({k.block_k, (uint64_t)((len + D.ratio - 1) / D.ratio) * D.ihd * 4});
        };
        for (uint32_t l = 0; l < c.num_hidden_layers; ++l) {
            if (layers[l].linear) {
                r.push_back({dn_state[layers[l].dn_idx], sn});
                r.push_back({dn_hist[layers[l].dn_idx], hn});
            } else {
                attn(kv[layers[l].at_idx], n);
            }
        }
        if (has_mtp) attn(mtp_kv, mtp_n);
        if (ple_ring) r.push_back({ple_ring, (uint64_t)ple_span * D.hh * 4});
        return r;
    }
    uint64_t state_bytes_at(uint32_t n, uint32_t mtp_n) const;
    void save_into(ChkPrefixState*& cp);
    void restore_prefix(const ChkPrefixState& cp);
    void clear_profile() {
        prof_collect();
        prof_kind = PROF_NONE;
        prof_ms = 0.0;
        prof_bytes = 0;
        prof_launches = 0;
    }

    // ------------------------------------------------------------ MTP
    // mtp_forward prelude (cpu.rs:344-369): hyper_g = fc_e(rms_norm_shift(e))
    // + fc_h(rms_norm_shift(h_g)); then one attention + MoE block with the
    // MTP layer's own KV, the MTP mixer and the shared LM head.
    void mtp_rows(int rows, const float* src_hyper, const uint32_t* d_tokens, uint32_t base_pos);
    void mtp_pass_trunk(int rows, uint32_t base_pos, const uint32_t* d_next);
    void prefill(const uint32_t* toks, uint32_t n, uint32_t next_after, bool all_logits, uint32_t* next,
                 uint32_t* draft);
    void prefill_rows(const uint32_t* toks, uint32_t n, uint32_t next_after, bool all_logits, uint32_t* next,
                      uint32_t* draft);
    void pf_keep_logits(uint32_t rows);
    uint64_t prefill_scratch_bytes(uint64_t rows, bool all_logits) const;
    uint32_t prefill_rows_fit(bool all_logits) const;
    // ------------------------------------------------- GEMM prefill
    bool pf_supported() const;
    // flash attention plans: workgroups per kv head, partial floats (at most
    // two pieces per workgroup of a kv head)
    uint64_t fa_wmax(uint64_t C) const {
        return std::min<uint64_t>((C + 15) / 16, std::max<uint32_t>(1, ncu / D.nkv));
    }
    uint64_t fa_part_floats(uint64_t C) const { return (uint64_t)D.nkv * 2 * fa_wmax(C) * 16 * (D.nh / D.nkv) * (2 + D.hd); }
    uint32_t pf_dense_rows(uint32_t T, uint32_t pos0) const;
    PfFlashLaunch pf_flash_launch(uint32_t T, uint32_t pos0);
    uint32_t pf_qsa_rows() const;
    void pf_alloc();
    void pf_hc_read(const HcDev& w, float* inj, uint32_t T, bool for_moe);
    void pf_out_proj(const Q4Mat& m, uint32_t K, uint32_t T);
    void pf_deltanet(const LayerDev& L, uint32_t T);
    void pf_attention(const LayerDev& L, uint32_t T, uint32_t pos0, const KvDev* kvo = nullptr);
    void pf_mtp(const uint32_t* toks, uint32_t c0, uint32_t T, uint32_t pos0, bool last, uint32_t next_after);
    void pf_moe(const LayerDev& L, uint32_t T);
    void pf_moe_flush();
    void prefill_gemm(const uint32_t* toks, uint32_t n, uint32_t next_after, bool all_logits, uint32_t* next);
    void mtp_draft(const uint32_t* next, uint32_t n, uint32_t chain, uint32_t* drafts, uint32_t* nd);
};

namespace chk {
void launch_mtp_prelude(const uint32_t* tokens, const Q4Mat& emb, const uint16_t* enorm, const uint16_t* hnorm,
                        const float* src_hyper, float* e_n, float* h_n, uint32_t H, uint32_t hc, float eps, int rows,
                        hipStream_t st);
void launch_mtp_fold(const float* fe, const float* fh, float* hyper, uint32_t H, uint32_t hc, int rows,
                     hipStream_t st);
}  // namespace chk

void ChkEngine::mtp_rows(int rows, const float* src_hyper, const uint32_t* d_tokens, uint32_t base_pos) {
    // e_n [rows][H] into mtp_fe's input slot (reuse mtp_hn layout: first
    // rows*H floats hold rms_norm_shift(e), then rows*hc*H the streams)
    float* en = s.mtp_hn;
    float* hn = s.mtp_hn + (uint64_t)MAX_NB * D.H;
    launch_mtp_prelude(d_tokens, embed, mtp_enorm, mtp_hnorm, src_hyper, en, hn, D.H, D.hc, D.eps, rows, st);
    // fc_e over rows, fc_h over rows * hc stream rows (in batches of 4)
    SegArgs a{};
    a.nseg = 1;
    a.seg[0] = Seg{fc_e, en, s.mtp_fe, D.H, D.H, 0, EPI_RAW};
    a.total = D.H;
    launch_qmv(a, rows, st);
    uint32_t nrows = rows * D.hc;
    for (uint32_t r0 = 0; r0 < nrows; r0 += MAX_NB) {
        int nbb = (int)std::min<uint32_t>(MAX_NB, nrows - r0);
        SegArgs f{};
        f.nseg = 1;
        f.seg[0] = Seg{fc_h, hn + (uint64_t)r0 * D.H, s.mtp_fh + (uint64_t)r0 * D.H, D.H, D.H, 0, EPI_RAW};
        f.total = D.H;
        launch_qmv(f, nbb, st);
    }
    launch_mtp_fold(s.mtp_fe, s.mtp_fh, s.mtp_hyper, D.H, D.hc, rows, st);
    const LayerDev& L = mtp_layer;
    KvDev kvs[MAX_NB];
    uint32_t rows_pos[MAX_NB];
    for (int b = 0; b < rows; ++b) {
        kvs[b] = mtp_kv;
        rows_pos[b] = base_pos + b;
    }
    HIPCHK(hipMemcpyAsync(s.rowpos_aux, rows_pos, rows * 4, hipMemcpyHostToDevice, st));
    hc_read(L.attn_hc, s.mtp_hyper, s.inj_a, rows);
    attention(L, s.mixed, rows, kvs, s.rowpos_aux, s.mtp_hyper, s.inj_a, nullptr);
    hc_read(L.mlp_hc, s.mtp_hyper, s.inj_m, rows);
    moe(L, c.num_hidden_layers, s.mixed, rows, s.mtp_hyper, s.inj_m, nullptr);
    const ActivityArgs aa{s.route_ids + (uint64_t)c.num_hidden_layers * MAX_NB * D.topk, 0, 1, (uint32_t)rows, D.topk,
                          D.E, c.num_hidden_layers, reinterpret_cast<unsigned long long*>(act)};
    hc_read(mtp_mixer, s.mtp_hyper, nullptr, rows, &aa);
    launch_lm_head(lm_head, s.mixed, s.mtp_logits, s.pv, s.pi, lm_parts, s.mtp_out, rows, st);
}

void ChkEngine::mtp_pass_trunk(int rows, uint32_t base_pos, const uint32_t* d_next) {
    mtp_rows(rows, s.hyper, d_next, base_pos);
}

// Gpu::mtp_draft (gpu/mtp.rs:11-78)
void ChkEngine::mtp_draft(const uint32_t* next, uint32_t n, uint32_t chain, uint32_t* drafts, uint32_t* nd) {
    ensure(has_mtp, "no MTP head");
    ensure(n >= 1 && n <= batch_nb, "MTP rows must match the committed rows");
    ensure(mtp_len == batch_pos,
           "MTP cache out of step: " + std::to_string(mtp_len) + " vs " + std::to_string(batch_pos));
    std::vector<uint32_t> out;
    uint32_t c0 = 0;
    bool first = true;
    uint32_t token = 0;
    // the MTP hyper source: the trunk rows (first pass) or the head's own
    // residual row (chained passes)
    if (folded_valid) {
        // the folded pass already ran over the trunk rows with the trunk's
        // predictions, which equal `next` for every accepted row
        folded_valid = false;
        mtp_len = batch_pos + n;
        first = false;
        token = folded[n - 1];
        if (chain > 0) out.push_back(token);
        c0 = 1;
        // the head residual of row n-1 becomes the chain source
        if (n - 1 != 0)
            HIPCHK(hipMemcpyAsync(s.mtp_hyper, s.mtp_hyper + (uint64_t)(n - 1) * D.hh, D.hh * 4,
                                  hipMemcpyDeviceToDevice, st));
    }
    for (uint32_t ci = c0; ci < std::max<uint32_t>(chain, 1); ++ci) {
        uint32_t rows = first ? n : 1;
        uint32_t base = first ? batch_pos : batch_pos + n - 1 + ci;
        ensure(base + rows <= max_t, "context capacity exceeded");
        if (first) {
            HIPCHK(hipMemcpyAsync(s.tokens, next, n * 4, hipMemcpyHostToDevice, st));
            mtp_rows((int)rows, s.hyper, s.tokens, base);
        } else {
            HIPCHK(hipMemcpyAsync(s.tokens, &token, 4, hipMemcpyHostToDevice, st));
            // chained: hidden input is the head's own residual row
            HIPCHK(hipMemcpyAsync(s.mtp_src, s.mtp_hyper, D.hh * 4, hipMemcpyDeviceToDevice, st));
            mtp_rows(1, s.mtp_src, s.tokens, base);
        }
        uint32_t res[MAX_NB];
        HIPCHK(hipMemcpyAsync(res, s.mtp_out, rows * 4, hipMemcpyDeviceToHost, st));
        HIPCHK(hipStreamSynchronize(st));
        uint32_t d = res[rows - 1];
        if (first) {
            mtp_len = batch_pos + n;
            if (rows - 1 != 0)
                HIPCHK(hipMemcpyAsync(s.mtp_hyper, s.mtp_hyper + (uint64_t)(rows - 1) * D.hh, D.hh * 4,
                                      hipMemcpyDeviceToDevice, st));
        }
        if (ci < chain) out.push_back(d);
        token = d;
        first = false;
        last_mtp_rows = rows;
    }
    HIPCHK(hipStreamSynchronize(st));
    for (size_t i = 0; i < out.size(); ++i) drafts[i] = out[i];
    *nd = (uint32_t)out.size();
    mtp_logits_fresh = false;
}

// Gpu::prefill_chunk (gpu/prefill.rs:196-464): the GEMM path wherever this
// engine implements it (every expert precision and the MTP head; not past
// the QSA budget), else the row path.  Both leave the same state behind
// (prefill.rs:13-15).  `next_after` (CHK_NO_TOKEN: none) is the token that
// follows the chunk, paired with its last row by the MTP head; without it
// the trunk's greedy token is (prefill.rs:354-355).  With `all_logits`
// every row's logits are kept for pf_logits_row.
void ChkEngine::prefill(const uint32_t* toks, uint32_t n, uint32_t next_after, bool all_logits, uint32_t* next,
                        uint32_t* draft) {
    ensure(n >= 1, "empty chunk");
    ensure(pos + n <= max_t, "context capacity exceeded");
    for (uint32_t i = 0; i < n; ++i) ensure(toks[i] < D.V, "token id out of range");
    ensure(next_after == CHK_NO_TOKEN || next_after < D.V, "token id out of range");
    pf_all_rows = 0;
    if (all_logits) pf_keep_logits(n);
    if (pf_supported()) {
        prefill_gemm(toks, n, next_after, all_logits, next);
        *draft = 0xffffffffu;
        if (has_mtp) HIPCHK(hipMemcpy(draft, s.mtp_out, 4, hipMemcpyDeviceToHost));
    } else {
        prefill_rows(toks, n, next_after, all_logits, next, draft);
    }
    if (all_logits) pf_all_rows = n;
    // like the reference, the chunk leaves no step in flight: its final
    // row's logits are logits_row(0)
    batch_pos = pos;
    batch_nb = 0;
    batch_snap = false;
    logit_rows = 1;
    logits_fresh = false;
    mtp_logits_fresh = false;
}

// The all-logits buffer: rows x vocab f32, grown to the largest chunk seen.
void ChkEngine::pf_keep_logits(uint32_t rows) {
    if (pf_all_cap >= rows) return;
    pf_all = pfalloc<float>((uint64_t)rows * D.V);
    pf_all_cap = rows;
}

// Prompt processing through the row path: rows of up to MAX_NB tokens,
// committed as they go, MTP cache kept in step (gpu/prefill.rs semantics:
// side effects identical to row stepping, prefill.rs:13-15).
void ChkEngine::prefill_rows(const uint32_t* toks, uint32_t n, uint32_t next_after, bool all_logits, uint32_t* next,
                             uint32_t* draft) {
    uint32_t saved_rows = trunk_rows;
    trunk_rows = MAX_NB;
    uint32_t last = 0;
    try {
        for (uint32_t i = 0; i < n; i += MAX_NB) {
            uint32_t m = std::min<uint32_t>(MAX_NB, n - i);
            uint32_t out[MAX_NB];
            step_rows(toks + i, m, false, false, out);
            if (all_logits)
                HIPCHK(hipMemcpyAsync(pf_all + (uint64_t)i * D.V, s.logits, (uint64_t)m * D.V * 4,
                                      hipMemcpyDeviceToDevice, st));
            commit(m);
            if (has_mtp) {
                // MTP cache rows for these positions pair each row with the
                // token after it: the next prompt token, `next_after` after
                // the chunk's last row, else the trunk's prediction
                uint32_t nx[MAX_NB];
                for (uint32_t r = 0; r < m; ++r) {
                    const uint32_t p = i + r + 1;
                    nx[r] = p < n ? toks[p] : (next_after != CHK_NO_TOKEN ? next_after : out[r]);
                }
                uint32_t d[4], nd = 0;
                mtp_draft(nx, m, i + m >= n ? 1 : 0, d, &nd);
                if (i + m >= n) *draft = nd ? d[0] : 0xffffffffu;
            }
            last = out[m - 1];
        }
    } catch (...) {
        trunk_rows = saved_rows;
        throw;
    }
    trunk_rows = saved_rows;
    // the final row's logits as logits_row(0)
    if (batch_nb > 1)
        HIPCHK(hipMemcpyAsync(s.logits, s.logits + (uint64_t)(batch_nb - 1) * D.V, (uint64_t)D.V * 4,
                              hipMemcpyDeviceToDevice, st));
    HIPCHK(hipStreamSynchronize(st));
    *next = last;
    if (!has_mtp) *draft = 0xffffffffu;
}

// K chunks of the prefill's DeltaNet a / b projections: the most (4 or 2)
// that keep whole 8-group scale blocks per chunk, else 1.
static uint32_t pf_ab_split(uint32_t H) {
    for (uint32_t ks : {4u, 2u})
        if ((H / 64) % ks == 0 && (H / 64 / ks) % 8 == 0) return ks;
    return 1;
}

// Scratch a prefill of `rows` rows per GEMM chunk allocates (pf_alloc's
// buffers, plus the all-logits rows).
uint64_t ChkEngine::prefill_scratch_bytes(uint64_t C, bool all_logits) const {
    const uint64_t slots = D.topk + 1, f = 4;
    uint64_t b = C * 8 + C * D.hh * f;
    if (has_mtp) b += C * 4 + C * (2ull * D.H + 3ull * D.hh) * f;
    const uint64_t plane = std::max({C * D.hh, C * D.v_dim, C * D.nh * D.hd, C * slots * D.I, C * D.SI, C * D.H});
    b += plane * 2 * 2 + plane / 64 * f + 3 * C * D.H * 2;
    b += C * (3ull * D.hc + D.lowrank + D.H + (uint64_t)D.hc * (D.lowrank + D.hc)) * f;
    b += C * D.lowrank / 8 * 32 + (C * D.lowrank / 64 + 1) * f;
    b += C * slots * D.I / 8 * 32 + (C * slots * D.I / 64 + 1) * f;
    const uint64_t dn = C * (2ull * D.conv_dim + 2ull * D.v_dim + (2ull * pf_ab_split(D.H) + 2) * D.nv);
    const uint64_t at = C * (2ull * D.nh * D.hd + 2ull * D.kv_row + D.idx_out + 2ull * D.nh * D.hd);
    b += std::max(dn, at) * f;
    b += C * (PF_ROUTER_CHUNKS * D.E + 1 + 2ull * D.topk) * f + (D.E + 1ull) * C * 4 +
         (PF_GCNT_STRIDE + 1ull) * (D.E + 1) * 4;
    b += (uint64_t)(pf_tile_bound((uint32_t)C, D.topk, D.E, 48) + pf_tile_bound((uint32_t)C, D.topk, D.E, 64)) * 12 +
         C * slots * (D.I + D.H) * f + C * slots * 4 + (D.E + 1) * 4;
    if (D.SI != D.I) b += C * D.SI * f;
    if (dc_supported(D.nk, D.nv, D.dk, D.dv)) b += dc_work_floats((uint32_t)C, D.nv, D.dv) * f;
    if (all_logits) b += C * D.V * f;
    {
        const uint64_t rmax = (C + 15) / 16, wmax = fa_wmax(C);
        b += (rmax * FA_MAXSEG + wmax) * 16 + fa_part_floats(C) * f;
    }
    if (ple_l >= 0) b += C * (ngram_heads + c.ple_embed_dim + 3ull * D.hh + D.H) * 4;
    if (D.qsa)
        b += (C * (D.inh * D.ihd + D.mask_words) +
              (uint64_t)pf_qsa_rows() * (D.max_blocks + D.mask_words + (uint64_t)D.nh * max_chunks * (D.hd + 2))) * 4;
    return b;
}

// Gpu::prefill_rows_fit (prefill/allocation.rs:150-169): the largest chunk
// (at most the context and 4096 rows, prefill.rs:116) whose scratch fits
// the device memory that is free now (this engine's own prefill scratch
// counts as free: it is reused or released before a replacement).
uint32_t ChkEngine::prefill_rows_fit(bool all_logits) const {
    size_t free_b = 0, total_b = 0;
    HIPCHK(hipMemGetInfo(&free_b, &total_b));
    uint64_t avail = (uint64_t)free_b + pf_alloc_bytes;
    // under a server budget, what the budget leaves (allocation.rs:154)
    if (mem_limit) avail = std::min<uint64_t>(avail, mem_limit - std::min(mem_limit, alloc_bytes - pf_alloc_bytes));
    uint32_t lo = 0, hi = std::min<uint32_t>(max_t, 4096);
    while (lo < hi) {
        const uint32_t mid = lo + (hi - lo + 1) / 2;
        if (prefill_scratch_bytes(mid, all_logits) <= avail) lo = mid;
        else hi = mid - 1;
    }
    ensure(lo > 0, "insufficient memory for prefill scratch; reduce expert pool or context capacity");
    return lo;
}

// ------------------------------------------------------- GEMM prefill
constexpr uint32_t PF_MAX_ROWS = 4096;                  // rows per chunk (gpu/prefill.rs:116)

bool ChkEngine::pf_supported() const {
    return (o.experts == 4 || o.experts == 3 || o.experts == 2) && D.lowrank % 64 == 0 && D.H % 64 == 0 && D.H <= 4096 && D.hc <= 4 &&
           (D.dv == 64 || D.dv == 128 || D.dv == 256) && D.I % 64 == 0 && (D.nh * D.hd) % 64 == 0 &&
           D.v_dim % 64 == 0 && D.E + 1 <= 513 && D.nh % D.nkv == 0 &&
           (D.nh / D.nkv == 1 || D.nh / D.nkv == 2 || D.nh / D.nkv == 4 || D.nh / D.nkv == 8) &&
           (D.hd == 128 || D.hd == 256);
}

// Rows whose QSA selection and attention partials one prefill launch holds:
// the partials of a row span every chunk of the context, so the group is
// sized to about 256 MB of them (4..64 rows, a multiple of 4).
uint32_t ChkEngine::pf_qsa_rows() const {
    const uint64_t per_row = ((uint64_t)D.nh * max_chunks * (D.hd + 2) + D.max_blocks + D.mask_words) * 4;
    const uint64_t fit = (256ull << 20) / std::max<uint64_t>(per_row, 1);
    return (uint32_t)std::max<uint64_t>(4, std::min<uint64_t>(64, fit) / 4 * 4);
}

void ChkEngine::pf_alloc() {
    if (pf.cap) return;
    // chunks of up to 4096 rows (prefill.rs:116); under a server budget, of
    // the rows the load kept room for (the prompt then runs in more chunks)
    uint64_t C = std::min<uint32_t>(max_t, PF_MAX_ROWS);
    if (mem_limit) C = std::min<uint64_t>(C, std::max<uint32_t>(1, budget_prefill_rows));
    const uint64_t slots = D.topk + 1;
    pf.tokens = pfalloc<uint32_t>(C);
    pf.pos = pfalloc<uint32_t>(C);
    pf.hyper = pfalloc<float>(C * D.hh);
    if (has_mtp) {
        pf.mtp_tok = pfalloc<uint32_t>(C);
        pf.mtp_en = pfalloc<float>(C * D.H);
        pf.mtp_hn = pfalloc<float>(C * D.hh);
        pf.mtp_fe = pfalloc<float>(C * D.H);
        pf.mtp_fh = pfalloc<float>(C * D.hh);
        pf.mtp_hyper = pfalloc<float>(C * D.hh);
    }
    const uint64_t plane = std::max({C * D.hh, C * D.v_dim, C * D.nh * D.hd, C * slots * D.I, C * D.SI, C * D.H});
    pf.hi = pfalloc<uint4>(plane / 8);
    pf.lo = pfalloc<uint4>(plane / 8);
    pf.xs = pfalloc<float>(plane / 64);
    pf.bhi = pfalloc<uint4>(C * D.H / 8);
    pf.bmid = pfalloc<uint4>(C * D.H / 8);
    pf.blo = pfalloc<uint4>(C * D.H / 8);
    pf.inv = pfalloc<float>(C * D.hc);
    pf.d = pfalloc<float>(C * D.lowrank);
    pf.dhi = pfalloc<uint4>(C * D.lowrank / 8);
    pf.dlo = pfalloc<uint4>(C * D.lowrank / 8);
    pf.dxs = pfalloc<float>(C * D.lowrank / 64 + 1);
    pf.ahi = pfalloc<uint4>(C * slots * D.I / 8);
    pf.alo = pfalloc<uint4>(C * slots * D.I / 8);
    pf.axs = pfalloc<float>(C * slots * D.I / 64 + 1);
    pf.hc_part = pfalloc<float>(C * D.hc * (D.lowrank + D.hc));
    pf.inj_a = pfalloc<float>(C * D.hc);
    pf.inj_m = pfalloc<float>(C * D.hc);
    pf.mixed = pfalloc<float>(C * D.H);
    pf.fa_seg = pfalloc<uint4>((C + 15) / 16 * FA_MAXSEG);
    pf.fa_merge = pfalloc<uint4>(fa_wmax(C));
    pf.fa_part = pfalloc<float>(fa_part_floats(C));
    pf.fa_key = ~0ull;
    // DeltaNet / attention arena
    const uint64_t dn = C * (2ull * D.conv_dim + 2ull * D.v_dim + (2ull * pf_ab_split(D.H) + 2) * D.nv);
    const uint64_t at = C * (2ull * D.nh * D.hd + 2ull * D.kv_row + D.idx_out + 2ull * D.nh * D.hd);
    float* arena = pfalloc<float>(std::max(dn, at));
    float* q = arena;
    pf.raw = q; q += C * D.conv_dim;
    pf.conv = q; q += C * D.conv_dim;
    pf.z = q; q += C * D.v_dim;
    pf.y = q; q += C * D.v_dim;
    pf.ab_split = pf_ab_split(D.H);
    pf.a = q;  // K chunk z of a at a + z 2 C nv, of b at b + z 2 C nv
    pf.b = q + C * D.nv;
    q += 2 * C * D.nv * pf.ab_split;
    pf.decay = q; q += C * D.nv;
    pf.beta = q;
    q = arena;
    pf.q_raw = q; q += C * 2 * D.nh * D.hd;
    pf.k_raw = q; q += C * D.kv_row;
    pf.v_raw = q; q += C * D.kv_row;
    pf.idx_raw = q; q += C * D.idx_out;
    pf.q_ready = q; q += C * D.nh * D.hd;
    pf.attn_out = q;
    pf.logits = pfalloc<float>(C * D.E * PF_ROUTER_CHUNKS);  // (K-chunk partials)
    pf.sg = pfalloc<float>(C);
    pf.wts = pfalloc<float>(C * D.topk);
    pf.ids = pfalloc<uint32_t>(C * D.topk);
    pf.list = pfalloc<uint32_t>((D.E + 1) * C);
    pf.count = pfalloc<uint32_t>(D.E + 1);
    pf.gcnt = pfalloc<uint32_t>((D.E + 1) * PF_GCNT_STRIDE);
    HIPCHK(hipMemset(pf.gcnt, 0, (D.E + 1) * PF_GCNT_STRIDE * 4));
    pf.tiles = pfalloc<uint32_t>(pf_tile_bound((uint32_t)C, D.topk, D.E, 48) + pf_tile_bound((uint32_t)C, D.topk, D.E, 64));
    pf.tinfo = pfalloc<uint2>(pf_tile_bound((uint32_t)C, D.topk, D.E, 48) + pf_tile_bound((uint32_t)C, D.topk, D.E, 64));
    pf.goff = pfalloc<uint32_t>(D.E + 1);
    pf.gpos = pfalloc<uint32_t>(C * slots);
    pf.ntiles = pfalloc<uint32_t>(2);
    pf.act = pfalloc<float>(C * slots * D.I);
    pf.act_sh = D.SI != D.I ? pfalloc<float>(C * D.SI) : nullptr;
    pf.yd = pfalloc<float>(C * slots * D.H);
    pf.dcw = dc_supported(D.nk, D.nv, D.dk, D.dv) ? pfalloc<float>(dc_work_floats((uint32_t)C, D.nv, D.dv)) : nullptr;
    if (D.qsa) {
        pf.qsa_rows = pf_qsa_rows();
        pf.iq_ready = pfalloc<float>(C * D.inh * D.ihd);
        pf.qsa_bscore = pfalloc<float>((uint64_t)pf.qsa_rows * D.max_blocks);
        pf.qsa_vmask = pfalloc<uint32_t>((uint64_t)pf.qsa_rows * D.mask_words);
        pf.qsa_rows_mask = pfalloc<uint32_t>(C * D.mask_words);
        pf.qsa_part = pfalloc<float>((uint64_t)pf.qsa_rows * D.nh * max_chunks * (D.hd + 2));
    }
    if (ple_l >= 0) {
        pf.ple_ids = pfalloc<uint32_t>(C * ngram_heads);
        pf.ple_e = pfalloc<float>(C * c.ple_embed_dim);
        pf.ple_key = pfalloc<float>(C * D.hh);
        pf.ple_value = pfalloc<float>(C * D.H);
        pf.ple_gated = pfalloc<float>(C * D.hh);
        pf.ple_gvn = pfalloc<float>(C * D.hh);
    }
    pf.cap = (uint32_t)C;
}

// gated_residual read (cpu.rs:461-500) over the chunk's rows: grouped
// RMSNorm into GEMM operands, [down; inject] GEMM with silu / 2 sigmoid,
// up GEMM with the sigmoid mix, then the mixed rows as the next operands.
void ChkEngine::pf_hc_read(const HcDev& w, float* inj, uint32_t T, bool for_moe) {
    const uint32_t mt = (T + 63) / 64;
    // a pending expert combine joins the norm pass (which reads and
    // rewrites every stream anyway) unless an out-projection is pending too
    PfCombine mc{};
    if (pf.moe_pend && pf.moe_pend == pf.hyper && pf.moe_pend_T == T && !pf.pend) {
        mc = PfCombine{pf.yd, pf.goff, pf.gpos, pf.wts, pf.sg, pf.inj_m, D.topk};
        pf.moe_pend = nullptr;
    }
    pf_moe_flush();
    launch_pf_hc_prep(pf.hyper, w.norm, D.H, D.hc, D.eps, pf.inv, pf.hi, pf.lo, pf.xs, T, pf.pend,
                      (uint64_t)pf.cap * D.H, pf.pend_split, pf.inj_a, st, mc);
    pf.pend = nullptr;
    // [down; inject] is narrow (lowrank + hc outputs) over a long K = hc H:
    // split K by stream, partials summed in stream order by the finisher
    const uint32_t N = D.lowrank + D.hc;
    PfGemmArgs g{};
    g.seg[0] = PfSeg{w.down, pf.hc_part, N, 0};
    g.seg[1] = PfSeg{w.inject, pf.hc_part + D.lowrank, N, D.lowrank};
    g.nseg = 2;
    g.N = N;
    g.K = D.hh;
    g.M = T;
    g.ksplit = D.hc;
    g.zstride = (uint64_t)T * N;
    g.xhi = pf.hi;
    g.xlo = pf.lo;
    g.xs = pf.xs;
    launch_pf_gemm_args(g, PE_STORE, mt, st);
    launch_pf_hc_down_finish(pf.hc_part, D.hc, T, D.lowrank, D.hc, 1.0f / (float)D.hc, pf.d, inj, pf.dhi, pf.dlo, pf.dxs,
                             st);
    PfGemmArgs u{};
    u.seg[0].m = w.up;
    u.nseg = 1;
    u.N = D.hh;
    u.K = D.lowrank;
    u.M = T;
    u.xhi = pf.dhi;
    u.xlo = pf.dlo;
    u.xs = pf.dxs;
    u.hyper = pf.hyper;
    u.inv = pf.inv;
    u.norm = w.norm;
    u.out = pf.mixed;
    u.H = D.H;
    u.hc = D.hc;
    if (D.H % 64 == 0 && (uintptr_t)w.norm % 16 == 0) {
        // the mixed rows leave as the next GEMM's operands (and the router's)
        u.phi = pf.hi;
        u.plo = pf.lo;
        u.pxs = pf.xs;
        if (for_moe) {
            u.pbhi = pf.bhi;
            u.pbmid = pf.bmid;
            u.pblo = pf.blo;
        }
    }
    // (false: the launch wrote the f32 rows, staged below)
    if (launch_pf_gemm_args(u, PE_HC_UP, mt, st) && u.phi) return;
    PfPrepArgs p{};
    p.x = pf.mixed;
    p.ldx = D.H;
    p.T = T;
    p.K = D.H;
    p.hi = pf.hi;
    p.lo = pf.lo;
    p.xs = pf.xs;
    if (for_moe) {
        p.bhi = pf.bhi;
        p.bmid = pf.bmid;
        p.blo = pf.blo;
    }
    launch_pf_prep(p, st);
}

// A block's out-projection (K inputs -> H) over the chunk's staged
// operands.  Its inject into the hc streams (cpu.rs:971-979) is left to the
// next hyper-connection read, which reads and rewrites every stream anyway:
// the GEMM stores K-chunk partials (two chunks: twice the workgroups of a
// one-pass launch, whose 8 column blocks x 64-row tiles gave the CUs one
// workgroup each) into yd, free until the expert down projection.
void ChkEngine::pf_out_proj(const Q4Mat& m, uint32_t K, uint32_t T) {
    if (pf.pend) throw std::runtime_error("an out-projection is already pending");
    pf_moe_flush();  // (its partials take yd)
    const uint32_t G = K / 64;
    PfGemmArgs o{};
    o.seg[0] = PfSeg{m, pf.yd, D.H, 0};
    o.nseg = 1;
    o.N = D.H;
    o.K = K;
    o.M = T;
    o.ksplit = G % 2 == 0 && (G / 2) % 8 == 0 ? 2 : 1;
    o.zstride = (uint64_t)pf.cap * D.H;
    o.xhi = pf.hi;
    o.xlo = pf.lo;
    o.xs = pf.xs;
    launch_pf_gemm_args(o, PE_STORE, (T + 63) / 64, st);
    pf.pend = pf.yd;
    pf.pend_split = o.ksplit;
}

// linear_attention (cpu.rs:745-826) over the chunk: the qkv and z input
// projections as one GEMM and the narrow a / b projections as a split-K
// one, conv + norms, the scan (chunked, 64 rows per chunk, for head dims of
// 128; else sequential), the gated norm into the out-projection's
// operands, out-projection + inject.
void ChkEngine::pf_deltanet(const LayerDev& L, uint32_t T) {
    const uint32_t mt = (T + 63) / 64, di = (uint32_t)L.dn_idx;
    PfGemmArgs g{};
    g.seg[0] = PfSeg{L.dn.qkv, pf.raw, D.conv_dim, 0};
    g.seg[1] = PfSeg{L.dn.z, pf.z, D.v_dim, D.conv_dim};
    g.nseg = 2;
    g.N = D.conv_dim + D.v_dim;
    g.K = D.H;
    g.M = T;
    g.xhi = pf.hi;
    g.xlo = pf.lo;
    g.xs = pf.xs;
    launch_pf_gemm_args(g, PE_STORE, mt, st);
    // a and b (2 nv outputs): as 64 more columns of the GEMM above they made
    // a last column block of workgroups, a whole extra pass over the CUs
    // at the 80B shape; split K, their workgroups are short
    PfGemmArgs ab = g;
    ab.seg[0] = PfSeg{L.dn.a, pf.a, D.nv, 0};
    ab.seg[1] = PfSeg{L.dn.b, pf.b, D.nv, D.nv};
    ab.N = 2 * D.nv;
    ab.ksplit = pf.ab_split;
    ab.zstride = 2ull * pf.cap * D.nv;
    launch_pf_gemm_args(ab, PE_STORE, mt, st);
    PfDnArgs a{};
    a.raw = pf.raw;
    a.ld_raw = D.conv_dim;
    a.a_raw = pf.a;
    a.b_raw = pf.b;
    a.ld_ab = D.nv;
    a.ab_split = pf.ab_split;
    a.ab_zstride = ab.zstride;
    a.conv_w = L.dn.conv;
    a.a_log = L.dn.a_log;
    a.dt_bias = L.dn.dt_bias;
    a.hist = dn_hist[di];
    a.conv = pf.conv;
    a.decay = pf.decay;
    a.beta = pf.beta;
    a.state = dn_state[di];
    a.y = pf.y;
    a.T = T;
    a.conv_dim = D.conv_dim;
    a.ck = D.ck;
    a.nk = D.nk;
    a.nv = D.nv;
    a.dv = D.dv;
    a.qk_dim = D.qk_dim;
    a.v_dim = D.v_dim;
    a.qscale = D.qscale;
    launch_pf_dn(a, pf.dcw, st);
    PfPrepArgs p{};
    p.x = pf.y;
    p.ldx = D.v_dim;
    p.T = T;
    p.K = D.v_dim;
    p.hi = pf.hi;
    p.lo = pf.lo;
    p.xs = pf.xs;
    p.z = pf.z;
    p.norm = L.dn.norm;
    p.dv = D.dv;
    launch_pf_prep(p, st);
    pf_out_proj(L.dn.out, D.v_dim, T);
}

// attention (cpu.rs:544-641) over the chunk: projections as one GEMM, the
// per-row prep writing the chunk's q8 K/V and index keys at their
// positions, causal attention of every row over the cache (sub-batches of
// rows sized to the partials buffer), o-projection + inject.
void ChkEngine::pf_attention(const LayerDev& L, uint32_t T, uint32_t pos0, const KvDev* kvo) {
    const KvDev& kvl = kvo ? *kvo : kv[L.at_idx];
    const uint32_t mt = (T + 63) / 64;
    PfGemmArgs g{};
    g.seg[0] = PfSeg{L.at.q, pf.q_raw, 2 * D.nh * D.hd, 0};
    g.seg[1] = PfSeg{L.at.k, pf.k_raw, D.kv_row, 2 * D.nh * D.hd};
    g.seg[2] = PfSeg{L.at.v, pf.v_raw, D.kv_row, 2 * D.nh * D.hd + D.kv_row};
    g.seg[3] = PfSeg{L.at.idx, pf.idx_raw, D.idx_out, 2 * D.nh * D.hd + 2 * D.kv_row};
    g.nseg = 4;
    g.N = 2 * D.nh * D.hd + 2 * D.kv_row + D.idx_out;
    g.K = D.H;
    g.M = T;
    g.xhi = pf.hi;
    g.xlo = pf.lo;
    g.xs = pf.xs;
    launch_pf_gemm_args(g, PE_STORE, mt, st);
    AttnArgs aa{};
    aa.q_raw = pf.q_raw;
    aa.k_raw = pf.k_raw;
    aa.v_raw = pf.v_raw;
    aa.idx_raw = pf.idx_raw;
    aa.q_norm = L.at.q_norm;
    aa.k_norm = L.at.k_norm;
    aa.q_ready = pf.q_ready;
    aa.kv[0] = kvl;
    aa.one_kv = 1;
    aa.pos = pf.pos;
    aa.out = pf.attn_out;
    aa.nh = D.nh;
    aa.nkv = D.nkv;
    aa.hd = D.hd;
    aa.rot = D.rot;
    aa.inh = D.inh;
    aa.ihd = D.ihd;
    aa.eps = D.eps;
    aa.theta = D.theta;
    aa.scale = D.attn_scale;
    aa.max_chunks = (pos0 + T - 1) / ATTN_CHUNK + 1;
    if (!D.qsa) {
        launch_attn_prep(aa, (int)T, st);
        launch_pf_flash(pf.q_ready, pf.q_raw, kvl, pf.attn_out, T, pos0, D.nh, D.nkv, D.hd, D.attn_scale,
                        pf_flash_launch(T, pos0), st);
    } else {
        // select_tokens (cpu.rs:643-719) over the chunk: every row's KV,
        // index key and index queries first, then the pooled keys of the
        // blocks the chunk completes (later chunks and decode steps read
        // them from block_k); rows still within the budget attend densely
        // (the flash kernel), later rows through the decode path's block
        // scores, top-kblk selection and masked partials, qsa_rows at a time
        set_qsa(aa, L);
        aa.iq_ready = pf.iq_ready;
        launch_attn_prep(aa, (int)T, st);
        launch_qsa_block_keys(aa, pos0 / D.ratio, (pos0 + T) / D.ratio, st);
        const uint32_t td = pf_dense_rows(T, pos0);
        if (td) {
            launch_pf_flash(pf.q_ready, pf.q_raw, kvl, pf.attn_out, td, pos0, D.nh, D.nkv, D.hd, D.attn_scale,
                            pf_flash_launch(td, pos0), st);
            launch_zero_f32(reinterpret_cast<float*>(pf.qsa_rows_mask), (uint64_t)td * D.mask_words, st);
        }
        for (uint32_t r0 = td; r0 < T; r0 += pf.qsa_rows) {
            const uint32_t nr = std::min(pf.qsa_rows, T - r0);
            AttnArgs ag = aa;
            ag.q_raw = pf.q_raw + (uint64_t)r0 * 2 * D.nh * D.hd;
            ag.q_ready = pf.q_ready + (uint64_t)r0 * D.nh * D.hd;
            ag.iq_ready = pf.iq_ready + (uint64_t)r0 * D.inh * D.ihd;
            ag.pos = pf.pos + r0;
            ag.out = pf.attn_out + (uint64_t)r0 * D.nh * D.hd;
            ag.bscore = pf.qsa_bscore;
            ag.vmask = pf.qsa_vmask;
            ag.part = pf.qsa_part;
            ag.max_chunks = (pos0 + r0 + nr - 1) / ATTN_CHUNK + 1;
            launch_qsa(ag, (int)nr, st);
            launch_copy_f32(reinterpret_cast<float*>(pf.qsa_rows_mask) + (uint64_t)r0 * D.mask_words,
                            reinterpret_cast<const float*>(pf.qsa_vmask), (uint64_t)nr * D.mask_words, st);
            launch_attn_core(ag, (int)nr, st);
        }
    }
    launch_pf_xprep(pf.attn_out, D.nh * D.hd, T, D.nh * D.hd, pf.hi, pf.lo, pf.xs, st);
    pf_out_proj(L.at.o, D.nh * D.hd, T);
}

// Rows of a chunk that attend densely (the flash kernel): all of them, or
// with QSA those before the first position whose blocks exceed the budget.
uint32_t ChkEngine::pf_dense_rows(uint32_t T, uint32_t pos0) const {
    if (!D.qsa) return T;
    const uint32_t first_sel = (D.kblk + 1) * D.ratio - 1;  // first position with nblk > kblk
    return first_sel <= pos0 ? 0 : std::min(T, first_sel - pos0);
}

// The flash plan for (T dense rows at pos0), made and uploaded when the key
// changes: at the start of a chunk, whose stream is then idle (the previous
// chunk ended with a stream synchronisation); a change within a chunk waits
// for the launches that may still read the old plan.
PfFlashLaunch ChkEngine::pf_flash_launch(uint32_t T, uint32_t pos0) {
    const uint64_t key = (uint64_t)T << 32 | pos0;
    if (key != pf.fa_key) {
        const PfFlashPlan p = pf_flash_plan(T, pos0, std::max<uint32_t>(1, ncu / D.nkv));
        const uint64_t rmax = (pf.cap + 15) / 16, wmax = fa_wmax(pf.cap);
        if (p.seg.size() > rmax * FA_MAXSEG || p.merge.size() > wmax || p.nslots > 2 * wmax)
            throw std::runtime_error("flash attention plan exceeds its buffers");
        HIPCHK(hipStreamSynchronize(st));
        HIPCHK(hipMemcpy(pf.fa_seg, p.seg.data(), p.seg.size() * sizeof(uint4), hipMemcpyHostToDevice));
        if (!p.merge.empty())
            HIPCHK(hipMemcpy(pf.fa_merge, p.merge.data(), p.merge.size() * sizeof(uint4), hipMemcpyHostToDevice));
        pf.fa_key = key;
        pf.fa_W = p.W;
        pf.fa_nslots = p.nslots;
        pf.fa_nmerge = (uint32_t)p.merge.size();
    }
    return PfFlashLaunch{pf.fa_seg, pf.fa_merge, pf.fa_part, pf.fa_W, pf.fa_nslots, pf.fa_nmerge};
}

// moe (cpu.rs:504-541) over the chunk: router GEMM, per-row top-k, entries
// grouped by expert, grouped gate/up GEMM (shared expert as the last
// group), grouped down GEMM per entry, weighted combine + inject.  The
// activations and down outputs are stored in grouped order (each expert's
// rows together), so the down GEMM's tiles read and write row ranges; the
// combine gathers each token's rows by their grouped positions.  A shared
// expert narrower or wider than the routed ones runs as two dense GEMMs of
// its own (gate/up over every row, then down into each row's shared slot).
void ChkEngine::pf_moe(const LayerDev& L, uint32_t T) {
    const uint32_t slots = D.topk + 1;
    launch_pf_router(L.moe.router, pf.bhi, pf.bmid, pf.blo, pf.logits, T, D.E, D.H, st);
    // the chunk's last row also as this layer's "last routes", as a row step leaves them
    const uint64_t roff = (uint64_t)L.moe.record_layer * MAX_NB * D.topk;
    const bool shared_grouped = D.SI == D.I;
    // (also places every entry in its expert's group: list, gpos)
    launch_pf_route(pf.logits, T, D.E, D.topk, D.norm_topk, pf.ids, pf.wts, s.route_ids + roff, s.route_w + roff,
                    L.moe.shared_gate, pf.bhi, pf.bmid, pf.blo, pf.sg, D.H, pf.gcnt, pf.list, pf.gpos, pf.cap,
                    shared_grouped, st);
    PfGemmArgs gu{};
    gu.seg[0] = PfSeg{L.moe.sh_gate, pf.act, D.I, 0};
    gu.seg[1].m = L.moe.sh_up;
    gu.nseg = 1;
    gu.N = D.I;
    gu.K = D.H;
    gu.xhi = pf.hi;
    gu.xlo = pf.lo;
    gu.xs = pf.xs;
    gu.list = pf.list;
    gu.tiles = pf.tiles;
    gu.tinfo = pf.tinfo;
    gu.ntiles = pf.ntiles;
    gu.cap = pf.cap;
    gu.div = slots;
    gu.X = experts_dev();
    gu.X4 = experts_dev(true);
    gu.kinds = o.experts == 4 || kinds_q4 == 0 ? nullptr : rec_kind;
    gu.record_layer = L.moe.record_layer;
    PfGemmArgs dn = gu;
    dn.seg[0] = PfSeg{L.moe.sh_down, pf.yd, D.H, 0};
    dn.seg[1] = PfSeg{};
    dn.N = D.H;
    dn.K = D.I;
    dn.list = nullptr;  // rows in grouped order: the tile's own range
    dn.div = 1;
    dn.xhi = pf.ahi;
    dn.xlo = pf.alo;
    dn.xs = pf.axs;
    // experts hold from one row to over a thousand (T k / E on average):
    // both GEMMs take 64-row tiles, whose empty 16-row slices the kernel
    // skips
    const uint32_t tr = 64;
    dn.tiles = pf.tiles + pf_tile_bound(T, D.topk, D.E, tr);
    dn.tinfo = pf.tinfo + pf_tile_bound(T, D.topk, D.E, tr);
    dn.ntiles = pf.ntiles + 1;
    // (also counts the layer's expert activity)
    launch_pf_group(pf.gcnt, T, D.topk, D.E, pf.cap, pf.count, pf.tiles, pf.ntiles, pf.tinfo, pf.goff, act,
                    L.moe.record_layer, tr, shared_grouped, st);
    // the activations leave as the down GEMM's operands where the form
    // allows, else as f32 rows staged by xprep
    gu.phi = pf.ahi;
    gu.plo = pf.alo;
    gu.pxs = pf.axs;
    const bool staged = launch_pf_gemm_args(gu, PE_SILU_MUL, pf_tile_bound(T, D.topk, D.E, tr), st);
    PfGemmArgs sh{};
    if (!shared_grouped) {
        sh.seg[0] = PfSeg{L.moe.sh_gate, pf.act_sh, D.SI, 0};
        sh.seg[1].m = L.moe.sh_up;
        sh.nseg = 1;
        sh.N = D.SI;
        sh.K = D.H;
        sh.M = T;
        sh.xhi = pf.hi;
        sh.xlo = pf.lo;
        sh.xs = pf.xs;
        launch_pf_gemm_args(sh, PE_SILU_MUL, (T + 63) / 64, st);
    }
    if (!staged) launch_pf_xprep(pf.act, D.I, T * slots, D.I, pf.ahi, pf.alo, pf.axs, st);
    launch_pf_gemm_args(dn, PE_STORE, pf_tile_bound(T, D.topk, D.E, 64), st);
    if (!shared_grouped) {
        // token t's shared slot of yd: grouped row T k + t, after the routed rows
        launch_pf_xprep(pf.act_sh, D.SI, T, D.SI, pf.hi, pf.lo, pf.xs, st);
        sh.seg[0] = PfSeg{L.moe.sh_down, pf.yd + (uint64_t)T * D.topk * D.H, D.H, 0};
        sh.seg[1] = PfSeg{};
        sh.N = D.H;
        sh.K = D.SI;
        launch_pf_gemm_args(sh, PE_STORE, (T + 63) / 64, st);
    }
    // the weighted combine and its inject (cpu.rs:527-540, 971-979) are
    // left to the next hyper-connection read; other readers of the streams
    // flush them first
    pf.moe_pend = pf.hyper;
    pf.moe_pend_T = T;
}

void ChkEngine::pf_moe_flush() {
    if (!pf.moe_pend) return;
    launch_pf_moe_combine(pf.yd, pf.goff, pf.gpos, pf.wts, pf.sg, pf.inj_m, pf.moe_pend, pf.moe_pend_T, D.H, D.topk,
                          D.hc, st);
    pf.moe_pend = nullptr;
}

void ChkEngine::prefill_gemm(const uint32_t* toks, uint32_t n, uint32_t next_after, bool all_logits,
                             uint32_t* next) {
    pf_alloc();
    folded_valid = false;
    tokens.resize(pos);
    for (uint32_t c0 = 0; c0 < n; c0 += pf.cap) {
        const uint32_t T = std::min(pf.cap, n - c0), pos0 = pos;
        pf.last_rows = T;
        pf.last_pos0 = pos0;
        std::vector<uint32_t> rp(T);
        for (uint32_t t = 0; t < T; ++t) rp[t] = pos0 + t;
        HIPCHK(hipMemcpy(pf.tokens, toks + c0, T * 4, hipMemcpyHostToDevice));
        HIPCHK(hipMemcpy(pf.pos, rp.data(), T * 4, hipMemcpyHostToDevice));
        if (ple_l >= 0) {
            // the chunk's n-gram rows need the history through each row
            tokens.insert(tokens.end(), toks + c0, toks + c0 + T);
            std::vector<uint32_t> ids((size_t)T * ngram_heads);
            ple_ids(pos0, T, ids.data(), ngram_heads);
            tokens.resize(pos0);
            HIPCHK(hipMemcpy(pf.ple_ids, ids.data(), ids.size() * 4, hipMemcpyHostToDevice));
        }
        pf.pend = nullptr;  // (an earlier failed chunk may have left one)
        pf.moe_pend = nullptr;
        HIPCHK(hipMemsetAsync(pf.gcnt, 0, (D.E + 1) * PF_GCNT_STRIDE * 4, st));  // (and its expert counts)
        // the chunk's flash plan, while the stream is idle
        if (const uint32_t td = pf_dense_rows(T, pos0)) pf_flash_launch(td, pos0);
        launch_pf_embed(pf.tokens, embed, pf.hyper, D.H, D.hc, T, st);
        for (uint32_t l = 0; l < c.num_hidden_layers; ++l) {
            const LayerDev& L = layers[l];
            if (L.has_ple) {
                pf_moe_flush();
                ple_rows(L.ple, pf.ple_ids, ngram_heads, pf.hyper, pf.pos, T, pf.ple_e, pf.ple_key, pf.ple_value, pf.ple_gated,
                         pf.ple_gvn, nullptr, true);
            }
            pf_hc_read(L.attn_hc, pf.inj_a, T, false);
            if (L.linear) pf_deltanet(L, T);
            else pf_attention(L, T, pos0);
            pf_hc_read(L.mlp_hc, pf.inj_m, T, true);
            pf_moe(L, T);
        }
        pf_moe_flush();
        if (all_logits) {
            // every row through the final mixer and the LM head, four rows
            // per launch pair (the decode kernels; a checking mode)
            for (uint32_t r0 = 0; r0 < T; r0 += MAX_NB) {
                const int nb = (int)std::min<uint32_t>(MAX_NB, T - r0);
                hc_read(final_mixer, pf.hyper + (uint64_t)r0 * D.hh, nullptr, nb);
                launch_lm_head(lm_head, s.mixed, pf_all + (uint64_t)(c0 + r0) * D.V, s.pv, s.pi, lm_parts, s.out_tok,
                               nb, st);
            }
        }
        const bool last = c0 + T >= n;
        if (last) {
            // final mixer and LM head on the chunk's last row (prefill.rs:308-334)
            hc_read(final_mixer, pf.hyper + (uint64_t)(T - 1) * D.hh, nullptr, 1);
            launch_lm_head(lm_head, s.mixed, s.logits, s.pv, s.pi, lm_parts, s.d_out, 1, st);
        }
        if (has_mtp) pf_mtp(toks, c0, T, pos0, last, next_after);
        HIPCHK(hipStreamSynchronize(st));
        HIPCHK(hipGetLastError());
        tokens.insert(tokens.end(), toks + c0, toks + c0 + T);
        pos = pos0 + T;
    }
    *next = s.h_out[0];
    if (has_mtp) {
        mtp_len = pos;
        last_mtp_rows = 1;
    }
}

// The MTP head over a prefill chunk (gpu/prefill.rs:335-446): row r pairs
// the trunk residual at pos0 + r with the token after it (the next prompt
// token; after the call's last row `next_after` when the caller knows it,
// else the trunk's greedy token),
// fc_e / fc_h as GEMMs over the chunk, the MTP layer through the prefill
// layer path on its own residual and KV cache, the last row's residual
// kept where chained drafts re-enter, and on the final chunk the MTP mixer
// and LM head on that row (the draft).
void ChkEngine::pf_mtp(const uint32_t* toks, uint32_t c0, uint32_t T, uint32_t pos0, bool last,
                       uint32_t next_after) {
    if (T > 1) HIPCHK(hipMemcpyAsync(pf.mtp_tok, toks + c0 + 1, (T - 1) * 4, hipMemcpyHostToDevice, st));
    if (!last) HIPCHK(hipMemcpyAsync(pf.mtp_tok + T - 1, toks + c0 + T, 4, hipMemcpyHostToDevice, st));
    else if (next_after != CHK_NO_TOKEN)
        HIPCHK(hipMemcpyAsync(pf.mtp_tok + T - 1, &next_after, 4, hipMemcpyHostToDevice, st));
    else HIPCHK(hipMemcpyAsync(pf.mtp_tok + T - 1, s.d_out, 4, hipMemcpyDeviceToDevice, st));
    launch_mtp_prelude(pf.mtp_tok, embed, mtp_enorm, mtp_hnorm, pf.hyper, pf.mtp_en, pf.mtp_hn, D.H, D.hc, D.eps,
                       (int)T, st);
    launch_pf_xprep(pf.mtp_en, D.H, T, D.H, pf.hi, pf.lo, pf.xs, st);
    launch_pf_gemm(fc_e, pf.hi, pf.lo, pf.xs, pf.mtp_fe, T, D.H, st);
    launch_pf_xprep(pf.mtp_hn, D.H, T * D.hc, D.H, pf.hi, pf.lo, pf.xs, st);
    launch_pf_gemm(fc_h, pf.hi, pf.lo, pf.xs, pf.mtp_fh, T * D.hc, D.H, st);
    launch_mtp_fold(pf.mtp_fe, pf.mtp_fh, pf.mtp_hyper, D.H, D.hc, (int)T, st);
    float* trunk = pf.hyper;
    pf.hyper = pf.mtp_hyper;
    try {
        const LayerDev& L = mtp_layer;
        pf_hc_read(L.attn_hc, pf.inj_a, T, false);
        pf_attention(L, T, pos0, &mtp_kv);
        pf_hc_read(L.mlp_hc, pf.inj_m, T, true);
        pf_moe(L, T);
        pf_moe_flush();
    } catch (...) {
        pf.hyper = trunk;
        pf.moe_pend = nullptr;
        throw;
    }
    pf.hyper = trunk;
    const float* tail = pf.mtp_hyper + (uint64_t)(T - 1) * D.hh;
    HIPCHK(hipMemcpyAsync(s.mtp_hyper, tail, D.hh * 4, hipMemcpyDeviceToDevice, st));
    if (last) {
        hc_read(mtp_mixer, tail, nullptr, 1);
        launch_lm_head(lm_head, s.mixed, s.mtp_logits, s.pv, s.pi, lm_parts, s.mtp_out, 1, st);
    }
}

// A sequence checkpoint (Gpu's PrefixState, gpu.rs:560-566): position, MTP
// length, the token history and a copy of every prefix region.  The copies
// stay in HBM (one device buffer per region, grown and reused by
// save_into), so a save or restore is a device-to-device copy.
struct ChkPrefixState {
    uint32_t pos = 0, mtp_len = 0;
    std::vector<uint32_t> tokens;
    struct Buf {
        void* ptr = nullptr;
        uint64_t bytes = 0, cap = 0;
    };
    std::vector<Buf> data;
    ~ChkPrefixState() {
        for (auto& b : data)
            if (b.ptr) hipFree(b.ptr);
    }
};

// Gpu::state_bytes_at (gpu/state.rs:130-137): the bytes a checkpoint at
// these lengths holds (regions, token history and the record itself).
uint64_t ChkEngine::state_bytes_at(uint32_t n, uint32_t mtp_n) const {
    uint64_t b = sizeof(ChkPrefixState) + (uint64_t)n * 4;
    for (const Region& r : prefix_regions(n, mtp_n)) b += r.bytes + sizeof(ChkPrefixState::Buf);
    return b;
}

// Gpu::save_prefix / save_into (gpu/state.rs:139-193): copy the regions at
// the current lengths, reusing the checkpoint's buffers where they are large
// enough (only initialised prefixes are copied).
void ChkEngine::save_into(ChkPrefixState*& cp) {
    std::unique_ptr<ChkPrefixState> fresh;
    if (!cp) {
        fresh.reset(new ChkPrefixState());
        cp = fresh.get();
    }
    try {
        const std::vector<Region> regs = prefix_regions(pos, mtp_len);
        cp->data.resize(regs.size());
        for (size_t i = 0; i < regs.size(); ++i) {
            ChkPrefixState::Buf& b = cp->data[i];
            if (b.cap < regs[i].bytes) {
                if (b.ptr) HIPCHK(hipFree(b.ptr));
                b.ptr = nullptr;
                b.cap = 0;
                HIPCHK(hipMalloc(&b.ptr, std::max<uint64_t>(regs[i].bytes, 256)));
                b.cap = std::max<uint64_t>(regs[i].bytes, 256);
            }
            b.bytes = regs[i].bytes;
            if (b.bytes) HIPCHK(hipMemcpyAsync(b.ptr, regs[i].ptr, b.bytes, hipMemcpyDeviceToDevice, st));
        }
        HIPCHK(hipStreamSynchronize(st));
    } catch (...) {
        if (fresh) cp = nullptr;
        throw;
    }
    cp->pos = pos;
    cp->mtp_len = mtp_len;
    cp->tokens.assign(tokens.begin(), tokens.begin() + std::min<size_t>(pos, tokens.size()));
    fresh.release();
}

// Gpu::restore_prefix (gpu/state.rs:195-230).
void ChkEngine::restore_prefix(const ChkPrefixState& cp) {
    ensure(cp.pos <= max_t && cp.mtp_len <= max_t, "prefix exceeds context");
    const std::vector<Region> regs = prefix_regions(cp.pos, cp.mtp_len);
    ensure(regs.size() == cp.data.size(), "prefix state layout mismatch");
    for (size_t i = 0; i < regs.size(); ++i) ensure(regs[i].bytes == cp.data[i].bytes, "prefix region mismatch");
    for (size_t i = 0; i < regs.size(); ++i)
        if (regs[i].bytes)
            HIPCHK(hipMemcpyAsync(regs[i].ptr, cp.data[i].ptr, regs[i].bytes, hipMemcpyDeviceToDevice, st));
    HIPCHK(hipStreamSynchronize(st));
    pos = cp.pos;
    mtp_len = cp.mtp_len;
    tokens = cp.tokens;
    batch_pos = pos;
    batch_nb = 0;
    folded_valid = false;
    logit_rows = 0;
}

// ===================================================================== C ABI

#define CHK_TRY(...)                   \
    try {                              \
        __VA_ARGS__;                   \
        return 0;                      \
    } catch (const std::exception& e_) { \
        chk::g_err = e_.what();        \
        return -1;                     \
    }

extern "C" {

const char* chk_last_error(void) { return chk::g_err.c_str(); }

int chk_engine_load(const ChkConfig* cfg, const ChkOptions* opt, ChkEngine** out) {
    *out = nullptr;
    auto e = std::make_unique<ChkEngine>();
    CHK_TRY(e->load(cfg, opt); *out = e.release())
}

void chk_engine_free(ChkEngine* e) { delete e; }

int chk_engine_load_store(const char* dir, const ChkOptions* opt, ChkEngine** out) {
    *out = nullptr;
    auto e = std::make_unique<ChkEngine>();
    CHK_TRY(e->load_store(dir, opt); *out = e.release())
}

int chk_engine_load_bounded(const ChkConfig* cfg, const ChkOptions* opt, uint64_t reserve, uint64_t memory_bytes,
                            uint32_t prefill_rows, ChkEngine** out) {
    *out = nullptr;
    auto e = std::make_unique<ChkEngine>();
    CHK_TRY(e->set_budget(reserve, memory_bytes, prefill_rows); e->load(cfg, opt); *out = e.release())
}

int chk_engine_load_store_bounded(const char* dir, const ChkOptions* opt, uint64_t reserve, uint64_t memory_bytes,
                                  uint32_t prefill_rows, ChkEngine** out) {
    *out = nullptr;
    auto e = std::make_unique<ChkEngine>();
    CHK_TRY(e->set_budget(reserve, memory_bytes, prefill_rows); e->load_store(dir, opt); *out = e.release())
}

int chk_store_config(const char* dir, ChkConfig* out) { CHK_TRY(*out = chk::open_store(dir)->cfg) }

int chk_step_rows(ChkEngine* e, const uint32_t* tokens, uint32_t n, int snap, int fold_mtp, uint32_t* out) {
    CHK_TRY(e->step_rows(tokens, n, snap != 0, fold_mtp != 0, out))
}

int chk_step(ChkEngine* e, uint32_t token, uint32_t* out) {
    CHK_TRY(e->step_rows(&token, 1, false, false, out); e->commit(1))
}

int chk_commit(ChkEngine* e, uint32_t n) { CHK_TRY(e->commit(n)) }

int chk_reset(ChkEngine* e) { CHK_TRY(e->reset_state(); HIPCHK(hipStreamSynchronize(e->st))) }

int chk_mtp_draft(ChkEngine* e, const uint32_t* next, uint32_t n, uint32_t chain, uint32_t* drafts,
                  uint32_t* n_drafts) {
    CHK_TRY(e->mtp_draft(next, n, chain, drafts, n_drafts))
}

int chk_mtp_chain(ChkEngine* e, uint32_t draft, uint32_t* out) {
    CHK_TRY({
        ensure(e->has_mtp, "no MTP head");
        ensure(e->pos + 1 <= e->max_t, "context capacity exceeded");
        HIPCHK(hipMemcpyAsync(e->s.tokens, &draft, 4, hipMemcpyHostToDevice, e->st));
        HIPCHK(hipMemcpyAsync(e->s.mtp_src, e->s.mtp_hyper, e->D.hh * 4, hipMemcpyDeviceToDevice, e->st));
        e->mtp_rows(1, e->s.mtp_src, e->s.tokens, e->pos);
        HIPCHK(hipMemcpyAsync(out, e->s.mtp_out, 4, hipMemcpyDeviceToHost, e->st));
        HIPCHK(hipStreamSynchronize(e->st));
        e->mtp_logits_fresh = false;
    })
}

int chk_prefill_chunk(ChkEngine* e, const uint32_t* tokens, uint32_t n, uint32_t next_after, int all_logits,
                      uint32_t* next, uint32_t* draft) {
    CHK_TRY(e->prefill(tokens, n, next_after, all_logits != 0, next, draft))
}

void chk_prefill_release(ChkEngine* e) { e->prefill_release(); }

// Gpu::debug_engine_blocks (gpu/prefill.rs:471-484): the blocks selected for
// row r of the last prefill chunk at its latest attention layer, from the
// block mask; rows that attend densely (within the budget) select none.
int chk_debug_engine_blocks(const ChkEngine* e, uint32_t r, uint32_t* out, uint32_t cap, uint32_t* n) {
    CHK_TRY({
        *n = 0;
        ensure(e->pf.cap, "prefill scratch released");
        ensure(r < e->pf.last_rows, "row out of range");
        if (!e->D.qsa) return 0;  // the budget covers every context: no selection
        std::vector<uint32_t> m(e->D.mask_words);
        HIPCHK(hipMemcpy(m.data(), e->pf.qsa_rows_mask + (uint64_t)r * e->D.mask_words, m.size() * 4,
                         hipMemcpyDeviceToHost));
        // the selection writes the mask words of the row's complete blocks
        // only (the attention reads no bit past them)
        const uint32_t nblk = std::min(e->D.max_blocks, (e->pf.last_pos0 + r + 1) / e->D.ratio);
        uint32_t k = 0;
        for (uint32_t j = 0; j < nblk; ++j)
            if ((m[j / 32] >> (j % 32)) & 1u) {
                if (k < cap) out[k] = j;
                ++k;
            }
        *n = k;
    })
}

// Gpu::debug_row_vis (gpu/prefill.rs:486-494): the tokens row r of the last
// row step attended to at its latest attention layer, ascending: every
// token while the row's complete blocks fit the budget, else the selected
// blocks' tokens and the incomplete tail (select_tokens, cpu.rs:643-719).
int chk_debug_row_vis(const ChkEngine* e, uint32_t r, uint32_t* out, uint32_t cap, uint32_t* n) {
    CHK_TRY({
        *n = 0;
        ensure(r < e->batch_nb, "row out of range");
        const Dims& D = e->D;
        const uint32_t t_len = e->batch_pos + r + 1, nblk = t_len / D.ratio;
        std::vector<uint32_t> m;
        const bool dense = !D.qsa || nblk <= D.kblk;
        if (!dense) {
            m.resize(D.mask_words);
            HIPCHK(hipMemcpy(m.data(), e->s.vmask + (uint64_t)r * D.mask_words, m.size() * 4, hipMemcpyDeviceToHost));
        }
        uint32_t k = 0;
        for (uint32_t t = 0; t < t_len; ++t) {
            const uint32_t j = t / D.ratio;
            if (dense || j >= nblk || ((m[j / 32] >> (j % 32)) & 1u)) {
                if (k < cap) out[k] = t;
                ++k;
            }
        }
        *n = k;
    })
}

int chk_prefill_rows_fit(const ChkEngine* e, int all_logits, uint32_t* rows) {
    CHK_TRY(*rows = e->prefill_rows_fit(all_logits != 0))
}

const float* chk_pf_logits_row(ChkEngine* e, uint32_t r) {
    if (!e->pf_all_rows) {
        chk::g_err = "prefill logits not kept";
        return nullptr;
    }
    if (r >= e->pf_all_rows) {
        chk::g_err = "prefill logits row out of range";
        return nullptr;
    }
    e->host_pf_row.resize(e->D.V);
    if (hipMemcpy(e->host_pf_row.data(), e->pf_all + (size_t)r * e->D.V, (size_t)e->D.V * 4, hipMemcpyDeviceToHost) !=
        hipSuccess) {
        chk::g_err = "logits copy failed";
        return nullptr;
    }
    return e->host_pf_row.data();
}

const float* chk_logits_row(ChkEngine* e, uint32_t r) {
    if (r >= e->logit_rows) {
        chk::g_err = "logits row out of range";
        return nullptr;
    }
    if (!e->logits_fresh) {
        if (hipMemcpy(e->host_logits.data(), e->s.logits, (size_t)e->logit_rows * e->D.V * 4, hipMemcpyDeviceToHost) !=
            hipSuccess) {
            chk::g_err = "logits copy failed";
            return nullptr;
        }
        e->logits_fresh = true;
    }
    return e->host_logits.data() + (size_t)r * e->D.V;
}

const float* chk_mtp_logits_row(ChkEngine* e, uint32_t r) {
    if (!e->has_mtp || r >= std::max<uint32_t>(e->last_mtp_rows, 1)) {
        chk::g_err = "MTP logits row out of range";
        return nullptr;
    }
    if (!e->mtp_logits_fresh) {
        if (hipMemcpy(e->host_mtp_logits.data(), e->s.mtp_logits, (size_t)e->last_mtp_rows * e->D.V * 4,
                      hipMemcpyDeviceToHost) != hipSuccess) {
            chk::g_err = "logits copy failed";
            return nullptr;
        }
        e->mtp_logits_fresh = true;
    }
    return e->host_mtp_logits.data() + (size_t)r * e->D.V;
}

uint32_t chk_pos(const ChkEngine* e) { return e->pos; }
uint32_t chk_eos_token(const ChkEngine* e) { return e->c.eos_token_id; }
uint32_t chk_vocab_size(const ChkEngine* e) { return e->c.vocab_size; }
uint32_t chk_max_t(const ChkEngine* e) { return e->max_t; }
uint32_t chk_trunk_rows(const ChkEngine* e) { return e->trunk_rows; }
int chk_has_mtp(const ChkEngine* e) { return e->has_mtp ? 1 : 0; }

const float* chk_logits(ChkEngine* e) { return chk_logits_row(e, 0); }

uint32_t chk_last_logits_row(const ChkEngine* e) { return e->batch_nb ? e->batch_nb - 1 : 0; }

double chk_allocated_gb(const ChkEngine* e) { return (double)e->alloc_bytes / 1e9; }

// kv_layer_bytes (gpu.rs:631-642) at n positions, for this engine's layout:
// q8 K and V with fp16 scales per 32 values, f32 index keys, and the pooled
// block keys when the context can pass the QSA budget
static uint64_t kv_layer_bytes(const ChkEngine* e, uint64_t n) {
    const Dims& D = e->D;
    uint64_t b = 2 * (n * D.kv_row + n * (D.kv_row / 32) * 2) + n * D.ihd * 4;
    if (D.qsa) b += (n + D.ratio - 1) / D.ratio * D.ihd * 4;
    return b;
}

uint64_t chk_kv_cache_bytes(const ChkEngine* e) {
    return e->kv.size() * kv_layer_bytes(e, e->pos) + (e->has_mtp ? kv_layer_bytes(e, e->mtp_len) : 0);
}

uint64_t chk_kv_cache_capacity(const ChkEngine* e) {
    return (e->kv.size() + (e->has_mtp ? 1 : 0)) * kv_layer_bytes(e, e->max_t);
}

double chk_kv_cache_fullness(const ChkEngine* e) {
    return (double)chk_kv_cache_bytes(e) / (double)std::max<uint64_t>(chk_kv_cache_capacity(e), 1);
}

double chk_context_fullness(const ChkEngine* e) { return (double)e->pos / (double)std::max<uint32_t>(e->max_t, 1); }

int chk_reset_request(ChkEngine* e) {
    CHK_TRY(e->reset_state(); e->clear_profile(); HIPCHK(hipStreamSynchronize(e->st)))
}

int chk_clear_profile(ChkEngine* e) { CHK_TRY(e->clear_profile()) }

uint64_t chk_prefix_state_bytes(const ChkEngine* e) { return e->state_bytes_at(e->pos, e->mtp_len); }

uint64_t chk_state_bytes_at(const ChkEngine* e, uint32_t pos, uint32_t mtp_len) {
    return e->state_bytes_at(pos, mtp_len);
}

int chk_save_prefix(ChkEngine* e, ChkPrefixState** out) {
    *out = nullptr;
    CHK_TRY(e->save_into(*out))
}

int chk_save_into(ChkEngine* e, ChkPrefixState** checkpoint) { CHK_TRY(e->save_into(*checkpoint)) }

int chk_restore_prefix(ChkEngine* e, const ChkPrefixState* state) {
    CHK_TRY({
        ensure(state != nullptr, "no checkpoint");
        e->restore_prefix(*state);
    })
}

void chk_prefix_free(ChkPrefixState* state) { delete state; }

uint32_t chk_prefix_pos(const ChkPrefixState* state) { return state->pos; }

uint32_t chk_prefix_mtp_len(const ChkPrefixState* state) { return state->mtp_len; }

uint32_t chk_prefix_tokens(const ChkPrefixState* state, uint32_t* out, uint32_t cap) {
    const uint32_t n = (uint32_t)state->tokens.size();
    for (uint32_t i = 0; i < std::min(n, cap); ++i) out[i] = state->tokens[i];
    return n;
}

int chk_memory_stats(const ChkEngine* e, ChkMemoryStats* m) {
    uint64_t nrec = (uint64_t)e->record_layers * e->D.E;
    m->dense = e->dense_bytes;
    m->experts = nrec * e->rl4.stride;
    m->experts_low_bit = e->experts_lo ? nrec * e->rllo.stride : 0;
    m->state = e->state_bytes;
    m->kv_cache = e->kv_bytes;
    m->scratch = e->scratch_bytes;
    m->total = m->dense + m->experts + m->experts_low_bit + m->state + m->kv_cache + m->scratch;
    return 0;
}

// ---- expert-cache interface (residency::Pool, gpu/residency.rs:255-460)
// over the all-resident HBM store: every record of the store is a member
// from load on, so acquire never needs a read, plan_reads plans none and
// finish has nothing to wait for.

static uint32_t pool_records(const ChkEngine* e) { return e->record_layers * e->D.E; }
static uint32_t pool_store_kind(const ChkEngine* e) { return e->o.experts == 3 ? 1u : (e->o.experts == 2 ? 2u : 0u); }

uint32_t chk_pool_slots(const ChkEngine* e) { return pool_records(e); }
uint32_t chk_pool_budget(const ChkEngine* e) { return pool_records(e); }
uint32_t chk_pool_resident(const ChkEngine* e) { return pool_records(e); }
int chk_pool_is_member(const ChkEngine* e, uint32_t rid) { return rid < pool_records(e) ? 1 : 0; }

int chk_pool_acquire(ChkEngine* e, const uint32_t* rids, uint32_t n, uint64_t step, uint32_t* need,
                     uint32_t* n_need) {
    CHK_TRY({
        (void)step;
        (void)need;
        for (uint32_t i = 0; i < n; ++i) ensure(rids[i] < pool_records(e), "record id out of range");
        *n_need = 0;  // every record is resident: nothing to read
    })
}

int chk_pool_plan_reads(const ChkEngine* e, const uint32_t* need, uint32_t n, uint32_t* n_reads, uint32_t* warm) {
    CHK_TRY({
        for (uint32_t i = 0; i < n; ++i) ensure(need[i] < pool_records(e), "record id out of range");
        *n_reads = 0;
        *warm = n;
    })
}

int chk_pool_finish(ChkEngine* e, const uint32_t* rids, uint32_t n) {
    CHK_TRY({
        for (uint32_t i = 0; i < n; ++i) ensure(rids[i] < pool_records(e), "record id out of range");
    })
}

// Kind of record rid: 0 (4-bit) unless a low-bit store is attached and the
// record uses it (Pool::kind, residency.rs:290-296).
static uint32_t pool_rec_kind(const ChkEngine* e, uint32_t rid) {
    return e->rec_kind_host ? e->rec_kind_host[rid] : 0u;
}

// Pool::addr (residency.rs:437-451): the record's device address in the
// store of its kind, tagged bit 63 for 3-bit and bit 62 for 2-bit.
uint64_t chk_pool_addr(const ChkEngine* e, uint32_t rid) {
    if (rid >= pool_records(e)) return 0;
    const uint32_t k = pool_rec_kind(e, rid);
    if (k == 0) return (uint64_t)(uintptr_t)e->experts4 + (uint64_t)rid * e->rl4.stride;
    const uint64_t tag = k == 1 ? (1ull << 63) : (1ull << 62);
    return ((uint64_t)(uintptr_t)e->experts_lo + (uint64_t)rid * e->rllo.stride) | tag;
}

int chk_pool_buf(const ChkEngine* e, uint32_t rid, void** base, uint64_t* offset) {
    CHK_TRY({
        ensure(rid < pool_records(e), "record id out of range");
        const bool q4 = pool_rec_kind(e, rid) == 0;
        *base = q4 ? (void*)e->experts4 : (void*)e->experts_lo;
        *offset = (uint64_t)rid * (q4 ? e->rl4.stride : e->rllo.stride);
    })
}

uint32_t chk_pool_kind(const ChkEngine* e, uint32_t rid) {
    return rid < pool_records(e) ? pool_rec_kind(e, rid) : 0u;
}

// Pool::set_kind (residency.rs:298-306): the store a record is decoded
// from, 0 (4-bit) or the attached low-bit store's kind; every record is
// resident, so any record may change.  The change reaches the device on
// the engine's stream ahead of the next step or prefill.
int chk_pool_set_kind(ChkEngine* e, uint32_t rid, uint32_t kind) {
    CHK_TRY({
        ensure(rid < pool_records(e), "record id out of range");
        ensure(kind <= 2, "kind must be 0 (4-bit), 1 (3-bit) or 2 (2-bit)");
        if (kind == 0 && !e->rec_kind_host) return 0;  // 4-bit store only: every record is kind 0
        ensure(e->rec_kind_host && (kind == 0 || kind == pool_store_kind(e)), "low-bit store of that kind not attached");
        const uint32_t was = e->rec_kind_host[rid];
        if (was == kind) return 0;
        e->rec_kind_host[rid] = (uint8_t)kind;
        HIPCHK(hipMemcpyAsync(e->rec_kind + rid, e->rec_kind_host + rid, 1, hipMemcpyHostToDevice, e->st));
        const uint32_t before = e->kinds_q4;
        e->kinds_q4 += kind == 0 ? 1 : 0;
        e->kinds_q4 -= was == 0 ? 1 : 0;
        if ((before == 0) != (e->kinds_q4 == 0)) e->drop_graphs();  // the kernels' form changes
    })
}

int chk_pool_store(const ChkEngine* e, uint32_t kind, void** base, uint64_t* stride) {
    CHK_TRY({
        if (kind == 0) {
            *base = e->experts4;
            *stride = e->rl4.stride;
        } else {
            ensure(e->experts_lo && kind == pool_store_kind(e), "low-bit store of that kind not attached");
            *base = e->experts_lo;
            *stride = e->rllo.stride;
        }
    })
}

// The bytes of every record in the store of its kind.
uint64_t chk_pool_bytes(const ChkEngine* e) {
    uint64_t n = 0;
    for (uint32_t rid = 0; rid < pool_records(e); ++rid) n += pool_rec_kind(e, rid) ? e->rllo.stride : e->rl4.stride;
    return n;
}

// Gpu::throttle_ms (gpu.rs:596-599): the wall time in ms of the second of
// two runs of the dependent-FMA probe (60,000 iterations per thread), from
// submission to completion, as MetalContext::throttle_probe times it.
int chk_throttle_ms(ChkEngine* e, double* ms) {
    CHK_TRY({
        float* out = nullptr;
        HIPCHK(hipMalloc(&out, 65536 * 4));
        double last = 0.0;
        try {
            for (int r = 0; r < 2; ++r) {
                HIPCHK(hipStreamSynchronize(e->st));
                const auto t0 = std::chrono::steady_clock::now();
                launch_clock_probe(out, 60000, e->st);
                HIPCHK(hipStreamSynchronize(e->st));
                last = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
            }
        } catch (...) {
            hipFree(out);
            throw;
        }
        HIPCHK(hipFree(out));
        *ms = last;
    })
}

// Gpu::working_set_limit_gb (gpu.rs:690-694): the device memory the engine
// may work in, in decimal GB (units.rs:7): the device's total memory.
double chk_working_set_limit_gb(const ChkEngine* e) {
    (void)e;
    size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) return 0.0;
    return (double)total_b / 1e9;
}

// Gpu::expert_activity (activity.rs:11-89, 110): cumulative per-record
// counters since load, records in record order (main layers, then the MTP
// layer; E per layer).  Every record is resident: a lookup is a hit, and
// nothing is prefetched or read.
int chk_expert_activity(const ChkEngine* e, ChkExpertCounters* records, uint32_t n, double* elapsed_seconds) {
    CHK_TRY({
        const uint32_t total = e->record_layers * e->D.E;
        ensure(n == total, "expert activity holds " + std::to_string(total) + " records");
        std::vector<uint64_t> h((size_t)total * 2);
        HIPCHK(hipStreamSynchronize(e->st));
        HIPCHK(hipMemcpy(h.data(), e->act, h.size() * 8, hipMemcpyDeviceToHost));
        for (uint32_t r = 0; r < total; ++r) {
            records[r] = ChkExpertCounters{};
            records[r].selected_rows = h[2 * r];
            records[r].cache_hits = h[2 * r + 1];
        }
        *elapsed_seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - e->act_started).count();
    })
}

int chk_last_routes(const ChkEngine* e, uint32_t layer, uint32_t r, uint32_t* ids, float* weights) {
    CHK_TRY({
        ensure(layer < e->record_layers, "layer out of range");
        ensure(r < MAX_NB, "row out of range");
        uint64_t off = ((uint64_t)layer * MAX_NB + r) * e->D.topk;
        HIPCHK(hipMemcpy(ids, e->s.route_ids + off, e->D.topk * 4, hipMemcpyDeviceToHost));
        if (weights) HIPCHK(hipMemcpy(weights, e->s.route_w + off, e->D.topk * 4, hipMemcpyDeviceToHost));
    })
}

int chk_last_probs(const ChkEngine* e, uint32_t layer, uint32_t r, float* probs) {
    CHK_TRY({
        ensure(layer < e->record_layers, "layer out of range");
        ensure(r < MAX_NB, "row out of range");
        const uint64_t off = ((uint64_t)layer * MAX_NB + r) * e->D.E;
        HIPCHK(hipMemcpy(probs, e->s.router_probs + off, e->D.E * 4, hipMemcpyDeviceToHost));
    })
}

// ------------------------------------------------------ kernel-level ABI

int chk_q4_matvec(const void* w, const void* s, const void* b, uint32_t out, uint32_t in, const float* x, float* y,
                  uint32_t nb, void* stream) {
    CHK_TRY({
        ensure(nb >= 1 && nb <= (uint32_t)MAX_NB, "nb must be 1..=4");
        ensure(in % 64 == 0 && in > 0 && out > 0, "in must be a positive multiple of 64");
        SegArgs a{};
        a.nseg = 1;
        a.seg[0] = Seg{Q4Mat{(const uint32_t*)w, (const uint16_t*)s, (const uint16_t*)b, out, in}, x, y, in, out, 0,
                       EPI_RAW};
        a.total = out;
        hipStream_t st = (hipStream_t)stream;
        launch_qmv(a, (int)nb, st);
        HIPCHK(hipStreamSynchronize(st));
        HIPCHK(hipGetLastError());
    })
}

int chk_lm_head_argmax(const void* w, const void* s, const void* b, uint32_t out, uint32_t in, const float* x,
                       uint32_t nb, float* logits, uint32_t* ids, void* stream) {
    CHK_TRY({
        ensure(nb >= 1 && nb <= (uint32_t)MAX_NB, "nb must be 1..=4");
        ensure(in % 64 == 0 && in > 0, "in must be a positive multiple of 64");
        ensure(out > 0 && out % 8 == 0, "out must be a positive multiple of 8");
        const uint32_t parts = 1024;
        hipStream_t st = (hipStream_t)stream;
        float* pv = nullptr;
        uint32_t* pi = nullptr;
        uint32_t* d_ids = nullptr;
        HIPCHK(hipMalloc(&pv, (size_t)nb * parts * 4));
        HIPCHK(hipMalloc(&pi, (size_t)nb * parts * 4));
        HIPCHK(hipMalloc(&d_ids, (size_t)nb * 4));
        launch_lm_head(Q4Mat{(const uint32_t*)w, (const uint16_t*)s, (const uint16_t*)b, out, in}, x, logits, pv, pi,
                       parts, d_ids, (int)nb, st);
        HIPCHK(hipMemcpyAsync(ids, d_ids, (size_t)nb * 4, hipMemcpyDeviceToDevice, st));
        HIPCHK(hipStreamSynchronize(st));
        HIPCHK(hipGetLastError());
        HIPCHK(hipFree(pv));
        HIPCHK(hipFree(pi));
        HIPCHK(hipFree(d_ids));
    })
}

int chk_attn_decode_q8(const float* q, const void* k, const void* v, const void* ks, const void* vs, uint32_t T,
                       uint32_t nh, uint32_t nkv, uint32_t hd, float* out, void* stream) {
    CHK_TRY({
        ensure(T > 0 && T <= (uint32_t)MAX_ATTN_CHUNKS * ATTN_CHUNK, "context must be 1..=262144 tokens");
        ensure(attn_shape_ok(nh, nkv, hd), "head_dim 128 or 256, 1, 2, 4, 8 or 12 query heads per kv head");
        hipStream_t st = (hipStream_t)stream;
        AttnArgs a{};
        a.nh = nh;
        a.nkv = nkv;
        a.hd = hd;
        a.max_chunks = (T + ATTN_CHUNK - 1) / ATTN_CHUNK;
        a.scale = powf((float)hd, -0.5f);
        a.q_raw = q;
        a.kv[0] = KvDev{(int8_t*)k, (int8_t*)v, (uint16_t*)ks, (uint16_t*)vs, nullptr};
        float* q_ready = nullptr;
        float* part = nullptr;
        uint32_t* pos = nullptr;
        HIPCHK(hipMalloc(&q_ready, (size_t)nh * hd * 4));
        HIPCHK(hipMalloc(&part, (size_t)nh * a.max_chunks * (hd + 2) * 4));
        HIPCHK(hipMalloc(&pos, 4));
        const uint32_t last = T - 1;
        HIPCHK(hipMemcpyAsync(pos, &last, 4, hipMemcpyHostToDevice, st));
        // the q halves of the per-head [q | gate] rows
        HIPCHK(hipMemcpy2DAsync(q_ready, (size_t)hd * 4, q, (size_t)2 * hd * 4, (size_t)hd * 4, nh,
                                hipMemcpyDeviceToDevice, st));
        a.q_ready = q_ready;
        a.part = part;
        a.pos = pos;
        a.out = out;
        launch_attn_core(a, 1, st);
        HIPCHK(hipStreamSynchronize(st));
        HIPCHK(hipGetLastError());
        HIPCHK(hipFree(q_ready));
        HIPCHK(hipFree(part));
        HIPCHK(hipFree(pos));
    })
}

int chk_dn_scan(const float* conv, const float* decay, const float* beta, float* state, float* y, uint32_t T,
                uint32_t nk, uint32_t nv, uint32_t dk, uint32_t dv, int chunked, void* stream) {
    CHK_TRY({
        ensure(T > 0 && T <= 65536, "1..=65536 rows");
        ensure(nk > 0 && nv % nk == 0 && dk == 128 && dv % 4 == 0 && dv > 0, "key head dim 128, nv a multiple of nk");
        ensure(!chunked || dc_supported(nk, nv, dk, dv), "the chunked scan needs key and value head dims of 128");
        hipStream_t st = (hipStream_t)stream;
        PfDnArgs a{};
        a.conv = const_cast<float*>(conv);
        a.decay = const_cast<float*>(decay);
        a.beta = const_cast<float*>(beta);
        a.state = state;
        a.y = y;
        a.T = T;
        a.nk = nk;
        a.nv = nv;
        a.dv = dv;
        a.qk_dim = nk * dk;
        a.v_dim = nv * dv;
        a.conv_dim = 2 * a.qk_dim + a.v_dim;
        float* work = nullptr;
        if (chunked) HIPCHK(hipMalloc(&work, dc_work_floats(T, nv, dv) * 4));
        launch_pf_dn_scan(a, work, st);
        HIPCHK(hipStreamSynchronize(st));
        HIPCHK(hipGetLastError());
        if (work) HIPCHK(hipFree(work));
    })
}

int chk_qsa_select(const float* scores, uint32_t t_len, uint32_t kblk, uint32_t ratio, uint32_t* vmask, void* stream) {
    CHK_TRY({
        ensure(ratio >= 1 && kblk >= 1, "ratio and kblk must be positive");
        ensure(t_len / ratio <= 65536, "at most 65536 blocks");
        hipStream_t st = (hipStream_t)stream;
        AttnArgs a{};
        a.qsa = 1;
        a.one_kv = 1;
        a.ratio = ratio;
        a.kblk = kblk;
        a.max_blocks = t_len / ratio + 1;
        a.mask_words = (a.max_blocks + 31) / 32;
        a.bscore = const_cast<float*>(scores);
        a.vmask = vmask;
        uint32_t* pos = nullptr;
        HIPCHK(hipMalloc(&pos, 4));
        const uint32_t last = t_len - 1;
        HIPCHK(hipMemcpyAsync(pos, &last, 4, hipMemcpyHostToDevice, st));
        a.pos = pos;
        launch_qsa_select(a, 1, st);
        HIPCHK(hipStreamSynchronize(st));
        HIPCHK(hipGetLastError());
        HIPCHK(hipFree(pos));
    })
}

static const LayerDev* layer_dev(ChkEngine* e, uint32_t layer) {
    if (layer < e->c.num_hidden_layers) return &e->layers[layer];
    if (layer == e->c.num_hidden_layers && e->has_mtp) return &e->mtp_layer;
    throw Error("layer out of range");
}

int chk_moe_block(ChkEngine* e, uint32_t layer, const float* x, uint32_t nb, float* out, uint32_t* top_ids,
                  float* top_w, float* probs) {
    CHK_TRY({
        ensure(nb >= 1 && nb <= (uint32_t)MAX_NB, "nb must be 1..=4");
        const LayerDev* L = layer_dev(e, layer);
        e->moe(*L, layer, x, (int)nb, nullptr, nullptr, out);
        uint64_t off = (uint64_t)layer * MAX_NB;
        if (top_ids)
            HIPCHK(hipMemcpyAsync(top_ids, e->s.route_ids + off * e->D.topk, nb * e->D.topk * 4,
                                  hipMemcpyDeviceToDevice, e->st));
        if (top_w)
            HIPCHK(hipMemcpyAsync(top_w, e->s.route_w + off * e->D.topk, nb * e->D.topk * 4, hipMemcpyDeviceToDevice,
                                  e->st));
        if (probs)
            HIPCHK(hipMemcpyAsync(probs, e->s.router_probs + off * e->D.E, nb * e->D.E * 4, hipMemcpyDeviceToDevice,
                                  e->st));
        HIPCHK(hipStreamSynchronize(e->st));
        HIPCHK(hipGetLastError());
    })
}

int chk_deltanet_block(ChkEngine* e, uint32_t layer, const float* x, uint32_t nb, int snap, float* out) {
    CHK_TRY({
        ensure(nb >= 1 && nb <= (uint32_t)MAX_NB, "nb must be 1..=4");
        ensure(layer < e->c.num_hidden_layers && e->layers[layer].linear, "not a DeltaNet layer");
        e->deltanet(e->layers[layer], x, (int)nb, snap != 0, nullptr, nullptr, out);
        HIPCHK(hipStreamSynchronize(e->st));
        HIPCHK(hipGetLastError());
    })
}

int chk_deltanet_state(ChkEngine* e, uint32_t layer, float* s_host, float* conv_host) {
    CHK_TRY({
        ensure(layer < e->c.num_hidden_layers && e->layers[layer].linear, "not a DeltaNet layer");
        int di = e->layers[layer].dn_idx;
        const Dims& D = e->D;
        if (s_host) {
            std::vector<float> t((size_t)D.nv * D.dv * D.dk);
            HIPCHK(hipMemcpy(t.data(), e->dn_state[di], t.size() * 4, hipMemcpyDeviceToHost));
            for (uint32_t h = 0; h < D.nv; ++h)
                for (uint32_t iv = 0; iv < D.dv; ++iv)
                    for (uint32_t ik = 0; ik < D.dk; ++ik)
                        s_host[((size_t)h * D.dk + ik) * D.dv + iv] = t[((size_t)h * D.dv + iv) * D.dk + ik];
        }
        if (conv_host)
            HIPCHK(hipMemcpy(conv_host, e->dn_hist[di], (size_t)D.conv_dim * (D.ck - 1) * 4, hipMemcpyDeviceToHost));
    })
}

int chk_deltanet_rollback(ChkEngine* e, uint32_t layer, uint32_t plane) {
    CHK_TRY({
        ensure(layer < e->c.num_hidden_layers && e->layers[layer].linear, "not a DeltaNet layer");
        ensure(plane < (uint32_t)MAX_SNAP, "snapshot plane out of range");
        int di = e->layers[layer].dn_idx;
        uint64_t sn = (uint64_t)e->D.nv * e->D.dv * e->D.dk, hn = (uint64_t)e->D.conv_dim * (e->D.ck - 1);
        launch_copy_f32(e->dn_state[di], e->dn_snap_state[di] + plane * sn, sn, e->st);
        launch_copy_f32(e->dn_hist[di], e->dn_snap_hist[di] + plane * hn, hn, e->st);
        HIPCHK(hipStreamSynchronize(e->st));
    })
}

int chk_attention_block(ChkEngine* e, uint32_t layer, const float* x, uint32_t nb, uint32_t pos, float* out) {
    CHK_TRY({
        ensure(nb >= 1 && nb <= (uint32_t)MAX_NB, "nb must be 1..=4");
        ensure(layer < e->c.num_hidden_layers && !e->layers[layer].linear, "not an attention layer");
        ensure(pos + nb <= e->max_t, "context capacity exceeded");
        const LayerDev& L = e->layers[layer];
        KvDev kvs[MAX_NB];
        uint32_t rp[MAX_NB];
        for (uint32_t b = 0; b < nb; ++b) {
            kvs[b] = e->kv[L.at_idx];
            rp[b] = pos + b;
        }
        HIPCHK(hipMemcpyAsync(e->s.rowpos_aux, rp, nb * 4, hipMemcpyHostToDevice, e->st));
        e->attention(L, x, (int)nb, kvs, e->s.rowpos_aux, nullptr, nullptr, out);
        HIPCHK(hipStreamSynchronize(e->st));
        HIPCHK(hipGetLastError());
    })
}

int chk_kv_fill(ChkEngine* e, uint32_t layer, uint32_t seq, const float* k, const float* v, uint32_t T) {
    CHK_TRY({
        ensure(layer < e->c.num_hidden_layers && !e->layers[layer].linear, "not an attention layer");
        ensure(seq <= 1, "sequence slot must be 0 or 1");
        ensure(T <= e->max_t, "context capacity exceeded");
        int ai = e->layers[layer].at_idx;
        if (seq == 1 && e->kv2.empty())
            for (size_t i = 0; i < e->kv.size(); ++i) e->kv2.push_back(e->alloc_kv());
        KvDev kv = seq == 0 ? e->kv[ai] : e->kv2[ai];
        launch_kv_fill(k, v, kv, e->D.kv_row, T, e->st);
        HIPCHK(hipStreamSynchronize(e->st));
        HIPCHK(hipGetLastError());
    })
}

int chk_attention_block2(ChkEngine* e, uint32_t layer, const float* x, const uint32_t* pos, float* out) {
    CHK_TRY({
        ensure(layer < e->c.num_hidden_layers && !e->layers[layer].linear, "not an attention layer");
        ensure(!e->kv2.empty(), "second sequence slot not initialised (chk_kv_fill seq 1)");
        ensure(pos[0] < e->max_t && pos[1] < e->max_t, "context capacity exceeded");
        const LayerDev& L = e->layers[layer];
        KvDev kvs[MAX_NB] = {e->kv[L.at_idx], e->kv2[L.at_idx]};
        uint32_t rp[MAX_NB] = {pos[0], pos[1]};
        HIPCHK(hipMemcpyAsync(e->s.rowpos_aux, rp, 2 * 4, hipMemcpyHostToDevice, e->st));
        e->attention(L, x, 2, kvs, e->s.rowpos_aux, nullptr, nullptr, out);
        HIPCHK(hipStreamSynchronize(e->st));
        HIPCHK(hipGetLastError());
    })
}

int chk_hc_read(ChkEngine* e, uint32_t layer, uint32_t which, const float* hyper, uint32_t nb, float* mixed,
                float* inj) {
    CHK_TRY({
        ensure(nb >= 1 && nb <= (uint32_t)MAX_NB, "nb must be 1..=4");
        const HcDev* w = nullptr;
        if (which == CHK_HC_FINAL) w = &e->final_mixer;
        else if (which == CHK_HC_MTP) {
            ensure(e->has_mtp, "no MTP head");
            w = &e->mtp_mixer;
        } else {
            const LayerDev* L = layer_dev(e, layer);
            w = which == CHK_HC_ATTN ? &L->attn_hc : &L->mlp_hc;
        }
        e->hc_read(*w, hyper, e->s.inj_a, (int)nb);
        HIPCHK(hipMemcpyAsync(mixed, e->s.mixed, (size_t)nb * e->D.H * 4, hipMemcpyDeviceToDevice, e->st));
        if (inj && w->has_inject)
            HIPCHK(hipMemcpyAsync(inj, e->s.inj_a, (size_t)nb * e->D.hc * 4, hipMemcpyDeviceToDevice, e->st));
        HIPCHK(hipStreamSynchronize(e->st));
        HIPCHK(hipGetLastError());
    })
}

int chk_expert_record(ChkEngine* e, uint32_t layer, uint32_t expert, uint32_t bits, void* host, uint64_t n) {
    CHK_TRY({
        ensure(layer < e->record_layers && expert < e->D.E, "record out of range");
        const uint8_t* base;
        uint64_t stride;
        if (bits == 4) {
            base = e->experts4;
            stride = e->rl4.stride;
        } else {
            ensure(e->experts_lo && bits == e->o.experts, "no low-bit store of that precision");
            base = e->experts_lo;
            stride = e->rllo.stride;
        }
        ensure(n <= stride, "copy larger than the record stride");
        HIPCHK(hipMemcpy(host, base + ((uint64_t)layer * e->D.E + expert) * stride, n, hipMemcpyDeviceToHost));
    })
}

uint64_t chk_record_stride(const ChkEngine* e, uint32_t bits) {
    if (bits == 4) return e->rl4.stride;
    return e->experts_lo && bits == e->o.experts ? e->rllo.stride : 0;
}

int chk_trace_enable(ChkEngine* e, int on) {
    CHK_TRY({
        e->tracing = on != 0;
        if (e->tracing && !e->s.trace)
            e->s.trace = e->dalloc<float>((uint64_t)e->c.num_hidden_layers * MAX_NB * e->D.hh);
    })
}

int chk_layer_hyper(ChkEngine* e, uint32_t layer, uint32_t r, float* host) {
    CHK_TRY({
        ensure(e->s.trace, "tracing is off");
        ensure(layer < e->c.num_hidden_layers && r < MAX_NB, "out of range");
        HIPCHK(hipMemcpy(host, e->s.trace + ((uint64_t)layer * MAX_NB + r) * e->D.hh, e->D.hh * 4,
                         hipMemcpyDeviceToHost));
    })
}

int chk_profile_kernel(ChkEngine* e, int kind) {
    CHK_TRY({
        ensure(kind >= 0 && kind <= 3, "unknown kernel class");
        e->prof_collect();
        e->prof_kind = kind;
        e->prof_ms = 0.0;
        e->prof_bytes = 0;
        e->prof_launches = 0;
    })
}

int chk_q4_gemm(const void* w, const void* s, const void* b, uint32_t out, uint32_t in, const float* x, uint32_t T,
                float* y, void* stream) {
    CHK_TRY({
        ensure(in % 64 == 0 && in > 0 && out > 0 && T > 0, "in must be a positive multiple of 64, out and T positive");
        hipStream_t st = (hipStream_t)stream;
        uint4 *hi = nullptr, *lo = nullptr;
        float* xs = nullptr;
        HIPCHK(hipMalloc(&hi, (size_t)T * in * 2));
        HIPCHK(hipMalloc(&lo, (size_t)T * in * 2));
        HIPCHK(hipMalloc(&xs, (size_t)T * (in / 64) * 4));
        // the GEMM addresses a matrix's codes, scales and biases by 32-bit
        // offsets from one base (the engine keeps them in one arena), so the
        // caller's three buffers are packed together first
        const size_t wb = (size_t)out * in / 2, sb = (size_t)out * (in / 64) * 2;
        const size_t so = (wb + 255) & ~(size_t)255, bo = so + ((sb + 255) & ~(size_t)255);
        uint8_t* pack = nullptr;
        HIPCHK(hipMalloc(&pack, bo + sb));
        HIPCHK(hipMemcpyAsync(pack, w, wb, hipMemcpyDeviceToDevice, st));
        HIPCHK(hipMemcpyAsync(pack + so, s, sb, hipMemcpyDeviceToDevice, st));
        HIPCHK(hipMemcpyAsync(pack + bo, b, sb, hipMemcpyDeviceToDevice, st));
        launch_pf_xprep(x, in, T, in, hi, lo, xs, st);
        launch_pf_gemm(Q4Mat{(const uint32_t*)pack, (const uint16_t*)(pack + so), (const uint16_t*)(pack + bo), out, in},
                       hi, lo, xs, y, T, out, st);
        HIPCHK(hipStreamSynchronize(st));
        HIPCHK(hipGetLastError());
        HIPCHK(hipFree(hi));
        HIPCHK(hipFree(lo));
        HIPCHK(hipFree(xs));
        HIPCHK(hipFree(pack));
    })
}

int chk_prefix_regions(const ChkEngine* e, uint32_t pos, uint32_t mtp_len, uint64_t* ptrs, uint64_t* bytes,
                       uint32_t cap, uint32_t* count) {
    CHK_TRY({
        ensure(pos <= e->max_t && mtp_len <= e->max_t, "prefix exceeds context");
        const auto regs = e->prefix_regions(pos, mtp_len);
        *count = (uint32_t)regs.size();
        for (uint32_t i = 0; i < std::min<uint32_t>(cap, (uint32_t)regs.size()); ++i) {
            ptrs[i] = (uint64_t)(uintptr_t)regs[i].ptr;
            bytes[i] = regs[i].bytes;
        }
    })
}

int chk_prefix_read(const ChkPrefixState* state, uint32_t i, void* host, uint64_t n) {
    CHK_TRY({
        ensure(i < state->data.size(), "region out of range");
        ensure(n <= state->data[i].bytes, "read past the region");
        if (n) HIPCHK(hipMemcpy(host, state->data[i].ptr, n, hipMemcpyDeviceToHost));
    })
}

int chk_fill_u8(void* dst, uint32_t value, uint64_t n, void* stream) {
    CHK_TRY({
        hipStream_t st = (hipStream_t)stream;
        launch_fill_u8((uint8_t*)dst, (uint8_t)value, n, st);
        HIPCHK(hipStreamSynchronize(st));
        HIPCHK(hipGetLastError());
    })
}

int chk_pf_flash_plan(uint32_t T, uint32_t pos0, uint32_t max_wg, uint32_t* W, uint32_t* nslots, uint32_t* seg,
                      uint64_t seg_cap, uint32_t* merge, uint64_t merge_cap, uint32_t* nmerge) {
    CHK_TRY({
        ensure(T >= 1 && max_wg >= 1, "T and max_wg must be positive");
        const PfFlashPlan p = pf_flash_plan(T, pos0, max_wg);
        ensure(p.seg.size() * 4 <= seg_cap && p.merge.size() * 4 <= merge_cap, "plan buffers too small");
        *W = p.W;
        *nslots = p.nslots;
        *nmerge = (uint32_t)p.merge.size();
        memcpy(seg, p.seg.data(), p.seg.size() * sizeof(uint4));
        if (!p.merge.empty()) memcpy(merge, p.merge.data(), p.merge.size() * sizeof(uint4));
    })
}

int chk_copy_f32(float* dst, const float* src, uint64_t n, void* stream) {
    CHK_TRY({
        hipStream_t st = (hipStream_t)stream;
        launch_copy_f32(dst, src, n, st);
        HIPCHK(hipStreamSynchronize(st));
        HIPCHK(hipGetLastError());
    })
}

int chk_profile_graph(ChkEngine* e, int kind, uint32_t reps, double* ms_total, uint64_t* launches,
                      uint64_t* bytes) {
    CHK_TRY({ *ms_total = e->profile_graph(kind, reps, *bytes, *launches); })
}

int chk_profile_read(ChkEngine* e, double* ms_total, uint64_t* launches, uint64_t* bytes) {
    CHK_TRY({
        e->prof_collect();
        *ms_total = e->prof_ms;
        *launches = e->prof_launches;
        *bytes = e->prof_bytes;
    })
}

// One captured graph runs the block of kind `kind` (2 MoE, 3 DeltaNet, 4
// attention) once for each of layers[0..n_layers), block i on input rows
// x + (i % nx) * nb * H, the way the decode step launches it; the graph is
// replayed `reps` times between two HIP events (after one untimed replay).
// Attention rows attend at positions pos[0..nb) over the engine's
// sequence (nb 1) or its two sequence slots (nb 2, chk_kv_fill seq 1);
// DeltaNet blocks with nb > 1 take the verify form (snapshots).
int chk_time_blocks(ChkEngine* e, int kind, uint32_t nb, const uint32_t* layers, uint32_t n_layers, const float* x,
                    uint32_t nx, const uint32_t* pos, uint32_t reps, float* us_per_block) {
    CHK_TRY({
        ensure(kind >= 2 && kind <= 4, "block kind must be 2 (MoE), 3 (DeltaNet) or 4 (attention)");
        ensure(nb >= 1 && nb <= e->trunk_rows, "rows per block must be 1..=" + std::to_string(e->trunk_rows));
        ensure(n_layers >= 1 && nx >= 1 && reps >= 1, "need layers, inputs and repetitions");
        ensure(!(kind == 4 && nb > 2), "attention blocks are timed at batch 1 or 2");
        ensure(!(kind == 4 && nb == 2 && e->kv2.empty()), "second sequence slot not initialised (chk_kv_fill seq 1)");
        for (uint32_t i = 0; i < n_layers; ++i) {
            ensure(layers[i] < e->c.num_hidden_layers || (kind == 2 && layers[i] == e->c.num_hidden_layers && e->has_mtp),
                   "layer out of range");
            if (kind == 3) ensure(e->layers[layers[i]].linear, "not a DeltaNet layer");
            if (kind == 4) ensure(!e->layers[layers[i]].linear, "not an attention layer");
        }
        if (kind == 4) {
            for (uint32_t b = 0; b < nb; ++b) ensure(pos[b] < e->max_t, "context capacity exceeded");
            HIPCHK(hipMemcpyAsync(e->s.rowpos_aux, pos, nb * 4, hipMemcpyHostToDevice, e->st));
        }
        float* out = e->s.mix_out;
        HIPCHK(hipStreamSynchronize(e->st));
        hipGraph_t g;
        HIPCHK(hipStreamBeginCapture(e->st, hipStreamCaptureModeThreadLocal));
        e->capturing = true;
        try {
            for (uint32_t i = 0; i < n_layers; ++i) {
                const LayerDev& L = layers[i] < e->c.num_hidden_layers ? e->layers[layers[i]] : e->mtp_layer;
                const float* xi = x + (uint64_t)(i % nx) * nb * e->D.H;
                if (kind == 2) {
                    e->moe(L, layers[i], xi, (int)nb, nullptr, nullptr, out);
                } else if (kind == 3) {
                    e->deltanet(L, xi, (int)nb, nb > 1, nullptr, nullptr, out);
                } else {
                    KvDev kvs[MAX_NB];
                    kvs[0] = e->kv[L.at_idx];
                    if (nb == 2) kvs[1] = e->kv2[L.at_idx];
                    e->attention(L, xi, (int)nb, kvs, e->s.rowpos_aux, nullptr, nullptr, out);
                }
            }
        } catch (...) {
            e->capturing = false;
            hipGraph_t dead;
            (void)hipStreamEndCapture(e->st, &dead);
            throw;
        }
        e->capturing = false;
        HIPCHK(hipStreamEndCapture(e->st, &g));
        hipGraphExec_t ge;
        HIPCHK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
        hipEvent_t a, b;
        HIPCHK(hipEventCreate(&a));
        HIPCHK(hipEventCreate(&b));
        HIPCHK(hipGraphLaunch(ge, e->st));  // warm
        HIPCHK(hipEventRecord(a, e->st));
        for (uint32_t r = 0; r < reps; ++r) HIPCHK(hipGraphLaunch(ge, e->st));
        HIPCHK(hipEventRecord(b, e->st));
        HIPCHK(hipEventSynchronize(b));
        float ms = 0.0f;
        HIPCHK(hipEventElapsedTime(&ms, a, b));
        *us_per_block = ms * 1e3f / (float)((uint64_t)reps * n_layers);
        (void)hipEventDestroy(a);
        (void)hipEventDestroy(b);
        HIPCHK(hipGraphExecDestroy(ge));
        HIPCHK(hipGraphDestroy(g));
        HIPCHK(hipGetLastError());
    })
}

int chk_time_decode(ChkEngine* e, uint32_t first_token, uint32_t steps, float* ms_per_step, uint32_t* last_token) {
    CHK_TRY({
        ensure(e->pos + steps <= e->max_t, "context capacity exceeded");
        hipEvent_t a, b;
        HIPCHK(hipEventCreate(&a));
        HIPCHK(hipEventCreate(&b));
        uint32_t tok = first_token;
        HIPCHK(hipEventRecord(a, e->st));
        for (uint32_t i = 0; i < steps; ++i) {
            uint32_t out;
            e->step_rows(&tok, 1, false, false, &out);
            e->commit(1);
            tok = out;
        }
        HIPCHK(hipEventRecord(b, e->st));
        HIPCHK(hipEventSynchronize(b));
        float ms = 0;
        HIPCHK(hipEventElapsedTime(&ms, a, b));
        *ms_per_step = steps ? ms / steps : 0.0f;
        *last_token = tok;
        hipEventDestroy(a);
        hipEventDestroy(b);
    })
}

}  // extern "C"
