// CPU ORACLE — test infrastructure only.
//
// A C++ restatement of the reference's f32 CPU forward for qwen4_exp:
//   /root/reference/src/nn.rs:6-56           (rms_norm, silu, sigmoid, softplus, softmax, l2_norm)
//   /root/reference/src/quant.rs:24-89        (QLinear::dequant_row, QLinear::matvec)
//   /root/reference/src/qwen4_exp/cpu.rs:276-1085 (forward_token, mtp_forward, gated_residual,
//                                               moe, attention, select_tokens, deltanet, helpers)
//   /root/reference/src/qwen4_exp/lowbit.rs:81-241 (Q3/Q2 record layout and packing)
// Loop orders, f32 arithmetic and per-row sequential sums follow the
// reference; output rows of a matvec are spread over OpenMP threads exactly
// where the reference uses rayon (quant.rs:62, cpu.rs:1033-1042), so results
// do not depend on the thread count.  Built with -ffp-contract=off.
//
// Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
// this library, and only as the checker (or the timed CPU baseline).  The
// product path never calls it.
//
// Weights are the seeded synthetic weights of include/cherenkov/synth.h.
// Dense tensors are generated at construction; routed-expert records (the
// reference's experts.bin records, pack.rs:351-393 layout) are generated on
// first use, so a full 48-layer x 512-expert model only materialises the
// records its tokens route to.
//
// Parity pins: every function here is checked by tests/test_oracle_*.py
// against the reference's own known-answer tests (quant.rs, lowbit.rs),
// against brute force / closed forms (top-k, DeltaNet invariants, attention
// with one token), or against an independent numpy restatement; the
// compositions (gated_residual, moe, deltanet, attention, select_tokens,
// mtp_forward, forward_token) by closed forms on special weights
// (tests/test_oracle_compositions.py); PLE (ngram_ids_from, ngram_row, ple)
// by hand-worked id cases and closed forms (tests/test_oracle_ple.py).
// The near-tie route hints (follow_route_hint; test-side, no counterpart in
// the reference) by tests/test_oracle_route_hints.py: an own-set hint is a
// bit-exact no-op, a boundary swap is taken exactly when the tolerance
// covers the gap, far or repeated experts are refused.

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <iterator>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "cherenkov/synth.h"
#include "cherenkov/types.h"

namespace {

constexpr size_t GROUP = 64;
constexpr size_t NIBBLES = 8;
constexpr size_t PAGE = 16384;

thread_local std::string g_err;

inline float bf(uint16_t h) { return chk_bf16_to_f32(h); }

// ---------------------------------------------------------------- nn.rs
// nn::rms_norm, src/nn.rs:6-15
void rms_norm(float* x, const uint16_t* w, size_t n, float eps) {
    float ss = 0.0f;
    for (size_t i = 0; i < n; ++i) ss += x[i] * x[i];
    float ms = ss / (float)n;
    float inv = 1.0f / sqrtf(ms + eps);
    for (size_t i = 0; i < n; ++i) x[i] = x[i] * inv * bf(w[i]);
}
// src/nn.rs:17-24
inline float silu(float v) { return v / (1.0f + expf(-v)); }
inline float sigmoid(float v) { return 1.0f / (1.0f + expf(-v)); }
// src/nn.rs:26-29
inline float softplus(float v) { return v > 20.0f ? v : log1pf(expf(v)); }
// src/nn.rs:32-46
void softmax(float* x, size_t n) {
    float mx = -3.40282347e+38f;  // f32::MIN
    for (size_t i = 0; i < n; ++i) mx = fmaxf(mx, x[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        x[i] = expf(x[i] - mx);
        sum += x[i];
    }
    float inv = 1.0f / sum;
    for (size_t i = 0; i < n; ++i) x[i] *= inv;
}
// src/nn.rs:49-56
void l2_norm(float* x, size_t n, float eps) {
    float ss = 0.0f;
    for (size_t i = 0; i < n; ++i) ss += x[i] * x[i];
    float inv = 1.0f / sqrtf(ss + eps);
    for (size_t i = 0; i < n; ++i) x[i] *= inv;
}

// ---------------------------------------------------------------- quant.rs
struct QL {
    uint32_t out = 0, in = 0;
    const uint32_t* w = nullptr;
    const uint16_t* s = nullptr;
    const uint16_t* b = nullptr;
};

// QLinear::dequant_row, src/quant.rs:24-45
void dequant_row(const QL& q, size_t row, float* dst) {
    size_t wpr = q.in / NIBBLES, gpr = q.in / GROUP;
    const uint32_t* words = q.w + row * wpr;
    const uint16_t* sc = q.s + row * gpr;
    const uint16_t* bi = q.b + row * gpr;
    for (size_t wi = 0; wi < wpr; ++wi) {
        uint32_t word = words[wi];
        size_t base = wi * NIBBLES;
        size_t g = base / GROUP;
        float scale = bf(sc[g]), bias = bf(bi[g]);
        for (size_t j = 0; j < NIBBLES; ++j) {
            uint32_t qv = (word >> (4 * j)) & 0xF;
            dst[base + j] = scale * (float)qv + bias;
        }
    }
}

// QLinear::matvec, src/quant.rs:49-88 (grouped form, rows in parallel)
void matvec(const QL& q, const float* x, float* y) {
    size_t gpr = q.in / GROUP, wpr = q.in / NIBBLES;
    std::vector<float> xs(gpr);
    for (size_t g = 0; g < gpr; ++g) {
        float s = 0.0f;
        for (size_t j = 0; j < GROUP; ++j) s += x[g * GROUP + j];
        xs[g] = s;
    }
    const float* xsums = xs.data();
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)q.out; ++r) {
        const uint32_t* words = q.w + (size_t)r * wpr;
        const uint16_t* sc = q.s + (size_t)r * gpr;
        const uint16_t* bi = q.b + (size_t)r * gpr;
        float acc = 0.0f;
        constexpr size_t WPG = GROUP / NIBBLES;
        for (size_t g = 0; g < gpr; ++g) {
            float qdot = 0.0f;
            const float* xg = x + g * GROUP;
            for (size_t wi = 0; wi < WPG; ++wi) {
                uint32_t word = words[g * WPG + wi];
                const float* xw = xg + wi * NIBBLES;
                for (size_t j = 0; j < NIBBLES; ++j) {
                    uint32_t qv = (word >> (4 * j)) & 0xF;
                    qdot += (float)qv * xw[j];
                }
            }
            acc += bf(sc[g]) * qdot + bf(bi[g]) * xsums[g];
        }
        y[r] = acc;
    }
}

// ---------------------------------------------------------------- lowbit.rs
// q2_slots, src/qwen4_exp/lowbit.rs:143-162
void q2_slots(int t_out[32], uint32_t off_out[32]) {
    for (int c = 0; c < 32; ++c) {
        int t = c / 16, r = c % 16, p, b;
        bool even = r % 2 == 0, low = r < 8;
        if (even && low) { p = 0; b = r / 2; }
        else if (even) { p = 1; b = (r - 8) / 2; }
        else if (low) { p = 2; b = (r - 1) / 2; }
        else { p = 3; b = (r - 9) / 2; }
        t_out[c] = t;
        off_out[c] = (uint32_t)(8 * b + 2 * p);
    }
}
// q3_slots, src/qwen4_exp/lowbit.rs:168-184
void q3_slots(int t_out[32], uint32_t up_out[32], uint32_t lo_out[32]) {
    for (int c = 0; c < 32; ++c) {
        int t = c / 16, r = c % 16, j, b;
        bool even = r % 2 == 0, low = r < 8;
        if (even && low) { j = 0; b = r / 2; }
        else if (even) { j = 1; b = (r - 8) / 2; }
        else if (low) { j = 2; b = (r - 1) / 2; }
        else { j = 3; b = (r - 9) / 2; }
        t_out[c] = t;
        up_out[c] = (uint32_t)(8 * b + 2 * j);
        lo_out[c] = (uint32_t)(8 * b + 4 * t + j);
    }
}
inline uint32_t rd32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
inline void wr32(uint8_t* p, uint32_t v) {
    p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); p[2] = (uint8_t)(v >> 16); p[3] = (uint8_t)(v >> 24);
}
// pack_matrix, src/qwen4_exp/lowbit.rs:188-241
void pack_matrix(const uint8_t* src, size_t codes, uint32_t bits, uint8_t* dst) {
    uint8_t q4[32];
    size_t chunks = codes / 32;
    if (bits == 2) {
        int t[32]; uint32_t off[32];
        q2_slots(t, off);
        for (size_t ch = 0; ch < chunks; ++ch) {
            for (int w = 0; w < 4; ++w) {
                uint32_t word = rd32(src + 4 * (ch * 4 + w));
                for (int j = 0; j < 8; ++j) q4[w * 8 + j] = (uint8_t)((word >> (4 * j)) & 0xF);
            }
            uint32_t pw[2] = {0, 0};
            for (int c = 0; c < 32; ++c) pw[t[c]] |= ((uint32_t)(q4[c] >> 2)) << off[c];
            wr32(dst + ch * 8, pw[0]);
            wr32(dst + ch * 8 + 4, pw[1]);
        }
    } else {
        int t[32]; uint32_t up[32], lo[32];
        q3_slots(t, up, lo);
        for (size_t ch = 0; ch < chunks; ++ch) {
            for (int w = 0; w < 4; ++w) {
                uint32_t word = rd32(src + 4 * (ch * 4 + w));
                for (int j = 0; j < 8; ++j) q4[w * 8 + j] = (uint8_t)((word >> (4 * j)) & 0xF);
            }
            uint32_t uw[2] = {0, 0}, lb = 0;
            for (int c = 0; c < 32; ++c) {
                uint32_t v = q4[c] >> 1;
                uw[t[c]] |= (v >> 1) << up[c];
                lb |= (v & 1u) << lo[c];
            }
            wr32(dst + ch * 12, uw[0]);
            wr32(dst + ch * 12 + 4, uw[1]);
            wr32(dst + ch * 12 + 8, lb);
        }
    }
}

// Low-bit expert matvec.  The reference CPU path has no low-bit matvec (the
// CPU oracle always reads experts.bin); its GPU kernels reconstruct each
// code at the midpoint of the Q4 range it covers, w = (2q + 0.5) s + b (Q3),
// (4q + 1.5) s + b (Q2) (lowbit.rs:6-10; kernels/qwen4_exp/experts.metal:
// 181-296; f64 oracle tests/unit/qwen4_exp/gpu/prefill.rs:177-198).  This
// restates that definition in the grouped form of QLinear::matvec:
// acc += s * sum(mid(q) x) + b * sum(x), decoding codes straight from the
// Q4 words (pack_matrix is pinned separately against the reference's
// round-trip test).
void lowbit_matvec_from_q4(const QL& q, uint32_t bits, const float* x, float* y) {
    size_t gpr = q.in / GROUP, wpr = q.in / NIBBLES;
    uint32_t shift = 4 - bits;
    float step = (float)(1u << shift), half = (float)((1u << shift) - 1) * 0.5f;
    std::vector<float> xs(gpr);
    for (size_t g = 0; g < gpr; ++g) {
        float s = 0.0f;
        for (size_t j = 0; j < GROUP; ++j) s += x[g * GROUP + j];
        xs[g] = s;
    }
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)q.out; ++r) {
        const uint32_t* words = q.w + (size_t)r * wpr;
        float acc = 0.0f;
        for (size_t g = 0; g < gpr; ++g) {
            float qdot = 0.0f;
            for (size_t wi = 0; wi < GROUP / NIBBLES; ++wi) {
                uint32_t word = words[g * (GROUP / NIBBLES) + wi];
                for (size_t j = 0; j < NIBBLES; ++j) {
                    uint32_t code = ((word >> (4 * j)) & 0xF) >> shift;
                    float mid = (float)code * step + half;
                    qdot += mid * x[g * GROUP + wi * NIBBLES + j];
                }
            }
            acc += bf(q.s[(size_t)r * gpr + g]) * qdot + bf(q.b[(size_t)r * gpr + g]) * xs[g];
        }
        y[r] = acc;
    }
}

// ---------------------------------------------------------------- storage
struct QStore {
    std::vector<uint32_t> w;
    std::vector<uint16_t> s, b;
    QL view;
};

void gen_qlinear(QStore& st, uint64_t seed, uint64_t id, uint32_t out, uint32_t in) {
    st.w.resize((size_t)out * in / NIBBLES);
    st.s.resize((size_t)out * in / GROUP);
    st.b.resize((size_t)out * in / GROUP);
    uint64_t kw = chk_key(seed, id, CHK_STREAM_W), ks = chk_key(seed, id, CHK_STREAM_S),
             kb = chk_key(seed, id, CHK_STREAM_B);
    uint32_t* w = st.w.data();
    uint16_t* s = st.s.data();
    uint16_t* b = st.b.data();
    long nw = (long)st.w.size(), ns = (long)st.s.size();
#pragma omp parallel for schedule(static)
    for (long i = 0; i < nw; ++i) w[i] = chk_q4_word(kw, (uint64_t)i);
#pragma omp parallel for schedule(static)
    for (long i = 0; i < ns; ++i) {
        s[i] = chk_normal_bf16(ks, (uint64_t)i, CHK_SCALE_SIGMA);
        b[i] = chk_normal_bf16(kb, (uint64_t)i, CHK_BIAS_SIGMA);
    }
    st.view = QL{out, in, st.w.data(), st.s.data(), st.b.data()};
}

std::vector<uint16_t> gen_bf16(uint64_t seed, uint32_t kind, uint32_t slot, uint32_t part, size_t n) {
    std::vector<uint16_t> v(n);
    uint64_t id = chk_tensor_id(kind, slot, 0, part);
    for (size_t i = 0; i < n; ++i) v[i] = chk_bf16_elem(seed, id, kind, i);
    return v;
}

struct HcW {
    std::vector<uint16_t> norm;
    QStore down, up, inject;
    bool has_inject = false;
};
struct AttnW {
    QStore q, k, v, o, idx;
    std::vector<uint16_t> q_norm, k_norm, idx_q_norm, idx_k_norm;
};
struct DeltaW {
    QStore qkv, z, a, b, out;
    std::vector<uint16_t> conv, a_log, dt_bias, norm;
};
struct MoeW {
    std::vector<uint16_t> router, shared_gate;
    QStore sh_gate, sh_up, sh_down;
    uint32_t record_layer = 0;
};
// PleWeights, src/qwen4_exp/cpu.rs:62-75
struct PleW {
    QStore key, value;
    std::vector<uint16_t> norm_key, norm_query, norm_conv, conv;  // conv [hh][kernel]
    uint32_t kernel = 0, dilation = 0;
    std::vector<int64_t> multipliers;
    std::vector<uint64_t> head_offsets, head_sizes;
};
// ngram.bin rows (NgramLayout, src/qwen4_exp/manifest.rs:42-55)
struct NgramTable {
    std::vector<uint8_t> bytes;
    uint64_t rows = 0, row_bytes = 0;
    uint32_t dim = 0, group = 0;
};
struct LayerW {
    HcW attn_hc, mlp_hc;
    bool linear = false;
    AttnW at;
    DeltaW dn;
    MoeW moe;
    bool has_ple = false;
    PleW ple;
};

struct KvCache {
    std::vector<float> k, v, index_k;
    size_t len = 0;
    // the tokens the latest query attended to (select_tokens' result), for
    // the tests of the engine's selection views
    std::vector<size_t> last_selected;
};
struct DeltaState {
    std::vector<float> s, conv;
};
// PleState, src/qwen4_exp/cpu.rs:302-310: the gvn ring of the dilated conv
struct PleRing {
    std::vector<float> hist;  // [span][hh]
    size_t span = 0, filled = 0;
};

}  // namespace

// Route hints (test-side, no counterpart in the reference): another
// implementation's expert choice per MoE layer for the next forward pass,
// taken only where it departs from this top-k by near-tied experts.
struct RouteHints {
    std::vector<uint32_t> ids;  // [layers + 1][k]; layer index == num_hidden_layers is the MTP layer
    std::vector<uint8_t> set;   // per layer: a hint is present
    float tol = 0.0f;
    uint64_t swaps = 0;         // layers whose routing followed a hint, cumulative
    // the routing each layer took in its latest pass: ids in rank order, softmax
    std::vector<uint32_t> last_ids;
    std::vector<float> last_probs;
};

struct OrcState {
    size_t pos = 0;
    std::vector<uint32_t> tokens;
    std::vector<KvCache> kv;
    std::vector<DeltaState> delta;
    std::vector<float> last_hyper;
    KvCache mtp_kv;
    PleRing ple;
    RouteHints hints;
};

struct OrcModel {
    ChkConfig c{};
    uint32_t expert_bits = 4;
    // per-record precision of the routed experts ([record layer][expert];
    // 0 = expert_bits), the mixed stores of Pool::set_kind
    // (src/qwen4_exp/gpu/residency.rs:298-306)
    std::vector<uint8_t> rec_bits;
    QStore embed, lm_head;
    std::vector<LayerW> layers;
    HcW final_mixer;
    bool has_mtp = false;
    std::vector<uint16_t> mtp_enorm, mtp_hnorm;
    QStore mtp_fc_e, mtp_fc_h;
    LayerW mtp_layer;
    HcW mtp_mixer;
    NgramTable ngram;
    // lazily generated Q4 expert records, pack.rs:351-393 layout
    size_t rec_gate_w = 0, rec_up_w = 0, rec_down_w = 0, rec_gate_s = 0, rec_gate_b = 0,
           rec_up_s = 0, rec_up_b = 0, rec_down_s = 0, rec_down_b = 0, rec_bytes = 0, rec_stride = 0;
    std::mutex mu;
    std::map<uint64_t, std::unique_ptr<std::vector<uint8_t>>> records;

    bool is_linear(uint32_t l) const { return (l + 1) % c.full_attention_interval != 0; }
    uint32_t hh() const { return c.hc_count * c.hidden_size; }

    const uint8_t* record(uint32_t rl, uint32_t e);
    QL expert_view(const uint8_t* rec, int part) const;
};

namespace {

void gen_hc(HcW& w, const ChkConfig& c, uint32_t slot, uint32_t part, bool inject) {
    uint32_t hh = c.hc_count * c.hidden_size;
    w.norm = gen_bf16(c.seed, CHK_T_HC_NORM, slot, part, hh);
    gen_qlinear(w.down, c.seed, chk_tensor_id(CHK_T_HC_DOWN, slot, 0, part), c.hc_lowrank, hh);
    gen_qlinear(w.up, c.seed, chk_tensor_id(CHK_T_HC_UP, slot, 0, part), hh, c.hc_lowrank);
    w.has_inject = inject;
    if (inject) gen_qlinear(w.inject, c.seed, chk_tensor_id(CHK_T_HC_INJECT, slot, 0, part), c.hc_count, hh);
}

void gen_layer(LayerW& L, const ChkConfig& c, uint32_t slot, bool linear, uint32_t record_layer) {
    uint64_t sd = c.seed;
    uint32_t h = c.hidden_size;
    gen_hc(L.attn_hc, c, slot, CHK_HC_ATTN, true);
    gen_hc(L.mlp_hc, c, slot, CHK_HC_MLP, true);
    L.linear = linear;
    if (linear) {
        uint32_t qk = c.linear_num_key_heads * c.linear_key_head_dim;
        uint32_t vd = c.linear_num_value_heads * c.linear_value_head_dim;
        uint32_t conv_dim = 2 * qk + vd;
        gen_qlinear(L.dn.qkv, sd, chk_tensor_id(CHK_T_DN_QKV, slot, 0, 0), conv_dim, h);
        gen_qlinear(L.dn.z, sd, chk_tensor_id(CHK_T_DN_Z, slot, 0, 0), vd, h);
        gen_qlinear(L.dn.a, sd, chk_tensor_id(CHK_T_DN_A, slot, 0, 0), c.linear_num_value_heads, h);
        gen_qlinear(L.dn.b, sd, chk_tensor_id(CHK_T_DN_B, slot, 0, 0), c.linear_num_value_heads, h);
        gen_qlinear(L.dn.out, sd, chk_tensor_id(CHK_T_DN_OUT, slot, 0, 0), h, vd);
        L.dn.conv = gen_bf16(sd, CHK_T_DN_CONV, slot, 0, (size_t)conv_dim * c.linear_conv_kernel_dim);
        L.dn.a_log = gen_bf16(sd, CHK_T_DN_ALOG, slot, 0, c.linear_num_value_heads);
        L.dn.dt_bias = gen_bf16(sd, CHK_T_DN_DTBIAS, slot, 0, c.linear_num_value_heads);
        L.dn.norm = gen_bf16(sd, CHK_T_DN_NORM, slot, 0, c.linear_value_head_dim);
    } else {
        uint32_t hd = c.head_dim;
        gen_qlinear(L.at.q, sd, chk_tensor_id(CHK_T_AT_Q, slot, 0, 0), 2 * c.num_attention_heads * hd, h);
        gen_qlinear(L.at.k, sd, chk_tensor_id(CHK_T_AT_K, slot, 0, 0), c.num_key_value_heads * hd, h);
        gen_qlinear(L.at.v, sd, chk_tensor_id(CHK_T_AT_V, slot, 0, 0), c.num_key_value_heads * hd, h);
        gen_qlinear(L.at.o, sd, chk_tensor_id(CHK_T_AT_O, slot, 0, 0), h, c.num_attention_heads * hd);
        gen_qlinear(L.at.idx, sd, chk_tensor_id(CHK_T_AT_IDX, slot, 0, 0),
                    (c.indexer_n_heads + 1) * c.indexer_head_dim, h);
        L.at.q_norm = gen_bf16(sd, CHK_T_AT_QNORM, slot, 0, hd);
        L.at.k_norm = gen_bf16(sd, CHK_T_AT_KNORM, slot, 0, hd);
        L.at.idx_q_norm = gen_bf16(sd, CHK_T_AT_IDX_QNORM, slot, 0, c.indexer_head_dim);
        L.at.idx_k_norm = gen_bf16(sd, CHK_T_AT_IDX_KNORM, slot, 0, c.indexer_head_dim);
    }
    L.moe.router = gen_bf16(sd, CHK_T_MOE_ROUTER, slot, 0, (size_t)c.num_experts * h);
    L.moe.shared_gate = gen_bf16(sd, CHK_T_MOE_SHARED_GATE, slot, 0, h);
    uint32_t si = c.shared_expert_intermediate_size;
    gen_qlinear(L.moe.sh_gate, sd, chk_tensor_id(CHK_T_MOE_SH_GATE_PROJ, slot, 0, 0), si, h);
    gen_qlinear(L.moe.sh_up, sd, chk_tensor_id(CHK_T_MOE_SH_UP, slot, 0, 0), si, h);
    gen_qlinear(L.moe.sh_down, sd, chk_tensor_id(CHK_T_MOE_SH_DOWN, slot, 0, 0), h, si);
    L.moe.record_layer = record_layer;
}

// The PLE block of decoder layer `slot` (cpu.rs:243-266) and the n-gram
// table's metadata, from the synthetic generator (synth.h).
void gen_ple(PleW& P, const ChkConfig& c, uint32_t slot) {
    const uint64_t sd = c.seed;
    const uint32_t h = c.hidden_size, hh = h * c.hc_count, E = c.ple_embed_dim;
    gen_qlinear(P.key, sd, chk_tensor_id(CHK_T_PLE_KEY, slot, 0, 0), hh, E);
    gen_qlinear(P.value, sd, chk_tensor_id(CHK_T_PLE_VALUE, slot, 0, 0), h, E);
    P.norm_key = gen_bf16(sd, CHK_T_PLE_NORM_KEY, slot, 0, hh);
    P.norm_query = gen_bf16(sd, CHK_T_PLE_NORM_QUERY, slot, 0, hh);
    P.norm_conv = gen_bf16(sd, CHK_T_PLE_NORM_CONV, slot, 0, hh);
    P.conv = gen_bf16(sd, CHK_T_PLE_CONV, slot, 0, (size_t)hh * c.ple_conv_kernel_size);
    P.kernel = c.ple_conv_kernel_size;
    P.dilation = c.ngram_size;
    const uint32_t heads = (c.ngram_size - 1) * c.heads_per_ngram;
    P.multipliers.resize(c.ngram_size);
    for (uint32_t k = 0; k < c.ngram_size; ++k) P.multipliers[k] = chk_ngram_multiplier(sd, k);
    P.head_offsets.resize(heads);
    P.head_sizes.resize(heads);
    uint64_t off = 0;
    for (uint32_t hd = 0; hd < heads; ++hd) {
        P.head_sizes[hd] = chk_ngram_head_size(c.ngram_head_rows, hd);
        P.head_offsets[hd] = off;
        off += P.head_sizes[hd];
    }
}

void gen_ngram(NgramTable& T, const ChkConfig& c, uint64_t rows) {
    const uint32_t heads = (c.ngram_size - 1) * c.heads_per_ngram;
    T.dim = c.ple_embed_dim / heads;
    T.group = c.ngram_group;
    T.rows = rows;
    T.row_bytes = chk_ngram_row_bytes(T.dim, T.group);
    T.bytes.assign(rows * T.row_bytes, 0);
    const uint64_t id = chk_tensor_id(CHK_T_NGRAM_TABLE, 0, 0, 0);
    const uint64_t kw = chk_key(c.seed, id, CHK_STREAM_W), ks = chk_key(c.seed, id, CHK_STREAM_S),
                   kb = chk_key(c.seed, id, CHK_STREAM_B);
    const uint32_t wpr = T.dim / 8, gpr = T.dim / T.group;
    uint8_t* base = T.bytes.data();
    const uint64_t rb = T.row_bytes;
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)rows; ++r) {
        uint8_t* rec = base + (uint64_t)r * rb;
        for (uint32_t j = 0; j < wpr; ++j) {
            const uint32_t w = chk_q4_word(kw, (uint64_t)r * wpr + j);
            memcpy(rec + 4 * j, &w, 4);
        }
        for (uint32_t g = 0; g < gpr; ++g) {
            const uint16_t sv = chk_normal_bf16(ks, (uint64_t)r * gpr + g, CHK_SCALE_SIGMA);
            const uint16_t bv = chk_normal_bf16(kb, (uint64_t)r * gpr + g, CHK_BIAS_SIGMA);
            memcpy(rec + 4 * wpr + 2 * g, &sv, 2);
            memcpy(rec + 4 * wpr + 2 * gpr + 2 * g, &bv, 2);
        }
    }
}

}  // namespace

const uint8_t* OrcModel::record(uint32_t rl, uint32_t e) {
    uint64_t key = ((uint64_t)rl << 32) | e;
    std::lock_guard<std::mutex> g(mu);
    auto it = records.find(key);
    if (it != records.end()) return it->second->data();
    auto rec = std::make_unique<std::vector<uint8_t>>(rec_stride, 0);
    uint8_t* base = rec->data();
    uint32_t I = c.moe_intermediate_size, H = c.hidden_size;
    struct P { size_t w, s, b, words, groups; } parts[3] = {
        {rec_gate_w, rec_gate_s, rec_gate_b, (size_t)I * H / 8, (size_t)I * H / 64},
        {rec_up_w, rec_up_s, rec_up_b, (size_t)I * H / 8, (size_t)I * H / 64},
        {rec_down_w, rec_down_s, rec_down_b, (size_t)H * I / 8, (size_t)H * I / 64}};
    for (uint32_t p = 0; p < 3; ++p) {
        uint64_t id = chk_tensor_id(CHK_T_EXPERT, rl, e, p);
        uint64_t kw = chk_key(c.seed, id, CHK_STREAM_W), ks = chk_key(c.seed, id, CHK_STREAM_S),
                 kb = chk_key(c.seed, id, CHK_STREAM_B);
        uint32_t* w = (uint32_t*)(base + parts[p].w);
        uint16_t* s = (uint16_t*)(base + parts[p].s);
        uint16_t* b = (uint16_t*)(base + parts[p].b);
        long nw = (long)parts[p].words, ng = (long)parts[p].groups;
#pragma omp parallel for schedule(static)
        for (long i = 0; i < nw; ++i) w[i] = chk_q4_word(kw, (uint64_t)i);
#pragma omp parallel for schedule(static)
        for (long i = 0; i < ng; ++i) {
            s[i] = chk_normal_bf16(ks, (uint64_t)i, CHK_SCALE_SIGMA);
            b[i] = chk_normal_bf16(kb, (uint64_t)i, CHK_BIAS_SIGMA);
        }
    }
    const uint8_t* out = base;
    records.emplace(key, std::move(rec));
    return out;
}

// Packed::expert, src/qwen4_exp/packed.rs:198-231
QL OrcModel::expert_view(const uint8_t* rec, int part) const {
    uint32_t I = c.moe_intermediate_size, H = c.hidden_size;
    if (part == 0) return QL{I, H, (const uint32_t*)(rec + rec_gate_w), (const uint16_t*)(rec + rec_gate_s), (const uint16_t*)(rec + rec_gate_b)};
    if (part == 1) return QL{I, H, (const uint32_t*)(rec + rec_up_w), (const uint16_t*)(rec + rec_up_s), (const uint16_t*)(rec + rec_up_b)};
    return QL{H, I, (const uint32_t*)(rec + rec_down_w), (const uint16_t*)(rec + rec_down_s), (const uint16_t*)(rec + rec_down_b)};
}

namespace {

// grouped_rms_norm, src/qwen4_exp/cpu.rs:1012-1027
std::vector<float> grouped_rms_norm(const float* x, const uint16_t* w, size_t n, size_t group, float eps) {
    std::vector<float> out(n, 0.0f);
    for (size_t g = 0; g * group < n; ++g) {
        const float* ch = x + g * group;
        float ss = 0.0f;
        for (size_t i = 0; i < group; ++i) ss += ch[i] * ch[i];
        float ms = ss / (float)group;
        float inv = 1.0f / sqrtf(ms + eps);
        for (size_t i = 0; i < group; ++i) out[g * group + i] = ch[i] * inv * bf(w[g * group + i]);
    }
    return out;
}

// rms_norm_shift, src/qwen4_exp/cpu.rs:999-1008
std::vector<float> rms_norm_shift(const float* x, const uint16_t* w, size_t n, float eps) {
    float ss = 0.0f;
    for (size_t i = 0; i < n; ++i) ss += x[i] * x[i];
    float ms = ss / (float)n;
    float inv = 1.0f / sqrtf(ms + eps);
    std::vector<float> out(n);
    for (size_t i = 0; i < n; ++i) out[i] = x[i] * inv * (1.0f + bf(w[i]));
    return out;
}

// bf16_matvec, src/qwen4_exp/cpu.rs:1029-1043
std::vector<float> bf16_matvec(const uint16_t* w, size_t rows, size_t cols, const float* x) {
    std::vector<float> y(rows);
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)rows; ++r) {
        float s = 0.0f;
        for (size_t j = 0; j < cols; ++j) s += bf(w[(size_t)r * cols + j]) * x[j];
        y[r] = s;
    }
    return y;
}

// bf16_dot, src/qwen4_exp/cpu.rs:1045-1047
float bf16_dot(const uint16_t* w, const float* x, size_t n) {
    float s = 0.0f;
    for (size_t i = 0; i < n; ++i) s += bf(w[i]) * x[i];
    return s;
}

// rope_partial, src/qwen4_exp/cpu.rs:1051-1063
void rope_partial(float* x, size_t pos, size_t rot, float theta) {
    size_t half = rot / 2;
    for (size_t j = 0; j < half; ++j) {
        float inv_freq = powf(theta, -(2.0f * (float)j) / (float)rot);
        float angle = (float)pos * inv_freq;
        float sn = sinf(angle), cs = cosf(angle);
        float a = x[j], b = x[j + half];
        x[j] = a * cs - b * sn;
        x[j + half] = b * cs + a * sn;
    }
}

// causal_conv, src/qwen4_exp/cpu.rs:1067-1085
void causal_conv(float* qkv, size_t n, const uint16_t* weights, float* history, size_t ck) {
    size_t km1 = ck - 1;
    for (size_t ch = 0; ch < n; ++ch) {
        const uint16_t* wrow = weights + ch * ck;
        float* hist = history + ch * km1;
        float cur = qkv[ch];
        float acc = bf(wrow[km1]) * cur;
        for (size_t j = 0; j < km1; ++j) acc += bf(wrow[j]) * hist[j];
        std::rotate(hist, hist + 1, hist + km1);
        hist[km1 - 1] = cur;
        qkv[ch] = silu(acc);
    }
}

// inject, src/qwen4_exp/cpu.rs:971-979
void inject(std::vector<float>& hyper, const std::vector<float>& out, const std::vector<float>& inj) {
    size_t h = out.size();
    for (size_t g = 0; g < inj.size(); ++g)
        for (size_t i = 0; i < h; ++i) hyper[g * h + i] += out[i] * inj[g];
}

// Rust f32::total_cmp as a strict weak order key.
inline int32_t total_key(float f) {
    int32_t i;
    memcpy(&i, &f, 4);
    return i ^ (int32_t)((uint32_t)(i >> 31) >> 1);
}

}  // namespace

namespace orc {

// gated_residual, src/qwen4_exp/cpu.rs:461-502
void gated_residual(const OrcModel& m, const HcW& w, const float* hyper, std::vector<float>& mixed,
                    std::vector<float>& inj) {
    const ChkConfig& c = m.c;
    size_t h = c.hidden_size, hc = c.hc_count;
    float eps = (float)c.rms_norm_eps;
    std::vector<float> normed = grouped_rms_norm(hyper, w.norm.data(), h * hc, h, eps);
    std::vector<float> d(w.down.view.out);
    matvec(w.down.view, normed.data(), d.data());
    for (float& v : d) v = silu(v / (float)hc);
    std::vector<float> u(w.up.view.out);
    matvec(w.up.view, d.data(), u.data());
    mixed.assign(h, 0.0f);
    for (size_t g = 0; g < hc; ++g)
        for (size_t i = 0; i < h; ++i) mixed[i] += sigmoid(u[g * h + i]) * normed[g * h + i];
    for (float& v : mixed) v /= (float)hc;
    inj.clear();
    if (w.has_inject) {
        std::vector<float> r(w.inject.view.out);
        matvec(w.inject.view, normed.data(), r.data());
        for (float v : r) inj.push_back(2.0f * sigmoid(v / (float)hc));
    }
}

// mlp, src/qwen4_exp/cpu.rs:981-997 (with the low-bit variant for Q3/Q2 stores)
std::vector<float> mlp(const QL& gate, const QL& up, const QL& down, const float* x, uint32_t bits) {
    std::vector<float> g(gate.out), u(up.out), out(down.out);
    if (bits == 4) {
        matvec(gate, x, g.data());
        matvec(up, x, u.data());
    } else {
        lowbit_matvec_from_q4(gate, bits, x, g.data());
        lowbit_matvec_from_q4(up, bits, x, u.data());
    }
    for (size_t i = 0; i < g.size(); ++i) g[i] = silu(g[i]) * u[i];
    if (bits == 4) matvec(down, g.data(), out.data());
    else lowbit_matvec_from_q4(down, bits, g.data(), out.data());
    return out;
}

// Routing of moe (src/qwen4_exp/cpu.rs:509-525): sort the softmax
// probabilities by f32::total_cmp descending with the expert index
// ascending on ties, keep the first k, renormalise by their sum when
// norm_topk_prob.
void route_topk(const float* probs, size_t E, size_t k, bool norm, uint32_t* ids, float* wts) {
    std::vector<uint32_t> idx(E);
    for (size_t i = 0; i < E; ++i) idx[i] = (uint32_t)i;
    std::sort(idx.begin(), idx.end(), [&](uint32_t a, uint32_t b) {
        int32_t ka = total_key(probs[a]), kb = total_key(probs[b]);
        if (ka != kb) return ka > kb;
        return a < b;
    });
    float sum = 0.0f;
    for (size_t i = 0; i < k; ++i) sum += probs[idx[i]];
    for (size_t i = 0; i < k; ++i) {
        ids[i] = idx[i];
        wts[i] = norm ? probs[idx[i]] / sum : probs[idx[i]];
    }
}

// One value head of the gated delta rule (src/qwen4_exp/cpu.rs:777-812):
// S <- decay S; kv = S^T k; delta = beta (v - kv); S <- S + k delta^T;
// y = S^T q.  S is [dk][dv] (the CPU order); y is accumulated into yh.
void delta_head_step(float* s, const float* qh, const float* kh, const float* vh, float decay, float beta,
                     size_t dk, size_t dv, float* yh) {
    std::vector<float> kv_mem(dv, 0.0f), delta(dv);
    for (size_t ik = 0; ik < dk; ++ik) {
        float* row = s + ik * dv;
        float kw = kh[ik];
        for (size_t iv = 0; iv < dv; ++iv) {
            row[iv] *= decay;
            kv_mem[iv] += row[iv] * kw;
        }
    }
    for (size_t iv = 0; iv < dv; ++iv) delta[iv] = (vh[iv] - kv_mem[iv]) * beta;
    for (size_t ik = 0; ik < dk; ++ik) {
        float* row = s + ik * dv;
        float kw = kh[ik], qw = qh[ik];
        for (size_t iv = 0; iv < dv; ++iv) {
            row[iv] += kw * delta[iv];
            yh[iv] += row[iv] * qw;
        }
    }
}

// Near-tie routing for the parity tests (no counterpart in the reference).
// Two f32 implementations of the same forward pass agree to rounding, so
// where the k-th and (k+1)-th router probabilities lie within rounding of
// each other they may pick different experts, after which their outputs
// part by far more than rounding.  `hint` is the other implementation's
// choice of k experts: when it differs from this top-k (ids, in rank order)
// only by experts whose probability is within `tol` (relative) of the k-th
// largest, the hinted set is taken, ranked by this model's probabilities
// (index ascending on equal keys) and weighted as route_topk weights its
// set.  Any other difference is a real disagreement and the hint is
// ignored.  Returns whether the routing changed.
bool follow_route_hint(const float* probs, size_t E, size_t k, bool norm, const uint32_t* hint, float tol,
                       uint32_t* ids, float* wts) {
    const float pk = probs[ids[k - 1]];
    std::vector<uint32_t> own(ids, ids + k), other(hint, hint + k);
    std::sort(own.begin(), own.end());
    std::sort(other.begin(), other.end());
    if (own == other) return false;
    if (std::adjacent_find(other.begin(), other.end()) != other.end()) return false;  // duplicate ids
    std::vector<uint32_t> diff;
    std::set_symmetric_difference(own.begin(), own.end(), other.begin(), other.end(), std::back_inserter(diff));
    for (uint32_t e : diff)
        if (e >= E || std::fabs(probs[e] - pk) > tol * pk) return false;
    std::sort(other.begin(), other.end(), [&](uint32_t a, uint32_t b) {
        int32_t ka = total_key(probs[a]), kb = total_key(probs[b]);
        if (ka != kb) return ka > kb;
        return a < b;
    });
    float sum = 0.0f;
    for (size_t i = 0; i < k; ++i) sum += probs[other[i]];
    for (size_t i = 0; i < k; ++i) {
        ids[i] = other[i];
        wts[i] = norm ? probs[other[i]] / sum : probs[other[i]];
    }
    return true;
}

// moe, src/qwen4_exp/cpu.rs:504-541.  Also reports the routing (top ids in
// rank order, renormalised weights, full softmax) for the parity tests.
// `hints`/`layer`: the near-tie hint of that layer, if one is set.
std::vector<float> moe(OrcModel& m, const MoeW& w, const float* x, uint32_t* top_out, float* w_out,
                       float* probs_out, RouteHints* hints = nullptr, size_t layer = 0) {
    const ChkConfig& c = m.c;
    size_t h = c.hidden_size, E = c.num_experts, k = c.num_experts_per_tok;
    std::vector<float> logits = bf16_matvec(w.router.data(), E, h, x);
    softmax(logits.data(), E);
    if (probs_out) memcpy(probs_out, logits.data(), E * 4);
    std::vector<uint32_t> idx(k);
    std::vector<float> wts(k);
    route_topk(logits.data(), E, k, c.norm_topk_prob != 0, idx.data(), wts.data());
    if (hints && layer < hints->set.size() && hints->set[layer] &&
        follow_route_hint(logits.data(), E, k, c.norm_topk_prob != 0, hints->ids.data() + layer * k, hints->tol,
                          idx.data(), wts.data()))
        hints->swaps += 1;
    if (hints) {
        const size_t n = c.num_hidden_layers + 1;
        hints->last_ids.resize(n * k);
        hints->last_probs.resize(n * E);
        std::copy(idx.begin(), idx.end(), hints->last_ids.begin() + layer * k);
        std::copy(logits.begin(), logits.end(), hints->last_probs.begin() + layer * E);
    }
    std::vector<float> out(h, 0.0f);
    for (size_t i = 0; i < k; ++i) {
        uint32_t ei = idx[i];
        float weight = wts[i];
        if (top_out) top_out[i] = ei;
        if (w_out) w_out[i] = weight;
        const uint8_t* rec = m.record(w.record_layer, ei);
        const size_t ri = (size_t)w.record_layer * E + ei;
        const uint32_t bits = ri < m.rec_bits.size() && m.rec_bits[ri] ? m.rec_bits[ri] : m.expert_bits;
        std::vector<float> y = mlp(m.expert_view(rec, 0), m.expert_view(rec, 1), m.expert_view(rec, 2), x, bits);
        for (size_t o = 0; o < h; ++o) out[o] += weight * y[o];
    }
    std::vector<float> shared = mlp(w.sh_gate.view, w.sh_up.view, w.sh_down.view, x, 4);
    float g = sigmoid(bf16_dot(w.shared_gate.data(), x, h));
    for (size_t o = 0; o < h; ++o) out[o] += g * shared[o];
    return out;
}

// The selection tail of select_tokens (cpu.rs:701-716): blocks sorted by
// (score desc, block asc), the first topk kept as token runs, the
// incomplete tail appended, tokens ascending.  Pinned by the reference's
// tie test (tests/unit/qwen4_exp/gpu/qsa.rs:300-372) restated in
// tests/test_oracle.py.
std::vector<size_t> qsa_pick(std::vector<std::pair<float, size_t>> bs, size_t topk, size_t ratio, size_t t_len) {
    const size_t blocks = t_len / ratio;
    std::sort(bs.begin(), bs.end(), [](const std::pair<float, size_t>& a, const std::pair<float, size_t>& b) {
        int32_t ka = total_key(a.first), kb = total_key(b.first);
        if (ka != kb) return ka > kb;
        return a.second < b.second;
    });
    std::vector<size_t> sel;
    for (size_t i = 0; i < topk; ++i)
        for (size_t t = bs[i].second * ratio; t < (bs[i].second + 1) * ratio; ++t) sel.push_back(t);
    for (size_t t = blocks * ratio; t < t_len; ++t) sel.push_back(t);
    std::sort(sel.begin(), sel.end());
    return sel;
}

// select_tokens, src/qwen4_exp/cpu.rs:643-719: dense while the complete
// blocks fit the budget, else block scores (pooled index keys,
// index_k_norm, rope at the block start, relu dots with the normed and
// roped index queries) and qsa_pick.  Scoring is pinned by closed forms
// in tests/test_oracle_compositions.py: block keys along chosen directions
// outside the rotated dims (a tie kept at the lower block, the relu's
// effect), and index queries and keys inside them, where the kept blocks
// follow the relative angle between the query rotated at pos and block b's
// key rotated at b * ratio (and change if either position is wrong).
std::vector<size_t> select_tokens(const OrcModel& m, const AttnW& w, const float* iq, const KvCache& cache,
                                  size_t pos) {
    const ChkConfig& c = m.c;
    size_t t_len = pos + 1, ratio = c.indexer_compress_ratio;
    size_t blocks = t_len / ratio, topk = c.indexer_budget / ratio;
    std::vector<size_t> sel;
    if (blocks <= topk) {
        for (size_t t = 0; t < t_len; ++t) sel.push_back(t);
        return sel;
    }
    size_t ihd = c.indexer_head_dim, inh = c.indexer_n_heads;
    size_t rot = (size_t)((double)c.head_dim * c.partial_rotary_factor);
    float theta = (float)c.rope_theta, eps = (float)c.rms_norm_eps;
    std::vector<float> q(iq, iq + inh * ihd);
    for (size_t hi = 0; hi < inh; ++hi) {
        rms_norm(q.data() + hi * ihd, w.idx_q_norm.data(), ihd, eps);
        rope_partial(q.data() + hi * ihd, pos, rot, theta);
    }
    std::vector<float> pooled(ihd);
    std::vector<std::pair<float, size_t>> bs;
    for (size_t b = 0; b < blocks; ++b) {
        std::fill(pooled.begin(), pooled.end(), 0.0f);
        for (size_t t = b * ratio; t < (b + 1) * ratio; ++t)
            for (size_t d = 0; d < ihd; ++d) pooled[d] += cache.index_k[t * ihd + d];
        for (float& v : pooled) v /= (float)ratio;
        rms_norm(pooled.data(), w.idx_k_norm.data(), ihd, eps);
        rope_partial(pooled.data(), b * ratio, rot, theta);
        float s = 0.0f;
        for (size_t hi = 0; hi < inh; ++hi) {
            float dot = 0.0f;
            for (size_t d = 0; d < ihd; ++d) dot += q[hi * ihd + d] * pooled[d];
            s += fmaxf(dot, 0.0f);
        }
        bs.push_back({s / sqrtf((float)ihd), b});
    }
    return qsa_pick(std::move(bs), topk, ratio, t_len);
}

// attention, src/qwen4_exp/cpu.rs:544-641.  With `kv_q8`, cached K/V rows
// are stored through the engine's int8 rule (d = amax/127 per 32 lanes,
// q = rint(v/d) clamped to +-127, fp16 d; kernels/common/attention.metal:
// 225-233) instead of f32 — the q8-aware restatement the attention parity
// tests compare against.
// The attention core of attention (src/qwen4_exp/cpu.rs:587-633): per q
// head h (kv head h / (nh / nkv)), scores = q.k_t * hd^-1/2 over the
// selected tokens, softmax, o = sum p v_t, then o *= sigmoid(gate).  qg
// holds each head's [q | gate] (2 hd values); k, v are [T][nkv hd].
void attend(const float* qg, const float* kc, const float* vc, const std::vector<size_t>& selected, size_t nh,
            size_t nkv, size_t hd, float* out) {
    size_t kv_row = nkv * hd, group = nh / nkv;
    float scale = powf((float)hd, -0.5f);
    std::vector<float> scores(selected.size());
    for (size_t hi = 0; hi < nh; ++hi) {
        size_t hk = hi / group;
        const float* q = qg + hi * 2 * hd;
        for (size_t si = 0; si < selected.size(); ++si) {
            const float* kt = kc + selected[si] * kv_row + hk * hd;
            float s = 0.0f;
            for (size_t d = 0; d < hd; ++d) s += q[d] * kt[d];
            scores[si] = scale * s;
        }
        softmax(scores.data(), scores.size());
        float* oh = out + hi * hd;
        for (size_t d = 0; d < hd; ++d) oh[d] = 0.0f;
        for (size_t si = 0; si < selected.size(); ++si) {
            const float* vt = vc + selected[si] * kv_row + hk * hd;
            float p = scores[si];
            for (size_t d = 0; d < hd; ++d) oh[d] += p * vt[d];
        }
        const float* gate = qg + hi * 2 * hd + hd;
        for (size_t d = 0; d < hd; ++d) oh[d] *= sigmoid(gate[d]);
    }
}

std::vector<float> attention(const OrcModel& m, const AttnW& w, const float* x, KvCache& cache, size_t pos,
                             bool kv_q8);

// deltanet, src/qwen4_exp/cpu.rs:720-829
std::vector<float> deltanet(const OrcModel& m, const DeltaW& w, const float* x, DeltaState& st) {
    const ChkConfig& c = m.c;
    size_t nk = c.linear_num_key_heads, nv = c.linear_num_value_heads;
    size_t dk = c.linear_key_head_dim, dv = c.linear_value_head_dim;
    size_t qk_dim = nk * dk, v_dim = nv * dv, conv_dim = 2 * qk_dim + v_dim, ck = c.linear_conv_kernel_dim;
    std::vector<float> qkv(conv_dim), gate_input(v_dim), decay_input(nv), beta_input(nv);
    matvec(w.qkv.view, x, qkv.data());
    matvec(w.z.view, x, gate_input.data());
    matvec(w.a.view, x, decay_input.data());
    matvec(w.b.view, x, beta_input.data());
    causal_conv(qkv.data(), conv_dim, w.conv.data(), st.conv.data(), ck);
    std::vector<float> q(qkv.begin(), qkv.begin() + qk_dim);
    std::vector<float> keys(qkv.begin() + qk_dim, qkv.begin() + 2 * qk_dim);
    const float* v = qkv.data() + 2 * qk_dim;
    float qscale = powf((float)dk, -0.5f);
    for (size_t hi = 0; hi < nk; ++hi) {
        float* qh = q.data() + hi * dk;
        l2_norm(qh, dk, 1e-6f);
        for (size_t i = 0; i < dk; ++i) qh[i] *= qscale;
        l2_norm(keys.data() + hi * dk, dk, 1e-6f);
    }
    size_t group = nv / nk;
    std::vector<float> y(v_dim, 0.0f);
    for (size_t hv = 0; hv < nv; ++hv) {
        size_t hk = hv / group;
        float beta = sigmoid(beta_input[hv]);
        float g = -(expf(bf(w.a_log[hv]))) * softplus(decay_input[hv] + bf(w.dt_bias[hv]));
        float decay = expf(g);
        float* yh = y.data() + hv * dv;
        delta_head_step(st.s.data() + hv * dk * dv, q.data() + hk * dk, keys.data() + hk * dk, v + hv * dv, decay,
                        beta, dk, dv, yh);
        rms_norm(yh, w.norm.data(), dv, 1e-6f);
        for (size_t iv = 0; iv < dv; ++iv) yh[iv] *= sigmoid(gate_input[hv * dv + iv]);
    }
    std::vector<float> o(w.out.view.out);
    matvec(w.out.view, y.data(), o.data());
    return o;
}

// IEEE binary16 round-to-nearest-even (the engine stores q8 scales as
// fp16; `half` crate / hardware cvt semantics), then widened back to f32.
inline uint16_t f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) {
        float af;
        memcpy(&af, &ax, 4);
        return (uint16_t)(sign | (uint32_t)rintf(af * 16777216.0f));
    }
    uint32_t h = ((((ax >> 23) - 127 + 15) << 10) | ((ax & 0x7fffffu) >> 13));
    uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}
inline float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
    float v;
    if (e == 0) {
        v = (float)mant * 5.9604645e-8f;
        return sign ? -v : v;
    }
    uint32_t x = sign | (e == 31 ? (0xffu << 23) | (mant << 13) : ((e - 15 + 127) << 23) | (mant << 13));
    memcpy(&v, &x, 4);
    return v;
}
inline float f16_round(float v) { return f16_to_f32(f32_to_f16(v)); }

void q8_roundtrip(float* row, size_t n) {
    for (size_t b = 0; b < n / 32; ++b) {
        float amax = 0.0f;
        for (size_t i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(row[b * 32 + i]));
        float d = amax / 127.0f;
        float dh = f16_round(d);
        for (size_t i = 0; i < 32; ++i) {
            float qv = d > 0.0f ? rintf(row[b * 32 + i] / d) : 0.0f;
            qv = fminf(fmaxf(qv, -127.0f), 127.0f);
            row[b * 32 + i] = qv * dh;
        }
    }
}

std::vector<float> attention(const OrcModel& m, const AttnW& w, const float* x, KvCache& cache, size_t pos,
                             bool kv_q8) {
    const ChkConfig& c = m.c;
    size_t nh = c.num_attention_heads, nkv = c.num_key_value_heads, hd = c.head_dim;
    size_t rot = (size_t)((double)hd * c.partial_rotary_factor);
    float theta = (float)c.rope_theta, eps = (float)c.rms_norm_eps;
    size_t ihd = c.indexer_head_dim, inh = c.indexer_n_heads;
    std::vector<float> qk(w.idx.view.out);
    matvec(w.idx.view, x, qk.data());
    cache.index_k.insert(cache.index_k.end(), qk.begin() + inh * ihd, qk.end());
    std::vector<float> qg(w.q.view.out), k(w.k.view.out), v(w.v.view.out);
    matvec(w.q.view, x, qg.data());
    matvec(w.k.view, x, k.data());
    matvec(w.v.view, x, v.data());
    for (size_t hi = 0; hi < nh; ++hi) {
        float* q = qg.data() + hi * 2 * hd;
        rms_norm(q, w.q_norm.data(), hd, eps);
        rope_partial(q, pos, rot, theta);
    }
    for (size_t hi = 0; hi < nkv; ++hi) {
        float* kh = k.data() + hi * hd;
        rms_norm(kh, w.k_norm.data(), hd, eps);
        rope_partial(kh, pos, rot, theta);
    }
    if (kv_q8) {
        q8_roundtrip(k.data(), k.size());
        q8_roundtrip(v.data(), v.size());
    }
    cache.k.insert(cache.k.end(), k.begin(), k.end());
    cache.v.insert(cache.v.end(), v.begin(), v.end());
    cache.len += 1;
    size_t t_len = cache.len;
    if (t_len != pos + 1) throw std::runtime_error("attention cache out of step");
    std::vector<size_t> selected = select_tokens(m, w, qk.data(), cache, pos);
    cache.last_selected = selected;
    std::vector<float> out(nh * hd, 0.0f);
    attend(qg.data(), cache.k.data(), cache.v.data(), selected, nh, nkv, hd, out.data());
    std::vector<float> o(w.o.view.out);
    matvec(w.o.view, out.data(), o.data());
    return o;
}

// CpuModel::ngram_ids_from, src/qwen4_exp/cpu.rs:848-887: the hashed
// n-gram row ids of the last token of tokens[0..n): bigram heads, then
// trigram heads.  shifted[k] is the token k back, or EOS when that reaches
// before the start or the window [t - k, t) holds an EOS; the products wrap
// like i64 and the head index is the Euclidean remainder.
std::vector<uint64_t> ngram_ids_from(const ChkConfig& c, const std::vector<int64_t>& mult,
                                     const std::vector<uint64_t>& offs, const std::vector<uint64_t>& sizes,
                                     const uint32_t* tokens, size_t n) {
    const uint32_t eos = c.eos_token_id;
    const size_t t = n - 1;
    std::vector<int64_t> shifted(c.ngram_size);
    for (size_t k = 0; k < c.ngram_size; ++k) {
        if (k == 0) {
            shifted[k] = (int64_t)tokens[t];
            continue;
        }
        bool before = t < k;
        for (size_t j = before ? t : t - k; j < t; ++j) before = before || tokens[j] == eos;
        shifted[k] = before ? (int64_t)eos : (int64_t)tokens[t - k];
    }
    std::vector<uint64_t> ids;
    for (size_t ng = 2; ng <= c.ngram_size; ++ng) {
        uint64_t mixed = (uint64_t)shifted[0] * (uint64_t)mult[0];
        for (size_t p = 1; p < ng; ++p) mixed ^= (uint64_t)shifted[p] * (uint64_t)mult[p];
        const int64_t mx = (int64_t)mixed;
        const size_t start = (ng - 2) * c.heads_per_ngram;
        for (size_t h = start; h < start + c.heads_per_ngram; ++h) {
            const int64_t size = (int64_t)sizes[h];
            int64_t r = mx % size;
            if (r < 0) r += size;
            ids.push_back((uint64_t)r + offs[h]);
        }
    }
    return ids;
}

// Packed::ngram_row, src/qwen4_exp/packed.rs:233-256
void ngram_row(const NgramTable& T, uint64_t id, float* dst) {
    if (id >= T.rows) throw std::runtime_error("n-gram id beyond the table");
    const uint8_t* rec = T.bytes.data() + id * T.row_bytes;
    const size_t wb = T.dim / 2, sb = T.dim / T.group * 2;
    for (size_t i = 0; i < T.dim; ++i) {
        const uint32_t word = rd32(rec + i / 8 * 4);
        const uint32_t q = (word >> (4 * (i % 8))) & 0xF;
        const size_t gi = i / T.group;
        const float sc = bf((uint16_t)(rec[wb + 2 * gi] | rec[wb + 2 * gi + 1] << 8));
        const float bi = bf((uint16_t)(rec[wb + sb + 2 * gi] | rec[wb + sb + 2 * gi + 1] << 8));
        dst[i] = sc * (float)q + bi;
    }
}

// CpuModel::ple, src/qwen4_exp/cpu.rs:889-967: the n-gram embedding of the
// current (last) token, key / value projections, per-stream gating of the
// value by sigmoid(sign(dot) sqrt(max(|dot|, 1e-6))) with dot = key_g .
// query_g / sqrt(h), the gated value's grouped RMSNorm (gvn), and the
// dilated causal depthwise conv over the gvn ring with SiLU, added to the
// gated value.  Returns the hc * h addend; `gvn_out` (optional) receives gvn.
std::vector<float> ple(const OrcModel& m, const PleW& w, const float* hyper, OrcState& st,
                       std::vector<float>* gvn_out) {
    const ChkConfig& c = m.c;
    const size_t h = c.hidden_size, hc = c.hc_count, hh = h * hc;
    const float eps = (float)c.rms_norm_eps;
    const size_t dim = m.ngram.dim;
    const std::vector<uint64_t> ids =
        ngram_ids_from(c, w.multipliers, w.head_offsets, w.head_sizes, st.tokens.data(), st.tokens.size());
    if (ids.size() * dim != c.ple_embed_dim) throw std::runtime_error("n-gram head layout mismatch");
    std::vector<float> e(c.ple_embed_dim, 0.0f);
    for (size_t hi = 0; hi < ids.size(); ++hi) ngram_row(m.ngram, ids[hi], e.data() + hi * dim);
    std::vector<float> key(w.key.view.out);
    matvec(w.key.view, e.data(), key.data());
    key = grouped_rms_norm(key.data(), w.norm_key.data(), key.size(), h, eps);
    std::vector<float> value(w.value.view.out);
    matvec(w.value.view, e.data(), value.data());
    const std::vector<float> query = grouped_rms_norm(hyper, w.norm_query.data(), hh, h, eps);
    std::vector<float> gated(hh);
    for (size_t g = 0; g < hc; ++g) {
        // Iterator::sum over f32 starts from -0.0 (Rust 1.98, the reference's
        // toolchain); only an all-(-0.0) sum keeps the sign
        float dot = -0.0f;
        for (size_t i = 0; i < h; ++i) dot += key[g * h + i] * query[g * h + i];
        dot /= sqrtf((float)h);
        const float gate = sqrtf(fmaxf(fabsf(dot), 1e-6f)) * copysignf(1.0f, dot);
        const float sg = sigmoid(gate);
        for (size_t i = 0; i < h; ++i) gated[g * h + i] = sg * value[i];
    }
    const std::vector<float> gvn = grouped_rms_norm(gated.data(), w.norm_conv.data(), hh, h, eps);
    PleRing& ps = st.ple;
    if (ps.span == 0) throw std::runtime_error("PLE state missing");
    const size_t span = ps.span, K = w.kernel;
    std::vector<float> out = gated;
    for (size_t ch = 0; ch < hh; ++ch) {
        const uint16_t* wrow = w.conv.data() + ch * K;
        float acc = bf(wrow[K - 1]) * gvn[ch];
        for (size_t k = 0; k + 1 < K; ++k) {
            const size_t back = (size_t)w.dilation * (K - 1 - k);
            if (back <= ps.filled) {
                const size_t slot = (ps.filled - back) % span;
                acc += bf(wrow[k]) * ps.hist[slot * hh + ch];
            }
        }
        out[ch] += silu(acc);
    }
    const size_t slot = ps.filled % span;
    std::copy(gvn.begin(), gvn.end(), ps.hist.begin() + slot * hh);
    ps.filled += 1;
    if (gvn_out) *gvn_out = gvn;
    return out;
}

}  // namespace orc

// ---------------------------------------------------------------- model
static bool validate(const ChkConfig& c) {
    if (c.hidden_size == 0 || c.hidden_size % 64 || c.hc_count < 2 || c.hc_lowrank % 64 ||
        c.moe_intermediate_size % 64 || c.shared_expert_intermediate_size % 64 ||
        c.full_attention_interval == 0 || c.ple_layer > c.num_hidden_layers) {
        g_err = "unsupported configuration";
        return false;
    }
    if (c.ple_layer) {
        const uint32_t heads = c.ngram_size >= 2 ? (c.ngram_size - 1) * c.heads_per_ngram : 0;
        if (heads == 0 || c.ple_embed_dim % 64 || c.ple_embed_dim % heads || c.ple_conv_kernel_size < 2 ||
            c.ngram_group == 0 || (c.ple_embed_dim / heads) % 8 || (c.ple_embed_dim / heads) % c.ngram_group ||
            c.ngram_head_rows <= heads) {
            g_err = "unsupported PLE configuration";
            return false;
        }
    }
    return true;
}

struct OrcModel* make_model(const ChkConfig* cfg, uint32_t bits) {
    auto m = std::make_unique<OrcModel>();
    m->c = *cfg;
    m->expert_bits = bits;
    const ChkConfig& c = m->c;
    uint32_t H = c.hidden_size, I = c.moe_intermediate_size, L = c.num_hidden_layers;
    size_t w_up = (size_t)I * H / 2, s_up = (size_t)I * (H / 64) * 2, s_down = (size_t)H * (I / 64) * 2;
    size_t off = 0;
    auto take = [&](size_t n) { size_t o = off; off += n; return o; };
    m->rec_gate_w = take(w_up); m->rec_up_w = take(w_up); m->rec_down_w = take(w_up);
    m->rec_gate_s = take(s_up); m->rec_gate_b = take(s_up); m->rec_up_s = take(s_up); m->rec_up_b = take(s_up);
    m->rec_down_s = take(s_down); m->rec_down_b = take(s_down);
    m->rec_bytes = off;
    m->rec_stride = (off + PAGE - 1) / PAGE * PAGE;
    gen_qlinear(m->embed, c.seed, chk_tensor_id(CHK_T_EMBED, 0, 0, 0), c.vocab_size, H);
    gen_qlinear(m->lm_head, c.seed, chk_tensor_id(CHK_T_LM_HEAD, 0, 0, 0), c.vocab_size, H);
    m->layers.resize(L);
    for (uint32_t l = 0; l < L; ++l) gen_layer(m->layers[l], c, l, m->is_linear(l), l);
    if (c.ple_layer) {
        LayerW& PL = m->layers[c.ple_layer - 1];
        PL.has_ple = true;
        gen_ple(PL.ple, c, c.ple_layer - 1);
        uint64_t rows = 0;
        for (uint64_t v : PL.ple.head_sizes) rows += v;
        gen_ngram(m->ngram, c, rows);
    }
    gen_hc(m->final_mixer, c, 0, CHK_HC_FINAL, false);
    m->has_mtp = c.mtp_num_hidden_layers > 0;
    if (m->has_mtp) {
        m->mtp_enorm = gen_bf16(c.seed, CHK_T_MTP_ENORM, L, 0, H);
        m->mtp_hnorm = gen_bf16(c.seed, CHK_T_MTP_HNORM, L, 0, (size_t)c.hc_count * H);
        gen_qlinear(m->mtp_fc_e, c.seed, chk_tensor_id(CHK_T_MTP_FC_E, L, 0, 0), H, H);
        gen_qlinear(m->mtp_fc_h, c.seed, chk_tensor_id(CHK_T_MTP_FC_H, L, 0, 0), H, H);
        gen_layer(m->mtp_layer, c, L, false, L);
        gen_hc(m->mtp_mixer, c, L, CHK_HC_MTP, false);
    }
    return m.release();
}

extern "C" {

const char* orc_last_error(void) { return g_err.c_str(); }

// qsa_pick over given block scores: vis receives the visible tokens
// (capacity topk * ratio + ratio), *nvis their count.
void orc_qsa_pick(const float* scores, uint32_t t_len, uint32_t topk, uint32_t ratio, uint32_t* vis, uint32_t* nvis) {
    const size_t blocks = t_len / ratio;
    std::vector<std::pair<float, size_t>> bs;
    for (size_t b = 0; b < blocks; ++b) bs.push_back({scores[b], b});
    const std::vector<size_t> sel = orc::qsa_pick(std::move(bs), topk, ratio, t_len);
    for (size_t i = 0; i < sel.size(); ++i) vis[i] = (uint32_t)sel[i];
    *nvis = (uint32_t)sel.size();
}

void* orc_model_new(const ChkConfig* cfg, uint32_t expert_bits) {
    if (!validate(*cfg) || (expert_bits != 2 && expert_bits != 3 && expert_bits != 4)) {
        if (g_err.empty()) g_err = "expert bits must be 2, 3 or 4";
        return nullptr;
    }
    try {
        return make_model(cfg, expert_bits);
    } catch (const std::exception& e) {
        g_err = e.what();
        return nullptr;
    }
}

void orc_model_free(void* m) { delete (OrcModel*)m; }

// CpuModel::new_state, src/qwen4_exp/cpu.rs:276-321
void* orc_state_new(void* mp) {
    OrcModel* m = (OrcModel*)mp;
    const ChkConfig& c = m->c;
    auto st = new OrcState();
    for (uint32_t l = 0; l < c.num_hidden_layers; ++l) {
        if (m->is_linear(l)) {
            DeltaState d;
            d.s.assign((size_t)c.linear_num_value_heads * c.linear_key_head_dim * c.linear_value_head_dim, 0.0f);
            d.conv.assign((size_t)(2 * c.linear_num_key_heads * c.linear_key_head_dim +
                                   c.linear_num_value_heads * c.linear_value_head_dim) *
                              (c.linear_conv_kernel_dim - 1),
                          0.0f);
            st->delta.push_back(std::move(d));
        } else {
            st->kv.emplace_back();
        }
    }
    if (c.ple_layer) {
        st->ple.span = (size_t)(c.ple_conv_kernel_size - 1) * c.ngram_size;
        st->ple.hist.assign(st->ple.span * c.hc_count * c.hidden_size, 0.0f);
    }
    return st;
}

void orc_state_free(void* s) { delete (OrcState*)s; }

// A synthetic sequence of n positions for timing decode at a long context
// (the CPU baseline of bench.py): every attention cache gets n rows of
// seeded N(0, 1) keys, values and index keys, the DeltaNet states small
// seeded values; no tokens are run.  Not a parity path.
int orc_state_fill_prefix(void* mp, void* sp, uint32_t n, uint64_t seed) {
    OrcModel* m = (OrcModel*)mp;
    OrcState* st = (OrcState*)sp;
    const ChkConfig& c = m->c;
    const size_t kv_row = (size_t)c.num_key_value_heads * c.head_dim;
    uint64_t key = chk_key(seed, 0x5eed, CHK_STREAM_S);
    uint64_t i = 0;
    auto next = [&](float sigma) { return chk_bf16_to_f32(chk_normal_bf16(key, i++, sigma)); };
    for (auto& kv : st->kv) {
        kv.k.resize(n * kv_row);
        kv.v.resize(n * kv_row);
        kv.index_k.resize((size_t)n * c.indexer_head_dim);
        for (auto& x : kv.k) x = next(1.0f);
        for (auto& x : kv.v) x = next(1.0f);
        for (auto& x : kv.index_k) x = next(1.0f);
        kv.len = n;
    }
    if (m->has_mtp) {
        st->mtp_kv.k.assign(n * kv_row, 0.0f);
        st->mtp_kv.v.assign(n * kv_row, 0.0f);
        st->mtp_kv.index_k.assign((size_t)n * c.indexer_head_dim, 0.0f);
        st->mtp_kv.len = n;
    }
    for (auto& d : st->delta)
        for (auto& x : d.s) x = next(0.01f);
    st->pos = n;
    st->tokens.assign(n, 0);
    return 0;
}

uint32_t orc_state_pos(void* s) { return (uint32_t)((OrcState*)s)->pos; }

// CpuModel::forward_token, src/qwen4_exp/cpu.rs:392-456.  `kv_q8` selects
// the q8-aware KV cache (see orc::attention).
int orc_forward_token(void* mp, void* sp, uint32_t token, int kv_q8, float* logits) {
    OrcModel* m = (OrcModel*)mp;
    OrcState* st = (OrcState*)sp;
    const ChkConfig& c = m->c;
    try {
        if (token >= c.vocab_size) throw std::runtime_error("token out of range");
        size_t h = c.hidden_size, hc = c.hc_count, hh = h * hc;
        std::vector<float> e(h);
        dequant_row(m->embed.view, token, e.data());
        std::vector<float> hyper(hh);
        for (size_t g = 0; g < hc; ++g) memcpy(hyper.data() + g * h, e.data(), h * 4);
        st->tokens.push_back(token);
        size_t kv_idx = 0, delta_idx = 0, li = 0;
        std::vector<float> mixed, inj;
        for (auto& layer : m->layers) {
            if (layer.has_ple) {
                const std::vector<float> add = orc::ple(*m, layer.ple, hyper.data(), *st, nullptr);
                for (size_t i = 0; i < hh; ++i) hyper[i] += add[i];
            }
            orc::gated_residual(*m, layer.attn_hc, hyper.data(), mixed, inj);
            std::vector<float> out;
            if (layer.linear) out = orc::deltanet(*m, layer.dn, mixed.data(), st->delta[delta_idx++]);
            else out = orc::attention(*m, layer.at, mixed.data(), st->kv[kv_idx++], st->pos, kv_q8 != 0);
            inject(hyper, out, inj);
            orc::gated_residual(*m, layer.mlp_hc, hyper.data(), mixed, inj);
            out = orc::moe(*m, layer.moe, mixed.data(), nullptr, nullptr, nullptr, &st->hints, li++);
            inject(hyper, out, inj);
        }
        if (!st->hints.set.empty()) std::fill(st->hints.set.begin(), st->hints.set.begin() + c.num_hidden_layers, 0);
        st->pos += 1;
        st->last_hyper = hyper;
        orc::gated_residual(*m, m->final_mixer, hyper.data(), mixed, inj);
        matvec(m->lm_head.view, mixed.data(), logits);
        return 0;
    } catch (const std::exception& ex) {
        g_err = ex.what();
        return -1;
    }
}

// The tokens the latest query of attention layer `layer` (a decoder layer
// index; num_hidden_layers: the MTP layer) attended to, ascending.
int orc_state_last_selection(void* mp, void* sp, uint32_t layer, uint32_t* out, uint32_t cap, uint32_t* n) {
    OrcModel* m = (OrcModel*)mp;
    OrcState* st = (OrcState*)sp;
    const KvCache* kc = nullptr;
    if (layer == m->c.num_hidden_layers && m->has_mtp) {
        kc = &st->mtp_kv;
    } else if (layer < m->c.num_hidden_layers && !m->layers[layer].linear) {
        size_t ki = 0;
        for (uint32_t l = 0; l < layer; ++l) ki += m->layers[l].linear ? 0 : 1;
        kc = &st->kv[ki];
    } else {
        g_err = "not an attention layer";
        return -1;
    }
    *n = (uint32_t)kc->last_selected.size();
    for (uint32_t i = 0; i < std::min<uint32_t>(*n, cap); ++i) out[i] = (uint32_t)kc->last_selected[i];
    return 0;
}

// Near-tie route hints for the next forward_token / mtp_forward (see
// follow_route_hint): ids[layers][k] for `layers` consecutive layers from
// layer 0 (num_hidden_layers + 1 includes the MTP layer), used once.
int orc_state_route_hints(void* mp, void* sp, const uint32_t* ids, uint32_t layers, float tol) {
    OrcModel* m = (OrcModel*)mp;
    OrcState* st = (OrcState*)sp;
    const size_t k = m->c.num_experts_per_tok, n = m->c.num_hidden_layers + 1;
    if (layers > n) { g_err = "more hinted layers than the model has"; return -1; }
    if (!(tol >= 0.0f)) { g_err = "tolerance must be >= 0"; return -1; }
    st->hints.ids.assign(n * k, 0);
    st->hints.set.assign(n, 0);
    std::copy(ids, ids + (size_t)layers * k, st->hints.ids.begin());
    std::fill(st->hints.set.begin(), st->hints.set.begin() + layers, 1);
    st->hints.tol = tol;
    return 0;
}

uint64_t orc_state_route_swaps(void* sp) { return ((OrcState*)sp)->hints.swaps; }

// The routing layer `layer` took in the state's latest pass: k ids in rank
// order and the E softmax probabilities (either output may be null).
int orc_state_last_routes(void* mp, void* sp, uint32_t layer, uint32_t* ids, float* probs) {
    OrcModel* m = (OrcModel*)mp;
    OrcState* st = (OrcState*)sp;
    const size_t k = m->c.num_experts_per_tok, E = m->c.num_experts;
    if ((size_t)layer * k >= st->hints.last_ids.size()) { g_err = "no routing recorded for that layer"; return -1; }
    if (ids) std::copy_n(st->hints.last_ids.begin() + (size_t)layer * k, k, ids);
    if (probs) std::copy_n(st->hints.last_probs.begin() + (size_t)layer * E, E, probs);
    return 0;
}

int orc_state_last_hyper(void* sp, float* out, size_t n) {
    OrcState* st = (OrcState*)sp;
    if (st->last_hyper.size() != n) { g_err = "hyper width"; return -1; }
    memcpy(out, st->last_hyper.data(), n * 4);
    return 0;
}

// CpuModel::mtp_forward, src/qwen4_exp/cpu.rs:328-389
int orc_mtp_forward(void* mp, void* sp, uint32_t token, const float* hyper_in, uint32_t pos, int kv_q8,
                    float* logits, float* hyper_out) {
    OrcModel* m = (OrcModel*)mp;
    OrcState* st = (OrcState*)sp;
    const ChkConfig& c = m->c;
    try {
        if (!m->has_mtp) throw std::runtime_error("no MTP head");
        size_t h = c.hidden_size, hc = c.hc_count;
        float eps = (float)c.rms_norm_eps;
        std::vector<float> e(h);
        dequant_row(m->embed.view, token, e.data());
        std::vector<float> en = rms_norm_shift(e.data(), m->mtp_enorm.data(), h, eps);
        std::vector<float> fe(h), fh(h), hyper(h * hc);
        matvec(m->mtp_fc_e.view, en.data(), fe.data());
        for (size_t g = 0; g < hc; ++g) {
            std::vector<float> hn = rms_norm_shift(hyper_in + g * h, m->mtp_hnorm.data() + g * h, h, eps);
            matvec(m->mtp_fc_h.view, hn.data(), fh.data());
            for (size_t i = 0; i < h; ++i) hyper[g * h + i] = fe[i] + fh[i];
        }
        LayerW& layer = m->mtp_layer;
        std::vector<float> mixed, inj;
        orc::gated_residual(*m, layer.attn_hc, hyper.data(), mixed, inj);
        std::vector<float> out = orc::attention(*m, layer.at, mixed.data(), st->mtp_kv, pos, kv_q8 != 0);
        inject(hyper, out, inj);
        orc::gated_residual(*m, layer.mlp_hc, hyper.data(), mixed, inj);
        out = orc::moe(*m, layer.moe, mixed.data(), nullptr, nullptr, nullptr, &st->hints, c.num_hidden_layers);
        if (st->hints.set.size() > c.num_hidden_layers) st->hints.set[c.num_hidden_layers] = 0;
        inject(hyper, out, inj);
        orc::gated_residual(*m, m->mtp_mixer, hyper.data(), mixed, inj);
        matvec(m->lm_head.view, mixed.data(), logits);
        if (hyper_out) memcpy(hyper_out, hyper.data(), hyper.size() * 4);
        return 0;
    } catch (const std::exception& ex) {
        g_err = ex.what();
        return -1;
    }
}

// ---- block-level entry points (the configs' isolated blocks) ----

static LayerW* layer_of(OrcModel* m, uint32_t layer) {
    if (layer < m->c.num_hidden_layers) return &m->layers[layer];
    if (layer == m->c.num_hidden_layers && m->has_mtp) return &m->mtp_layer;
    return nullptr;
}

// The MoE block on an already-normalised input x[h]; reports routing.
// The precision of one routed-expert record (4, 3 or 2 bits; 0 restores
// the model's expert_bits).
int orc_set_record_bits(void* mp, uint32_t record_layer, uint32_t e, uint32_t bits) {
    OrcModel* m = (OrcModel*)mp;
    const size_t E = m->c.num_experts, n = (m->c.num_hidden_layers + 1) * E;
    if (record_layer > m->c.num_hidden_layers || e >= E || (bits && bits != 2 && bits != 3 && bits != 4)) {
        g_err = "record or bits out of range";
        return -1;
    }
    if (m->rec_bits.size() != n) m->rec_bits.assign(n, 0);
    m->rec_bits[(size_t)record_layer * E + e] = (uint8_t)bits;
    return 0;
}

int orc_moe(void* mp, uint32_t layer, const float* x, float* out, uint32_t* top_idx, float* top_w, float* probs) {
    OrcModel* m = (OrcModel*)mp;
    LayerW* L = layer_of(m, layer);
    if (!L) { g_err = "layer out of range"; return -1; }
    std::vector<float> o = orc::moe(*m, L->moe, x, top_idx, top_w, probs);
    memcpy(out, o.data(), o.size() * 4);
    return 0;
}

int orc_gated_residual(void* mp, uint32_t layer, uint32_t which, const float* hyper, float* mixed_out,
                       float* inj_out) {
    OrcModel* m = (OrcModel*)mp;
    const HcW* w = nullptr;
    if (which == CHK_HC_FINAL) w = &m->final_mixer;
    else if (which == CHK_HC_MTP) w = m->has_mtp ? &m->mtp_mixer : nullptr;
    else {
        LayerW* L = layer_of(m, layer);
        if (L) w = which == CHK_HC_ATTN ? &L->attn_hc : &L->mlp_hc;
    }
    if (!w) { g_err = "no such hyper-connection"; return -1; }
    std::vector<float> mixed, inj;
    orc::gated_residual(*m, *w, hyper, mixed, inj);
    memcpy(mixed_out, mixed.data(), mixed.size() * 4);
    if (inj_out) memcpy(inj_out, inj.data(), inj.size() * 4);
    return 0;
}

// One DeltaNet mixer call on decoder layer `layer` with state from `sp`.
int orc_deltanet(void* mp, void* sp, uint32_t layer, const float* x, float* out) {
    OrcModel* m = (OrcModel*)mp;
    OrcState* st = (OrcState*)sp;
    if (layer >= m->c.num_hidden_layers || !m->is_linear(layer)) { g_err = "not a DeltaNet layer"; return -1; }
    size_t di = 0;
    for (uint32_t l = 0; l < layer; ++l) di += m->is_linear(l) ? 1 : 0;
    std::vector<float> o = orc::deltanet(*m, m->layers[layer].dn, x, st->delta[di]);
    memcpy(out, o.data(), o.size() * 4);
    return 0;
}

int orc_delta_state(void* mp, void* sp, uint32_t layer, float* s_out, float* conv_out) {
    OrcModel* m = (OrcModel*)mp;
    OrcState* st = (OrcState*)sp;
    if (layer >= m->c.num_hidden_layers || !m->is_linear(layer)) { g_err = "not a DeltaNet layer"; return -1; }
    size_t di = 0;
    for (uint32_t l = 0; l < layer; ++l) di += m->is_linear(l) ? 1 : 0;
    if (s_out) memcpy(s_out, st->delta[di].s.data(), st->delta[di].s.size() * 4);
    if (conv_out) memcpy(conv_out, st->delta[di].conv.data(), st->delta[di].conv.size() * 4);
    return 0;
}

// One attention mixer call at `pos` (the state's cache must hold pos rows).
int orc_attention(void* mp, void* sp, uint32_t layer, const float* x, uint32_t pos, int kv_q8, float* out) {
    OrcModel* m = (OrcModel*)mp;
    OrcState* st = (OrcState*)sp;
    try {
        if (layer >= m->c.num_hidden_layers || m->is_linear(layer)) throw std::runtime_error("not an attention layer");
        size_t ki = 0;
        for (uint32_t l = 0; l < layer; ++l) ki += m->is_linear(l) ? 0 : 1;
        std::vector<float> o = orc::attention(*m, m->layers[layer].at, x, st->kv[ki], pos, kv_q8 != 0);
        memcpy(out, o.data(), o.size() * 4);
        return 0;
    } catch (const std::exception& ex) {
        g_err = ex.what();
        return -1;
    }
}

// Attention at position T over an explicit cache of T rows (k, v f32
// [T][nkv * hd]; passed through the q8 rule when kv_q8): the isolated
// attention-decode block (configs with a prefilled KV cache).
int orc_attention_kv(void* mp, uint32_t layer, const float* x, uint32_t rows, const float* k, const float* v, uint32_t T,
                     int kv_q8, float* out) {
    OrcModel* m = (OrcModel*)mp;
    try {
        if (layer >= m->c.num_hidden_layers || m->is_linear(layer)) throw std::runtime_error("not an attention layer");
        size_t kv_row = (size_t)m->c.num_key_value_heads * m->c.head_dim;
        KvCache cache;
        cache.k.assign(k, k + (size_t)T * kv_row);
        cache.v.assign(v, v + (size_t)T * kv_row);
        if (kv_q8) {
            for (size_t t = 0; t < T; ++t) {
                orc::q8_roundtrip(cache.k.data() + t * kv_row, kv_row);
                orc::q8_roundtrip(cache.v.data() + t * kv_row, kv_row);
            }
        }
        cache.index_k.assign((size_t)T * m->c.indexer_head_dim, 0.0f);
        cache.len = T;
        // rows r > 0 are later positions of the same sequence: each appends
        // its own K/V before the next attends (a verify batch)
        size_t H = m->c.hidden_size;
        for (uint32_t r = 0; r < rows; ++r) {
            std::vector<float> o = orc::attention(*m, m->layers[layer].at, x + r * H, cache, T + r, kv_q8 != 0);
            memcpy(out + r * H, o.data(), o.size() * 4);
        }
        return 0;
    } catch (const std::exception& ex) {
        g_err = ex.what();
        return -1;
    }
}

// ---- primitives exposed for the known-answer tests ----

void orc_q4_matvec(const uint32_t* w, const uint16_t* s, const uint16_t* b, uint32_t out, uint32_t in,
                   const float* x, float* y) {
    matvec(QL{out, in, w, s, b}, x, y);
}

void orc_q4_dequant_row(const uint32_t* w, const uint16_t* s, const uint16_t* b, uint32_t out, uint32_t in,
                        uint32_t row, float* dst) {
    dequant_row(QL{out, in, w, s, b}, row, dst);
}

void orc_lowbit_matvec(const uint32_t* w, const uint16_t* s, const uint16_t* b, uint32_t out, uint32_t in,
                       uint32_t bits, const float* x, float* y) {
    lowbit_matvec_from_q4(QL{out, in, w, s, b}, bits, x, y);
}

void orc_pack_matrix(const uint8_t* src, uint64_t codes, uint32_t bits, uint8_t* dst) {
    pack_matrix(src, (size_t)codes, bits, dst);
}

void orc_q2_slots(int32_t* t, uint32_t* off) {
    int tt[32];
    uint32_t oo[32];
    q2_slots(tt, oo);
    for (int i = 0; i < 32; ++i) { t[i] = tt[i]; off[i] = oo[i]; }
}

void orc_q3_slots(int32_t* t, uint32_t* up, uint32_t* lo) {
    int tt[32];
    uint32_t uu[32], ll[32];
    q3_slots(tt, uu, ll);
    for (int i = 0; i < 32; ++i) { t[i] = tt[i]; up[i] = uu[i]; lo[i] = ll[i]; }
}

void orc_softmax(float* x, uint32_t n) { softmax(x, n); }
void orc_rms_norm(float* x, const uint16_t* w, uint32_t n, float eps) { rms_norm(x, w, n, eps); }
void orc_l2_norm(float* x, uint32_t n, float eps) { l2_norm(x, n, eps); }
void orc_rope_partial(float* x, uint32_t pos, uint32_t rot, float theta) { rope_partial(x, pos, rot, theta); }
float orc_softplus(float v) { return softplus(v); }
void orc_attend(const float* qg, const float* k, const float* v, uint32_t T, uint32_t nh, uint32_t nkv, uint32_t hd,
                float* out) {
    std::vector<size_t> all(T);
    for (uint32_t t = 0; t < T; ++t) all[t] = t;
    orc::attend(qg, k, v, all, nh, nkv, hd, out);
}
void orc_route_topk(const float* probs, uint32_t E, uint32_t k, int norm, uint32_t* ids, float* wts) {
    orc::route_topk(probs, E, k, norm != 0, ids, wts);
}
void orc_delta_head_step(float* s, const float* q, const float* k, const float* v, float decay, float beta,
                         uint32_t dk, uint32_t dv, float* y) {
    orc::delta_head_step(s, q, k, v, decay, beta, dk, dv, y);
}
void orc_q8_roundtrip(float* row, uint32_t n) { orc::q8_roundtrip(row, n); }
uint16_t orc_f32_to_f16(float v) { return orc::f32_to_f16(v); }
void orc_causal_conv(float* qkv, uint32_t n, const uint16_t* w, float* hist, uint32_t ck) {
    causal_conv(qkv, n, w, hist, ck);
}

// ---- weight access (to check the device generator byte for byte) ----

// Copies the Q4 record (layer, expert) into dst[rec_stride].
int orc_expert_record(void* mp, uint32_t record_layer, uint32_t e, uint8_t* dst, uint64_t cap) {
    OrcModel* m = (OrcModel*)mp;
    if (cap < m->rec_stride) { g_err = "buffer too small"; return -1; }
    memcpy(dst, m->record(record_layer, e), m->rec_stride);
    return 0;
}

uint64_t orc_record_stride(void* mp) { return ((OrcModel*)mp)->rec_stride; }

// ---- weight overrides (the closed-form pins of tests/test_oracle.py) ----
// Replace one tensor of the synthetic model with caller-given values of
// the same shape, so a composed function can be run on special weights
// whose result has a closed form.  `layer` selects the decoder layer
// (num_hidden_layers: the MTP layer); model-level tensors ignore it.
static HcW* hc_of(OrcModel* m, uint32_t layer, const std::string& grp) {
    if (grp == "final") return &m->final_mixer;
    if (grp == "mtp_mixer") return &m->mtp_mixer;
    LayerW* L = layer_of(m, layer);
    if (!L) return nullptr;
    if (grp == "attn_hc") return &L->attn_hc;
    if (grp == "mlp_hc") return &L->mlp_hc;
    return nullptr;
}

static QStore* q4_of(OrcModel* m, uint32_t layer, const std::string& name) {
    if (name == "embed") return &m->embed;
    if (name == "lm_head") return &m->lm_head;
    if (name == "mtp.fc_e") return &m->mtp_fc_e;
    if (name == "mtp.fc_h") return &m->mtp_fc_h;
    const size_t dot = name.find('.');
    if (dot == std::string::npos) return nullptr;
    const std::string grp = name.substr(0, dot), t = name.substr(dot + 1);
    if (HcW* h = hc_of(m, layer, grp)) {
        if (t == "down") return &h->down;
        if (t == "up") return &h->up;
        if (t == "inject") return h->has_inject ? &h->inject : nullptr;
        return nullptr;
    }
    LayerW* L = layer_of(m, layer);
    if (!L) return nullptr;
    if (grp == "dn" && L->linear) {
        if (t == "qkv") return &L->dn.qkv;
        if (t == "z") return &L->dn.z;
        if (t == "a") return &L->dn.a;
        if (t == "b") return &L->dn.b;
        if (t == "out") return &L->dn.out;
    }
    if (grp == "at" && !L->linear) {
        if (t == "q") return &L->at.q;
        if (t == "k") return &L->at.k;
        if (t == "v") return &L->at.v;
        if (t == "o") return &L->at.o;
        if (t == "idx") return &L->at.idx;
    }
    if (grp == "ple" && L->has_ple) {
        if (t == "key") return &L->ple.key;
        if (t == "value") return &L->ple.value;
    }
    if (grp == "moe") {
        if (t == "sh_gate") return &L->moe.sh_gate;
        if (t == "sh_up") return &L->moe.sh_up;
        if (t == "sh_down") return &L->moe.sh_down;
    }
    return nullptr;
}

static std::vector<uint16_t>* bf16_of(OrcModel* m, uint32_t layer, const std::string& name) {
    if (name == "mtp.enorm") return &m->mtp_enorm;
    if (name == "mtp.hnorm") return &m->mtp_hnorm;
    const size_t dot = name.find('.');
    if (dot == std::string::npos) return nullptr;
    const std::string grp = name.substr(0, dot), t = name.substr(dot + 1);
    if (HcW* h = hc_of(m, layer, grp)) return t == "norm" ? &h->norm : nullptr;
    LayerW* L = layer_of(m, layer);
    if (!L) return nullptr;
    if (grp == "dn" && L->linear) {
        if (t == "conv") return &L->dn.conv;
        if (t == "a_log") return &L->dn.a_log;
        if (t == "dt_bias") return &L->dn.dt_bias;
        if (t == "norm") return &L->dn.norm;
    }
    if (grp == "at" && !L->linear) {
        if (t == "q_norm") return &L->at.q_norm;
        if (t == "k_norm") return &L->at.k_norm;
        if (t == "idx_q_norm") return &L->at.idx_q_norm;
        if (t == "idx_k_norm") return &L->at.idx_k_norm;
    }
    if (grp == "ple" && L->has_ple) {
        if (t == "norm_key") return &L->ple.norm_key;
        if (t == "norm_query") return &L->ple.norm_query;
        if (t == "norm_conv") return &L->ple.norm_conv;
        if (t == "conv") return &L->ple.conv;
    }
    if (grp == "moe") {
        if (t == "router") return &L->moe.router;
        if (t == "shared_gate") return &L->moe.shared_gate;
    }
    return nullptr;
}

int orc_set_q4(void* mp, uint32_t layer, const char* name, const uint32_t* w, const uint16_t* s, const uint16_t* b,
               uint64_t n_words) {
    OrcModel* m = (OrcModel*)mp;
    QStore* q = q4_of(m, layer, name);
    if (!q) {
        g_err = std::string("no Q4 tensor ") + name;
        return -1;
    }
    if (n_words != q->w.size()) {
        g_err = std::string("shape mismatch for ") + name;
        return -1;
    }
    std::copy(w, w + q->w.size(), q->w.begin());
    std::copy(s, s + q->s.size(), q->s.begin());
    std::copy(b, b + q->b.size(), q->b.begin());
    return 0;
}

int orc_set_bf16(void* mp, uint32_t layer, const char* name, const uint16_t* v, uint64_t n) {
    OrcModel* m = (OrcModel*)mp;
    std::vector<uint16_t>* t = bf16_of(m, layer, name);
    if (!t) {
        g_err = std::string("no bf16 tensor ") + name;
        return -1;
    }
    if (n != t->size()) {
        g_err = std::string("shape mismatch for ") + name;
        return -1;
    }
    std::copy(v, v + n, t->begin());
    return 0;
}

// Read one tensor back (the packed-store writer of the tests).
int orc_get_q4(void* mp, uint32_t layer, const char* name, uint32_t* w, uint16_t* s, uint16_t* b, uint64_t n_words) {
    OrcModel* m = (OrcModel*)mp;
    QStore* q = q4_of(m, layer, name);
    if (!q || n_words != q->w.size()) {
        g_err = std::string("no Q4 tensor of that shape: ") + name;
        return -1;
    }
    std::copy(q->w.begin(), q->w.end(), w);
    std::copy(q->s.begin(), q->s.end(), s);
    std::copy(q->b.begin(), q->b.end(), b);
    return 0;
}

int orc_get_bf16(void* mp, uint32_t layer, const char* name, uint16_t* v, uint64_t n) {
    OrcModel* m = (OrcModel*)mp;
    std::vector<uint16_t>* t = bf16_of(m, layer, name);
    if (!t || n != t->size()) {
        g_err = std::string("no bf16 tensor of that size: ") + name;
        return -1;
    }
    std::copy(t->begin(), t->end(), v);
    return 0;
}

// ---- PLE ----
static PleW* ple_of(OrcModel* m) {
    if (!m->c.ple_layer) {
        g_err = "the model has no PLE block";
        return nullptr;
    }
    return &m->layers[m->c.ple_layer - 1].ple;
}

// ngram_ids_from over tokens[0..n) (the ids of its last token); cap >= the
// number of heads
int orc_ngram_ids(void* mp, const uint32_t* tokens, uint32_t n, uint64_t* ids, uint32_t cap, uint32_t* n_ids) {
    OrcModel* m = (OrcModel*)mp;
    PleW* P = ple_of(m);
    if (!P) return -1;
    if (n == 0) {
        g_err = "no tokens";
        return -1;
    }
    const std::vector<uint64_t> v =
        orc::ngram_ids_from(m->c, P->multipliers, P->head_offsets, P->head_sizes, tokens, n);
    if (v.size() > cap) {
        g_err = "id buffer too small";
        return -1;
    }
    std::copy(v.begin(), v.end(), ids);
    *n_ids = (uint32_t)v.size();
    return 0;
}

// The PLE block alone for the next token: appends `token` to the state's
// history, runs CpuModel::ple on `hyper` (hc * h), writes the addend and
// gvn (each hc * h) and advances the ring; the position is untouched.
int orc_ple(void* mp, void* sp, uint32_t token, const float* hyper, float* add, float* gvn) {
    OrcModel* m = (OrcModel*)mp;
    OrcState* st = (OrcState*)sp;
    PleW* P = ple_of(m);
    if (!P) return -1;
    try {
        st->tokens.push_back(token);
        std::vector<float> g;
        const std::vector<float> a = orc::ple(*m, *P, hyper, *st, &g);
        std::copy(a.begin(), a.end(), add);
        std::copy(g.begin(), g.end(), gvn);
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

// The hash metadata (multipliers [ngram_size], head offsets and sizes
// [heads]): copied out, or replaced when `set`.
int orc_ngram_meta(void* mp, int64_t* mult, uint64_t* offs, uint64_t* sizes, int set) {
    OrcModel* m = (OrcModel*)mp;
    PleW* P = ple_of(m);
    if (!P) return -1;
    if (set) {
        std::copy(mult, mult + P->multipliers.size(), P->multipliers.begin());
        std::copy(offs, offs + P->head_offsets.size(), P->head_offsets.begin());
        std::copy(sizes, sizes + P->head_sizes.size(), P->head_sizes.begin());
    } else {
        std::copy(P->multipliers.begin(), P->multipliers.end(), mult);
        std::copy(P->head_offsets.begin(), P->head_offsets.end(), offs);
        std::copy(P->head_sizes.begin(), P->head_sizes.end(), sizes);
    }
    return 0;
}

uint64_t orc_ngram_table_bytes(void* mp) { return ((OrcModel*)mp)->ngram.bytes.size(); }

// Packed::ngram_row of table row `id` (dim floats).
int orc_ngram_row(void* mp, uint64_t id, float* dst) {
    try {
        orc::ngram_row(((OrcModel*)mp)->ngram, id, dst);
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

// The n-gram table's bytes (ngram.bin layout): copied out, or replaced
// when `set` (n must be the table's size).
int orc_ngram_table(void* mp, uint8_t* buf, uint64_t n, int set) {
    OrcModel* m = (OrcModel*)mp;
    if (n != m->ngram.bytes.size()) {
        g_err = "n-gram table size mismatch";
        return -1;
    }
    if (set) std::copy(buf, buf + n, m->ngram.bytes.begin());
    else std::copy(m->ngram.bytes.begin(), m->ngram.bytes.end(), buf);
    return 0;
}

int orc_set_record(void* mp, uint32_t record_layer, uint32_t e, const uint8_t* src, uint64_t n) {
    OrcModel* m = (OrcModel*)mp;
    if (n > m->rec_stride) {
        g_err = "record larger than the stride";
        return -1;
    }
    uint8_t* dst = const_cast<uint8_t*>(m->record(record_layer, e));
    std::copy(src, src + n, dst);
    return 0;
}

}  // extern "C"
