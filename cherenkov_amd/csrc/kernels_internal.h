// Argument blocks and launchers of the decode kernels (internal).
#pragma once

#include "internal.h"

namespace chk {

constexpr int MAX_SEG = 5;

enum Epi { EPI_RAW = 0, EPI_DN_CONV = 1, EPI_DN_DECAY = 2, EPI_DN_BETA = 3 };

struct Seg {
    Q4Mat m;
    const float* x;
    float* y;
    uint32_t xs, ys;  // row strides of x and y (elements)
    uint32_t row0;    // first global row of this segment
    int epi;
};

struct SegArgs {
    Seg seg[MAX_SEG];
    int nseg;
    uint32_t total;
    // EPI_DN_CONV
    const uint16_t* conv_w;
    float* hist;
    float* snap_hist;
    uint32_t ck, conv_dim;
    int snap;
    // EPI_DN_DECAY
    const uint16_t* a_log;
    const uint16_t* dt_bias;
};

struct DnScanArgs {
    float* state;       // [nv][dv][dk]
    float* snap_state;  // [MAX_SNAP][nv][dv][dk]
    const float* conv_out;  // [nb][conv_dim] (q | k | v after conv + silu)
    const float* decay;     // [nb][nv]
    const float* beta;      // [nb][nv]
    const float* z;         // [nb][v_dim]
    const uint16_t* norm;   // [dv]
    float* y;               // [nb][v_dim] gated-normed output
    uint32_t nk, nv, dv, qk_dim, conv_dim;
    float qscale;
    int snap;
};

struct RouterArgs {
    const uint16_t* router;       // [E][H]
    const uint16_t* shared_gate;  // [H]
    const float* x;               // [nb][H]
    float* logits;                // [nb][E]
    float* probs;                 // [nb][E]
    float* sg;                    // [nb]
    uint32_t* ids;                // [nb][topk]
    float* w;                     // [nb][topk]
    uint32_t* counter;
    uint32_t E, H, topk;
    int norm_topk;
};

struct MoeArgs {
    ExpertsDev X;
    uint32_t record_layer;
    Q4Mat sh_gate, sh_up, sh_down;
    const float* x;        // [nb][H]
    const uint32_t* ids;   // [nb][topk]
    const float* w;        // [nb][topk]
    const float* sg;       // [nb] shared gate logit
    float* act;            // [nb][topk + 1][I]
    float* hyper;          // [nb][hc H] (null: no inject)
    const float* inj;      // [nb][hc]
    float* raw_out;        // [nb][H] (optional)
    uint32_t nb, H, I, topk, hc;
};

// Softmax over E logits then top-k by (probability desc, index asc),
// renormalised (cpu.rs:508-525); one wave, rows b < nb.
CHK_DEV void topk_wave(const float* logits, float* probs, uint32_t E, uint32_t k, int norm, uint32_t* ids,
                       float* w, int nb, int lane) {
    constexpr int MAXE = 16;  // up to 1024 experts per wave
    for (int b = 0; b < nb; ++b) {
        const float* l = logits + (size_t)b * E;
        float v[MAXE];
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < MAXE; ++j) {
            uint32_t e = lane + 64 * j;
            v[j] = e < E ? l[e] : -INFINITY;
            mx = fmaxf(mx, v[j]);
        }
        mx = wave_max(mx);
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < MAXE; ++j) {
            uint32_t e = lane + 64 * j;
            v[j] = e < E ? expf(v[j] - mx) : 0.0f;
            sum += v[j];
        }
        sum = wave_sum(sum);
        float inv = 1.0f / sum;
#pragma unroll
        for (int j = 0; j < MAXE; ++j) {
            uint32_t e = lane + 64 * j;
            v[j] = e < E ? v[j] * inv : -1.0f;
            if (e < E) probs[(size_t)b * E + e] = v[j];
        }
        // ranks are written as found; lane 0 renormalises afterwards
        float topsum = 0.0f;
        for (uint32_t r = 0; r < k; ++r) {
            float bv = -2.0f;
            uint32_t bi = 0xffffffffu;
#pragma unroll
            for (int j = 0; j < MAXE; ++j) {
                uint32_t e = lane + 64 * j;
                if (e < E && (v[j] > bv || (v[j] == bv && e < bi))) { bv = v[j]; bi = e; }
            }
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) {
                float ov = __shfl_xor(bv, m, 64);
                uint32_t oi = __shfl_xor(bi, m, 64);
                if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
            }
            if (bi >= E) bi = 0;  // only reachable with NaN logits; keeps ids in range
            topsum += bv;
            if (lane == 0) {
                ids[b * k + r] = bi;
                w[b * k + r] = bv;
            }
#pragma unroll
            for (int j = 0; j < MAXE; ++j)
                if (lane + 64 * j == bi) v[j] = -1.0f;
        }
        if (lane == 0 && norm)
            for (uint32_t r = 0; r < k; ++r) w[b * k + r] = w[b * k + r] / topsum;
    }
}

struct AttnArgs {
    // projections output
    const float* q_raw;    // [nb][nh * 2 * hd]  (per head: q | gate)
    const float* k_raw;    // [nb][nkv * hd]
    const float* v_raw;    // [nb][nkv * hd]
    const float* idx_raw;  // [nb][(inh + 1) * ihd]
    const uint16_t* q_norm;
    const uint16_t* k_norm;
    float* q_ready;        // [nb][nh][hd]
    KvDev kv[MAX_NB];      // cache of each row's sequence
    uint32_t pos[MAX_NB];  // position of each row (its KV row index)
    float* part;           // [nb][nh][max_chunks][hd + 2]
    float* out;            // [nb][nh * hd] gated
    uint32_t nh, nkv, hd, rot, inh, ihd, max_chunks;
    float eps, theta, scale;
};

void launch_embed(const uint32_t* tokens, const Q4Mat& emb, float* hyper, uint32_t H, uint32_t hc, int nb,
                  hipStream_t st);
void launch_hc_down(const HcDev& w, const float* hyper, float* d, float* inj, float* inv, uint32_t H, uint32_t hc,
                    float eps, int nb, hipStream_t st);
void launch_hc_up_mix(const HcDev& w, const float* hyper, const float* inv, const float* d, float* mixed,
                      uint32_t H, uint32_t hc, int nb, hipStream_t st);
void launch_qmv(const SegArgs& a, int nb, hipStream_t st);
void launch_qmv_inject(const Q4Mat& m, const float* x, uint32_t xs, float* hyper, const float* inj, uint32_t hc,
                       float* raw_out, int nb, hipStream_t st);
void launch_dn_scan(const DnScanArgs& a, int nb, hipStream_t st);
void launch_router(const RouterArgs& a, int nb, hipStream_t st);
void launch_moe(const MoeArgs& a, hipStream_t st);
void launch_lm_head(const Q4Mat& m, const float* x, float* logits, float* pv, uint32_t* pi, uint32_t nparts,
                    uint32_t* out, int nb, hipStream_t st);
void launch_attn(const AttnArgs& a, int nb, hipStream_t st);
void launch_copy_f32(float* dst, const float* src, uint64_t n, hipStream_t st);
void launch_kv_fill(const float* k, const float* v, KvDev kv, uint32_t kv_row, uint32_t T, hipStream_t st);
void launch_zero_f32(float* dst, uint64_t n, hipStream_t st);

}  // namespace chk
