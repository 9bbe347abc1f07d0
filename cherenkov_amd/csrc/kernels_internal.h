// Argument blocks and launchers of the decode kernels (internal).
#pragma once

#include <vector>

#include "internal.h"

namespace chk {

constexpr int MAX_SEG = 5;

// Value lanes per DeltaNet scan workgroup: 32, so each workgroup's outputs
// are one nibble-plane chunk for the out-projection.
constexpr int DN_SCAN_COLS = 32;

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
    const float* z;         // [nb][v_dim] output gate input
    const uint16_t* norm;   // [dv] gated-norm weight
    float* y;               // [nb][v_dim] y * w * sigmoid(z) (before the 1/rms)
    XqChunk* y_xq;          // [nb][v_dim / 32] the same in nibble planes (optional)
    float* ssq;             // [nb][nv][dv / 16] partial sums of y^2
    uint32_t nk, nv, dv, qk_dim, conv_dim;
    float qscale;
    int snap;
};

enum XMode { XM_PLAIN = 0, XM_DN_GATED = 1 };

struct InjArgs {
    Q4Mat m;
    const float* x;  // [nb][in]
    uint32_t xs;
    int xmode;
    // XM_DN_GATED: gated RMSNorm of the DeltaNet output per value head
    const float* z;         // [nb][in] (same stride as x)
    const uint16_t* norm;   // [dv]
    const float* ssq;       // [nb][nheads][ssq_blocks]
    const XqChunk* x_xq;    // [nb][in / 32] x in nibble planes before the 1/rms (optional)
    uint32_t dv, nheads, ssq_blocks;
    float* hyper;  // [nb][hc H] (null: no inject)
    const float* inj;
    uint32_t hc;
    float* raw_out;  // [nb][H] (optional)
};

struct RouterArgs {
    const uint16_t* router;       // [E][H]
    const uint16_t* shared_gate;  // [H]
    const float* x;               // [nb][H]
    float* logits;                // [nb][E]
    float* sg;                    // [nb]
    uint32_t E, H;
};

// Routed-expert records of mixed precision (residency.rs:290-310, 437-451):
// X is the store the launch decodes at X.bits; with a low-bit X, kinds
// [record layers][experts] (0 = 4-bit, else X's low-bit kind) sends each
// record with kind 0 to its 4-bit copy in X4 instead.  kinds is null for
// 4-bit launches.
struct MoeArgs {
    ExpertsDev X;
    ExpertsDev X4;
    const uint8_t* kinds;
    uint32_t record_layer;
    Q4Mat sh_gate, sh_up, sh_down;
    const float* x;        // [nb][H]
    // routing: the gate/up kernel computes it from the router logits and
    // publishes ids/w; the down kernel reads them back
    const float* logits;   // [nb][E]
    float* probs;          // [nb][E]
    uint32_t E;
    int norm_topk;
    uint32_t* ids_out;     // [nb][topk]
    float* w_out;          // [nb][topk]
    const uint32_t* ids;   // [nb][topk]
    const float* w;        // [nb][topk]
    const float* sg;       // [nb] shared gate logit
    // a row's act: topk routed slots of I values, then the shared
    // expert's SI (rows of topk I + SI values; act_xq likewise in 32-value
    // chunks)
    float* act;            // [nb][topk I + SI]
    XqChunk* act_xq;       // [nb][(topk I + SI) / 32] act in nibble planes
    float* hyper;          // [nb][hc H] (null: no inject)
    const float* inj;      // [nb][hc]
    float* raw_out;        // [nb][H] (optional)
    uint32_t nb, H, I, topk, hc;
    uint32_t SI;           // the shared expert's width
};

// Wave64 reductions through DPP (quad_perm, row_ror, row_bcast): no LDS
// round trips.  The result is valid in every lane.
#define CHK_DPP(v, ctrl, rmask, old) \
    __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), ctrl, rmask, 0xf, false))

CHK_DEV float wave_max_dpp(float v) {
    v = fmaxf(v, CHK_DPP(v, 0xb1, 0xf, v));  // quad_perm [1,0,3,2]
    v = fmaxf(v, CHK_DPP(v, 0x4e, 0xf, v));  // quad_perm [2,3,0,1]
    v = fmaxf(v, CHK_DPP(v, 0x124, 0xf, v)); // row_ror:4
    v = fmaxf(v, CHK_DPP(v, 0x128, 0xf, v)); // row_ror:8
    v = fmaxf(v, CHK_DPP(v, 0x142, 0xa, v)); // row_bcast:15 into rows 1, 3
    v = fmaxf(v, CHK_DPP(v, 0x143, 0xc, v)); // row_bcast:31 into rows 2, 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

CHK_DEV float wave_sum_dpp(float v) {
    v += CHK_DPP(v, 0xb1, 0xf, 0.0f);
    v += CHK_DPP(v, 0x4e, 0xf, 0.0f);
    v += CHK_DPP(v, 0x124, 0xf, 0.0f);
    v += CHK_DPP(v, 0x128, 0xf, 0.0f);
    v += CHK_DPP(v, 0x142, 0xa, 0.0f);
    v += CHK_DPP(v, 0x143, 0xc, 0.0f);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Wave64 max of ints through DPP (the lanes outside a row mask keep their
// own value); valid in every lane.
CHK_DEV int wave_max_i32(int v) {
    // the moved value defaults to INT_MIN (max's identity) where a row mask
    // excludes a lane, so the compiler can fold each move into its v_max
    // as a DPP operand (one instruction per step instead of two)
    constexpr int LO = -2147483647 - 1;
    v = max(v, __builtin_amdgcn_update_dpp(LO, v, 0xb1, 0xf, 0xf, false));   // quad_perm [1,0,3,2]
    v = max(v, __builtin_amdgcn_update_dpp(LO, v, 0x4e, 0xf, 0xf, false));   // quad_perm [2,3,0,1]
    v = max(v, __builtin_amdgcn_update_dpp(LO, v, 0x124, 0xf, 0xf, false));  // row_ror:4
    v = max(v, __builtin_amdgcn_update_dpp(LO, v, 0x128, 0xf, 0xf, false));  // row_ror:8
    v = max(v, __builtin_amdgcn_update_dpp(LO, v, 0x142, 0xa, 0xf, false));  // row_bcast:15 into rows 1, 3
    v = max(v, __builtin_amdgcn_update_dpp(LO, v, 0x143, 0xc, 0xf, false));  // row_bcast:31 into rows 2, 3
    return __builtin_amdgcn_readlane(v, 63);
}

// take in the lanes of `mask`, keep elsewhere: a single v_cndmask_b32 (as
// an explicit instruction, so the compiler cannot turn a run of them over
// neighbouring array slots into index-select chains)
CHK_DEV uint32_t lane_pick(uint32_t keep, uint32_t take, uint64_t mask) {
    uint32_t r;
    asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(r) : "v"(keep), "v"(take), "s"(mask));
    return r;
}

// Routing of one row by one wave (moe, cpu.rs:508-525): softmax of E <=
// 512 router logits in f32 (E a multiple of 8), then the order
// (probability desc, index asc) down to rank need - 1.  Lane l holds
// experts 8l..8l+7 (two float4 loads), sorts them with a branch-free
// 19-comparator network, and each round a DPP wave max pops the best
// head; the lowest lane wins ties, i.e. the lowest index.  On return lane
// r < need holds rank r's expert id and probability.  probs (optional)
// receives the softmax.
CHK_DEV void rank_swap(float& va, uint32_t& ia, float& vb, uint32_t& ib) {
    const bool sw = (vb > va) | ((vb == va) & (ib < ia));
    const float tv = sw ? vb : va;
    const uint32_t ti = sw ? ib : ia;
    vb = sw ? va : vb;
    ib = sw ? ia : ib;
    va = tv;
    ia = ti;
}

// NZ > 1: the logits arrive as NZ K-chunk partials zs floats apart,
// summed here in chunk order.
template <int NZ = 1>
CHK_DEV void route_row(const float* __restrict__ l, uint32_t E, uint32_t need, int lane, float* probs,
                       uint32_t& my_id, float& my_p, size_t zs = 0) {
    constexpr int PER = 8;
    const uint32_t base = (uint32_t)lane * PER;
    const bool live = base < E;
    const float4* lp = reinterpret_cast<const float4*>(l + (live ? base : 0));
    float4 l0 = lp[0], l1 = lp[1];
#pragma unroll
    for (int z = 1; z < NZ; ++z) {
        const float4* q = reinterpret_cast<const float4*>(l + z * zs + (live ? base : 0));
        const float4 q0 = q[0], q1 = q[1];
        l0 = make_float4(l0.x + q0.x, l0.y + q0.y, l0.z + q0.z, l0.w + q0.w);
        l1 = make_float4(l1.x + q1.x, l1.y + q1.y, l1.z + q1.z, l1.w + q1.w);
    }
    float v[PER] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
    uint32_t ix[PER];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        ix[j] = base + j;
        v[j] = live ? v[j] : -INFINITY;
        mx = fmaxf(mx, v[j]);
    }
    mx = wave_max_dpp(mx);
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        v[j] = expf(v[j] - mx);  // 0 for the -inf padding
        sum += v[j];
    }
    const float inv = 1.0f / wave_sum_dpp(sum);
#pragma unroll
    for (int j = 0; j < PER; ++j) v[j] = live ? v[j] * inv : -1.0f;
    if (probs && live) {
        float4* pp = reinterpret_cast<float4*>(probs + base);
        pp[0] = make_float4(v[0], v[1], v[2], v[3]);
        pp[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
#define CS(a, c) rank_swap(v[a], ix[a], v[c], ix[c])
    CS(0, 2); CS(1, 3); CS(4, 6); CS(5, 7);
    CS(0, 4); CS(1, 5); CS(2, 6); CS(3, 7);
    CS(0, 1); CS(2, 3); CS(4, 5); CS(6, 7);
    CS(2, 4); CS(3, 5);
    CS(1, 4); CS(3, 6);
    CS(1, 2); CS(3, 4); CS(5, 6);
#undef CS
    // pops on int keys: probabilities are >= 0, so their bit patterns order
    // like the floats; the padding (< 0) never wins while real entries remain
    int key[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) key[j] = __float_as_int(v[j]);
    my_id = 0;
    my_p = 0.0f;
    for (uint32_t r = 0; r < need; ++r) {
        const int m = wave_max_i32(key[0]);
        const uint64_t ball = __ballot(key[0] == m);
        const int win = (int)__builtin_ctzll(ball);
        const uint32_t idx = (uint32_t)__builtin_amdgcn_readlane((int)ix[0], win);
        if ((uint32_t)lane == r) {
            my_id = idx;
            my_p = __int_as_float(m);
        }
        // the winning lane drops its head: one v_cndmask per slot on the
        // winner's lane mask
        const uint64_t pm = 1ull << win;
#pragma unroll
        for (int j = 0; j + 1 < PER; ++j) {
            key[j] = (int)lane_pick((uint32_t)key[j], (uint32_t)key[j + 1], pm);
            ix[j] = lane_pick(ix[j], ix[j + 1], pm);
        }
        key[PER - 1] = (int)lane_pick((uint32_t)key[PER - 1], 0xffffffffu, pm);
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
    const uint32_t* pos;   // [nb] device: position of each row (its KV row index)
    float* part;           // [nb][nh][max_chunks][hd + 2]
    float* out;            // [nb][nh * hd] gated
    uint32_t nh, nkv, hd, rot, inh, ihd, max_chunks;
    float eps, theta, scale;
    int one_kv;            // every row belongs to kv[0]'s sequence (prefill rows)
    // QSA indexer (cpu.rs:643-719); qsa = 0 keeps every row dense
    int qsa;
    const uint16_t* iq_norm;  // [ihd]
    const uint16_t* ik_norm;  // [ihd]
    float* iq_ready;          // [nb][inh][ihd] normed, roped index queries
    float* bscore;            // [nb][max_blocks] block scores
    uint32_t* vmask;          // [nb][mask_words] selected complete blocks
    uint32_t ratio, kblk, max_blocks, mask_words;
};

// ------------------------------------------------------------- prefill
enum PfEpi { PE_STORE = 0, PE_HC_UP = 2, PE_SILU_MUL = 3 };

// Operand preparation of one activation matrix (k_pf_prep).
struct PfPrepArgs {
    const float* x;    // [T][ldx]
    uint32_t ldx, T, K;
    uint4* hi;         // [T][K/8] fp16, permuted 8-blocks
    uint4* lo;
    float* xs;         // [T][K/64]
    uint4* bhi;        // optional bf16 natural-order planes [T][K/8] (hi + mid + lo)
    uint4* bmid;
    uint4* blo;
    // DeltaNet gated norm (z non-null): x = y, z same stride
    const float* z;
    const uint16_t* norm;
    uint32_t dv;
};

// One output segment of a concatenated projection: outputs [n0, n0 + m.out).
struct PfSeg {
    Q4Mat m;
    float* y;
    uint32_t ldy, n0;
    uint32_t wo, so, bo;  // set by the launcher: element offsets of m from wbase / sbase
};

struct PfGemmArgs {
    PfSeg seg[4];      // PE_SILU_MUL: seg[0].m gate, seg[1].m up (shared expert), output seg[0].y
    uint32_t nseg, N, K, M;
    uint32_t ksplit;         // K chunks (grid z); PE_STORE then writes chunk z at y + z zstride
    uint64_t zstride;
    const uint4* xhi;
    const uint4* xlo;
    const float* xs;
    // grouped rows (tinfo non-null)
    const uint32_t* list;    // [groups][cap] entries: A row list[g][m] / div (else off + m)
    const uint32_t* tiles;   // (group << 16 | tile)
    const uint2* tinfo;      // per tile: (group's first row in grouped order, group's row count)
    const uint32_t* ntiles;
    uint32_t cap, div;
    ExpertsDev X;            // routed-expert records for groups < X.experts
    ExpertsDev X4;           // their 4-bit copies, for records whose kind is 0
    const uint8_t* kinds;    // [record layers][experts] with a low-bit X (else null)
    uint32_t record_layer;
    const uint32_t* wbase;   // set by the launcher (dense matrices' common bases)
    const uint16_t* sbase;
    // PE_HC_UP
    float* hyper;            // [M][hc H]
    const float* inv;        // [M][hc]
    const uint16_t* norm;    // [hc H]
    float* out;              // [M][H]
    uint32_t H, hc;
    // PE_HC_UP / PE_SILU_MUL with phi set: the rows leave as the next
    // GEMM's operands (k_pf_prep's planes: hi, lo, xs; with pbhi also the
    // router's three bf16 planes, PE_HC_UP) instead of f32 rows
    uint4 *phi, *plo, *pbhi, *pbmid, *pblo;
    float* pxs;
    uint32_t vec4;           // set by the launcher: outputs leave as 16-byte stores
};

// DeltaNet prefill (conv, decay/beta, sequential scan) over T rows.
struct PfDnArgs {
    const float* raw;      // [T][ld_raw] qkv projection (pre-conv)
    uint32_t ld_raw;
    const float* a_raw;    // [ab_split][.. ab_zstride][T][ld_ab]: K-chunk partials, summed in order
    const float* b_raw;
    uint32_t ld_ab, ab_split = 1;
    uint64_t ab_zstride;
    const uint16_t* conv_w;
    const uint16_t* a_log;
    const uint16_t* dt_bias;
    float* hist;           // [conv_dim][ck - 1]
    float* conv;           // [T][conv_dim] after conv, silu, q/k norms
    float* decay;          // [T][nv]
    float* beta;           // [T][nv]
    float* state;          // [nv][dv][dk]
    float* y;              // [T][v_dim]
    uint32_t T, conv_dim, ck, nk, nv, dv, qk_dim, v_dim;
    float qscale;
};

// Per-step inputs written by the host into pinned, device-mapped memory
// (read once per step by the first kernel, so a captured graph replays
// with new tokens and positions).
constexpr uint32_t MAX_NGRAM_IDS = 32;  // n-gram heads of a PLE block
struct StepIn {
    uint32_t tokens[MAX_NB];
    uint32_t pos;
    uint32_t pad[3];
    uint32_t ngram[MAX_NB][MAX_NGRAM_IDS];  // PLE table rows of each row's token
};

void launch_embed(const StepIn* in, uint32_t* tokens, uint32_t* rowpos, const Q4Mat& emb, float* hyper, uint32_t H,
                  uint32_t hc, int nb, hipStream_t st);

// Cumulative routed-expert activity (ExpertCounters::lookup, activity.rs:
// 31-35) of `layers` record layers from layer0 on: per layer, how many of
// the step's `rows` rows chose each expert (ids [rows][topk] at
// ids + l * layer_stride) goes to the expert's selected rows and, when
// non-zero, one lookup (a hit: every record is resident).  act: [record
// layers][E][2].  Null `act`: nothing to count.
struct ActivityArgs {
    const uint32_t* ids;
    uint64_t layer_stride;
    uint32_t layers, rows, topk, E, layer0;
    unsigned long long* act;
};
constexpr uint32_t ACT_MAX_E = 512;

// One workgroup's share: record layer layer0 + l, counted in `hist` (LDS,
// ACT_MAX_E entries) by threads t < nt.
CHK_DEV void expert_activity_layer(const ActivityArgs& a, uint32_t l, uint32_t t, uint32_t nt, uint32_t* hist) {
    for (uint32_t e = t; e < a.E; e += nt) hist[e] = 0;
    __syncthreads();
    const uint32_t* li = a.ids + (uint64_t)l * a.layer_stride;
    for (uint32_t i = t; i < a.rows * a.topk; i += nt) {
        const uint32_t e = li[i];
        if (e < a.E) atomicAdd(&hist[e], 1u);
    }
    __syncthreads();
    unsigned long long* c = a.act + (uint64_t)(a.layer0 + l) * a.E * 2;
    for (uint32_t e = t; e < a.E; e += nt)
        if (hist[e]) {
            c[2 * e] += hist[e];
            c[2 * e + 1] += 1;
        }
}

// The hyper-connection read's first half; with `act` set, `act.layers`
// more workgroups count the step's expert activity alongside it (the
// step's last read, after every layer's routing), so the count costs no
// dependent launch of its own.
void launch_hc_down(const HcDev& w, const float* hyper, float* d, float* inj, float* inv, uint32_t H, uint32_t hc,
                    float eps, int nb, hipStream_t st, const ActivityArgs* act = nullptr);
void launch_hc_up_mix(const HcDev& w, const float* hyper, const float* inv, const float* d, float* mixed,
                      uint32_t H, uint32_t hc, int nb, hipStream_t st);
void launch_qmv(const SegArgs& a, int nb, hipStream_t st);
void launch_qmv_inject(const InjArgs& a, int nb, hipStream_t st);
void launch_dn_scan(const DnScanArgs& a, int nb, hipStream_t st);
void launch_router(const RouterArgs& a, int nb, hipStream_t st);
// ev_start / ev_stop (optional): HIP events the dispatch itself records at
// the kernel's start and end (hipExtLaunchKernelGGL)
void launch_moe_gate_up(const MoeArgs& a, hipStream_t st, hipEvent_t ev_start = nullptr,
                        hipEvent_t ev_stop = nullptr);
void launch_moe_down(const MoeArgs& a, hipStream_t st);
void launch_lm_head(const Q4Mat& m, const float* x, float* logits, float* pv, uint32_t* pi, uint32_t nparts,
                    uint32_t* out, int nb, hipStream_t st);
void launch_attn(const AttnArgs& a, int nb, hipStream_t st);
void launch_pf_prep(const PfPrepArgs& a, hipStream_t st);
void launch_pf_xprep(const float* x, uint32_t ldx, uint32_t T, uint32_t K, uint4* hi, uint4* lo, float* xs,
                     hipStream_t st);
// An expert block's output left for the next hyper-connection read to
// combine and inject (launch_pf_moe_combine's inputs); yd null: none.
struct PfCombine {
    const float* yd = nullptr;
    const uint32_t* goff = nullptr;
    const uint32_t* pos = nullptr;
    const float* wts = nullptr;
    const float* sg = nullptr;
    const float* inj = nullptr;
    uint32_t topk = 0;
};
void launch_pf_hc_prep(float* hyper, const uint16_t* norm, uint32_t H, uint32_t hc, float eps, float* inv,
                       uint4* hi, uint4* lo, float* xs, uint32_t T, const float* part, uint64_t pzs, uint32_t nsplit,
                       const float* pinj, hipStream_t st, const PfCombine& mc = PfCombine{});
// false when the caller asked for operand planes (phi) and the launch wrote
// its f32 rows instead
bool launch_pf_gemm_args(const PfGemmArgs& a, int epi, uint32_t grid_y, hipStream_t st);
// Causal flash attention over a prefill chunk.  Its (row block, token
// tile) steps are dealt to the workgroups by a plan made on the host
// (pf_flash_plan, the same for every kv head): per workgroup up to
// FA_MAXSEG segments (row block, first tile, end tile, partial slot or ~0
// for a whole block; row block ~0 ends the list), and per split row block
// a merge entry (row block, first slot, pieces, 0).
constexpr uint32_t FA_MAXSEG = 6;
constexpr int FA_MAXP = 4;  // pieces of a split row block
struct PfFlashPlan {
    uint32_t W = 0;            // workgroups per kv head
    uint32_t nslots = 0;       // partial slots per kv head
    std::vector<uint4> seg;    // [W][FA_MAXSEG]
    std::vector<uint4> merge;  // [split row blocks]
};
PfFlashPlan pf_flash_plan(uint32_t T, uint32_t pos0, uint32_t max_wg);
struct PfFlashLaunch {         // a plan uploaded to the device
    const uint4* seg;
    const uint4* merge;
    float* part;               // [nkv][nslots][16][nh / nkv][2 + hd]
    uint32_t W, nslots, nmerge;
};
void launch_pf_flash(const float* q_ready, const float* q_raw, const KvDev& kv, float* out, uint32_t T, uint32_t pos0,
                     uint32_t nh, uint32_t nkv, uint32_t hd, float scale, const PfFlashLaunch& plan, hipStream_t st);
void launch_pf_gemm(const Q4Mat& w, const uint4* xhi, const uint4* xlo, const float* xs, float* y, uint32_t T,
                    uint32_t ldy, hipStream_t st);
// [down; inject] partials -> inj and d, d staged as the up GEMM's operands
// (hi, lo, xs) with d as the scratch of the unfused form
void launch_pf_hc_down_finish(const float* part, uint32_t nsplit, uint32_t T, uint32_t lowrank, uint32_t hc,
                              float alpha, float* d, float* inj, uint4* hi, uint4* lo, float* xs, hipStream_t st);
// The prefill router's plan: column blocks of 64 PF_ROUTER_CT experts and
// PF_ROUTER_CHUNKS K chunks where the shape allows (the logits then leave
// as that many partials, T E floats apart, summed by the routing pass),
// else 64-expert blocks over the whole K (grid z = 1).
constexpr uint32_t PF_ROUTER_CT = 2;
constexpr uint32_t PF_ROUTER_CHUNKS = 2;
dim3 pf_router_plan(uint32_t T, uint32_t E, uint32_t H);
void launch_pf_router(const uint16_t* router, const uint4* bhi, const uint4* bmid, const uint4* blo, float* logits,
                      uint32_t T, uint32_t E, uint32_t H, hipStream_t st);
void launch_pf_route(const float* logits, uint32_t T, uint32_t E, uint32_t topk, int norm_topk, uint32_t* ids,
                     float* wts, uint32_t* last_ids, float* last_wts, const uint16_t* shared_gate, const uint4* bhi,
                     const uint4* bmid, const uint4* blo, float* sg, uint32_t H, uint32_t* gcnt, uint32_t* list,
                     uint32_t* pos, uint32_t cap, bool shared, hipStream_t st);
// words between two experts' entry counters of the routing pass (gcnt)
constexpr uint32_t PF_GCNT_STRIDE = 32;
void launch_pf_group(uint32_t* gcnt, uint32_t T, uint32_t topk, uint32_t E, uint32_t cap, uint32_t* count,
                     uint32_t* tiles, uint32_t* ntiles, uint2* tinfo, uint32_t* goff, uint64_t* act, uint32_t layer,
                     uint32_t tr, bool shared, hipStream_t st);
uint32_t pf_tile_bound(uint32_t T, uint32_t topk, uint32_t E, uint32_t tr);
void launch_pf_moe_combine(const float* yd, const uint32_t* goff, const uint32_t* pos, const float* wts, const float* sg,
                           const float* inj, float* hyper, uint32_t T, uint32_t H, uint32_t topk, uint32_t hc,
                           hipStream_t st);
void launch_pf_embed(const uint32_t* tokens, const Q4Mat& emb, float* hyper, uint32_t H, uint32_t hc, uint32_t T,
                     hipStream_t st);
// conv + norms, decay / beta, then the scan: chunked (dnscan.hip) when
// `work` is given and the head dims allow it, else the sequential kernel.
void launch_pf_dn(const PfDnArgs& a, float* work, hipStream_t st);
void launch_pf_dn_scan(const PfDnArgs& a, float* work, hipStream_t st);
bool dc_supported(uint32_t nk, uint32_t nv, uint32_t dk, uint32_t dv);
uint64_t dc_work_floats(uint32_t T, uint32_t nv, uint32_t dv);
void launch_dc_scan(const PfDnArgs& a, float* work, hipStream_t st);
void launch_attn_prep(const AttnArgs& a, int nb, hipStream_t st);
void launch_qsa_select(const AttnArgs& a, int nb, hipStream_t st);
// block keys + scores + selection of nb rows (a no-op without QSA)
void launch_qsa(const AttnArgs& a, int nb, hipStream_t st);
// pooled keys of blocks [blk0, blk1) of kv[0]'s sequence
void launch_qsa_block_keys(const AttnArgs& a, uint32_t blk0, uint32_t blk1, hipStream_t st);
void launch_attn_core(const AttnArgs& a, int nb, hipStream_t st);
bool attn_shape_ok(uint32_t nh, uint32_t nkv, uint32_t hd);
void launch_copy_f32(float* dst, const float* src, uint64_t n, hipStream_t st);
void launch_kv_fill(const float* k, const float* v, KvDev kv, uint32_t kv_row, uint32_t T, hipStream_t st);
void launch_zero_f32(float* dst, uint64_t n, hipStream_t st);
// dependent-FMA clock probe over 65536 threads (out: 65536 floats)
void launch_clock_probe(float* out, uint32_t iters, hipStream_t st);
// PLE n-gram block (ple.hip)
void gen_ngram_table(uint8_t* table, uint64_t rows, uint32_t dim, uint32_t group, uint64_t seed, hipStream_t st);
// ids: row r's table rows at ids[r * ids_stride ..]
void launch_ple_gather(const uint32_t* ids, uint32_t ids_stride, uint32_t nids, const uint8_t* table,
                       uint64_t row_bytes, uint32_t dim, uint32_t group, float* e, uint32_t rows, hipStream_t st);
void launch_ple_gate(const float* key, const float* hyper, uint64_t hyper_stride, const float* value,
                     const uint16_t* wk, const uint16_t* wq, const uint16_t* wc, float* gated, float* gvn, uint32_t H,
                     uint32_t hc, float eps, uint32_t rows, hipStream_t st);
void launch_ple_conv(const float* gated, const float* gvn, const uint16_t* conv, const float* ring, float* hyper,
                     uint64_t hyper_stride, const uint32_t* pos, uint32_t hh, uint32_t K, uint32_t dil, uint32_t span,
                     uint32_t rows, hipStream_t st);
void launch_ple_ring(const float* gvn, float* ring, float* backup, const uint32_t* pos, uint32_t hh, uint32_t span,
                     uint32_t rows, hipStream_t st);
void launch_fill_u8(uint8_t* dst, uint8_t v, uint64_t n, hipStream_t st);

}  // namespace chk
