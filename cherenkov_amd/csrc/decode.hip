// Decode / verify kernels for the qwen4_exp token loop on gfx950 (wave64).
//
// One step runs `nb` <= 4 rows (one committed token plus drafts).  Every
// weight matrix is streamed from HBM once per step for all rows.  Batch-1
// decode is a chain of HBM-bound matvecs, so each wave keeps its slice of
// the input vector in VGPRs and issues the weight loads of R rows before it
// consumes any of them (R x 16 B in flight per lane), on grids that stride
// over row blocks instead of spawning a wave per row.
//
// Reference semantics: /root/reference/src/qwen4_exp/cpu.rs (forward_token
// and the blocks it calls); the Metal dispatch plan this replaces:
// src/qwen4_exp/gpu/decode.rs:13-294 and kernels/{common,qwen4_exp}/*.metal.
#include <algorithm>
#include <stdexcept>
#include <type_traits>

#include "kernels_internal.h"

namespace chk {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

CHK_DEV uint4 ldw4(const uint32_t* p) {
    u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

CHK_DEV void ldx32(const float* p, float* x) {
    const float4* p4 = reinterpret_cast<const float4*>(p);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        float4 v = p4[k];
        x[4 * k] = v.x; x[4 * k + 1] = v.y; x[4 * k + 2] = v.z; x[4 * k + 3] = v.w;
    }
}

// This lane's input chunks (ch = lir + c * LPR, c < CPL) of NB input rows
// and their sums.  Lanes past the last chunk read chunk nch-1 (a valid
// address) and zero it, so the loads stay unconditional.
template <int NB, int CPL>
struct XFrag {
    float v[NB][CPL][32];
    float s[NB][CPL];
    h2 hi[NB][CPL][16], lo[NB][CPL][16];  // the fp16 dot's pairs (x_pairs)

    template <int LPR>
    CHK_DEV void load(const float* __restrict__ x, uint32_t xs, uint32_t nch, int lir) {
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const uint32_t ch = lir + c * LPR;
            const uint32_t cc = ch < nch ? ch : nch - 1;
#pragma unroll
            for (int b = 0; b < NB; ++b) ldx32(x + (size_t)b * xs + cc * 32, v[b][c]);
            if (ch >= nch)
#pragma unroll
                for (int b = 0; b < NB; ++b)
#pragma unroll
                    for (int j = 0; j < 32; ++j) v[b][c][j] = 0.0f;
        }
    }
    // chunk sums and fp16 pairs of the (possibly rescaled) loaded inputs
    CHK_DEV void sums() {
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                float t = 0.0f;
#pragma unroll
                for (int j = 0; j < 32; ++j) t += v[b][c][j];
                s[b][c] = t;
                x_pairs(v[b][c], hi[b][c], lo[b][c]);
            }
    }
};

template <int LPR, int CPL, int NB>
CHK_DEV void load_x(const float* __restrict__ x, uint32_t xs, uint32_t nch, int lir, XFrag<NB, CPL>& xf) {
    xf.template load<LPR>(x, xs, nch, lir);
    xf.sums();
}

// This lane's input chunks (ch = lir + c * LPR) of NB rows in nibble-plane
// form, read from the workgroup's LDS image (xq_prep: [row][nch] chunks).
// Lanes past the last chunk read chunk nch-1; the weight side masks them.
template <int NB, int CPL>
struct XqFrag {
    XqChunk c[NB][CPL];

    template <int LPR>
    CHK_DEV void read(const XqChunk* lds, uint32_t nch, int lir) {
#pragma unroll
        for (int k = 0; k < CPL; ++k) {
            const uint32_t ch = lir + k * LPR;
            const uint32_t cc = ch < nch ? ch : nch - 1;
#pragma unroll
            for (int b = 0; b < NB; ++b) c[b][k] = lds[b * nch + cc];
        }
    }
};

// Dynamic LDS of the matvec kernels: the nibble-plane image of their inputs.
extern __shared__ XqChunk xq_lds[];

// R rows of a Q4 matrix as this lane sees them: issue() starts every load
// (unconditionally, raw bf16 scale/bias kept undecoded so nothing waits),
// dot() consumes them against the lane's input chunks and reduces over the
// LPR lanes of a row.  Splitting the two lets callers put independent
// prologue/epilogue loads between them.
template <int LPR, int CPL, int R>
struct Q4Frag {
    uint4 wq[R][CPL];
    // raw bf16 scale and bias, one per 32-bit register: packing two into
    // one register (or converting them where they load) would make the
    // wave wait for them, and for every load issued before, right there
    uint32_t s16[R][CPL], b16[R][CPL];
    bool ok[CPL];

    CHK_DEV void issue(const Q4Mat& m, const uint32_t (&rows)[R], int lir) {
        const uint32_t wpr = m.in >> 3, gpr = m.in >> 6, nch = m.in >> 5;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const uint32_t ch = lir + c * LPR;
            ok[c] = ch < nch;
            const uint32_t cc = ok[c] ? ch : nch - 1;
#pragma unroll
            for (int i = 0; i < R; ++i) {
                wq[i][c] = ldw4(m.w + (size_t)rows[i] * wpr + cc * 4);
                s16[i][c] = m.s[(size_t)rows[i] * gpr + (cc >> 1)];
                b16[i][c] = m.b[(size_t)rows[i] * gpr + (cc >> 1)];
            }
        }
    }

    // against inputs in nibble planes (the u4 dot8 form, device.h)
    template <int NB>
    CHK_DEV void dot(const XqFrag<NB, CPL>& xf, float (&acc)[R][NB]) const {
#pragma unroll
        for (int i = 0; i < R; ++i)
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                float a = 0.0f;
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    const float p = q4_dot8(wq[i][c], xf.c[b][c], __uint_as_float(s16[i][c] << 16),
                                            __uint_as_float(b16[i][c] << 16));
                    a += ok[c] ? p : 0.0f;
                }
                acc[i][b] = group_sum<LPR>(a);
            }
    }
};

template <int LPR, int CPL, int R, int NB>
CHK_DEV void q4_block(const Q4Mat& m, const uint32_t (&rows)[R], const XqFrag<NB, CPL>& xr, int lir,
                      float (&acc)[R][NB]) {
    Q4Frag<LPR, CPL, R> f;
    f.issue(m, rows, lir);
    f.template dot<NB>(xr, acc);
}

// Low-bit (Q3/Q2) 32-code chunk in the lowbit.rs layout (q2_slots /
// q3_slots, lowbit.rs:143-184).  Codes reconstruct at the midpoint of the
// Q4 range they cover, w = mid * s + b with mid = 2q + 0.5 (Q3) or
// 4q + 1.5 (Q2), so a chunk contributes s * (step * sum(q x) + half * sum(x)) + b * sum(x).
template <int BITS>
CHK_DEV float lowbit_chunk(uint32_t w0, uint32_t w1, uint32_t lo, const float* x, float xs, float s, float b) {
    float qd = 0.0f;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const uint32_t w = t ? w1 : w0;
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
#pragma unroll
            for (int byte = 0; byte < 4; ++byte) {
                uint32_t code = (w >> (8 * byte + 2 * pp)) & 3u;
                if (BITS == 3) code = 2u * code + ((lo >> (8 * byte + 4 * t + pp)) & 1u);
                const int r = pp == 0 ? 2 * byte : pp == 1 ? 2 * byte + 8 : pp == 2 ? 2 * byte + 1 : 2 * byte + 9;
                qd += (float)code * x[16 * t + r];
            }
        }
    }
    const float step = BITS == 2 ? 4.0f : 2.0f, half = BITS == 2 ? 1.5f : 0.5f;
    return s * (step * qd + half * xs) + b * xs;
}

// The same chunk's codes as Q4-order nibble words (word k holds inputs
// 8k .. 8k + 7, lowest nibble first), for the dot8 form.  Byte b of word t
// holds, at 2-bit positions pp = 0, 2, the codes of inputs 16 t + 2b and
// 16 t + 2b + 1 (nibbles 2b, 2b + 1 of word 2t: mask 0x33 keeps exactly
// them) and at pp = 1, 3 those of inputs 16 t + 2b + 8, + 9 (word 2t + 1).
// Q3 codes are 2 code + lo bit (8 byte + 4 t + pp).
template <int BITS>
CHK_DEV uint4 lowbit_nibbles(uint32_t w0, uint32_t w1, uint32_t lo) {
    constexpr uint32_t M = 0x33333333u;
    if (BITS == 2) return make_uint4(w0 & M, (w0 >> 2) & M, w1 & M, (w1 >> 2) & M);
    // lo bits sh and sh + 2 of every byte -> bits 0 and 4 of that byte
    auto lob = [&](int sh) { return ((lo >> sh) & 0x01010101u) | (((lo >> (sh + 2)) & 0x01010101u) << 4); };
    return make_uint4(((w0 & M) << 1) | lob(0), (((w0 >> 2) & M) << 1) | lob(1), ((w1 & M) << 1) | lob(4),
                      (((w1 >> 2) & M) << 1) | lob(5));
}

// A routed-expert projection inside its record: Q4 view or low-bit pointers.
struct ExpMat {
    const uint8_t* w;
    const uint16_t* s;
    const uint16_t* b;
    uint32_t out, in;
};

CHK_DEV ExpMat expert_mat(const ExpertsDev& X, const uint8_t* rec, int part, uint32_t out, uint32_t in) {
    const uint64_t woff = part == 0 ? X.gate_w : part == 1 ? X.up_w : X.down_w;
    const uint64_t soff = part == 0 ? X.gate_s : part == 1 ? X.up_s : X.down_s;
    const uint64_t boff = part == 0 ? X.gate_b : part == 1 ? X.up_b : X.down_b;
    return ExpMat{rec + woff, (const uint16_t*)(rec + soff), (const uint16_t*)(rec + boff), out, in};
}

// R rows of an expert projection (any precision), split like Q4Frag.
template <int LPR, int CPL, int R, int BITS>
struct ExpFrag {
    Q4Frag<LPR, CPL, R> q;
    uint32_t w0[BITS == 4 ? 1 : R][CPL], w1[BITS == 4 ? 1 : R][CPL], lo[BITS == 4 ? 1 : R][CPL];

    CHK_DEV void issue(const ExpMat& m, const uint32_t (&rows)[R], int lir) {
        if (BITS == 4) {
            Q4Mat qm{(const uint32_t*)m.w, m.s, m.b, m.out, m.in};
            q.issue(qm, rows, lir);
            return;
        }
        const uint32_t nch = m.in >> 5, gpr = m.in >> 6, cb = BITS == 2 ? 8 : 12;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const uint32_t ch = lir + c * LPR;
            q.ok[c] = ch < nch;
            const uint32_t cc = q.ok[c] ? ch : nch - 1;
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const int ii = BITS == 4 ? 0 : i;
                const uint8_t* p = m.w + ((size_t)rows[i] * nch + cc) * cb;
                if (BITS == 2) {
                    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
                    u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
                    w0[ii][c] = v.x; w1[ii][c] = v.y; lo[ii][c] = 0;
                } else {
                    const uint32_t* qq = reinterpret_cast<const uint32_t*>(p);
                    w0[ii][c] = __builtin_nontemporal_load(qq);
                    w1[ii][c] = __builtin_nontemporal_load(qq + 1);
                    lo[ii][c] = __builtin_nontemporal_load(qq + 2);
                }
                q.s16[i][c] = m.s[(size_t)rows[i] * gpr + (cc >> 1)];
                q.b16[i][c] = m.b[(size_t)rows[i] * gpr + (cc >> 1)];
            }
        }
    }

    // inputs in nibble planes: Q4 words as they are, Q3/Q2 codes expanded
    // to nibbles, the midpoint rule folded into the scale and bias
    // (step s, half s + b)
    template <int NB>
    CHK_DEV void dot(const XqFrag<NB, CPL>& xr, float (&acc)[R][NB]) const {
        if constexpr (BITS == 4) {
            q.template dot<NB>(xr, acc);
        } else {
            constexpr float step = BITS == 2 ? 4.0f : 2.0f, half = BITS == 2 ? 1.5f : 0.5f;
#pragma unroll
            for (int i = 0; i < R; ++i) {
                uint4 wn[CPL];
                float s2[CPL], b2[CPL];
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    wn[c] = lowbit_nibbles<BITS>(w0[i][c], w1[i][c], lo[i][c]);
                    const float sc = bf16f(q.s16[i][c]);
                    s2[c] = step * sc;
                    b2[c] = fmaf(half, sc, bf16f(q.b16[i][c]));
                }
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    float a = 0.0f;
#pragma unroll
                    for (int c = 0; c < CPL; ++c) {
                        const float p = q4_dot8(wn[c], xr.c[b][c], s2[c], b2[c]);
                        a += q.ok[c] ? p : 0.0f;
                    }
                    acc[i][b] = group_sum<LPR>(a);
                }
            }
        }
    }

    // Q3/Q2 records: f32 inputs
    template <int NB>
    CHK_DEV void dot(const XFrag<NB, CPL>& xr, float (&acc)[R][NB]) const {
        static_assert(BITS != 4, "Q4 records take nibble-plane inputs");
#pragma unroll
        for (int i = 0; i < R; ++i)
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int ii = BITS == 4 ? 0 : i;
                float a = 0.0f;
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    const float p = lowbit_chunk<BITS>(w0[ii][c], w1[ii][c], lo[ii][c], xr.v[b][c], xr.s[b][c],
                                                       bf16f(q.s16[i][c]), bf16f(q.b16[i][c]));
                    a += q.ok[c] ? p : 0.0f;
                }
                acc[i][b] = group_sum<LPR>(a);
            }
    }
};



// ------------------------------------------------------------------ embed
// embed.dequant_row + replicate into hc streams (cpu.rs:399-407).  Uses
// explicitly rounded mul/add so hyper starts bit-identical to the oracle.
__global__ void __launch_bounds__(256) k_embed(const StepIn* __restrict__ in, uint32_t* __restrict__ tok_out,
                                               uint32_t* __restrict__ rowpos, Q4Mat emb, float* __restrict__ hyper,
                                               uint32_t H, uint32_t hc) {
    uint32_t b = blockIdx.y, i = blockIdx.x * CHK_WG + threadIdx.x;
    const uint32_t tok = in->tokens[b];
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        tok_out[b] = tok;
        rowpos[b] = in->pos + b;
    }
    if (i >= H) return;
    uint32_t word = emb.w[(size_t)tok * (H / 8) + i / 8];
    uint32_t g = i / 64;
    float s = bf16f(emb.s[(size_t)tok * (H / 64) + g]), bb = bf16f(emb.b[(size_t)tok * (H / 64) + g]);
    float q = (float)((word >> (4 * (i % 8))) & 15u);
    float e = __fadd_rn(__fmul_rn(s, q), bb);
    for (uint32_t k = 0; k < hc; ++k) hyper[(size_t)b * hc * H + k * H + i] = e;
}

// ---------------------------------------------------------- hc read (down)
// gated_residual first half (cpu.rs:461-475, 493-500): normed = grouped
// RMSNorm(hyper) * w, d = silu(down(normed) / hc), inj = 2 sigmoid(inject(normed) / hc).
// A workgroup takes HR consecutive rows of [down; inject]; wave g takes hc
// stream g, so its RMS is a wave reduction, its normalised inputs are
// prepared once for all HR rows, and the per-stream partial dots meet in LDS.
constexpr int HR = 2;

template <int CPL, int NB>
__global__ void __launch_bounds__(256) k_hc_down(HcDev w, const float* __restrict__ hyper, float* __restrict__ d,
                                                 float* __restrict__ inj, float* __restrict__ inv_out, uint32_t H,
                                                 uint32_t hc, float eps, ActivityArgs act) {
    __shared__ float red[4][HR][NB];
    __shared__ uint32_t hist[ACT_MAX_E];
    const int lane = threadIdx.x & 63, g = (int)wave_id();
    const uint32_t total = w.down.out + (w.has_inject ? w.inject.out : 0u);
    const uint32_t groups = (total + HR - 1) / HR;
    if (blockIdx.x >= groups) {  // the expert-activity workgroups past the rows
        expert_activity_layer(act, blockIdx.x - groups, threadIdx.x, blockDim.x, hist);
        return;
    }
    const uint32_t r0 = blockIdx.x * HR;
    const uint32_t hh = H * hc, nch = H >> 5;  // chunks per stream
    // this stream's inputs first, then every weight load of the HR rows:
    // the RMS and the normalised pairs are formed while the weights fly
    float xin[NB][CPL][32];
    uint4 nrm[CPL][4];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const uint32_t cc = min(lane + 64u * c, nch - 1);
#pragma unroll
        for (int b = 0; b < NB; ++b) ldx32(hyper + (size_t)b * hh + (size_t)g * H + cc * 32, xin[b][c]);
        const uint4* np = reinterpret_cast<const uint4*>(w.norm + (size_t)g * H + cc * 32);
#pragma unroll
        for (int q = 0; q < 4; ++q) nrm[c][q] = np[q];
    }
    asm volatile("" ::: "memory");  // compiler-only: weight loads stay behind these
    uint4 wq[HR][CPL];
    uint32_t s16[HR][CPL], b16[HR][CPL];  // raw bf16, one per register
#pragma unroll
    for (int i = 0; i < HR; ++i) {
        const uint32_t row = min(r0 + i, total - 1);
        const Q4Mat& m = row < w.down.out ? w.down : w.inject;
        const uint32_t r = row < w.down.out ? row : row - w.down.out;
        const uint32_t* wr = m.w + (size_t)r * (hh >> 3) + (size_t)g * (H >> 3);
        const uint16_t* sr = m.s + (size_t)r * (hh >> 6) + (size_t)g * (H >> 6);
        const uint16_t* br = m.b + (size_t)r * (hh >> 6) + (size_t)g * (H >> 6);
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const uint32_t ch = min(lane + 64 * c, nch - 1);
            wq[i][c] = ldw4(wr + ch * 4);
            s16[i][c] = sr[ch >> 1];
            b16[i][c] = br[ch >> 1];
        }
    }
    // compiler-only: the input work below may not be hoisted above the
    // weight loads
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int j = 0; j < 32; ++j) asm volatile("" : "+v"(xin[b][c][j])::"memory");
#pragma unroll
        for (int q = 0; q < 4; ++q)
            asm volatile("" : "+v"(nrm[c][q].x), "+v"(nrm[c][q].y), "+v"(nrm[c][q].z), "+v"(nrm[c][q].w)::"memory");
    }
    const Q4Consts k;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        float sq4[4] = {0.0f, 0.0f, 0.0f, 0.0f}, xs[CPL];
        h2 hi[CPL][16], lo[CPL][16];
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const uint32_t ch = lane + 64 * c, cc = min(ch, nch - 1);
            float (&xv)[32] = xin[b][c];
            // four independent partial sums per reduction (short chains)
            float t4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint4 nv = nrm[c][q];
                const uint32_t nn[4] = {nv.x, nv.y, nv.z, nv.w};
#pragma unroll
                for (int h = 0; h < 8; ++h) {
                    const int j = q * 8 + h;
                    const float wn = __uint_as_float(h & 1 ? nn[h >> 1] & 0xffff0000u : nn[h >> 1] << 16);
                    const float xj = ch < nch ? xv[j] : 0.0f;
                    sq4[h & 3] += xj * xj;
                    xv[j] = xj * wn;
                    t4[h & 3] += xv[j];
                }
            }
            xs[c] = (t4[0] + t4[1]) + (t4[2] + t4[3]);
            x_pairs(xv, hi[c], lo[c]);
        }
        const float sq = (sq4[0] + sq4[1]) + (sq4[2] + sq4[3]);
        const float inv = 1.0f / sqrtf(wave_sum(sq) / (float)H + eps);
        if (blockIdx.x == 0 && lane == 0) inv_out[b * hc + g] = inv;
#pragma unroll
        for (int i = 0; i < HR; ++i) {
            float part = 0.0f;
#pragma unroll
            for (int c = 0; c < CPL; ++c)
                part += q4_chunk_h(wq[i][c], hi[c], lo[c], xs[c], bf16f(s16[i][c]), bf16f(b16[i][c]), k);
            part = wave_sum(part) * inv;
            if (lane == 0) red[g][i][b] = part;
        }
    }
    __syncthreads();
    if (threadIdx.x < HR * NB) {
        const uint32_t i = threadIdx.x / NB, b = threadIdx.x % NB, row = r0 + i;
        if (row < total) {
            float tot = 0.0f;
            for (uint32_t gg = 0; gg < hc; ++gg) tot += red[gg][i][b];
            const float v = tot / (float)hc;
            if (row < w.down.out) d[(size_t)b * w.down.out + row] = siluf_(v);
            else inj[b * hc + (row - w.down.out)] = 2.0f * sigmoidf_(v);
        }
    }
}

// ------------------------------------------------------ hc read (up + mix)
// mixed[i] = (1/hc) sum_g sigmoid(up(d)[g H + i]) * normed[g H + i]
// (cpu.rs:477-491).  A wave has RPW = 64/LPR row slots; slot k serves
// stream k % hc of output group k / hc, R outputs per group.
template <int LPR, int R, int NB>
__global__ void __launch_bounds__(256) k_hc_up_mix(HcDev w, const float* __restrict__ hyper, const float* __restrict__ inv,
                            const float* __restrict__ d, float* __restrict__ mixed, uint32_t H, uint32_t hc) {
    constexpr int RPW = 64 / LPR;
    __shared__ float red[4][NB][64];
    const int lane = threadIdx.x & 63, wv = (int)wave_id(), lir = lane % LPR, k = lane / LPR;
    const uint32_t groups = RPW / hc;
    const uint32_t o0 = global_wave() * groups * R;
    const uint32_t g = k % hc, og = k / hc;
    const bool slot_ok = (uint32_t)k < groups * hc;
    uint32_t rows[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
        uint32_t o = o0 + og * R + i;
        rows[i] = g * H + (o < H ? o : H - 1);
    }
    // d first: its quantisation then overlaps the up rows' flight
    XqStaged<1, 256> xs;
    const bool staged = xs.fits(w.up.in, NB);
    if (staged) xs.load(d, w.down.out, w.up.in, NB);
    Q4Frag<LPR, 1, R> f;
    f.issue(w.up, rows, lir);
    // the row-group leader prefetches hyper, inv and w for its outputs'
    // normed = hyper * inv * w, formed only at the end (using them here
    // would wait for every weight load issued above)
    float hyv[R][NB], invv[NB];
    uint32_t wnr[R];  // raw bf16, one per register (packing would wait)
    if (lir == 0 && slot_ok) {
#pragma unroll
        for (int b = 0; b < NB; ++b) invv[b] = inv[b * hc + g];
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const uint32_t o = min(o0 + og * R + i, H - 1);
            const size_t j = (size_t)g * H + o;
            wnr[i] = w.norm[j];
#pragma unroll
            for (int b = 0; b < NB; ++b) hyv[i][b] = hyper[(size_t)b * H * hc + j];
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (staged) xs.store(w.up.in, NB, xq_lds, XqIdentity{});
    else xq_prep(d, w.down.out, w.up.in, NB, xq_lds, XqIdentity{});
    XqFrag<NB, 1> xr;
    xr.template read<LPR>(xq_lds, w.up.in >> 5, lir);
    float acc[R][NB];
    f.template dot<NB>(xr, acc);
    if (lir == 0 && slot_ok) {
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const uint32_t o = o0 + og * R + i;
#pragma unroll
            for (int b = 0; b < NB; ++b)
                red[wv][b][(og * R + i) * hc + g] =
                    o < H ? sigmoidf_(acc[i][b]) * (hyv[i][b] * invv[b] * __uint_as_float(wnr[i] << 16)) : 0.0f;
        }
    }
    __syncthreads();
    if ((uint32_t)lane < groups * R) {
        const uint32_t o = o0 + lane;
        if (o < H)
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                float s = 0.0f;
                for (uint32_t gg = 0; gg < hc; ++gg) s += red[wv][b][lane * hc + gg];
                mixed[(size_t)b * H + o] = s / (float)hc;
            }
    }
}

// ------------------------------------------------- multi-segment Q4 matvec
// Several matrices over one input width in one launch (horizontal fusion),
// R rows per wave per grid-stride step, per-segment epilogues.
// Per-row epilogue inputs, fetched by lane i for row i while the weights
// are in flight.
// The bf16 parameters stay raw, one per 32-bit register, until the
// epilogue: converting (or packing) them at the load would make the wave
// wait for each one, and for every weight load issued before it, there.
struct EpiIn {
    float hist[8];
    uint32_t cw[9];
    uint32_t p0, p1;
};

CHK_DEV void epi_prefetch(const SegArgs& a, const Seg& sg, uint32_t r, EpiIn& e) {
    if (sg.epi == EPI_DN_CONV) {
        const uint32_t km1 = a.ck - 1;
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j)
            if (j < km1) e.hist[j] = a.hist[(size_t)r * km1 + j];
#pragma unroll
        for (uint32_t j = 0; j < 9; ++j)
            if (j < a.ck) e.cw[j] = a.conv_w[(size_t)r * a.ck + j];
        // compiler-only, in each branch: without it the two branches' last
        // load-and-store (cw[8] here, p1 below) are merged into one store
        // through a pointer phi, which keeps EpiIn in scratch memory
        asm volatile("" ::: "memory");
    } else if (sg.epi == EPI_DN_DECAY) {
        e.p0 = a.a_log[r];
        e.p1 = a.dt_bias[r];
        asm volatile("" ::: "memory");
    }
    asm volatile("" ::: "memory");  // compiler-only: later loads stay behind these
    __builtin_amdgcn_sched_barrier(0);
}

template <int NB>
CHK_DEV void seg_epilogue(const SegArgs& a, const Seg& sg, uint32_t r, const float (&acc)[NB], EpiIn& e) {
    // compiler-only: the prefetched values are redefined here, so no work
    // on them (exp(A_log), the history products) is hoisted to the
    // prefetch, where it would wait for the whole weight stream
#pragma unroll
    for (int j = 0; j < 8; ++j) asm volatile("" : "+v"(e.hist[j]));
#pragma unroll
    for (int j = 0; j < 9; ++j) asm volatile("" : "+v"(e.cw[j]));
    asm volatile("" : "+v"(e.p0), "+v"(e.p1));
    switch (sg.epi) {
    case EPI_RAW:
#pragma unroll
        for (int b = 0; b < NB; ++b) sg.y[(size_t)b * sg.ys + r] = acc[b];
        break;
    case EPI_DN_CONV: {
        // causal_conv (cpu.rs:1067-1085) for channel r, rows in order;
        // history snapshots after every row but the last (conv_b,
        // deltanet.metal:37-42).
        // history slots are shifted with compile-time indices (km1 <= 8)
        const uint32_t km1 = a.ck - 1;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const float cur = acc[b];
            float wl = 0.0f;
#pragma unroll
            for (uint32_t j = 0; j < 9; ++j)
                if (j == km1) wl = __uint_as_float(e.cw[j] << 16);
            float s = wl * cur;
#pragma unroll
            for (uint32_t j = 0; j < 8; ++j)
                if (j < km1) s += __uint_as_float(e.cw[j] << 16) * e.hist[j];
#pragma unroll
            for (uint32_t j = 0; j < 7; ++j)
                if (j + 1 < km1) e.hist[j] = e.hist[j + 1];
#pragma unroll
            for (uint32_t j = 0; j < 8; ++j)
                if (j + 1 == km1) e.hist[j] = cur;
            sg.y[(size_t)b * sg.ys + r] = siluf_(s);
            if (a.snap && b + 1 < NB) {
                float* sp = a.snap_hist + (size_t)b * a.conv_dim * km1 + (size_t)r * km1;
#pragma unroll
                for (uint32_t j = 0; j < 8; ++j)
                    if (j < km1) sp[j] = e.hist[j];
            }
        }
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j)
            if (j < km1) a.hist[(size_t)r * km1 + j] = e.hist[j];
        break;
    }
    case EPI_DN_DECAY:
        // g = -exp(A_log) * softplus(a + dt_bias), decay = e^g (cpu.rs:775-777)
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const float gg = -expf(__uint_as_float(e.p0 << 16)) * softplusf_(acc[b] + __uint_as_float(e.p1 << 16));
            sg.y[(size_t)b * sg.ys + r] = expf(gg);
        }
        break;
    case EPI_DN_BETA:
#pragma unroll
        for (int b = 0; b < NB; ++b) sg.y[(size_t)b * sg.ys + r] = sigmoidf_(acc[b]);
        break;
    }
}

template <int CPL, int R, int NB>
__global__ void __launch_bounds__(256) k_qmv(SegArgs a) {
    const int lane = threadIdx.x & 63;
    const uint32_t groups = (a.total + R - 1) / R;
    const uint32_t nch = a.seg[0].m.in >> 5;  // every segment shares x (launch_qmv checks)
    XqFrag<NB, CPL> xr;
    // First pass: the epilogue inputs, then x, then the weights go out, and
    // the workgroup quantises x while the weights fly (waves without a
    // group still join that prep).  The epilogue loads come first because
    // their count differs between segments: behind x they would make the
    // compiler's wait for x cover the weights.  The pass is peeled: a loop
    // around it would make the compiler wait at the loop head for x too.
    XqStaged<NB, 256> xs;
    const bool staged = xs.fits(a.seg[0].m.in, NB);
    auto pass_body = [&](uint32_t grp, auto first) {
        constexpr bool FIRST = decltype(first)::value;
        const bool live = grp < groups;
        const uint32_t row0 = (live ? grp : 0) * R;
        int si = 0;
#pragma unroll
        for (int k = 1; k < MAX_SEG; ++k)
            if (k < a.nseg && row0 >= a.seg[k].row0) si = k;
        const Seg& sg = a.seg[si];
        // segments hold whole blocks of R rows except a lone segment's tail
        uint32_t rows[R];
#pragma unroll
        for (int i = 0; i < R; ++i) rows[i] = min(row0 - sg.row0 + i, sg.m.out - 1);
        // lane i < R owns row i's epilogue; its inputs load ahead of the weights
        uint32_t my_row = rows[0];
#pragma unroll
        for (int i = 1; i < R; ++i)
            if (lane == i) my_row = rows[i];
        EpiIn e;
        if (live && lane < R) epi_prefetch(a, sg, my_row, e);
        if constexpr (FIRST) {
            if (staged) xs.load(a.seg[0].x, a.seg[0].xs, a.seg[0].m.in, NB);
        }
        Q4Frag<64, CPL, R> f;
        f.issue(sg.m, rows, lane);  // dead waves load clamped rows, unused
        if constexpr (FIRST) {
            if (staged) xs.store(a.seg[0].m.in, NB, xq_lds, XqIdentity{});
            else xq_prep(a.seg[0].x, a.seg[0].xs, a.seg[0].m.in, NB, xq_lds, XqIdentity{});
            xr.template read<64>(xq_lds, nch, lane);
        }
        if (!live) return;
        float acc[R][NB];
        f.template dot<NB>(xr, acc);
        float mine[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            mine[b] = acc[0][b];
#pragma unroll
            for (int i = 1; i < R; ++i)
                if (lane == i) mine[b] = acc[i][b];
        }
        if (lane < R && row0 - sg.row0 + lane < sg.m.out) seg_epilogue<NB>(a, sg, my_row, mine, e);
    };
    pass_body(global_wave(), std::true_type{});
    for (uint32_t grp = global_wave() + total_waves(); grp < groups; grp += total_waves())
        pass_body(grp, std::false_type{});
}

// --------------------------------------------- Q4 matvec + hyper inject
// out = W x; hyper[b][g H + r] += out * inj[b][g] (inject, cpu.rs:971-979).
// XM_DN_GATED: x is the DeltaNet core output y, gated here as
// rmsnorm(y_head) * w * sigmoid(z) (cpu.rs:814-826, eps 1e-6), the head's
// sum of squares coming from the scan's per-block partials.
// XM_DN_GATED input transform: scale 8 inputs by their value head's
// 1/sqrt(mean(y^2) + 1e-6), the head's sum of squares summed from the
// scan's per-block partials.
struct DnGateScale {
    const InjArgs* a;
    CHK_DEV void operator()(uint32_t b, uint32_t e, float (&v)[8]) const {
        const uint32_t head = e / a->dv;
        const float4* sp = reinterpret_cast<const float4*>(a->ssq + ((size_t)b * a->nheads + head) * a->ssq_blocks);
        float ss = 0.0f;
        for (uint32_t k = 0; k < a->ssq_blocks / 4; ++k) {
            const float4 q = sp[k];
            ss += (q.x + q.y) + (q.z + q.w);
        }
        const float inv = 1.0f / sqrtf(ss / (float)a->dv + 1e-6f);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] *= inv;
    }
};

template <int CPL, int R, int NB, int XM>
__global__ void __launch_bounds__(256) k_qmv_inject(InjArgs a) {
    const int lane = threadIdx.x & 63;
    const Q4Mat& m = a.m;
    const uint32_t nch = m.in >> 5, H = m.out;
    const uint32_t groups = m.out / R;
    // lane (i, g) = (lane / hc, lane % hc) owns hyper[b][g H + row_i]
    const uint32_t li = lane / a.hc, lg = lane % a.hc;
    const bool owner = li < (uint32_t)R && a.hyper;
    XqFrag<NB, CPL> xr;
    // plain inputs load ahead of the weights (see XqStaged)
    // (first pass peeled, and the hyper loads ahead of x, as in k_qmv)
    XqStaged<(NB < 2 ? 2 : NB), 256> xs;
    const bool staged = XM != XM_DN_GATED && xs.fits(m.in, NB);
    auto pass_body = [&](uint32_t grp, auto first) {
        constexpr bool FIRST = decltype(first)::value;
        const bool live = grp < groups;
        const uint32_t g0 = live ? grp : 0;
        uint32_t rows[R];
#pragma unroll
        for (int i = 0; i < R; ++i) rows[i] = g0 * R + i;
        float hy[NB], ij[NB];
        if (live && owner)
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                hy[b] = a.hyper[(size_t)b * H * a.hc + lg * H + g0 * R + li];
                ij[b] = a.inj[b * a.hc + lg];
            }
        asm volatile("" ::: "memory");  // compiler-only: x and the weights stay behind
        // the scan's chunks and the first SQ float4 of their heads' sums of
        // squares load ahead of the weights too (branch-free), so neither
        // waits behind them
        constexpr uint32_t SQ = 2;
        XqChunk q0[NB][CPL];
        float4 sq0[NB][CPL][SQ];
        const bool chunks = XM == XM_DN_GATED && a.x_xq;
        if constexpr (FIRST) {
            if (staged) xs.load(a.x, a.xs, m.in, NB);
            if (chunks) {
                const uint32_t nq = a.ssq_blocks / 4;
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    const uint32_t cc = min(lane + 64u * c, nch - 1);
                    const uint32_t head = cc * 32 / a.dv;
#pragma unroll
                    for (int b = 0; b < NB; ++b) {
                        q0[b][c] = a.x_xq[(size_t)b * nch + cc];
                        const float4* sp =
                            reinterpret_cast<const float4*>(a.ssq + ((size_t)b * a.nheads + head) * a.ssq_blocks);
#pragma unroll
                        for (uint32_t k = 0; k < SQ; ++k) sq0[b][c][k] = sp[min(k, nq - 1)];
                    }
                }
            }
            asm volatile("" ::: "memory");  // compiler-only: the weights stay behind these
        }
        Q4Frag<64, CPL, R> f;
        f.issue(m, rows, lane);  // dead waves load clamped rows, unused
        if constexpr (FIRST) {
            if (chunks) {
                // the scan's chunks of y w sigmoid(z), scaled by their head's
                // 1/rms: a common factor of m, d and the chunk sum
                const uint32_t nq = a.ssq_blocks / 4;
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    const uint32_t cc = min(lane + 64u * c, nch - 1);
                    const uint32_t head = cc * 32 / a.dv;
#pragma unroll
                    for (int b = 0; b < NB; ++b) {
                        XqChunk q = q0[b][c];
                        const float4* sp =
                            reinterpret_cast<const float4*>(a.ssq + ((size_t)b * a.nheads + head) * a.ssq_blocks);
                        float ss = 0.0f;
#pragma unroll
                        for (uint32_t k = 0; k < SQ; ++k)
                            if (k < nq) ss += (sq0[b][c][k].x + sq0[b][c][k].y) + (sq0[b][c][k].z + sq0[b][c][k].w);
                        for (uint32_t k = SQ; k < nq; ++k) {
                            const float4 v = sp[k];
                            ss += (v.x + v.y) + (v.z + v.w);
                        }
                        const float inv = 1.0f / sqrtf(ss / (float)a.dv + 1e-6f);
                        q.prm.x *= inv;
                        q.prm.y *= inv;
                        q.prm.z *= inv;
                        xr.c[b][c] = q;
                    }
                }
            } else {
                if (XM == XM_DN_GATED) xq_prep(a.x, a.xs, m.in, NB, xq_lds, DnGateScale{&a});
                else if (staged) xs.store(m.in, NB, xq_lds, XqIdentity{});
                else xq_prep(a.x, a.xs, m.in, NB, xq_lds, XqIdentity{});
                xr.template read<64>(xq_lds, nch, lane);
            }
        }
        if (!live) return;
        float acc[R][NB];
        f.template dot<NB>(xr, acc);
        if (a.raw_out && lane < R) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                float v = acc[0][b];
#pragma unroll
                for (int i = 1; i < R; ++i)
                    if (lane == i) v = acc[i][b];
                a.raw_out[(size_t)b * H + rows[0] + lane] = v;
            }
        }
        if (owner) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                float v = acc[0][b];
#pragma unroll
                for (int i = 1; i < R; ++i)
                    if (li == (uint32_t)i) v = acc[i][b];
                a.hyper[(size_t)b * H * a.hc + lg * H + grp * R + li] = hy[b] + v * ij[b];
            }
        }
    };
    pass_body(global_wave(), std::true_type{});
    for (uint32_t grp = global_wave() + total_waves(); grp < groups; grp += total_waves())
        pass_body(grp, std::false_type{});
}

// ------------------------------------------------------- DeltaNet step
// One wave per (value head, 16 value lanes): that slice of the head's fp32
// state [dv][dk] (transposed relative to cpu.rs, as delta_scan2 keeps it)
// lives in VGPRs, 4 lanes per value lane, 32 key lanes each.  Per row:
// L2-normalise the key head's q (times dk^-1/2) and k (eps 1e-6),
// S <- decay S, delta = beta (v - S^T k), S <- S + k delta^T, y = S^T q
// (cpu.rs:745-812); snapshots after rows < nb-1.  The gated RMSNorm needs
// the whole head, so each wave leaves its share of sum(y^2) for the
// out-projection's prologue.
// A workgroup (two waves) takes 32 value lanes of one head, so each row's
// gated outputs form one 32-value chunk that leaves in nibble planes too.
template <int NB>
__global__ void __launch_bounds__(DN_SCAN_COLS * 4) k_dn_scan(DnScanArgs a) {
    constexpr int DK = 128, TPC = 4, KPT = DK / TPC, COLS = DN_SCAN_COLS;
    __shared__ float ys[COLS];
    const uint32_t blocks = a.dv / COLS;
    const uint32_t hv = blockIdx.x / blocks, blk = blockIdx.x % blocks;
    const int t = threadIdx.x, p = t % TPC;
    const uint32_t iv = blk * COLS + t / TPC;
    const uint32_t hk = hv / (a.nv / a.nk);
    float S[KPT];
    float* sp = a.state + ((size_t)hv * a.dv + iv) * DK + p * KPT;
#pragma unroll
    for (int k = 0; k < KPT; k += 4) {
        float4 v = *reinterpret_cast<const float4*>(sp + k);
        S[k] = v.x; S[k + 1] = v.y; S[k + 2] = v.z; S[k + 3] = v.w;
    }
    for (int b = 0; b < NB; ++b) {
        const float* row = a.conv_out + (size_t)b * a.conv_dim;
        float q[KPT], kk[KPT];
        float sq = 0.0f, sk = 0.0f;
#pragma unroll
        for (int j = 0; j < KPT; j += 4) {
            float4 qv = *reinterpret_cast<const float4*>(row + hk * DK + p * KPT + j);
            float4 kv = *reinterpret_cast<const float4*>(row + a.qk_dim + hk * DK + p * KPT + j);
            q[j] = qv.x; q[j + 1] = qv.y; q[j + 2] = qv.z; q[j + 3] = qv.w;
            kk[j] = kv.x; kk[j + 1] = kv.y; kk[j + 2] = kv.z; kk[j + 3] = kv.w;
        }
        // every other input of the row too (the state above for the first):
        // one round trip, not one per use
        const float decay = a.decay[b * a.nv + hv], beta = a.beta[b * a.nv + hv];
        const float v = row[2 * a.qk_dim + hv * a.dv + iv];
        const size_t jy = (size_t)b * a.nv * a.dv + hv * a.dv + iv;
        const float zr = a.z[jy];
        const uint32_t nr = a.norm[iv];
        asm volatile("" ::: "memory");  // compiler-only: no load sinks below this
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < KPT; ++j) {
            sq += q[j] * q[j];
            sk += kk[j] * kk[j];
        }
        sq = group_sum<TPC>(sq);
        sk = group_sum<TPC>(sk);
        const float iq = 1.0f / sqrtf(sq + 1e-6f), ik = 1.0f / sqrtf(sk + 1e-6f);
#pragma unroll
        for (int j = 0; j < KPT; ++j) {
            q[j] = q[j] * iq * a.qscale;
            kk[j] *= ik;
        }
        float kvm = 0.0f;
#pragma unroll
        for (int j = 0; j < KPT; ++j) {
            S[j] *= decay;
            kvm += S[j] * kk[j];
        }
        kvm = group_sum<TPC>(kvm);
        const float delta = (v - kvm) * beta;
        float y = 0.0f;
#pragma unroll
        for (int j = 0; j < KPT; ++j) {
            S[j] += kk[j] * delta;
            y += S[j] * q[j];
        }
        y = group_sum<TPC>(y);
        if (a.snap && b + 1 < NB) {
            float* pp = a.snap_state + (size_t)b * a.nv * a.dv * DK + ((size_t)hv * a.dv + iv) * DK + p * KPT;
#pragma unroll
            for (int k = 0; k < KPT; k += 4)
                *reinterpret_cast<float4*>(pp + k) = make_float4(S[k], S[k + 1], S[k + 2], S[k + 3]);
        }
        // gated RMSNorm numerator: y * w * sigmoid(z); the head's
        // 1/rms (from the partial sums of y^2, one per 16 value lanes) is
        // applied by the consumer
        const float ss = wave_sum(p == 0 ? y * y : 0.0f);
        if (p == 0) {
            const float yv = y * __uint_as_float(nr << 16) * sigmoidf_(zr);
            a.y[jy] = yv;
            ys[t / TPC] = yv;
        }
        if ((t & 63) == 0) a.ssq[((size_t)b * a.nv + hv) * (a.dv / 16) + blk * (COLS / 16) + (t >> 6)] = ss;
        {
            __syncthreads();
            if (t < 64) xq_chunk_store(ys, a.y_xq + (size_t)b * (a.nv * a.dv / COLS) + hv * blocks + blk, t);
            __syncthreads();
        }
    }
#pragma unroll
    for (int k = 0; k < KPT; k += 4) *reinterpret_cast<float4*>(sp + k) = make_float4(S[k], S[k + 1], S[k + 2], S[k + 3]);
}

// ------------------------------------------------------------ router
// logits = W_r x (bf16 [E][H]) and the shared-expert gate dot as row E
// (cpu.rs:506-508, 534-535).  Softmax/top-k happen in the experts
// kernel's prologue.
template <int R, int NB>
__global__ void __launch_bounds__(256) k_router(RouterArgs a) {
    const int lane = threadIdx.x & 63;
    const uint32_t H = a.H, nch = H >> 5, rows_total = a.E + 1;
    const uint32_t groups = (rows_total + R - 1) / R;
    for (uint32_t grp = global_wave(); grp < groups; grp += total_waves()) {
        float acc[R][NB];
#pragma unroll
        for (int i = 0; i < R; ++i)
#pragma unroll
            for (int b = 0; b < NB; ++b) acc[i][b] = 0.0f;
        // lane l takes input chunk c0 + l (32 inputs) of each pass; one pass
        // covers 2048 inputs
        for (uint32_t c0 = 0; c0 < nch; c0 += 64) {
            uint4 wq[R][4];
            const uint32_t ch = c0 + lane;
#pragma unroll
            for (int i = 0; i < R; ++i) {
                uint32_t row = grp * R + i;
                if (row > a.E) row = a.E;
                const uint16_t* wr = row < a.E ? a.router + (size_t)row * H : a.shared_gate;
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    wq[i][k] = ch < nch ? ldw4(reinterpret_cast<const uint32_t*>(wr + ch * 32) + 4 * k)
                                        : make_uint4(0, 0, 0, 0);
            }
            XFrag<NB, 1> xr;
            xr.template load<64>(a.x + (size_t)c0 * 32, H, nch - c0, lane);
#pragma unroll
            for (int i = 0; i < R; ++i) {
#pragma unroll
                for (int b = 0; b < NB; ++b) {
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const uint32_t uu[4] = {wq[i][k].x, wq[i][k].y, wq[i][k].z, wq[i][k].w};
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            acc[i][b] += __uint_as_float(uu[j] << 16) * xr.v[b][0][k * 8 + 2 * j];
                            acc[i][b] += __uint_as_float(uu[j] & 0xffff0000u) * xr.v[b][0][k * 8 + 2 * j + 1];
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const uint32_t row = grp * R + i;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const float t = wave_sum(acc[i][b]);
                if (lane == 0 && row <= a.E) {
                    if (row < a.E) a.logits[(size_t)b * a.E + row] = t;
                    else a.sg[b] = t;
                }
            }
        }
    }
}

// ----------------------------------------------------- experts: gate/up
// act[b][slot][i] = silu(gate_i . x_b) * (up_i . x_b) for the top-k routed
// experts of row b (slots 0..k-1) and the shared expert (slot k) (mlp,
// cpu.rs:981-992).  One task per wave: (row, slot, R consecutive i), the
// gate and up rows of all R loaded together.  A routed wave ranks its own
// row's experts (route_row) down to its slot while its x loads are in
// flight; the wave of slot k-1, i0 = 0 ranks all k and publishes the
// routing (ids, renormalised weights) for the down kernel.
// The routing of row b for the down kernel: ids in rank order and weights
// renormalised by the chosen probabilities summed in rank order
// (cpu.rs:516-525); lane r holds rank r (route_row).
CHK_DEV void publish_routing(const MoeArgs& a, uint32_t b, int lane, uint32_t my_id, float my_p) {
    float topsum = 0.0f;
    for (uint32_t r = 0; r < a.topk; ++r) topsum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_p), (int)r));
    if ((uint32_t)lane < a.topk) {
        a.ids_out[b * a.topk + lane] = my_id;
        a.w_out[b * a.topk + lane] = a.norm_topk ? my_p / topsum : my_p;
    }
}

// A workgroup of GU_WAVES waves covers one 32-row chunk of one (row, slot),
// R = 32 / GU_WAVES rows per wave, so the chunk's act values meet in LDS
// and leave quantised (act_xq, the down kernel's input form) as well as
// in f32.
#ifndef CHK_GU_WAVES
#define CHK_GU_WAVES 8
#endif
constexpr uint32_t GU_WAVES = CHK_GU_WAVES;
constexpr uint32_t GU_WG = 64 * GU_WAVES;

// CPL: input chunks per lane (hidden sizes up to 2048 CPL).
// MIXED: a low-bit launch whose records may be switched to their 4-bit
// copies (a.kinds set); else every routed record is decoded at X.bits.
template <int R, int BITS, int CPL, bool MIXED>
__global__ void __launch_bounds__(GU_WG) k_moe_gate_up(MoeArgs a) {
    static_assert(R * GU_WAVES == 32, "a workgroup covers one 32-row chunk");
    __shared__ float act_s[32];
    const int lane = threadIdx.x & 63;
    const uint32_t w = wave_id();
    // a row's tasks: topk routed slots of cpr chunks, then the shared
    // expert's cps chunks
    const uint32_t cpr = a.I / 32, cps = a.SI / 32, per_row = a.topk * cpr + cps;
    const uint32_t task = blockIdx.x;
    const uint32_t b = task / per_row, t = task % per_row;
    const bool shared_task = t >= a.topk * cpr;
    const uint32_t slot = shared_task ? a.topk : t / cpr, c = shared_task ? t - a.topk * cpr : t % cpr;
    const size_t act_off = (size_t)b * (a.topk * a.I + a.SI) + slot * a.I;  // this slot's act values
    const size_t xq_off = (size_t)b * per_row + slot * cpr;                  // and its chunks
    const uint32_t i0 = c * 32 + w * R;
    uint32_t rows[R];
#pragma unroll
    for (int i = 0; i < R; ++i) rows[i] = i0 + i;
    const uint32_t nch = a.H >> 5;
    const bool routed = slot < a.topk;
    const bool publish = slot + 1 == a.topk && c == 0 && w == 0;
    // x (independent of the routing) first, so its quantisation overlaps
    // the expert weights' flight
    XqStaged<2, GU_WG> xs;
    const bool staged = xs.fits(a.H, a.nb);
    if (staged) xs.load(a.x, a.H, a.H, a.nb);
    // mixed stores: this lane's 8 experts' kinds (the lanes' expert split of
    // route_row), in flight with the logits
    uint32_t kw0 = 0, kw1 = 0;
    if (MIXED && routed) {
        const uint2 kv = *reinterpret_cast<const uint2*>(a.kinds + (size_t)a.record_layer * a.E +
                                                         min((uint32_t)lane * 8u, a.E - 8u));
        kw0 = kv.x;
        kw1 = kv.y;
    }
    uint32_t my_id = 0;
    float my_p = 0.0f;
    if (routed)
        route_row(a.logits + (size_t)b * a.E, a.E, publish ? a.topk : slot + 1, lane,
                  publish && a.probs ? a.probs + (size_t)b * a.E : nullptr, my_id, my_p);
    const uint32_t e = routed ? min((uint32_t)__builtin_amdgcn_readlane((int)my_id, (int)slot), a.X.experts - 1) : 0u;
    // a low-bit launch decodes routed records of kind != 0 at X.bits and the
    // rest from their 4-bit copies (the kind byte of expert e: lane e / 8)
    bool low = BITS != 4 && routed;
    if (MIXED && routed) {
        const uint32_t kw = (uint32_t)__builtin_amdgcn_readlane((int)((e & 4u) ? kw1 : kw0), (int)(e >> 3));
        low = ((kw >> (8u * (e & 3u))) & 0xffu) != 0u;
    }
    const uint8_t* rec = a.X.base + ((size_t)a.record_layer * a.X.experts + e) * a.X.stride;
    float g[R][1], u[R][1];
    // Q4 routed and shared rows share one straight path (only the matrices
    // differ); low-bit routed rows take their own fragments.  The prep sits
    // outside both so every wave reaches its barrier at the same point.
    const bool q4path = BITS == 4 || !low;
    Q4Frag<64, CPL, R> fg, fu;
    ExpFrag<64, CPL, R, BITS> lg, lu;
    if (q4path) {
        Q4Mat mg = a.sh_gate, mu = a.sh_up;
        if ((BITS == 4 || MIXED) && routed) {
            const ExpertsDev& XQ = BITS == 4 ? a.X : a.X4;
            const uint8_t* rq = XQ.base + ((size_t)a.record_layer * XQ.experts + e) * XQ.stride;
            const ExpMat eg = expert_mat(XQ, rq, 0, a.I, a.H), eu = expert_mat(XQ, rq, 1, a.I, a.H);
            mg = Q4Mat{(const uint32_t*)eg.w, eg.s, eg.b, a.I, a.H};
            mu = Q4Mat{(const uint32_t*)eu.w, eu.s, eu.b, a.I, a.H};
        }
        fg.issue(mg, rows, lane);
        fu.issue(mu, rows, lane);
    } else if (BITS != 4) {
        lg.issue(expert_mat(a.X, rec, 0, a.I, a.H), rows, lane);
        lu.issue(expert_mat(a.X, rec, 1, a.I, a.H), rows, lane);
    }
    if (publish) publish_routing(a, b, lane, my_id, my_p);
    if (staged) xs.store(a.H, a.nb, xq_lds, XqIdentity{});
    else xq_prep<GU_WG>(a.x, a.H, a.H, a.nb, xq_lds, XqIdentity{});
    XqFrag<1, CPL> xq;
    xq.template read<64>(xq_lds + b * nch, nch, lane);
    if (q4path) {
        fg.template dot<1>(xq, g);
        fu.template dot<1>(xq, u);
    } else if constexpr (BITS != 4) {
        lg.template dot<1>(xq, g);
        lu.template dot<1>(xq, u);
    }
    if (lane < R) {
        float gv = g[0][0], uv = u[0][0];
#pragma unroll
        for (int i = 1; i < R; ++i)
            if (lane == i) {
                gv = g[i][0];
                uv = u[i][0];
            }
        const float act = siluf_(gv) * uv;
        a.act[act_off + i0 + lane] = act;
        act_s[w * R + lane] = act;
    }
    __syncthreads();
    if (w == 0) xq_chunk_store(act_s, a.act_xq + xq_off + c, lane);
}

// ------------------------------------------------- experts: down + combine
// out[r] = sum_j w_j down_j(act_j)[r] + sigmoid(shared_gate . x) shared_down(act_k)[r]
// (cpu.rs:527-540), then hyper[g H + r] += out * inj_g.  A wave covers R
// output rows; its 64/LPR lane groups take one expert slot each per pass.
// Two dependent round trips: the routing (ids, weights), then every pass's
// weight rows and activations at once.
template <int LPR, int R, int BITS, int PASSES, bool MIXED>
__global__ void __launch_bounds__(256) k_moe_down(MoeArgs a) {
    constexpr int G = 64 / LPR;
    const int lane = threadIdx.x & 63, grp = lane / LPR, lir = lane % LPR;
    const uint32_t slots = a.topk + 1;
    // act_xq rows: topk routed slots of nch chunks, then the shared
    // expert's nchs
    const uint32_t groups = a.H / R, nch = a.I >> 5, nchs = a.SI >> 5, xrow = a.topk * nch + nchs;
    const uint32_t li = lane / a.hc, lg = lane % a.hc;
    const bool owner = li < (uint32_t)R && a.hyper;
    // routing of every row (lane j < topk: slot j's id and weight; lane
    // topk: the shared expert's gate), loaded raw together with the first
    // (group, row)'s hyper inputs so that one round trip precedes the
    // weights; act comes quantised from gate/up
    // (branch-free clamped loads: a loaded value merged with a default at
    // a branch join is copied there, which waits for the load)
    uint32_t rid[4];
    float rw[4], sgv[4];
    const uint32_t rl = min((uint32_t)lane, a.topk - 1);
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const uint32_t bb = min((uint32_t)b, a.nb - 1);
        rid[b] = a.ids[bb * a.topk + rl];
        rw[b] = a.w[bb * a.topk + rl];
        sgv[b] = a.sg[bb];
    }
    // mixed stores: lane l holds the kinds of experts 8l..8l+7
    uint32_t kw0 = 0, kw1 = 0;
    if (MIXED) {
        const uint2 kv = *reinterpret_cast<const uint2*>(a.kinds + (size_t)a.record_layer * a.E +
                                                         min((uint32_t)lane * 8u, a.E - 8u));
        kw0 = kv.x;
        kw1 = kv.y;
    }
    const uint32_t gi0 = global_wave();
    // the first row's activation chunks do not depend on the routing either
    XqFrag<1, 1> xq0[PASSES];
#pragma unroll
    for (int pass = 0; pass < PASSES; ++pass) {
        const uint32_t slot = grp + pass * G, sl = slot < slots ? slot : slots - 1;
        xq0[pass].template read<LPR>(a.act_xq + (size_t)sl * nch, sl < a.topk ? nch : nchs, lir);
    }
    float hy0 = 0.0f, ij0 = 0.0f;
    if (a.hyper) {
        hy0 = a.hyper[lg * a.H + min(gi0 * R + min(li, (uint32_t)R - 1), a.H - 1)];
        ij0 = a.inj[lg];
    }
    asm volatile("" ::: "memory");  // compiler-only: the weight loads stay behind these
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const bool live = (uint32_t)b < a.nb;
        rid[b] = live && (uint32_t)lane < a.topk ? min(rid[b], a.X.experts - 1) : 0u;
        rw[b] = !live ? 0.0f : (uint32_t)lane < a.topk ? rw[b] : (uint32_t)lane == a.topk ? sigmoidf_(sgv[b]) : 0.0f;
    }
    for (uint32_t gi = gi0; gi < groups; gi += total_waves()) {
        uint32_t rows[R];
#pragma unroll
        for (int i = 0; i < R; ++i) rows[i] = gi * R + i;
        for (uint32_t b = 0; b < a.nb; ++b) {
            uint32_t my_id = rid[0];
            float my_w = rw[0];
#pragma unroll
            for (int k = 1; k < 4; ++k)
                if (b == (uint32_t)k) {
                    my_id = rid[k];
                    my_w = rw[k];
                }
            // hyper of this wave's rows, for the inject below
            float hy = hy0, ij = ij0;
            if (owner && (gi != gi0 || b != 0)) {
                hy = a.hyper[(size_t)b * a.H * a.hc + lg * a.H + rows[0] + li];
                ij = a.inj[b * a.hc + lg];
            }
            // Q4: routed and shared slots share one path (per-lane matrices);
            // low-bit routed slots take their own fragments and f32 inputs
            Q4Frag<LPR, 1, R> fq[PASSES];
            ExpFrag<LPR, 1, R, BITS> fl[PASSES];
            XqFrag<1, 1> xq[PASSES];
            float wgt[PASSES];
            bool low[PASSES];  // a routed slot decoded at X.bits (its kind != 0)
#pragma unroll
            for (int pass = 0; pass < PASSES; ++pass) {
                const uint32_t slot = grp + pass * G;
                const uint32_t sl = slot < slots ? slot : slots - 1;
                const uint32_t e = __shfl(my_id, sl < a.topk ? sl : 0, 64);
                wgt[pass] = __shfl(my_w, sl, 64);
                if (slot >= slots) wgt[pass] = 0.0f;
                low[pass] = BITS != 4 && sl < a.topk;
                if (MIXED) {
                    const uint32_t k0 = __shfl(kw0, (int)(e >> 3), 64), k1 = __shfl(kw1, (int)(e >> 3), 64);
                    low[pass] = low[pass] && ((((e & 4u) ? k1 : k0) >> (8u * (e & 3u))) & 0xffu) != 0u;
                }
                const uint8_t* rec = a.X.base + ((size_t)a.record_layer * a.X.experts + e) * a.X.stride;
                if (BITS != 4 && low[pass]) {
                    fl[pass].issue(expert_mat(a.X, rec, 2, a.H, a.I), rows, lir);
                } else {
                    // the shared expert, or a routed record's 4-bit copy
                    Q4Mat mm = a.sh_down;
                    if ((BITS == 4 || MIXED) && sl < a.topk) {
                        const ExpertsDev& XQ = BITS == 4 ? a.X : a.X4;
                        const uint8_t* rq = XQ.base + ((size_t)a.record_layer * XQ.experts + e) * XQ.stride;
                        const ExpMat em = expert_mat(XQ, rq, 2, a.H, a.I);
                        mm = Q4Mat{(const uint32_t*)em.w, em.s, em.b, a.H, a.I};
                    }
                    fq[pass].issue(mm, rows, lir);
                }
                if (gi == gi0 && b == 0) xq[pass] = xq0[pass];
                else xq[pass].template read<LPR>(a.act_xq + (size_t)b * xrow + sl * nch, sl < a.topk ? nch : nchs, lir);
            }
            float tot[R];
#pragma unroll
            for (int i = 0; i < R; ++i) tot[i] = 0.0f;
#pragma unroll
            for (int pass = 0; pass < PASSES; ++pass) {
                float acc[R][1];
                if constexpr (BITS != 4) {
                    if (low[pass]) fl[pass].template dot<1>(xq[pass], acc);
                    else fq[pass].template dot<1>(xq[pass], acc);
                } else {
                    fq[pass].template dot<1>(xq[pass], acc);
                }
#pragma unroll
                for (int i = 0; i < R; ++i) tot[i] += wgt[pass] * acc[i][0];
            }
            float mine = 0.0f;
#pragma unroll
            for (int i = 0; i < R; ++i) {
                float v = tot[i];
#pragma unroll
                for (int m = LPR; m < 64; m <<= 1) v += __shfl_xor(v, m, 64);
                if (li == (uint32_t)i) mine = v;
                if (a.raw_out && lane == i) a.raw_out[(size_t)b * a.H + rows[i]] = v;
            }
            asm volatile("" : "+v"(hy), "+v"(ij));  // compiler-only: not consumed earlier
            if (owner) a.hyper[(size_t)b * a.H * a.hc + lg * a.H + rows[0] + li] = hy + mine * ij;
        }
    }
}

// ------------------------------------------------------- LM head + argmax
// logits = W_lm mixed; greedy argmax with the lowest index winning ties
// (argmax_partial/argmax_final, kernels/common/sampling.metal:10-84).
// CPL: input chunks per lane (inputs up to 2048 CPL).
template <int R, int NB, int CPL>
__global__ void __launch_bounds__(256) k_lm_head(Q4Mat m, const float* __restrict__ x, float* __restrict__ logits, float* __restrict__ pv,
                          uint32_t* __restrict__ pi) {
    __shared__ float sv[NB][4];
    __shared__ uint32_t si[NB][4];
    const int lane = threadIdx.x & 63, wv = (int)wave_id();
    float bv[NB];
    uint32_t bi[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) { bv[b] = -INFINITY; bi[b] = 0xffffffffu; }
    const uint32_t groups = m.out / R, nch = m.in >> 5;
    // each wave's next row group is in flight while it reduces the current
    // one; x loads first, then the first group's, then the workgroup
    // quantises x
    XqStaged<NB, 256> xs;
    const bool staged = xs.fits(m.in, NB);
    if (staged) xs.load(x, m.in, m.in, NB);
    uint32_t grp = global_wave();
    uint32_t rows[R];
#pragma unroll
    for (int i = 0; i < R; ++i) rows[i] = grp * R + i;
    Q4Frag<64, CPL, R> f;
    if (grp < groups) f.issue(m, rows, lane);
    if (staged) xs.store(m.in, NB, xq_lds, XqIdentity{});
    else xq_prep(x, m.in, m.in, NB, xq_lds, XqIdentity{});
    XqFrag<NB, CPL> xr;
    xr.template read<64>(xq_lds, nch, lane);
    while (grp < groups) {
        const uint32_t nxt = grp + total_waves();
        uint32_t nrows[R];
#pragma unroll
        for (int i = 0; i < R; ++i) nrows[i] = nxt * R + i;
        Q4Frag<64, CPL, R> fn;
        if (nxt < groups) fn.issue(m, nrows, lane);
        float acc[R][NB];
        f.template dot<NB>(xr, acc);
#pragma unroll
        for (int i = 0; i < R; ++i)
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if (lane == i) logits[(size_t)b * m.out + rows[i]] = acc[i][b];
                if (acc[i][b] > bv[b] || (acc[i][b] == bv[b] && rows[i] < bi[b])) { bv[b] = acc[i][b]; bi[b] = rows[i]; }
            }
        f = fn;
        grp = nxt;
#pragma unroll
        for (int i = 0; i < R; ++i) rows[i] = nrows[i];
    }
    if (lane == 0)
#pragma unroll
        for (int b = 0; b < NB; ++b) { sv[b][wv] = bv[b]; si[b][wv] = bi[b]; }
    __syncthreads();
    if (threadIdx.x < NB) {
        const int b = threadIdx.x;
        float v = sv[b][0];
        uint32_t i = si[b][0];
        for (int k = 1; k < (int)(CHK_WG >> 6); ++k)
            if (sv[b][k] > v || (sv[b][k] == v && si[b][k] < i)) { v = sv[b][k]; i = si[b][k]; }
        pv[(size_t)b * gridDim.x + blockIdx.x] = v;
        pi[(size_t)b * gridDim.x + blockIdx.x] = i;
    }
}

__global__ void __launch_bounds__(256) k_argmax_final(const float* __restrict__ pv, const uint32_t* __restrict__ pi, uint32_t n,
                               uint32_t* __restrict__ out) {
    __shared__ float sv[256];
    __shared__ uint32_t si[256];
    const uint32_t b = blockIdx.x;
    float v = -INFINITY;
    uint32_t i = 0xffffffffu;
    for (uint32_t k = threadIdx.x; k < n; k += CHK_WG) {
        const float x = pv[(size_t)b * n + k];
        const uint32_t xi = pi[(size_t)b * n + k];
        if (x > v || (x == v && xi < i)) { v = x; i = xi; }
    }
    sv[threadIdx.x] = v;
    si[threadIdx.x] = i;
    __syncthreads();
    for (uint32_t s = CHK_WG / 2; s > 0; s >>= 1) {
        if (threadIdx.x < s) {
            const float x = sv[threadIdx.x + s];
            const uint32_t xi = si[threadIdx.x + s];
            if (x > sv[threadIdx.x] || (x == sv[threadIdx.x] && xi < si[threadIdx.x])) {
                sv[threadIdx.x] = x;
                si[threadIdx.x] = xi;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) out[b] = si[0] == 0xffffffffu ? 0u : si[0];
}

// --------------------------------------------------------------- launchers

#define CHK_NB_SWITCH(nb, CALL) \
    switch (nb) {               \
    case 1: { constexpr int NB = 1; CALL; } break; \
    case 2: { constexpr int NB = 2; CALL; } break; \
    case 3: { constexpr int NB = 3; CALL; } break; \
    default: { constexpr int NB = 4; CALL; } break; \
    }

static uint32_t grid_for(uint32_t waves_needed, uint32_t cap = 2048) {
    uint32_t g = (waves_needed + 3) / 4;
    return std::max<uint32_t>(1, std::min(g, cap));
}

// Dynamic LDS of a kernel that stages nrows input rows of K floats as
// nibble planes (xq_prep), checked against gfx950's per-workgroup limit;
// plain matvecs split their rows above XQ_LDS_SPLIT to keep occupancy.
constexpr size_t XQ_LDS_MAX = 160 * 1024;
constexpr size_t XQ_LDS_SPLIT = 64 * 1024;

static size_t xq_bytes(uint32_t nrows, uint32_t K) {
    if (K % 32) throw std::runtime_error("matvec input width must be a multiple of 32");
    const size_t b = (size_t)nrows * (K / 32) * sizeof(XqChunk);
    if (b > XQ_LDS_MAX) throw std::runtime_error("matvec inputs exceed the workgroup's LDS budget");
    return b;
}

void launch_embed(const StepIn* in, uint32_t* tokens, uint32_t* rowpos, const Q4Mat& emb, float* hyper, uint32_t H,
                  uint32_t hc, int nb, hipStream_t st) {
    dim3 grid((H + 255) / 256, nb);
    k_embed<<<grid, 256, 0, st>>>(in, tokens, rowpos, emb, hyper, H, hc);
}

void launch_hc_down(const HcDev& w, const float* hyper, float* d, float* inj, float* inv, uint32_t H, uint32_t hc,
                    float eps, int nb, hipStream_t st, const ActivityArgs* act) {
    const uint32_t rows = w.down.out + (w.has_inject ? w.inject.out : 0);
    const uint32_t cpl = (H / 32 + 63) / 64;
    if (hc > 4 || cpl > 2) throw std::runtime_error("hyper-connection read supports hc <= 4 and hidden <= 4096");
    ActivityArgs a{};
    if (act && act->act && act->layers && act->rows) {
        if (act->E > ACT_MAX_E) throw std::runtime_error("expert activity counts at most 512 experts per layer");
        a = *act;
    }
    const uint32_t grid = (rows + HR - 1) / HR + a.layers;
    if (cpl <= 1) {
        CHK_NB_SWITCH(nb, (k_hc_down<1, NB><<<grid, 64 * hc, 0, st>>>(w, hyper, d, inj, inv, H, hc, eps, a)))
    } else {
        CHK_NB_SWITCH(nb, (k_hc_down<2, NB><<<grid, 64 * hc, 0, st>>>(w, hyper, d, inj, inv, H, hc, eps, a)))
    }
}

void launch_hc_up_mix(const HcDev& w, const float* hyper, const float* inv, const float* d, float* mixed,
                      uint32_t H, uint32_t hc, int nb, hipStream_t st) {
    const uint32_t nch = w.up.in / 32;
    int lpr = 2;
    while (lpr < (int)nch) lpr <<= 1;
    // a wave holds 64 / lpr row slots, one per stream at least
    if (w.up.in % 32 || lpr > 16 || (uint32_t)lpr * hc > 64)
        throw std::runtime_error("hyper-connection low rank must be a multiple of 32 up to 512 (16 lanes a stream)");
    constexpr int R = 2;
    const uint32_t outs_pw = (64 / lpr) / hc * R;
    const uint32_t grid = grid_for((H + outs_pw - 1) / outs_pw, 1u << 20);
    const size_t lds = xq_bytes(nb, w.up.in);
#define UPMIX(L) CHK_NB_SWITCH(nb, (k_hc_up_mix<L, R, NB><<<grid, 256, lds, st>>>(w, hyper, inv, d, mixed, H, hc)))
    switch (lpr) {
    case 2: UPMIX(2); break;
    case 4: UPMIX(4); break;
    case 8: UPMIX(8); break;
    default: UPMIX(16); break;
    }
#undef UPMIX
}

void launch_qmv(const SegArgs& a, int nb, hipStream_t st) {
    const uint32_t in = a.seg[0].m.in;
    const uint32_t cpl = (in / 32 + 63) / 64;
    if (cpl > 4) throw std::runtime_error("matvec input wider than 8192");
    bool raw = true;
    for (int k = 0; k < a.nseg; ++k) {
        if (a.seg[k].x != a.seg[0].x || a.seg[k].xs != a.seg[0].xs || a.seg[k].m.in != in)
            throw std::runtime_error("segments of one matvec launch must share their input");
        raw = raw && a.seg[k].epi == EPI_RAW;
    }
    // rows of plain segments are independent: split a launch whose staged
    // inputs exceed the LDS budget (only wide test shapes reach this)
    if (nb > 1 && raw && (size_t)nb * (in / 32) * sizeof(XqChunk) > XQ_LDS_SPLIT) {
        const int h = nb / 2;
        SegArgs lo = a, hi = a;
        for (int k = 0; k < a.nseg; ++k) {
            hi.seg[k].x += (size_t)h * a.seg[k].xs;
            hi.seg[k].y += (size_t)h * a.seg[k].ys;
        }
        launch_qmv(lo, h, st);
        launch_qmv(hi, nb - h, st);
        return;
    }
    const size_t lds = xq_bytes(nb, in);
    // 1-2 rows take R rows per wave, 3-4 rows half that (only the row
    // counts each shape serves are instantiated)
#define QMV(C, R, NB) k_qmv<C, R, NB><<<grid_for((a.total + R - 1) / R), 256, lds, st>>>(a)
#define QMV_LO(C, R) (nb == 1 ? (void)QMV(C, R, 1) : (void)QMV(C, R, 2))
#define QMV_HI(C, R) (nb == 3 ? (void)QMV(C, R, 3) : (void)QMV(C, R, 4))
    if (nb <= 2) {
        if (cpl <= 1) QMV_LO(1, 4);
        else if (cpl == 2) QMV_LO(2, 4);
        else QMV_LO(4, 2);
    } else {
        if (cpl <= 1) QMV_HI(1, 2);
        else if (cpl == 2) QMV_HI(2, 2);
        else QMV_HI(4, 1);
    }
#undef QMV_HI
#undef QMV_LO
#undef QMV
}

void launch_qmv_inject(const InjArgs& a, int nb, hipStream_t st) {
    const uint32_t cpl = (a.m.in / 32 + 63) / 64;
    if (a.m.in % 32 || cpl > 4) throw std::runtime_error("out-projection input must be a multiple of 32 up to 8192");
    if (cpl > 2 && nb > 2) {
        // inputs past 4096 take four chunks per lane, whose 3-4 row forms
        // would spill: rows are independent, so two launches of <= 2 rows
        InjArgs hi = a;
        hi.x += (size_t)2 * a.xs;
        if (hi.z) hi.z += (size_t)2 * a.xs;
        if (hi.x_xq) hi.x_xq += (size_t)2 * (a.m.in / 32);
        if (hi.ssq) hi.ssq += (size_t)2 * a.nheads * a.ssq_blocks;
        if (hi.hyper) hi.hyper += (size_t)2 * a.m.out * a.hc;
        if (hi.inj) hi.inj += (size_t)2 * a.hc;
        if (hi.raw_out) hi.raw_out += (size_t)2 * a.m.out;
        launch_qmv_inject(a, 2, st);
        launch_qmv_inject(hi, nb - 2, st);
        return;
    }
    constexpr int R = 2;
    const uint32_t grid = grid_for(a.m.out / R);
    if (a.xmode == XM_DN_GATED && !a.x_xq)
        throw std::runtime_error("the gated-norm input comes as the scan's nibble-plane chunks");
    const size_t lds = (a.xmode == XM_DN_GATED && a.x_xq) ? 0 : xq_bytes(nb, a.m.in);
    if (a.x_xq && a.xs != a.m.in) throw std::runtime_error("chunked inputs must be dense rows");
#define INJ(C, X) CHK_NB_SWITCH(nb, (k_qmv_inject<C, R, NB, X><<<grid, 256, lds, st>>>(a)))
    // one, two or four 32-input chunks per lane (lanes past the last chunk
    // are masked)
    if (a.xmode == XM_DN_GATED) {
        if (cpl <= 1) {
            INJ(1, XM_DN_GATED);
        } else if (cpl == 2) {
            INJ(2, XM_DN_GATED);
        } else if (nb == 1) {
            k_qmv_inject<4, R, 1, XM_DN_GATED><<<grid, 256, lds, st>>>(a);
        } else {
            k_qmv_inject<4, R, 2, XM_DN_GATED><<<grid, 256, lds, st>>>(a);
        }
    } else {
        if (cpl <= 1) {
            INJ(1, XM_PLAIN);
        } else if (cpl == 2) {
            INJ(2, XM_PLAIN);
        } else if (nb == 1) {
            k_qmv_inject<4, R, 1, XM_PLAIN><<<grid, 256, lds, st>>>(a);
        } else {
            k_qmv_inject<4, R, 2, XM_PLAIN><<<grid, 256, lds, st>>>(a);
        }
    }
#undef INJ
}

void launch_dn_scan(const DnScanArgs& a, int nb, hipStream_t st) {
    if (a.dv % 32) throw std::runtime_error("value head width must be a multiple of 32");
    if (!a.y_xq) throw std::runtime_error("the DeltaNet scan writes its outputs as nibble-plane chunks");
    CHK_NB_SWITCH(nb, (k_dn_scan<NB><<<a.nv * (a.dv / DN_SCAN_COLS), DN_SCAN_COLS * 4, 0, st>>>(a)));
}

void launch_router(const RouterArgs& a, int nb, hipStream_t st) {
    if (a.H % 32) throw std::runtime_error("router input width must be a multiple of 32");
    // one wave per workgroup so the 2 MiB matrix spreads over every CU
    constexpr int R = 2;
    const uint32_t grid = (a.E + 1 + R - 1) / R;
    CHK_NB_SWITCH(nb, (k_router<R, NB><<<grid, 64, 0, st>>>(a)));
}

void launch_moe_gate_up(const MoeArgs& a, hipStream_t st, hipEvent_t ev_start, hipEvent_t ev_stop) {
    constexpr int RG = 32 / GU_WAVES;
    if (a.topk >= 64 || a.E > 512 || a.E % 8 || a.I % RG) throw std::runtime_error("routing too wide");
    if (a.I % 32) throw std::runtime_error("expert width must be a multiple of 32");
    if (!a.act_xq) throw std::runtime_error("the gate/up kernel needs the act chunk buffer");
    if (a.H % 32 || a.H > 4096) throw std::runtime_error("expert input width must be a multiple of 32 up to 4096");
    if (a.SI % 32) throw std::runtime_error("shared expert width must be a multiple of 32");
    const uint32_t grid = a.nb * (a.topk * (a.I / 32) + a.SI / 32);  // one 32-row chunk per workgroup
    const size_t lds = xq_bytes(a.nb, a.H);
    const bool wide = a.H > 2048;
    const bool mixed = a.kinds != nullptr;
#define GU_FN(B, M) (wide ? (const void*)k_moe_gate_up<RG, B, 2, M> : (const void*)k_moe_gate_up<RG, B, 1, M>)
    const void* fn = a.X.bits == 3   ? (mixed ? GU_FN(3, true) : GU_FN(3, false))
                     : a.X.bits == 2 ? (mixed ? GU_FN(2, true) : GU_FN(2, false))
                                     : GU_FN(4, false);
#undef GU_FN
    MoeArgs arg = a;
    void* args[] = {&arg};
    // with events: recorded by the dispatch itself (the kernel's own start and end)
    const hipError_t e = ev_start ? hipExtLaunchKernel(fn, dim3(grid), dim3(GU_WG), args, lds, st, ev_start, ev_stop, 0)
                                  : hipLaunchKernel(fn, dim3(grid), dim3(GU_WG), args, lds, st);
    if (e != hipSuccess) throw std::runtime_error(std::string("gate/up launch: ") + hipGetErrorString(e));
}

void launch_moe_down(const MoeArgs& a, hipStream_t st) {
    constexpr int RD = 2;
    if (a.I % 32 || a.SI % 32) throw std::runtime_error("expert widths must be multiples of 32");
    const uint32_t nch = std::max(a.I, a.SI) / 32;  // lanes of a row: the wider expert's chunks
    int lpr = 2;
    while (lpr < (int)nch) lpr <<= 1;
    if (lpr > 32) throw std::runtime_error("expert width above 1024 is not supported");
    const uint32_t slots = a.topk + 1, groups_per_wave = 64 / lpr;
    const uint32_t passes = (slots + groups_per_wave - 1) / groups_per_wave;
    if (passes > 4) throw std::runtime_error("too many experts per token for the down kernel");
    if (a.topk >= 64 || a.hc * RD > 64) throw std::runtime_error("routing too wide");
    const uint32_t gdown = grid_for(a.H / RD, 1024);
    if (a.nb > 4) throw std::runtime_error("the down kernel takes at most 4 rows");
#define DOWN(L, B, P, M) k_moe_down<L, RD, B, P, M><<<gdown, 256, 0, st>>>(a)
#define DOWNP(L, B, M)                        \
    switch (passes) {                         \
    case 1: DOWN(L, B, 1, M); break;          \
    case 2: DOWN(L, B, 2, M); break;          \
    case 3: DOWN(L, B, 3, M); break;          \
    default: DOWN(L, B, 4, M); break;         \
    }
#define DOWNB(B, M)                           \
    switch (lpr) {                            \
    case 2: DOWNP(2, B, M); break;            \
    case 4: DOWNP(4, B, M); break;            \
    case 8: DOWNP(8, B, M); break;            \
    case 16: DOWNP(16, B, M); break;          \
    default: DOWNP(32, B, M); break;          \
    }
    const bool mixed = a.kinds != nullptr;
    switch (a.X.bits) {
    case 3:
        if (mixed) DOWNB(3, true) else DOWNB(3, false)
        break;
    case 2:
        if (mixed) DOWNB(2, true) else DOWNB(2, false)
        break;
    default: DOWNB(4, false); break;
    }
#undef DOWNB
#undef DOWNP
#undef DOWN
}

void launch_lm_head(const Q4Mat& m, const float* x, float* logits, float* pv, uint32_t* pi, uint32_t nparts,
                    uint32_t* out, int nb, hipStream_t st) {
    if (m.out % 4) throw std::runtime_error("LM head rows must be a multiple of 4");
    const size_t lds = xq_bytes(nb, m.in);
    if (m.in > 4096) throw std::runtime_error("LM head input wider than 4096");
    if (m.in <= 2048) {
        CHK_NB_SWITCH(nb, (k_lm_head<4, NB, 1><<<nparts, 256, lds, st>>>(m, x, logits, pv, pi)));
    } else {  // two chunks per lane: two rows per wave keep the registers
        CHK_NB_SWITCH(nb, (k_lm_head<2, NB, 2><<<nparts, 256, lds, st>>>(m, x, logits, pv, pi)));
    }
    k_argmax_final<<<nb, 256, 0, st>>>(pv, pi, nparts, out);
}

}  // namespace chk
