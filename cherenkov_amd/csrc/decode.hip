// Decode / verify kernels for the qwen4_exp token loop on gfx950 (wave64).
//
// One step runs `nb` <= 4 rows (one committed token plus drafts).  Every
// weight matrix is streamed from HBM once per step for all rows: the row
// loop sits inside each wave, after the weight load.  Reference semantics:
// /root/reference/src/qwen4_exp/cpu.rs (forward_token and the blocks it
// calls); the Metal dispatch plan it replaces: src/qwen4_exp/gpu/decode.rs:
// 13-294 and kernels/{common,qwen4_exp}/*.metal.
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

// Row r of a Q4 matrix dotted with NB input rows; LPR lanes per matrix row,
// lane `lir` takes 32-input chunks lir, lir + LPR, ...  Returns the full dot
// in every lane of the row group.
template <int LPR, int NB>
CHK_DEV void q4_dot(const Q4Mat& m, uint32_t r, const float* __restrict__ x, uint32_t xs, int lir, float* acc) {
    const uint32_t nch = m.in >> 5;
    const uint32_t* wr = m.w + (size_t)r * (m.in >> 3);
    const uint16_t* sr = m.s + (size_t)r * (m.in >> 6);
    const uint16_t* br = m.b + (size_t)r * (m.in >> 6);
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = 0.0f;
    for (uint32_t c = lir; c < nch; c += LPR) {
        uint4 wq = ldw4(wr + c * 4);
        float s = bf16f(sr[c >> 1]), bb = bf16f(br[c >> 1]);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            float xv[32];
            ldx32(x + (size_t)b * xs + c * 32, xv);
            acc[b] += q4_chunk(wq, xv, s, bb);
        }
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = group_sum<LPR>(acc[b]);
}

// Low-bit (Q3/Q2) 32-code chunk in the lowbit.rs layout; codes reconstruct
// at the midpoint (2q + 0.5 or 4q + 1.5) of the Q4 range they cover:
// w = mid * s + b, so the chunk partial is s * (step * sum(q x) + half * sum(x)) + b * sum(x).
template <int BITS>
CHK_DEV float lowbit_chunk(const uint8_t* p, const float* x, float s, float b) {
    float qd = 0.0f, xs = 0.0f;
    uint32_t w0, w1, lo = 0;
    if (BITS == 2) {
        uint2 v = *reinterpret_cast<const uint2*>(p);
        w0 = v.x; w1 = v.y;
    } else {
        const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
        w0 = q[0]; w1 = q[1]; lo = q[2];
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        uint32_t w = t ? w1 : w0;
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
#pragma unroll
            for (int byte = 0; byte < 4; ++byte) {
                uint32_t code = (w >> (8 * byte + 2 * pp)) & 3u;
                if (BITS == 3) code = 2u * code + ((lo >> (8 * byte + 4 * t + pp)) & 1u);
                int r = pp == 0 ? 2 * byte : pp == 1 ? 2 * byte + 8 : pp == 2 ? 2 * byte + 1 : 2 * byte + 9;
                float xv = x[16 * t + r];
                qd += (float)code * xv;
            }
        }
    }
#pragma unroll
    for (int j = 0; j < 32; ++j) xs += x[j];
    const float step = BITS == 2 ? 4.0f : 2.0f, half = BITS == 2 ? 1.5f : 0.5f;
    return s * (step * qd + half * xs) + b * xs;
}

// Expert projection `part` (0 gate, 1 up, 2 down) row r, Q4 or low-bit.
template <int LPR, int NB, int BITS>
CHK_DEV void expert_dot(const ExpertsDev& X, const uint8_t* rec, int part, uint32_t out, uint32_t in, uint32_t r,
                        const float* __restrict__ x, uint32_t xs, int lir, float* acc) {
    uint64_t woff = part == 0 ? X.gate_w : part == 1 ? X.up_w : X.down_w;
    uint64_t soff = part == 0 ? X.gate_s : part == 1 ? X.up_s : X.down_s;
    uint64_t boff = part == 0 ? X.gate_b : part == 1 ? X.up_b : X.down_b;
    if (BITS == 4) {
        Q4Mat m{(const uint32_t*)(rec + woff), (const uint16_t*)(rec + soff), (const uint16_t*)(rec + boff), out, in};
        q4_dot<LPR, NB>(m, r, x, xs, lir, acc);
        return;
    }
    const uint32_t nch = in >> 5, cb = BITS == 2 ? 8 : 12;
    const uint8_t* wr = rec + woff + (size_t)r * nch * cb;
    const uint16_t* sr = (const uint16_t*)(rec + soff) + (size_t)r * (in >> 6);
    const uint16_t* br = (const uint16_t*)(rec + boff) + (size_t)r * (in >> 6);
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = 0.0f;
    for (uint32_t c = lir; c < nch; c += LPR) {
        float s = bf16f(sr[c >> 1]), bb = bf16f(br[c >> 1]);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            float xv[32];
            ldx32(x + (size_t)b * xs + c * 32, xv);
            acc[b] += lowbit_chunk<BITS>(wr + (size_t)c * cb, xv, s, bb);
        }
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = group_sum<LPR>(acc[b]);
}

// ------------------------------------------------------------------ embed
// embed.dequant_row + replicate into hc streams (cpu.rs:399-407).  Uses
// explicitly rounded mul/add so hyper starts bit-identical to the oracle.
__global__ void k_embed(const uint32_t* __restrict__ tokens, Q4Mat emb, float* __restrict__ hyper, uint32_t H,
                        uint32_t hc) {
    uint32_t b = blockIdx.y, i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= H) return;
    uint32_t tok = tokens[b];
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
// One wave per row of [down; inject]; each wave reads the whole hyper row,
// so the per-stream RMS is a wave reduction (no extra pass).
template <int NB>
__global__ void k_hc_down(HcDev w, const float* __restrict__ hyper, float* __restrict__ d, float* __restrict__ inj,
                          float* __restrict__ inv_out, uint32_t H, uint32_t hc, float eps) {
    const int lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const uint32_t nrow = w.down.out + (w.has_inject ? w.inject.out : 0);
    if (row >= nrow) return;
    const Q4Mat& m = row < w.down.out ? w.down : w.inject;
    const uint32_t r = row < w.down.out ? row : row - w.down.out;
    const uint32_t hh = H * hc, nch = hh >> 5;
    float acc[NB][8], ss[NB][8];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int g = 0; g < 8; ++g) { acc[b][g] = 0.0f; ss[b][g] = 0.0f; }
    const uint32_t* wr = m.w + (size_t)r * (hh >> 3);
    const uint16_t* sr = m.s + (size_t)r * (hh >> 6);
    const uint16_t* br = m.b + (size_t)r * (hh >> 6);
    for (uint32_t c = lane; c < nch; c += 64) {
        uint4 wq = ldw4(wr + c * 4);
        float s = bf16f(sr[c >> 1]), bb = bf16f(br[c >> 1]);
        uint32_t g = (c * 32) / H;
        float nw[32];
#pragma unroll
        for (int j = 0; j < 32; ++j) nw[j] = bf16f(w.norm[c * 32 + j]);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            float xv[32];
            ldx32(hyper + (size_t)b * hh + c * 32, xv);
            float sq = 0.0f;
#pragma unroll
            for (int j = 0; j < 32; ++j) {
                sq += xv[j] * xv[j];
                xv[j] *= nw[j];
            }
            float part = q4_chunk(wq, xv, s, bb);
#pragma unroll
            for (int gg = 0; gg < 8; ++gg)
                if (gg == (int)g) { acc[b][gg] += part; ss[b][gg] += sq; }
        }
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        float tot = 0.0f;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            if (g < (int)hc) {
                float s2 = wave_sum(ss[b][g]);
                float inv = 1.0f / sqrtf(s2 / (float)H + eps);
                tot += inv * wave_sum(acc[b][g]);
                if (row == 0 && lane == 0) inv_out[b * hc + g] = inv;
            }
        }
        if (lane == 0) {
            float v = tot / (float)hc;
            if (row < w.down.out) d[(size_t)b * w.down.out + r] = siluf_(v);
            else inj[b * hc + r] = 2.0f * sigmoidf_(v);
        }
    }
}

// ------------------------------------------------------ hc read (up + mix)
// mixed[i] = (1/hc) sum_g sigmoid(up(d)[g H + i]) * normed[g H + i]
// (cpu.rs:477-491).  A wave covers RPW = 64/LPR rows: RPW/hc outputs x hc streams.
template <int LPR, int NB>
__global__ void k_hc_up_mix(HcDev w, const float* __restrict__ hyper, const float* __restrict__ inv,
                            const float* __restrict__ d, float* __restrict__ mixed, uint32_t H, uint32_t hc) {
    constexpr int RPW = 64 / LPR;
    __shared__ float red[4][NB][64];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, lir = lane % LPR, k = lane / LPR;
    const uint32_t outs_pw = RPW / hc;
    const uint32_t o0 = (blockIdx.x * (blockDim.x >> 6) + wv) * outs_pw;
    const uint32_t i = o0 + k / hc, g = k % hc;
    const bool active = (uint32_t)k < outs_pw * hc && i < H;
    float acc[NB];
    if (active) {
        q4_dot<LPR, NB>(w.up, g * H + i, d, w.down.out, lir, acc);
    }
    if (lir == 0) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            float v = 0.0f;
            if (active) {
                size_t j = (size_t)g * H + i;
                float normed = hyper[(size_t)b * H * hc + j] * inv[b * hc + g] * bf16f(w.norm[j]);
                v = sigmoidf_(acc[b]) * normed;
            }
            red[wv][b][k] = v;
        }
    }
    __syncthreads();
    if ((uint32_t)lane < outs_pw && o0 + lane < H) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            float s = 0.0f;
            for (uint32_t gg = 0; gg < hc; ++gg) s += red[wv][b][lane * hc + gg];
            mixed[(size_t)b * H + o0 + lane] = s / (float)hc;
        }
    }
}

// ------------------------------------------------- multi-segment Q4 matvec
// Several matrices over inputs of one width in one launch (horizontal
// fusion), one wave per output row, with per-segment epilogues.
template <int NB>
__global__ void k_qmv(SegArgs a) {
    const int lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= a.total) return;
    int si = 0;
#pragma unroll
    for (int k = 1; k < MAX_SEG; ++k)
        if (k < a.nseg && row >= a.seg[k].row0) si = k;
    const Seg& sg = a.seg[si];
    const uint32_t r = row - sg.row0;
    float acc[NB];
    q4_dot<64, NB>(sg.m, r, sg.x, sg.xs, lane, acc);
    if (lane != 0) return;
    switch (sg.epi) {
    case EPI_RAW:
#pragma unroll
        for (int b = 0; b < NB; ++b) sg.y[(size_t)b * sg.ys + r] = acc[b];
        break;
    case EPI_DN_CONV: {
        // causal_conv (cpu.rs:1067-1085) for channel r, rows in order;
        // history snapshots after every row but the last (conv_b,
        // deltanet.metal:37-42).
        const uint32_t km1 = a.ck - 1;
        float hist[8];
        float* hp = a.hist + (size_t)r * km1;
        for (uint32_t j = 0; j < km1; ++j) hist[j] = hp[j];
        const uint16_t* cw = a.conv_w + (size_t)r * a.ck;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            float cur = acc[b];
            float s = bf16f(cw[km1]) * cur;
            for (uint32_t j = 0; j < km1; ++j) s += bf16f(cw[j]) * hist[j];
            for (uint32_t j = 0; j + 1 < km1; ++j) hist[j] = hist[j + 1];
            hist[km1 - 1] = cur;
            sg.y[(size_t)b * sg.ys + r] = siluf_(s);
            if (a.snap && b + 1 < NB) {
                float* sp = a.snap_hist + (size_t)b * a.conv_dim * km1 + (size_t)r * km1;
                for (uint32_t j = 0; j < km1; ++j) sp[j] = hist[j];
            }
        }
        for (uint32_t j = 0; j < km1; ++j) hp[j] = hist[j];
        break;
    }
    case EPI_DN_DECAY:
        // g = -exp(A_log) * softplus(a + dt_bias), decay = e^g (cpu.rs:775-777)
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            float g = -expf(bf16f(a.a_log[r])) * softplusf_(acc[b] + bf16f(a.dt_bias[r]));
            sg.y[(size_t)b * sg.ys + r] = expf(g);
        }
        break;
    case EPI_DN_BETA:
#pragma unroll
        for (int b = 0; b < NB; ++b) sg.y[(size_t)b * sg.ys + r] = sigmoidf_(acc[b]);
        break;
    }
}

// --------------------------------------------- Q4 matvec + hyper inject
// out = W x; hyper[b][g H + r] += out * inj[b][g] (inject, cpu.rs:971-979).
template <int NB>
__global__ void k_qmv_inject(Q4Mat m, const float* __restrict__ x, uint32_t xs, float* __restrict__ hyper,
                             const float* __restrict__ inj, uint32_t hc, float* __restrict__ raw_out) {
    const int lane = threadIdx.x & 63;
    const uint32_t r = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (r >= m.out) return;
    float acc[NB];
    q4_dot<64, NB>(m, r, x, xs, lane, acc);
    if (lane != 0) return;
    const uint32_t H = m.out;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        if (raw_out) raw_out[(size_t)b * H + r] = acc[b];
        if (hyper)
            for (uint32_t g = 0; g < hc; ++g) hyper[(size_t)b * H * hc + g * H + r] += acc[b] * inj[b * hc + g];
    }
}

// ------------------------------------------------------- DeltaNet step
// One workgroup per value head: the head's fp32 state [dv][dk] (transposed
// relative to cpu.rs, as delta_scan2 keeps it) lives in VGPRs, 4 threads
// per value lane, 32 key lanes each.  Per row: L2-normalise q, k of the
// key head, S <- decay S, delta = beta (v - S^T k), S <- S + k delta^T,
// y = S^T q (cpu.rs:745-812); snapshots after rows < nb-1; then the gated
// RMSNorm y = rmsnorm(y) * w * sigmoid(z) (cpu.rs:814-826, eps 1e-6).
template <int NB>
__global__ void __launch_bounds__(512) k_dn_scan(DnScanArgs a) {
    constexpr int DK = 128, TPC = 4, KPT = DK / TPC;
    __shared__ float red[8];
    const uint32_t hv = blockIdx.x;
    const int t = threadIdx.x, iv = t / TPC, p = t % TPC;
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
        for (int j = 0; j < KPT; ++j) {
            q[j] = row[hk * DK + p * KPT + j];
            kk[j] = row[a.qk_dim + hk * DK + p * KPT + j];
            sq += q[j] * q[j];
            sk += kk[j] * kk[j];
        }
        sq = group_sum<TPC>(sq);
        sk = group_sum<TPC>(sk);
        float iq = 1.0f / sqrtf(sq + 1e-6f), ik = 1.0f / sqrtf(sk + 1e-6f);
#pragma unroll
        for (int j = 0; j < KPT; ++j) {
            q[j] = q[j] * iq * a.qscale;
            kk[j] *= ik;
        }
        const float decay = a.decay[b * a.nv + hv], beta = a.beta[b * a.nv + hv];
        const float v = row[2 * a.qk_dim + hv * a.dv + iv];
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
            for (int k = 0; k < KPT; k += 4) *reinterpret_cast<float4*>(pp + k) = make_float4(S[k], S[k + 1], S[k + 2], S[k + 3]);
        }
        float ss = block_sum(p == 0 ? y * y : 0.0f, red);
        float inv = 1.0f / sqrtf(ss / (float)a.dv + 1e-6f);
        if (p == 0) {
            float z = a.z[(size_t)b * a.nv * a.dv + hv * a.dv + iv];
            a.y[(size_t)b * a.nv * a.dv + hv * a.dv + iv] = y * inv * bf16f(a.norm[iv]) * sigmoidf_(z);
        }
    }
#pragma unroll
    for (int k = 0; k < KPT; k += 4) *reinterpret_cast<float4*>(sp + k) = make_float4(S[k], S[k + 1], S[k + 2], S[k + 3]);
}

// ------------------------------------------------------------ router
// logits = W_r x (bf16 [E][H]) and the shared-expert gate dot (cpu.rs:
// 506-508, 534-535).  The last workgroup to finish runs softmax and top-k
// (desc probability, lowest index on ties, renormalised; cpu.rs:508-525).
template <int NB>
__global__ void k_router(RouterArgs a) {
    const int lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const uint32_t H = a.H;
    if (row <= a.E) {
        const uint16_t* wr = row < a.E ? a.router + (size_t)row * H : a.shared_gate;
        float acc[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[b] = 0.0f;
        for (uint32_t c = lane; c < H / 32; c += 64) {
            const uint4* wp = reinterpret_cast<const uint4*>(wr + c * 32);
            float wv[32];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                uint4 u = wp[k];
                uint32_t uu[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    wv[k * 8 + 2 * j] = __uint_as_float(uu[j] << 16);
                    wv[k * 8 + 2 * j + 1] = __uint_as_float(uu[j] & 0xffff0000u);
                }
            }
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                float xv[32];
                ldx32(a.x + (size_t)b * H + c * 32, xv);
#pragma unroll
                for (int j = 0; j < 32; ++j) acc[b] += wv[j] * xv[j];
            }
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            float s = wave_sum(acc[b]);
            if (lane == 0) {
                if (row < a.E) a.logits[(size_t)b * a.E + row] = s;
                else a.sg[b] = s;
            }
        }
    }
    // last-block-done: the final workgroup computes the routing
    __shared__ uint32_t ticket;
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) ticket = atomicAdd(a.counter, 1u);
    __syncthreads();
    if (ticket != gridDim.x - 1) return;
    __threadfence();
    if (threadIdx.x >= 64) return;
    if (lane == 0) *a.counter = 0u;
    topk_wave(a.logits, a.probs, a.E, a.topk, a.norm_topk, a.ids, a.w, NB, lane);
}

// ----------------------------------------------------- experts: gate/up
// act[b][slot][i] = silu(gate_i . x_b) * (up_i . x_b) for the top-k routed
// experts of row b (slots 0..k-1) and the shared expert (slot k) (mlp,
// cpu.rs:981-992).  One wave per (row, slot, i).
template <int NB1, int BITS>
__global__ void k_moe_gate_up(MoeArgs a) {
    const int lane = threadIdx.x & 63;
    const uint32_t t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const uint32_t slots = a.topk + 1;
    if (t >= a.nb * slots * a.I) return;
    const uint32_t b = t / (slots * a.I), slot = (t / a.I) % slots, i = t % a.I;
    const float* x = a.x + (size_t)b * a.H;
    float g, u;
    if (slot < a.topk) {
        uint32_t e = min(a.ids[b * a.topk + slot], a.X.experts - 1);
        const uint8_t* rec = a.X.base + ((size_t)a.record_layer * a.X.experts + e) * a.X.stride;
        float acc[1];
        expert_dot<64, 1, BITS>(a.X, rec, 0, a.I, a.H, i, x, 0, lane, acc);
        g = acc[0];
        expert_dot<64, 1, BITS>(a.X, rec, 1, a.I, a.H, i, x, 0, lane, acc);
        u = acc[0];
    } else {
        float acc[1];
        q4_dot<64, 1>(a.sh_gate, i, x, 0, lane, acc);
        g = acc[0];
        q4_dot<64, 1>(a.sh_up, i, x, 0, lane, acc);
        u = acc[0];
    }
    if (lane == 0) a.act[((size_t)b * slots + slot) * a.I + i] = siluf_(g) * u;
}

// ------------------------------------------------- experts: down + combine
// out[r] = sum_j w_j down_j(act_j)[r] + sigmoid(shared_gate . x) shared_down(act_k)[r]
// (cpu.rs:527-540), then hyper[g H + r] += out * inj_g.  One wave per
// output row; LPR lanes per expert row, 64/LPR experts in flight.
template <int LPR, int NB1, int BITS>
__global__ void k_moe_down(MoeArgs a) {
    constexpr int G = 64 / LPR;
    const int lane = threadIdx.x & 63, grp = lane / LPR, lir = lane % LPR;
    const uint32_t r = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (r >= a.H) return;
    const uint32_t slots = a.topk + 1;
    for (uint32_t b = 0; b < a.nb; ++b) {
        float tot = 0.0f;
        for (uint32_t slot = grp; slot < slots; slot += G) {
            const float* act = a.act + ((size_t)b * slots + slot) * a.I;
            float acc[1], wgt;
            if (slot < a.topk) {
                uint32_t e = min(a.ids[b * a.topk + slot], a.X.experts - 1);
                const uint8_t* rec = a.X.base + ((size_t)a.record_layer * a.X.experts + e) * a.X.stride;
                expert_dot<LPR, 1, BITS>(a.X, rec, 2, a.H, a.I, r, act, 0, lir, acc);
                wgt = a.w[b * a.topk + slot];
            } else {
                q4_dot<LPR, 1>(a.sh_down, r, act, 0, lir, acc);
                wgt = sigmoidf_(a.sg[b]);
            }
            tot += wgt * acc[0];
        }
#pragma unroll
        for (int m = LPR; m < 64; m <<= 1) tot += __shfl_xor(tot, m, 64);
        if (lane == 0) {
            if (a.raw_out) a.raw_out[(size_t)b * a.H + r] = tot;
            if (a.hyper)
                for (uint32_t g = 0; g < a.hc; ++g)
                    a.hyper[(size_t)b * a.H * a.hc + g * a.H + r] += tot * a.inj[b * a.hc + g];
        }
    }
}

// ------------------------------------------------------- LM head + argmax
// logits = W_lm mixed; greedy argmax with the lowest index winning ties
// (argmax_partial/argmax_final, kernels/common/sampling.metal:10-84).
template <int NB>
__global__ void k_lm_head(Q4Mat m, const float* __restrict__ x, float* __restrict__ logits, float* __restrict__ pv,
                          uint32_t* __restrict__ pi) {
    __shared__ float sv[NB][4];
    __shared__ uint32_t si[NB][4];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t nw = gridDim.x * (blockDim.x >> 6);
    float bv[NB];
    uint32_t bi[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) { bv[b] = -INFINITY; bi[b] = 0xffffffffu; }
    for (uint32_t r = blockIdx.x * (blockDim.x >> 6) + wv; r < m.out; r += nw) {
        float acc[NB];
        q4_dot<64, NB>(m, r, x, m.in, lane, acc);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (lane == 0) logits[(size_t)b * m.out + r] = acc[b];
            if (acc[b] > bv[b] || (acc[b] == bv[b] && r < bi[b])) { bv[b] = acc[b]; bi[b] = r; }
        }
    }
    if (lane == 0)
#pragma unroll
        for (int b = 0; b < NB; ++b) { sv[b][wv] = bv[b]; si[b][wv] = bi[b]; }
    __syncthreads();
    if (threadIdx.x < NB) {
        int b = threadIdx.x;
        float v = sv[b][0];
        uint32_t i = si[b][0];
        for (int k = 1; k < (int)(blockDim.x >> 6); ++k)
            if (sv[b][k] > v || (sv[b][k] == v && si[b][k] < i)) { v = sv[b][k]; i = si[b][k]; }
        pv[(size_t)b * gridDim.x + blockIdx.x] = v;
        pi[(size_t)b * gridDim.x + blockIdx.x] = i;
    }
}

__global__ void k_argmax_final(const float* __restrict__ pv, const uint32_t* __restrict__ pi, uint32_t n,
                               uint32_t* __restrict__ out) {
    __shared__ float sv[256];
    __shared__ uint32_t si[256];
    const uint32_t b = blockIdx.x;
    float v = -INFINITY;
    uint32_t i = 0xffffffffu;
    for (uint32_t k = threadIdx.x; k < n; k += blockDim.x) {
        float x = pv[(size_t)b * n + k];
        uint32_t xi = pi[(size_t)b * n + k];
        if (x > v || (x == v && xi < i)) { v = x; i = xi; }
    }
    sv[threadIdx.x] = v;
    si[threadIdx.x] = i;
    __syncthreads();
    for (uint32_t s = blockDim.x / 2; s > 0; s >>= 1) {
        if (threadIdx.x < s) {
            float x = sv[threadIdx.x + s];
            uint32_t xi = si[threadIdx.x + s];
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

void launch_embed(const uint32_t* tokens, const Q4Mat& emb, float* hyper, uint32_t H, uint32_t hc, int nb,
                  hipStream_t st) {
    dim3 grid((H + 255) / 256, nb);
    k_embed<<<grid, 256, 0, st>>>(tokens, emb, hyper, H, hc);
}

void launch_hc_down(const HcDev& w, const float* hyper, float* d, float* inj, float* inv, uint32_t H, uint32_t hc,
                    float eps, int nb, hipStream_t st) {
    uint32_t rows = w.down.out + (w.has_inject ? w.inject.out : 0);
    CHK_NB_SWITCH(nb, (k_hc_down<NB><<<(rows + 3) / 4, 256, 0, st>>>(w, hyper, d, inj, inv, H, hc, eps)));
}

void launch_hc_up_mix(const HcDev& w, const float* hyper, const float* inv, const float* d, float* mixed,
                      uint32_t H, uint32_t hc, int nb, hipStream_t st) {
    uint32_t nch = w.up.in / 32;
    int lpr = 1;
    while (lpr < (int)nch) lpr <<= 1;
    if (lpr > 64) lpr = 64;
    uint32_t outs_pw = (64 / lpr) / hc;
    uint32_t waves = (H + outs_pw - 1) / outs_pw;
    uint32_t grid = (waves + 3) / 4;
#define UPMIX(L) CHK_NB_SWITCH(nb, (k_hc_up_mix<L, NB><<<grid, 256, 0, st>>>(w, hyper, inv, d, mixed, H, hc)))
    switch (lpr) {
    case 1: case 2: UPMIX(2); break;
    case 4: UPMIX(4); break;
    case 8: UPMIX(8); break;
    case 16: UPMIX(16); break;
    default: UPMIX(16); break;
    }
#undef UPMIX
}

void launch_qmv(const SegArgs& a, int nb, hipStream_t st) {
    uint32_t grid = (a.total + 3) / 4;
    CHK_NB_SWITCH(nb, (k_qmv<NB><<<grid, 256, 0, st>>>(a)));
}

void launch_qmv_inject(const Q4Mat& m, const float* x, uint32_t xs, float* hyper, const float* inj, uint32_t hc,
                       float* raw_out, int nb, hipStream_t st) {
    uint32_t grid = (m.out + 3) / 4;
    CHK_NB_SWITCH(nb, (k_qmv_inject<NB><<<grid, 256, 0, st>>>(m, x, xs, hyper, inj, hc, raw_out)));
}

void launch_dn_scan(const DnScanArgs& a, int nb, hipStream_t st) {
    CHK_NB_SWITCH(nb, (k_dn_scan<NB><<<a.nv, a.dv * 4, 0, st>>>(a)));
}

void launch_router(const RouterArgs& a, int nb, hipStream_t st) {
    uint32_t grid = (a.E + 1 + 3) / 4;
    CHK_NB_SWITCH(nb, (k_router<NB><<<grid, 256, 0, st>>>(a)));
}

void launch_moe(const MoeArgs& a, hipStream_t st) {
    uint32_t tasks = a.nb * (a.topk + 1) * a.I;
    uint32_t grid = (tasks + 3) / 4;
    uint32_t nch = a.I / 32;
    int lpr = 1;
    while (lpr < (int)nch) lpr <<= 1;
    if (lpr > 64) lpr = 64;
    if (lpr < 2) lpr = 2;
    uint32_t gdown = (a.H + 3) / 4;
#define DOWN(L, B) k_moe_down<L, 1, B><<<gdown, 256, 0, st>>>(a)
#define DOWNB(B)                              \
    switch (lpr) {                            \
    case 2: DOWN(2, B); break;                \
    case 4: DOWN(4, B); break;                \
    case 8: DOWN(8, B); break;                \
    case 16: DOWN(16, B); break;              \
    case 32: DOWN(32, B); break;              \
    default: DOWN(64, B); break;              \
    }
    switch (a.X.bits) {
    case 3:
        k_moe_gate_up<1, 3><<<grid, 256, 0, st>>>(a);
        DOWNB(3);
        break;
    case 2:
        k_moe_gate_up<1, 2><<<grid, 256, 0, st>>>(a);
        DOWNB(2);
        break;
    default:
        k_moe_gate_up<1, 4><<<grid, 256, 0, st>>>(a);
        DOWNB(4);
        break;
    }
#undef DOWNB
#undef DOWN
}

void launch_lm_head(const Q4Mat& m, const float* x, float* logits, float* pv, uint32_t* pi, uint32_t nparts,
                    uint32_t* out, int nb, hipStream_t st) {
    CHK_NB_SWITCH(nb, (k_lm_head<NB><<<nparts, 256, 0, st>>>(m, x, logits, pv, pi)));
    k_argmax_final<<<nb, 256, 0, st>>>(pv, pi, nparts, out);
}

}  // namespace chk
