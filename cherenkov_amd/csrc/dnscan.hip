// Chunked gated delta rule for the prefill (64 rows per chunk).
//
// The recurrence of cpu.rs:745-812 (the reference prefill runs it row by
// row, gpu/prefill/deltanet.rs:80-95), per value head with the state S
// [dk][dv] and, for row t, decay d_t, beta b_t, normed q_t, k_t and v_t:
//   delta_t = b_t (v_t - d_t S^T k_t),  S <- d_t S + k_t delta_t^T,
//   y_t = S^T q_t.
// Over a chunk of C rows that starts from S0, with G_t = sum_{s<=t} log d_s
// (so gamma_t = e^{G_t} and gamma_t / gamma_i = e^{G_t - G_i} <= 1 for
// i <= t), unrolling the recurrence gives
//   (I + A) Delta = diag(b) V - diag(b gamma) K S0,
//       A[t][i] = b_t e^{G_t - G_i} (k_t . k_i) for i < t,
//   Y  = diag(gamma) Q S0 + P Delta,  P[t][i] = e^{G_t - G_i} (q_t . k_i), i <= t,
//   S_C = gamma_C S0 + K^T diag(gamma_C / gamma) Delta.
// With U = (I + A)^-1 diag(b) V and W = (I + A)^-1 diag(b gamma) K,
// Delta = U - W S0.  U, W and P do not depend on the state, so
// k_dc_prep builds them for every (head, chunk) at once; k_dc_scan then
// walks the chunks in order with four matrix products per chunk.
//
// Both kernels run on v_mfma_f32_16x16x4_f32 (f32 operands, f32
// accumulation).  Layouts (16 x 16 tiles, lane l): A[l % 16][k = l / 16],
// B[k = l / 16][l % 16], D rows 4 (l / 16) .. + 4 of column l % 16.  The k
// index of one MFMA may stand for any position of the contraction as long
// as A and B agree; lane group l / 16 takes a contiguous quarter of it so
// each lane reads its operands as float4 runs.
#include <algorithm>
#include <cstdint>
#include <stdexcept>
#include <type_traits>

#include "kernels_internal.h"

namespace chk {

typedef float f4v __attribute__((ext_vector_type(4)));

constexpr int DC_C = 64;          // rows per chunk
constexpr int DC_DK = 128;        // key head dim
constexpr int DC_DV = 128;        // value head dim
constexpr int DC_KP = DC_DK + 4;  // padded LDS row (floats)
constexpr int DC_PP = DC_C + 4;

CHK_DEV f4v mfma4(float a, float b, f4v c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }

// Per (value head, chunk) workspace: U [C][dv], W [C][dk], P [C][C],
// QG = diag(gamma) Q [C][dk], KF = (diag(gamma_C / gamma) K)^T [dk][C],
// then gamma_C and 3 pad.  Each matrix is stored in the order the chunk
// walk's lanes load it, so one load instruction of a wave reads 1 KB in
// one piece: an A operand M [rows][K] (W, QG: K = dk; P, KF: K = C) as
// float4 number (((row / 16) K / 16 + (k % (K / 4)) / 4) 16 + row % 16) 4 + k / (K / 4),
// i.e. the 16 rows of a tile, lane group l / 16 holding the k quarter
// (K / 4) (l / 16) ..; U as float4 number ((col / 16) 4 + t / 16) 16 + col % 16) 4 + (t % 16) / 4.
constexpr size_t DC_OFF_W = 0;  // offsets after U (dv dependent)
constexpr size_t DC_OFF_P = DC_OFF_W + DC_C * DC_DK;
constexpr size_t DC_OFF_QG = DC_OFF_P + DC_C * DC_C;
constexpr size_t DC_OFF_KF = DC_OFF_QG + DC_C * DC_DK;
constexpr size_t DC_OFF_E = DC_OFF_KF + DC_DK * DC_C;
__host__ __device__ constexpr size_t dc_task_floats(uint32_t dv) { return (size_t)DC_C * dv + DC_OFF_E + 4; }

// float index of element (row, k) of an A operand with K = 128 (W, QG) or 64 (P, KF)
CHK_DEV uint32_t dc_a128(uint32_t row, uint32_t k) {
    return ((((row >> 4) * 8 + ((k & 31) >> 2)) * 16 + (row & 15)) * 4 + (k >> 5)) * 4 + (k & 3);
}
CHK_DEV uint32_t dc_a64(uint32_t row, uint32_t k) {
    return ((((row >> 4) * 4 + ((k & 15) >> 2)) * 16 + (row & 15)) * 4 + (k >> 4)) * 4 + (k & 3);
}


// ------------------------------------------------------------ chunk prep
// One workgroup per (value head, chunk).  K and Q rows of the chunk go to
// LDS and out again as QG and KF with the decays folded in; the lower 16 x 16 tiles of K K^T and Q K^T (10 each) are split over
// the four waves; A overwrites the Q rows, P goes out.  (I + A) X = B for
// the 256 right-hand-side columns [b V | b gamma K] is solved by blocks of
// 16 rows: the four diagonal blocks L_ii = I + A_ii are inverted by
// substitution (one column per lane), then
//   X_i = L_ii^-1 (B_i - sum_{j<i} A_ij X_j),
// every product on MFMA, wave w holding columns 64 w .. 64 w + 63.  An
// MFMA's D tile (rows 4 (l / 16) + r) is the next product's B operand as
// it stands when the A operand takes its k index as 4 (l / 16) + step.
__global__ void __launch_bounds__(256) k_dc_prep(PfDnArgs a, float* __restrict__ work) {
    __shared__ __align__(16) float Ks[DC_C][DC_KP];
    __shared__ __align__(16) float Qs[DC_C][DC_KP];  // Q rows, then A rows
    __shared__ __align__(16) float Li[4][16][20];    // inverted diagonal blocks
    __shared__ float Gs[DC_C], Bs[DC_C], Es[DC_C], Fs[DC_C];
    const uint32_t nch = (a.T + DC_C - 1) / DC_C;
    const uint32_t hv = blockIdx.x / nch, c = blockIdx.x % nch;
    const uint32_t hk = hv / (a.nv / a.nk);
    const uint32_t t0 = c * DC_C, n = min((uint32_t)DC_C, a.T - t0);
    const int tid = threadIdx.x, lane = tid & 63, i16 = lane & 15, kq = lane >> 4;
    const int w = (int)wave_id();
    float* const Uw = work + (size_t)blockIdx.x * dc_task_floats(a.dv);
    float* const Ww = Uw + DC_C * a.dv + DC_OFF_W;
    float* const Pw = Uw + DC_C * a.dv + DC_OFF_P;
    float* const QGw = Uw + DC_C * a.dv + DC_OFF_QG;
    float* const KFw = Uw + DC_C * a.dv + DC_OFF_KF;
    float* const Ew = Uw + DC_C * a.dv + DC_OFF_E;
    // waves 0-1 fetch their V right-hand sides (D layout: rows
    // 16 bi + 4 kq + r of column tile ct) now, so the loads land while the
    // factors below are built; padding rows repeat the last row (their
    // beta is 0)
    const bool vcol = w < 2;
    float vr[4][4][4];
    if (vcol) {
#pragma unroll
        for (int bi = 0; bi < 4; ++bi)
#pragma unroll
            for (int ct = 0; ct < 4; ++ct)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t t = min((uint32_t)(16 * bi + 4 * kq + r), n - 1);
                    vr[bi][ct][r] = a.conv[(size_t)(t0 + t) * a.conv_dim + 2 * (size_t)a.qk_dim + (size_t)hv * a.dv +
                                           64 * (w & 1) + 16 * ct + i16];
                }
    }
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        const int idx = tid + 256 * m, r = idx >> 5, f = idx & 31;
        float4 qv = make_float4(0.0f, 0.0f, 0.0f, 0.0f), kv = qv;
        if ((uint32_t)r < n) {
            const float* row = a.conv + (size_t)(t0 + r) * a.conv_dim + hk * DC_DK + f * 4;
            qv = *reinterpret_cast<const float4*>(row);
            kv = *reinterpret_cast<const float4*>(row + a.qk_dim);
        }
        *reinterpret_cast<float4*>(&Qs[r][f * 4]) = qv;
        *reinterpret_cast<float4*>(&Ks[r][f * 4]) = kv;
    }
    if (w == 0) {
        // padding rows: decay 1, beta 0 (they leave the state alone)
        float g = 0.0f, b = 0.0f;
        if ((uint32_t)lane < n) {
            g = fmaxf(logf(a.decay[(size_t)(t0 + lane) * a.nv + hv]), -80.0f);
            b = a.beta[(size_t)(t0 + lane) * a.nv + hv];
        }
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const float o = __shfl_up(g, off, 64);
            if (lane >= off) g += o;
        }
        Gs[lane] = g;
        Bs[lane] = b;
        const float gc = __shfl(g, DC_C - 1, 64);
        Es[lane] = expf(g);
        Fs[lane] = expf(gc - g);
        if (lane == 0) Ew[0] = expf(gc);
    }
    __syncthreads();
    // QG and KF (row t of K scaled by gamma_C / gamma_t), one float4 of the
    // load order per thread and step
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        const int idx = tid + 256 * m;
        const int t = 16 * (idx >> 9) + ((idx >> 2) & 15), k0 = 32 * (idx & 3) + 4 * ((idx >> 6) & 7);
        float4 qv = *reinterpret_cast<const float4*>(&Qs[t][k0]);
        const float e = Es[t];
        qv.x *= e;
        qv.y *= e;
        qv.z *= e;
        qv.w *= e;
        *reinterpret_cast<float4*>(QGw + 4 * idx) = qv;
    }
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        const int idx = tid + 256 * m;
        const int d = 16 * (idx >> 8) + ((idx >> 2) & 15), t0 = 16 * (idx & 3) + 4 * ((idx >> 6) & 3);
        *reinterpret_cast<float4*>(KFw + 4 * idx) = make_float4(Ks[t0][d] * Fs[t0], Ks[t0 + 1][d] * Fs[t0 + 1],
                                                                Ks[t0 + 2][d] * Fs[t0 + 2], Ks[t0 + 3][d] * Fs[t0 + 3]);
    }
    // lower tiles (ti >= tj) in the order (0,0) (1,0) (1,1) (2,0) ... (3,3);
    // wave w takes tiles w, w + 4, w + 8
    constexpr int TI[10] = {0, 1, 1, 2, 2, 2, 3, 3, 3, 3};
    constexpr int TJ[10] = {0, 0, 1, 0, 1, 2, 0, 1, 2, 3};
    f4v kk[3], qk[3];
#pragma unroll
    for (int u = 0; u < 3; ++u) {
        kk[u] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
        qk[u] = kk[u];
        const int tile = w + 4 * u;
        if (tile >= 10) continue;
        const float* ka = &Ks[16 * TI[tile] + i16][kq * 32];
        const float* qa = &Qs[16 * TI[tile] + i16][kq * 32];
        const float* kb = &Ks[16 * TJ[tile] + i16][kq * 32];
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const float4 x = *reinterpret_cast<const float4*>(ka + 4 * m);
            const float4 q = *reinterpret_cast<const float4*>(qa + 4 * m);
            const float4 y = *reinterpret_cast<const float4*>(kb + 4 * m);
            kk[u] = mfma4(x.x, y.x, kk[u]);
            qk[u] = mfma4(q.x, y.x, qk[u]);
            kk[u] = mfma4(x.y, y.y, kk[u]);
            qk[u] = mfma4(q.y, y.y, qk[u]);
            kk[u] = mfma4(x.z, y.z, kk[u]);
            qk[u] = mfma4(q.z, y.z, qk[u]);
            kk[u] = mfma4(x.w, y.w, kk[u]);
            qk[u] = mfma4(q.w, y.w, qk[u]);
        }
    }
    __syncthreads();  // every Q read is done: A may overwrite the Q rows
#pragma unroll
    for (int u = 0; u < 3; ++u) {
        const int tile = w + 4 * u;
        if (tile >= 10) continue;
        const int i = 16 * TJ[tile] + i16;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = 16 * TI[tile] + 4 * kq + r;
            const float e = expf(Gs[t] - Gs[i]);
            Qs[t][i] = i < t ? Bs[t] * e * kk[u][r] : 0.0f;
            Pw[dc_a64(t, i)] = i <= t ? e * qk[u][r] : 0.0f;
        }
    }
    // the upper tiles of P are zero
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const int idx = tid + 256 * m;
        const int t = 16 * (idx >> 8) + ((idx >> 2) & 15), i0 = 16 * (idx & 3) + 4 * ((idx >> 6) & 3);
        if ((i0 >> 4) > (t >> 4)) *reinterpret_cast<float4*>(Pw + 4 * idx) = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    __syncthreads();
    // wave w inverts diagonal block w: lane c < 16 takes column c
    if (lane < 16) {
        float x[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) x[r] = r == lane ? 1.0f : 0.0f;
#pragma unroll
        for (int r = 1; r < 16; ++r) {
            const float* ar = &Qs[16 * w + r][16 * w];
            float acc = 0.0f;
#pragma unroll
            for (int q = 0; q < r; ++q) acc = fmaf(ar[q], x[q], acc);
            x[r] -= acc;
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) Li[w][r][lane] = x[r];
    }
    __syncthreads();
    // right-hand sides (D layout: rows 16 bi + 4 kq + r of column tile ct):
    // waves 0-1 b V (value columns), waves 2-3 b gamma K
    f4v X[4][4];
#pragma unroll
    for (int bi = 0; bi < 4; ++bi) {
        f4v acc[4];
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
            const int col = 64 * (w & 1) + 16 * ct + i16;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = 16 * bi + 4 * kq + r;
                acc[ct][r] = vcol ? Bs[t] * vr[bi][ct][r] : Bs[t] * Es[t] * Ks[t][col];
            }
        }
        // B_i - sum_{j < i} A_ij X_j
#pragma unroll
        for (int bj = 0; bj < bi; ++bj) {
            const float4 av = *reinterpret_cast<const float4*>(&Qs[16 * bi + i16][16 * bj + 4 * kq]);
#pragma unroll
            for (int ct = 0; ct < 4; ++ct) {
                acc[ct] = mfma4(-av.x, X[bj][ct][0], acc[ct]);
                acc[ct] = mfma4(-av.y, X[bj][ct][1], acc[ct]);
                acc[ct] = mfma4(-av.z, X[bj][ct][2], acc[ct]);
                acc[ct] = mfma4(-av.w, X[bj][ct][3], acc[ct]);
            }
        }
        const float4 lv = *reinterpret_cast<const float4*>(&Li[bi][i16][4 * kq]);
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
            f4v xo = {0.0f, 0.0f, 0.0f, 0.0f};
            xo = mfma4(lv.x, acc[ct][0], xo);
            xo = mfma4(lv.y, acc[ct][1], xo);
            xo = mfma4(lv.z, acc[ct][2], xo);
            xo = mfma4(lv.w, acc[ct][3], xo);
            X[bi][ct] = xo;
        }
    }
    // U: a D tile's four rows are one float4 of the load order; W element-wise
#pragma unroll
    for (int bi = 0; bi < 4; ++bi)
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
            const int col = 64 * (w & 1) + 16 * ct + i16;
            if (vcol) {
                *reinterpret_cast<f4v*>(Uw + 4 * ((((col >> 4) * 4 + bi) * 16 + i16) * 4 + kq)) = X[bi][ct];
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) Ww[dc_a128(16 * bi + 4 * kq + r, col)] = X[bi][ct][r];
            }
        }
}

// ------------------------------------------------------------ chunk walk
// One workgroup of eight waves per (value head, 16 value columns): the
// state block S [dk][16] lives in every wave's registers as the B operand
// (lane (j, q) holds rows 32 q .. 32 q + 31 of column j) and in LDS
// column-major for the exchange.  Per chunk:
//   waves 0-3: WS = W S for rows 16 w ..,  Delta = U - WS  (to LDS)
//   waves 4-7: QS = QG S for rows 16 (w - 4) .., then Y = QS + P Delta
//   every wave: rows 16 w .. of S = gamma_C S + KF Delta
// Every operand comes from global memory straight into the MFMA layouts
// (no LDS staging), two chunks ahead.  The eight column blocks of a head share their chunk
// operands, so they go to one XCD (workgroups are dealt to the XCDs round
// robin) and meet in its L2.
constexpr int DC_WG = 512;

__global__ void __launch_bounds__(DC_WG) k_dc_scan(PfDnArgs a, const float* __restrict__ work) {
    __shared__ __align__(16) float Ss[16][DC_KP];  // [column][k]
    __shared__ __align__(16) float Ds[16][DC_PP];  // [column][row]
    const uint32_t ncb = a.dv / 16, nch = (a.T + DC_C - 1) / DC_C;
    uint32_t hv, cb;
    if (a.nv % 8 == 0) {
        const uint32_t rest = blockIdx.x >> 3;
        hv = (rest / ncb) * 8 + (blockIdx.x & 7);
        cb = rest % ncb;
    } else {
        hv = blockIdx.x / ncb;
        cb = blockIdx.x % ncb;
    }
    const uint32_t j0 = cb * 16;
    const int lane = threadIdx.x & 63, i16 = lane & 15, kq = lane >> 4;
    const int w = (int)wave_id(), wr = w & 3;
    const bool wsw = w < 4;  // W S / Delta wave, else Q S / Y wave
    const size_t tf = dc_task_floats(a.dv);
    const float* const wbase = work + (size_t)hv * nch * tf;
    float S[32];
    {
        const float* sp = a.state + ((size_t)hv * a.dv + j0 + i16) * DC_DK + kq * 32;
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const float4 v = *reinterpret_cast<const float4*>(sp + 4 * m);
            S[4 * m] = v.x;
            S[4 * m + 1] = v.y;
            S[4 * m + 2] = v.z;
            S[4 * m + 3] = v.w;
            if (w == 0) *reinterpret_cast<float4*>(&Ss[i16][kq * 32 + 4 * m]) = v;
        }
    }
    // Per-chunk operands, two chunks in flight (set c & 1 holds chunk c;
    // chunk c + 2 loads into it piece by piece right after chunk c's MFMAs
    // have read each piece, so the loads stream under the products):
    //   A1: W rows (waves 0-3) or QG rows (waves 4-7) 16 wr + i16, k 32 kq ..
    //   PA: P rows 16 wr + i16, columns 16 kq .. (waves 4-7); waves 0-3 hold
    //       U of rows 16 wr + 4 kq .. in PA[.][0] (the same float4 four
    //       times, so every wave issues the same loads)
    //   KA: KF row 16 w + i16, columns 16 kq .., and EC = gamma_C
    f4v A1[2][8], PA[2][4], KA[2][4];
    float EC[2];
    const float* const tb = wbase + DC_C * a.dv;
    // float4 number m of this lane in the load order of each operand
    const uint32_t lq = (uint32_t)(i16 * 4 + kq) * 4;
    auto a1_src = [&](uint32_t c, int m) __attribute__((always_inline)) {
        return tb + c * tf + (wsw ? DC_OFF_W : DC_OFF_QG) + (wr * 8 + m) * 256 + lq;
    };
    auto pa_src = [&](uint32_t c, int m) __attribute__((always_inline)) {
        return wsw ? wbase + c * tf + (cb * 4 + wr) * 256 + lq : tb + c * tf + DC_OFF_P + (wr * 4 + m) * 256 + lq;
    };
    auto ka_src = [&](uint32_t c, int m) __attribute__((always_inline)) {
        return tb + c * tf + DC_OFF_KF + (w * 4 + m) * 256 + lq;
    };
    auto load_all = [&](auto B, uint32_t c) __attribute__((always_inline)) {
        constexpr int b = decltype(B)::value;
#pragma unroll
        for (int m = 0; m < 8; ++m) A1[b][m] = *reinterpret_cast<const f4v*>(a1_src(c, m));
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            PA[b][m] = *reinterpret_cast<const f4v*>(pa_src(c, m));
            KA[b][m] = *reinterpret_cast<const f4v*>(ka_src(c, m));
        }
        EC[b] = tb[c * tf + DC_OFF_E];
    };
    auto chunk = [&](auto B, uint32_t c) __attribute__((always_inline)) {
        constexpr int b = decltype(B)::value;
        // the next loads into this set: chunk c + 2, or again the last chunk
        // (unconditional, so the waits on them count exactly)
        const uint32_t cn = min(c + 2, nch - 1);
        f4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            acc = mfma4(A1[b][m][0], S[4 * m], acc);
            acc = mfma4(A1[b][m][1], S[4 * m + 1], acc);
            acc = mfma4(A1[b][m][2], S[4 * m + 2], acc);
            acc = mfma4(A1[b][m][3], S[4 * m + 3], acc);
            A1[b][m] = *reinterpret_cast<const f4v*>(a1_src(cn, m));
        }
        if (wsw)
            *reinterpret_cast<float4*>(&Ds[i16][16 * wr + 4 * kq]) =
                make_float4(PA[b][0][0] - acc[0], PA[b][0][1] - acc[1], PA[b][0][2] - acc[2], PA[b][0][3] - acc[3]);
        __syncthreads();
        // Delta as the B operand: lane (j, q) holds rows 16 q .. 16 q + 15
        float dv[16];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const float4 v = *reinterpret_cast<const float4*>(&Ds[i16][16 * kq + 4 * m]);
            dv[4 * m] = v.x;
            dv[4 * m + 1] = v.y;
            dv[4 * m + 2] = v.z;
            dv[4 * m + 3] = v.w;
        }
        if (!wsw) {
            f4v ya = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                ya = mfma4(PA[b][m][0], dv[4 * m], ya);
                ya = mfma4(PA[b][m][1], dv[4 * m + 1], ya);
                ya = mfma4(PA[b][m][2], dv[4 * m + 2], ya);
                ya = mfma4(PA[b][m][3], dv[4 * m + 3], ya);
            }
            const uint32_t t0 = c * DC_C, n = min((uint32_t)DC_C, a.T - t0);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t t = 16 * wr + 4 * kq + r;
                if (t < n) a.y[(size_t)(t0 + t) * a.v_dim + (size_t)hv * a.dv + j0 + i16] = acc[r] + ya[r];
            }
        }
        f4v sa = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            sa = mfma4(KA[b][m][0], dv[4 * m], sa);
            sa = mfma4(KA[b][m][1], dv[4 * m + 1], sa);
            sa = mfma4(KA[b][m][2], dv[4 * m + 2], sa);
            sa = mfma4(KA[b][m][3], dv[4 * m + 3], sa);
            KA[b][m] = *reinterpret_cast<const f4v*>(ka_src(cn, m));
            PA[b][m] = *reinterpret_cast<const f4v*>(pa_src(cn, m));
        }
        const float ec = EC[b];
        EC[b] = tb[cn * tf + DC_OFF_E];
        float4* sp = reinterpret_cast<float4*>(&Ss[i16][16 * w + 4 * kq]);
        const float4 so = *sp;
        *sp = make_float4(fmaf(ec, so.x, sa[0]), fmaf(ec, so.y, sa[1]), fmaf(ec, so.z, sa[2]), fmaf(ec, so.w, sa[3]));
        __syncthreads();
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const float4 v = *reinterpret_cast<const float4*>(&Ss[i16][kq * 32 + 4 * m]);
            S[4 * m] = v.x;
            S[4 * m + 1] = v.y;
            S[4 * m + 2] = v.z;
            S[4 * m + 3] = v.w;
        }
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    load_all(I0{}, 0);
    load_all(I1{}, min(1u, nch - 1));
    // pairs of chunks, then an odd last one outside the loop, so the loop
    // body has one path and its waits on the loads two chunks back stay exact
    uint32_t c = 0;
    for (; c + 1 < nch; c += 2) {
        chunk(I0{}, c);
        chunk(I1{}, c + 1);
    }
    if (c < nch) chunk(I0{}, c);
    if (w == 0) {
        float* sp = a.state + ((size_t)hv * a.dv + j0 + i16) * DC_DK + kq * 32;
#pragma unroll
        for (int m = 0; m < 8; ++m)
            *reinterpret_cast<float4*>(sp + 4 * m) = make_float4(S[4 * m], S[4 * m + 1], S[4 * m + 2], S[4 * m + 3]);
    }
}

// -------------------------------------------------------------- launchers

bool dc_supported(uint32_t nk, uint32_t nv, uint32_t dk, uint32_t dv) {
    return dk == DC_DK && dv == DC_DV && nk > 0 && nv % nk == 0;
}

uint64_t dc_work_floats(uint32_t T, uint32_t nv, uint32_t dv) {
    return (uint64_t)nv * ((T + DC_C - 1) / DC_C) * dc_task_floats(dv);
}

void launch_dc_scan(const PfDnArgs& a, float* work, hipStream_t st) {
    if (!a.T) return;
    if (!dc_supported(a.nk, a.nv, a.qk_dim / std::max(a.nk, 1u), a.dv) || a.qk_dim != a.nk * DC_DK ||
        a.conv_dim != 2 * a.qk_dim + a.nv * a.dv || a.v_dim != a.nv * a.dv)
        throw std::runtime_error("chunked scan needs key and value head dims of 128");
    if (!work) throw std::runtime_error("chunked scan needs its workspace");
    const uint32_t nch = (a.T + DC_C - 1) / DC_C;
    k_dc_prep<<<a.nv * nch, 256, 0, st>>>(a, work);
    k_dc_scan<<<a.nv * (a.dv / 16), DC_WG, 0, st>>>(a, work);
}

}  // namespace chk
