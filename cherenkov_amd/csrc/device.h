// Device-side helpers shared by the gfx950 kernels: bf16/fp16 conversion,
// wave64 reductions, MLX-affine Q4 group-64 chunk dots.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "cherenkov/synth.h"

#define CHK_DEV __device__ __forceinline__

namespace chk {

constexpr int WAVE = 64;

CHK_DEV float bf16f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

CHK_DEV float sigmoidf_(float v) { return 1.0f / (1.0f + expf(-v)); }
CHK_DEV float siluf_(float v) { return v / (1.0f + expf(-v)); }
CHK_DEV float softplusf_(float v) { return v > 20.0f ? v : log1pf(expf(v)); }

// DPP lane moves (quad_perm / row_* / row_bcast, GFX9 encodings): the
// source lane's value, or `old` where the row mask or bounds exclude it.
#define CHK_DPPF(v, ctrl, rmask, old) \
    __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), ctrl, rmask, 0xf, false))

// Sum over groups of WIDTH adjacent lanes (a power of two <= 64), valid in
// every lane of the group: DPP within 16-lane rows, row_bcast across rows.
template <int WIDTH>
CHK_DEV float group_sum(float v) {
    if (WIDTH >= 2) v += CHK_DPPF(v, 0xb1, 0xf, 0.0f);   // quad_perm [1,0,3,2]
    if (WIDTH >= 4) v += CHK_DPPF(v, 0x4e, 0xf, 0.0f);   // quad_perm [2,3,0,1]
    if (WIDTH >= 8) v += CHK_DPPF(v, 0x141, 0xf, 0.0f);  // row_half_mirror
    if (WIDTH >= 16) v += CHK_DPPF(v, 0x140, 0xf, 0.0f); // row_mirror
    if (WIDTH == 32) v += __shfl_xor(v, 16, 64);
    if (WIDTH == 64) {
        v += CHK_DPPF(v, 0x142, 0xa, 0.0f);  // row_bcast:15 into rows 1, 3
        v += CHK_DPPF(v, 0x143, 0xc, 0.0f);  // row_bcast:31 into rows 2, 3
        v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
    }
    return v;
}
CHK_DEV float wave_sum(float v) { return group_sum<64>(v); }

template <int WIDTH>
CHK_DEV float group_max(float v) {
#pragma unroll
    for (int m = WIDTH / 2; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, WAVE));
    return v;
}
CHK_DEV float wave_max(float v) { return group_max<64>(v); }

// Every kernel on the step path launches CHK_WG threads per workgroup.  The
// size is a compile-time constant on purpose: reading blockDim.x costs a
// vector memory load of the dispatch packet, and its wait would sit in front
// of every kernel's first weight load.
constexpr uint32_t CHK_WG = 256;

// The wave index, marked wave-uniform so that everything derived from it
// (task ids, segment descriptors) stays in SGPRs and kernel arguments are
// read with scalar loads.
CHK_DEV uint32_t wave_id() { return (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }
// Task order across the grid: consecutive tasks go to different workgroups
// (and so CUs) before a workgroup takes a second one.
CHK_DEV uint32_t global_wave() { return wave_id() * gridDim.x + blockIdx.x; }
CHK_DEV uint32_t total_waves() { return gridDim.x * (CHK_WG >> 6); }

// Block-wide sum of one value per thread over a CHK_WG-thread workgroup;
// `red` is LDS of >= CHK_WG / 64 floats.
CHK_DEV float block_sum(float v, float* red) {
    v = wave_sum(v);
    constexpr int nw = CHK_WG >> 6;
    int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float s = 0.0f;
    for (int i = 0; i < nw; ++i) s += red[i];
    return s;
}
CHK_DEV float block_max(float v, float* red) {
    v = wave_max(v);
    constexpr int nw = CHK_WG >> 6;
    int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float s = red[0];
    for (int i = 1; i < nw; ++i) s = fmaxf(s, red[i]);
    return s;
}

// A quantised linear layer in HBM (MLX affine, bits 4, group 64):
// w u32 [out][in/8] (8 nibbles LSB-first along in), s/b bf16 [out][in/64].
struct Q4Mat {
    const uint32_t* w;
    const uint16_t* s;
    const uint16_t* b;
    uint32_t out, in;
};

// Partial of one 32-input chunk (half a group): s * sum(q x) + b * sum(x),
// with sum(x) precomputed once per chunk (it does not depend on the row).
// f32 reference form, used where the inputs are only needed once.
CHK_DEV float q4_chunk(uint4 wq, const float* x, float xsum, float s, float b) {
    float qd = 0.0f;
    uint32_t ws[4] = {wq.x, wq.y, wq.z, wq.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
#pragma unroll
        for (int j = 0; j < 8; ++j) qd += (float)((ws[k] >> (4 * j)) & 15u) * x[k * 8 + j];
    }
    return s * qd + b * xsum;
}

// ---- the same chunk on the packed fp16 dot (v_dot2_f32_f16)
//
// A u32 weight word holds nibbles q0..q7.  OR-ing the word (or the word
// shifted right by 8), masked to 0x000F000F or 0x00F000F0, into the fp16
// pair 1024.0|1024.0 yields the pairs (1024 + q0, 1024 + q4) and
// (1024 + 16 q1, 1024 + 16 q5), and from w >> 8 (q2, q6) and 16 (q3, q7).
// One packed fp16 subtract removes the 1024 exactly, so each pair holds
// small integers.  The inputs are split as x = hi + lo, two fp16
// round-to-nearest-even values (about 22 significant bits), with the x of
// the 16 q pairs pre-divided by 16 (exact).  Every product of two fp16
// values is exact in f32, and v_dot2_f32_f16 accumulates in f32, so the
// chunk's q . x keeps f32-grade accuracy: 4 v_and_or_b32, 4 v_pk_add_f16
// and 8 v_dot2 per weight word instead of 8 extract + 8 convert + 8 fma.
// Inputs must stay below 65504 / 16 in magnitude (activations here do).
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

struct Q4Consts {
    uint32_t m1, m2, magic;
    h2 off;
    CHK_DEV Q4Consts() : m1(0x000F000Fu), m2(0x00F000F0u), magic(0x64006400u) {
        // the masks as SGPR operands and the magic in a VGPR: one
        // v_and_or_b32 per pair without a second constant-bus operand
        asm volatile("" : "+s"(m1), "+s"(m2), "+v"(magic));
        off = h2{(_Float16)1024.0f, (_Float16)1024.0f};
    }
};

// hi/lo pairs of one lane's 32 inputs in the order the weight words unpack.
CHK_DEV void x_pairs(const float (&v)[32], h2 (&hi)[16], h2 (&lo)[16]) {
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float a = v[8 * m + k], c = v[8 * m + k + 4];
            if (k & 1) {
                a *= 0.0625f;
                c *= 0.0625f;
            }
            const _Float16 ha = (_Float16)a, hc = (_Float16)c;
            hi[4 * m + k] = h2{ha, hc};
            lo[4 * m + k] = h2{(_Float16)(a - (float)ha), (_Float16)(c - (float)hc)};
        }
}

CHK_DEV float q4_chunk_h(uint4 wq, const h2 (&hi)[16], const h2 (&lo)[16], float xsum, float s, float b,
                         const Q4Consts& k) {
    const uint32_t ws[4] = {wq.x, wq.y, wq.z, wq.w};
    // hi and lo products in two independent chains (half the dependent depth)
    float dh = 0.0f, dl = 0.0f;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const uint32_t w = ws[m], w8 = w >> 8;
        const h2 q[4] = {__builtin_bit_cast(h2, (w & k.m1) | k.magic) - k.off,
                         __builtin_bit_cast(h2, (w & k.m2) | k.magic) - k.off,
                         __builtin_bit_cast(h2, (w8 & k.m1) | k.magic) - k.off,
                         __builtin_bit_cast(h2, (w8 & k.m2) | k.magic) - k.off};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            dh = __builtin_amdgcn_fdot2(q[j], hi[4 * m + j], dh, false);
            dl = __builtin_amdgcn_fdot2(q[j], lo[4 * m + j], dl, false);
        }
    }
    return s * (dh + dl) + b * xsum;
}

// ---- inputs as fixed-point nibble planes (the u4 dot8 product)
//
// A 32-input chunk x_0..x_31 is held as u_j = rint((x_j - m) / d) in
// [0, 2^(4 XQ_PLANES) - 1] with m = min_j x_j and d = (max - min) / (2^(4 XQ_PLANES) - 1),
// split into XQ_PLANES planes of nibbles: plane p, word k holds bits
// 4p..4p+3 of u_{8k+j} in nibble j.  A packed Q4 weight word holds q_{8k+j}
// in nibble j, so v_dot8_u32_u4(word, plane p) = sum_j q_j nibble_p(u_j)
// exactly, and
//   sum_j q_j x_j ~= m Q + d sum_p 16^p dot8(w, plane_p),   Q = dot8(w, 0x11111111).
// The plane sums are combined in two exact integer halves (planes 0-2 and
// 3-5, each < 15 * 4095 * 32 < 2^21) before the f32 scale.  The one
// approximation is the input's quantisation, |x - (m + d u)| <= d / 2: with
// six planes, 2^-25 of the chunk's range, on a par with the f32 inputs'
// own rounding.  The bias term uses the exact f32 chunk sum.  Per weight
// word: 7 v_dot8 instead of the 16 VALU ops of the fp16 pair form above,
// which is what keeps batch-1 matvecs HBM-bound.
constexpr int XQ_PLANES = 6;
constexpr float XQ_LEVELS = (float)((1u << (4 * XQ_PLANES)) - 1u);

struct XqChunk {
    uint4 p[XQ_PLANES];  // planes, words k = 0..3
    float4 prm;          // (m, d, sum of the chunk's x, 0)
};

// Product of one Q4 weight chunk (4 words = 32 weights of one row) with an
// input chunk, scaled: s * sum(q x) + b * sum(x) (quant.rs:70-85 per half group).
CHK_DEV float q4_dot8(const uint4& w, const XqChunk& xc, float s, float b) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    uint32_t a[XQ_PLANES], q = 0u;
#pragma unroll
    for (int p = 0; p < XQ_PLANES; ++p) a[p] = 0u;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
#pragma unroll
        for (int p = 0; p < XQ_PLANES; ++p) {
            const uint4 P = xc.p[p];
            const uint32_t pk = k == 0 ? P.x : k == 1 ? P.y : k == 2 ? P.z : P.w;
            a[p] = __builtin_amdgcn_udot8(ws[k], pk, a[p], false);
        }
        q = __builtin_amdgcn_udot8(ws[k], 0x11111111u, q, false);
    }
    uint32_t lo = 0u, hi = 0u;
#pragma unroll
    for (int p = 0; p < XQ_PLANES; ++p) {
        if (p < 3) lo += a[p] << (4 * p);
        else hi += a[p] << (4 * (p - 3));
    }
    const float U = XQ_PLANES > 3 ? fmaf((float)hi, 4096.0f, (float)lo) : (float)lo;
    return s * fmaf(xc.prm.x, (float)q, xc.prm.y * U) + b * xc.prm.z;
}

// Quantise one thread's 8 consecutive inputs (a quarter chunk; the four
// quarters of a chunk sit in one lane quad) into its plane words.  Every
// lane of the wave must call it (DPP quad reductions).  Returns the plane
// words; the quad's lane 0 also gets the chunk's (m, d, sum).
CHK_DEV void xq_quarter(const float (&v)[8], uint32_t (&P)[XQ_PLANES], float4& prm) {
    float mn = v[0], mx = v[0], sm = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        mn = fminf(mn, v[j]);
        mx = fmaxf(mx, v[j]);
        sm += v[j];
    }
    mn = fminf(mn, CHK_DPPF(mn, 0xb1, 0xf, mn));
    mn = fminf(mn, CHK_DPPF(mn, 0x4e, 0xf, mn));
    mx = fmaxf(mx, CHK_DPPF(mx, 0xb1, 0xf, mx));
    mx = fmaxf(mx, CHK_DPPF(mx, 0x4e, 0xf, mx));
    sm += CHK_DPPF(sm, 0xb1, 0xf, 0.0f);
    sm += CHK_DPPF(sm, 0x4e, 0xf, 0.0f);
    const float range = mx - mn;
    // v_rcp (1 ulp) instead of an IEEE divide: u only has to be a rounding
    // of (x - m) / d to within a level, and d below is range / levels
    const float inv = range > 0.0f ? XQ_LEVELS * __builtin_amdgcn_rcpf(range) : 0.0f;
    constexpr uint32_t top = (1u << (4 * XQ_PLANES)) - 1u;
    static_assert(XQ_PLANES == 6, "the byte transpose below is written for six planes");
    // u = round-half-up((x - m) / d), 24 bits
    uint32_t u[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) u[j] = min((uint32_t)fmaf(v[j] - mn, inv, 0.5f), top);
    // Pair (u_2j, u_2j+1) -> t_j holds byte j of planes 0, 2, 4 in its
    // bytes 0, 1, 2 (low nibble from u_2j, high nibble from u_2j+1), s_j the
    // same for planes 1, 3, 5; v_perm_b32 then gathers byte j of the four
    // pairs into each plane word.
    uint32_t t[4], sv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        t[j] = (u[2 * j] & 0x0F0F0Fu) | ((u[2 * j + 1] << 4) & 0xF0F0F0u);
        sv[j] = ((u[2 * j] >> 4) & 0x0F0F0Fu) | (u[2 * j + 1] & 0xF0F0F0u);
    }
    // perm(a, b, sel): result byte i = byte sel_i of {a:b} (b is bytes 0-3)
    const uint32_t a01 = __builtin_amdgcn_perm(t[1], t[0], 0x05010400u);   // t0.0 t1.0 t0.1 t1.1
    const uint32_t a23 = __builtin_amdgcn_perm(t[3], t[2], 0x05010400u);
    const uint32_t b01 = __builtin_amdgcn_perm(t[1], t[0], 0x07030602u);   // t0.2 t1.2 -- --
    const uint32_t b23 = __builtin_amdgcn_perm(t[3], t[2], 0x07030602u);
    const uint32_t c01 = __builtin_amdgcn_perm(sv[1], sv[0], 0x05010400u);
    const uint32_t c23 = __builtin_amdgcn_perm(sv[3], sv[2], 0x05010400u);
    const uint32_t d01 = __builtin_amdgcn_perm(sv[1], sv[0], 0x07030602u);
    const uint32_t d23 = __builtin_amdgcn_perm(sv[3], sv[2], 0x07030602u);
    P[0] = __builtin_amdgcn_perm(a23, a01, 0x05040100u);
    P[2] = __builtin_amdgcn_perm(a23, a01, 0x07060302u);
    P[4] = __builtin_amdgcn_perm(b23, b01, 0x05040100u);
    P[1] = __builtin_amdgcn_perm(c23, c01, 0x05040100u);
    P[3] = __builtin_amdgcn_perm(c23, c01, 0x07060302u);
    P[5] = __builtin_amdgcn_perm(d23, d01, 0x05040100u);
    prm = make_float4(mn, range * (1.0f / XQ_LEVELS), sm, 0.0f);
}

// Workgroup-cooperative quantisation of nrows input rows of K floats (row
// stride xs) into LDS chunks out[b * K/32 + c].  `xform(b, e, v)` may
// rescale the 8 inputs starting at element e of row b before quantisation
// (identity for plain inputs).  Every thread of the WGS-thread workgroup
// must call it with the same arguments; it ends with a barrier.  K must be
// a multiple of 32.
template <uint32_t WGS = CHK_WG, class F>
CHK_DEV void xq_prep(const float* __restrict__ x, uint32_t xs, uint32_t K, uint32_t nrows, XqChunk* out, F&& xform) {
    const uint32_t nblk = K >> 3, total = nrows * nblk;
    for (uint32_t base = 0; base < total; base += WGS) {
        const uint32_t i = base + threadIdx.x;
        const bool live = i < total;
        const uint32_t ii = live ? i : total - 1;
        const uint32_t b = ii / nblk, e = (ii % nblk) * 8;
        const float4* p4 = reinterpret_cast<const float4*>(x + (size_t)b * xs + e);
        const float4 v0 = p4[0], v1 = p4[1];
        float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        xform(b, e, v);
        uint32_t P[XQ_PLANES];
        float4 prm;
        xq_quarter(v, P, prm);
        if (live) {
            const uint32_t c = ii >> 2, k = ii & 3;
            uint32_t* dst = reinterpret_cast<uint32_t*>(out + c);
#pragma unroll
            for (int p = 0; p < XQ_PLANES; ++p) dst[4 * p + k] = P[p];
            if (k == 0) out[c].prm = prm;
        }
    }
    __syncthreads();
}

// One wave quantises 32 values (v32, e.g. in LDS) into the chunk *dst in
// global memory: lanes 0..3 take 8 values each (the other quads repeat them
// so the quad reductions stay defined), lanes 0..3 store the plane words
// and lane 0 the chunk parameters.  Every lane of the wave must call it.
CHK_DEV void xq_chunk_store(const float* v32, XqChunk* dst, int lane) {
    const int k = lane & 3;
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = v32[8 * k + j];
    uint32_t P[XQ_PLANES];
    float4 prm;
    xq_quarter(v, P, prm);
    if (lane < 4) {
        uint32_t* d = reinterpret_cast<uint32_t*>(dst);
#pragma unroll
        for (int p = 0; p < XQ_PLANES; ++p) d[4 * p + k] = P[p];
        if (lane == 0) dst->prm = prm;
    }
}

struct XqIdentity {
    CHK_DEV void operator()(uint32_t, uint32_t, float (&)[8]) const {}
};

// xq_prep in two steps, for a workgroup that issues its input loads ahead
// of its weight loads.  Vector loads return in issue order, so inputs
// issued first can be quantised while the weights are still in flight;
// issued after them, the quantisation waits for every weight as well.
// load() reads up to IT * WGS blocks of 8 inputs into registers (fits()
// says whether the shape is covered; otherwise use xq_prep), store()
// quantises them into LDS exactly as xq_prep does and ends with a barrier.
template <int IT, uint32_t WGS>
struct XqStaged {
    float v[IT][8];

    CHK_DEV static bool fits(uint32_t K, uint32_t nrows) { return nrows * (K >> 3) <= IT * WGS; }

    // Compiler-only ordering (no instruction is emitted): load() ends with
    // a memory clobber so the caller's weight loads stay behind the input
    // loads, and store() starts by redefining the inputs under another, so
    // the quantisation is not hoisted above those weight loads (which
    // would make the wave wait for its inputs before issuing them).
    CHK_DEV void load(const float* __restrict__ x, uint32_t xs, uint32_t K, uint32_t nrows) {
        const uint32_t nblk = K >> 3, total = nrows * nblk;
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            if (it * WGS >= total) break;
            const uint32_t i = it * WGS + threadIdx.x, ii = i < total ? i : total - 1;
            const uint32_t b = ii / nblk, e = (ii % nblk) * 8;
            const float4* p4 = reinterpret_cast<const float4*>(x + (size_t)b * xs + e);
            const float4 v0 = p4[0], v1 = p4[1];
            v[it][0] = v0.x;
            v[it][1] = v0.y;
            v[it][2] = v0.z;
            v[it][3] = v0.w;
            v[it][4] = v1.x;
            v[it][5] = v1.y;
            v[it][6] = v1.z;
            v[it][7] = v1.w;
        }
        asm volatile("" ::: "memory");
    }

    template <class F>
    CHK_DEV void store(uint32_t K, uint32_t nrows, XqChunk* out, F&& xform) {
        const uint32_t nblk = K >> 3, total = nrows * nblk;
#pragma unroll
        for (int it = 0; it < IT; ++it)
#pragma unroll
            for (int j = 0; j < 8; ++j) asm volatile("" : "+v"(v[it][j])::"memory");
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            if (it * WGS >= total) break;
            const uint32_t i = it * WGS + threadIdx.x;
            const bool live = i < total;
            const uint32_t ii = live ? i : total - 1;
            const uint32_t b = ii / nblk, e = (ii % nblk) * 8;
            float w[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) w[j] = v[it][j];
            xform(b, e, w);
            uint32_t P[XQ_PLANES];
            float4 prm;
            xq_quarter(w, P, prm);
            if (live) {
                const uint32_t c = ii >> 2, k = ii & 3;
                uint32_t* dst = reinterpret_cast<uint32_t*>(out + c);
#pragma unroll
                for (int p = 0; p < XQ_PLANES; ++p) dst[4 * p + k] = P[p];
                if (k == 0) out[c].prm = prm;
            }
        }
        __syncthreads();
    }
};

}  // namespace chk
