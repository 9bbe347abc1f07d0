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
    float d = 0.0f;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const uint32_t w = ws[m], w8 = w >> 8;
        const h2 q[4] = {__builtin_bit_cast(h2, (w & k.m1) | k.magic) - k.off,
                         __builtin_bit_cast(h2, (w & k.m2) | k.magic) - k.off,
                         __builtin_bit_cast(h2, (w8 & k.m1) | k.magic) - k.off,
                         __builtin_bit_cast(h2, (w8 & k.m2) | k.magic) - k.off};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            d = __builtin_amdgcn_fdot2(q[j], hi[4 * m + j], d, false);
            d = __builtin_amdgcn_fdot2(q[j], lo[4 * m + j], d, false);
        }
    }
    return s * d + b * xsum;
}

}  // namespace chk
