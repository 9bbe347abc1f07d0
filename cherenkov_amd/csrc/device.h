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

// Block-wide sum of one value per thread; `red` is LDS of >= blockDim/64 floats.
CHK_DEV float block_sum(float v, float* red) {
    v = wave_sum(v);
    int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float s = 0.0f;
    for (int i = 0; i < nw; ++i) s += red[i];
    return s;
}
CHK_DEV float block_max(float v, float* red) {
    v = wave_max(v);
    int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
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

}  // namespace chk
