// MTP prelude/fold and the q8 KV fill used by the attention block tests.
#include <stdexcept>

#include "kernels_internal.h"

namespace chk {

// rms_norm_shift (cpu.rs:999-1008, the (1 + w) convention) of the next
// token's embedding (item 0) and of each trunk stream g (items 1..hc)
// (mtp_forward, cpu.rs:344-369).
__global__ void __launch_bounds__(256) k_mtp_prelude(const uint32_t* __restrict__ tokens, Q4Mat emb,
                                                     const uint16_t* __restrict__ enorm,
                                                     const uint16_t* __restrict__ hnorm,
                                                     const float* __restrict__ src, float* __restrict__ en,
                                                     float* __restrict__ hn, uint32_t H, uint32_t hc, float eps) {
    __shared__ float red[8];
    const uint32_t b = blockIdx.y, item = blockIdx.x;
    float ss = 0.0f;
    if (item == 0) {
        const uint32_t tok = tokens[b];
        for (uint32_t i = threadIdx.x; i < H; i += CHK_WG) {
            uint32_t word = emb.w[(size_t)tok * (H / 8) + i / 8];
            float s = bf16f(emb.s[(size_t)tok * (H / 64) + i / 64]), bb = bf16f(emb.b[(size_t)tok * (H / 64) + i / 64]);
            float e = __fadd_rn(__fmul_rn(s, (float)((word >> (4 * (i % 8))) & 15u)), bb);
            en[(size_t)b * H + i] = e;
            ss += e * e;
        }
        float tot = block_sum(ss, red);
        float inv = 1.0f / sqrtf(tot / (float)H + eps);
        for (uint32_t i = threadIdx.x; i < H; i += CHK_WG)
            en[(size_t)b * H + i] = en[(size_t)b * H + i] * inv * (1.0f + bf16f(enorm[i]));
    } else {
        const uint32_t g = item - 1;
        const float* x = src + (size_t)b * H * hc + (size_t)g * H;
        for (uint32_t i = threadIdx.x; i < H; i += CHK_WG) ss += x[i] * x[i];
        float tot = block_sum(ss, red);
        float inv = 1.0f / sqrtf(tot / (float)H + eps);
        float* o = hn + ((size_t)b * hc + g) * H;
        for (uint32_t i = threadIdx.x; i < H; i += CHK_WG) o[i] = x[i] * inv * (1.0f + bf16f(hnorm[(size_t)g * H + i]));
    }
}

__global__ void __launch_bounds__(256) k_mtp_fold(const float* __restrict__ fe, const float* __restrict__ fh, float* __restrict__ hyper,
                           uint32_t H, uint32_t hc) {
    const uint32_t b = blockIdx.y, i = blockIdx.x * CHK_WG + threadIdx.x;
    if (i >= H) return;
    for (uint32_t g = 0; g < hc; ++g)
        hyper[(size_t)b * H * hc + g * H + i] = fe[(size_t)b * H + i] + fh[((size_t)b * hc + g) * H + i];
}

// q8 quantisation of whole cache rows (the kv_append_q8 rule).
__global__ void __launch_bounds__(256) k_kv_fill(const float* __restrict__ k, const float* __restrict__ v, KvDev kv, uint64_t n,
                          uint32_t kv_row) {
    const uint64_t i = (uint64_t)blockIdx.x * CHK_WG + threadIdx.x;
    const int side = blockIdx.y;
    const float x = i < n ? (side == 0 ? k[i] : v[i]) : 0.0f;
    float amax = group_max<32>(fabsf(x));
    float dq = amax / 127.0f;
    float qv = dq > 0.0f ? rintf(x / dq) : 0.0f;
    qv = fminf(fmaxf(qv, -127.0f), 127.0f);
    if (i >= n) return;
    (side == 0 ? kv.k : kv.v)[i] = (int8_t)qv;
    if ((i & 31) == 0) (side == 0 ? kv.ks : kv.vs)[i / 32] = __half_as_ushort(__float2half_rn(dq));
}

void launch_mtp_prelude(const uint32_t* tokens, const Q4Mat& emb, const uint16_t* enorm, const uint16_t* hnorm,
                        const float* src_hyper, float* e_n, float* h_n, uint32_t H, uint32_t hc, float eps, int rows,
                        hipStream_t st) {
    k_mtp_prelude<<<dim3(1 + hc, rows), 256, 0, st>>>(tokens, emb, enorm, hnorm, src_hyper, e_n, h_n, H, hc, eps);
}

void launch_mtp_fold(const float* fe, const float* fh, float* hyper, uint32_t H, uint32_t hc, int rows,
                     hipStream_t st) {
    k_mtp_fold<<<dim3((H + 255) / 256, rows), 256, 0, st>>>(fe, fh, hyper, H, hc);
}

void launch_kv_fill(const float* k, const float* v, KvDev kv, uint32_t kv_row, uint32_t T, hipStream_t st) {
    uint64_t n = (uint64_t)T * kv_row;
    if (!n) return;
    k_kv_fill<<<dim3((uint32_t)((n + 255) / 256), 2), 256, 0, st>>>(k, v, kv, n, kv_row);
}


// Dependent-FMA clock probe (Gpu::throttle_ms, gpu.rs:596-599 over
// MetalContext::throttle_probe, metal.rs:167-212): 65536 threads each run
// `iters` pairs of dependent FMAs; a slower run means lower clocks.
__global__ void __launch_bounds__(256) k_clock_probe(float* __restrict__ out, uint32_t iters) {
    const uint32_t gid = blockIdx.x * 256 + threadIdx.x;
    float x = 1.0f + (float)gid * 1e-9f;
    for (uint32_t i = 0; i < iters; ++i) {
        x = fmaf(x, 1.0000001f, 1e-7f);
        x = fmaf(x, 0.9999999f, -1e-7f);
    }
    out[gid] = x;
}

void launch_clock_probe(float* out, uint32_t iters, hipStream_t st) {
    k_clock_probe<<<65536 / 256, 256, 0, st>>>(out, iters);
}

}  // namespace chk
