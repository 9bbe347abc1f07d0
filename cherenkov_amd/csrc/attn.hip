// Gated attention decode over the int8 (q8) KV cache.
//
// Reference semantics: attention (cpu.rs:544-641) with the engine's q8 KV
// rule (kv_append_q8, kernels/common/attention.metal:187-234): per 32-lane
// block d = amax/127, q = rint(v/d) clamped to +-127 (0 when d = 0), d kept
// as fp16, dequantised as q * fp16(d).  The split-T flash-decode shape
// (partials (m, l, o) per chunk, then an LSE merge with the sigmoid output
// gate) replaces attn_part2_q8/attn_combine (attention.metal:138-310).
#include "kernels_internal.h"

namespace chk {

// Per head: q RMSNorm + partial RoPE -> q_ready; k RMSNorm + RoPE -> q8 K
// row; v -> q8 V row; the raw indexer key -> index cache.  One workgroup of
// hd threads per (row, item): items [0, nh) q heads, [nh, nh + nkv) k heads,
// [nh + nkv, nh + 2 nkv) v heads, nh + 2 nkv the index key.
__global__ void __launch_bounds__(256) k_attn_prep(AttnArgs a) {
    __shared__ float red[8];
    __shared__ float sx[512];
    const uint32_t b = blockIdx.y, item = blockIdx.x, d = threadIdx.x, hd = a.hd;
    const uint32_t pos = a.pos[b];
    const KvDev& kv = a.kv[b];
    if (item == a.nh + 2 * a.nkv) {
        if (d < a.ihd) kv.index_k[(size_t)pos * a.ihd + d] = a.idx_raw[(size_t)b * (a.inh + 1) * a.ihd + a.inh * a.ihd + d];
        return;
    }
    const bool is_q = item < a.nh, is_k = !is_q && item < a.nh + a.nkv;
    float x;
    if (is_q) x = a.q_raw[(size_t)b * a.nh * 2 * hd + item * 2 * hd + d];
    else if (is_k) x = a.k_raw[(size_t)b * a.nkv * hd + (item - a.nh) * hd + d];
    else x = a.v_raw[(size_t)b * a.nkv * hd + (item - a.nh - a.nkv) * hd + d];
    if (is_q || is_k) {
        // nn::rms_norm (nn.rs:6-15) then rope_partial (cpu.rs:1051-1063)
        float ss = block_sum(x * x, red);
        float inv = 1.0f / sqrtf(ss / (float)hd + a.eps);
        x = x * inv * bf16f(is_q ? a.q_norm[d] : a.k_norm[d]);
        sx[d] = x;
        __syncthreads();
        const uint32_t half = a.rot / 2;
        if (d < a.rot) {
            uint32_t j = d < half ? d : d - half;
            float inv_freq = powf(a.theta, -(2.0f * (float)j) / (float)a.rot);
            float ang = (float)pos * inv_freq;
            float sn = sinf(ang), cs = cosf(ang);
            float av = sx[j], bv = sx[j + half];
            x = d < half ? av * cs - bv * sn : bv * cs + av * sn;
        }
    }
    if (is_q) {
        a.q_ready[((size_t)b * a.nh + item) * hd + d] = x;
        return;
    }
    // q8: 32-lane blocks are half-waves
    float amax = group_max<32>(fabsf(x));
    float dq = amax / 127.0f;
    float qv = dq > 0.0f ? rintf(x / dq) : 0.0f;
    qv = fminf(fmaxf(qv, -127.0f), 127.0f);
    const uint32_t kvh = is_k ? item - a.nh : item - a.nh - a.nkv;
    const uint32_t kv_row = a.nkv * hd;
    int8_t* plane = is_k ? kv.k : kv.v;
    uint16_t* sc = is_k ? kv.ks : kv.vs;
    plane[(size_t)pos * kv_row + kvh * hd + d] = (int8_t)qv;
    if ((d & 31) == 0) sc[(size_t)pos * (kv_row / 32) + (kvh * hd + d) / 32] = __half_as_ushort(__float2half_rn(dq));
}

CHK_DEV float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }

// Partials over one chunk of ATTN_CHUNK tokens for (row b, q head h).
__global__ void __launch_bounds__(256) k_attn_part(AttnArgs a) {
    __shared__ float red[8];
    __shared__ float sq[512];
    __shared__ float sp[ATTN_CHUNK];
    const uint32_t h = blockIdx.x, c = blockIdx.y, b = blockIdx.z, t = threadIdx.x, hd = a.hd;
    const uint32_t T = a.pos[b] + 1;  // causal: rows see positions <= their own
    const uint32_t t0 = c * ATTN_CHUNK;
    float* part = a.part + (((size_t)b * a.nh + h) * a.max_chunks + c) * (hd + 2);
    if (t0 >= T) return;
    const KvDev& kv = a.kv[b];
    const uint32_t hk = h / (a.nh / a.nkv), kv_row = a.nkv * hd;
    for (uint32_t d = t; d < hd; d += blockDim.x) sq[d] = a.q_ready[((size_t)b * a.nh + h) * hd + d];
    __syncthreads();
    const uint32_t tok = t0 + t;
    float s = -INFINITY;
    if (tok < T) {
        const int8_t* kr = kv.k + (size_t)tok * kv_row + hk * hd;
        const uint16_t* ks = kv.ks + (size_t)tok * (kv_row / 32) + hk * hd / 32;
        float acc = 0.0f;
        for (uint32_t blk = 0; blk < hd / 32; ++blk) {
            const int4* p = reinterpret_cast<const int4*>(kr + blk * 32);
            int4 u0 = p[0], u1 = p[1];
            int w[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
            float part_acc = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    float kvv = (float)(int8_t)((w[j] >> (8 * k)) & 0xff);
                    part_acc += sq[blk * 32 + j * 4 + k] * kvv;
                }
            }
            acc += part_acc * h2f(ks[blk]);
        }
        s = acc * a.scale;
    }
    float m = block_max(s, red);
    float p = tok < T ? expf(s - m) : 0.0f;
    sp[t] = p;
    float l = block_sum(p, red);
    const uint32_t n = min(ATTN_CHUNK, T - t0);
    for (uint32_t d = t; d < hd; d += blockDim.x) {
        float o = 0.0f;
        const uint32_t blkd = (hk * hd + d) / 32;
        for (uint32_t j = 0; j < n; ++j) {
            uint32_t tk = t0 + j;
            float vv = (float)kv.v[(size_t)tk * kv_row + hk * hd + d] * h2f(kv.vs[(size_t)tk * (kv_row / 32) + blkd]);
            o += sp[j] * vv;
        }
        part[2 + d] = o;
    }
    if (t == 0) {
        part[0] = m;
        part[1] = l;
    }
}

// LSE merge of the chunk partials and the per-dim sigmoid gate
// (cpu.rs:629-633: the gate is the second half of each head's q_proj rows).
__global__ void __launch_bounds__(256) k_attn_combine(AttnArgs a) {
    const uint32_t h = blockIdx.x, b = blockIdx.y, hd = a.hd;
    const uint32_t T = a.pos[b] + 1, nc = (T + ATTN_CHUNK - 1) / ATTN_CHUNK;
    const float* part = a.part + ((size_t)b * a.nh + h) * a.max_chunks * (hd + 2);
    float M = -INFINITY;
    for (uint32_t c = 0; c < nc; ++c) M = fmaxf(M, part[c * (hd + 2)]);
    float L = 0.0f;
    for (uint32_t c = 0; c < nc; ++c) L += part[c * (hd + 2) + 1] * expf(part[c * (hd + 2)] - M);
    for (uint32_t d = threadIdx.x; d < hd; d += blockDim.x) {
        float o = 0.0f;
        for (uint32_t c = 0; c < nc; ++c) o += part[c * (hd + 2) + 2 + d] * expf(part[c * (hd + 2)] - M);
        float gate = a.q_raw[(size_t)b * a.nh * 2 * hd + h * 2 * hd + hd + d];
        a.out[(size_t)b * a.nh * hd + h * hd + d] = o / L * sigmoidf_(gate);
    }
}

__global__ void __launch_bounds__(256) k_copy_f32(float* __restrict__ dst, const float* __restrict__ src, uint64_t n) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

__global__ void __launch_bounds__(256) k_zero_f32(float* __restrict__ dst, uint64_t n) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = 0.0f;
}

// Positions come from device memory and the chunk grid covers the whole
// context capacity (chunks past a row's length exit at once), so the
// launch is the same every step and can live in a captured graph.
void launch_attn(const AttnArgs& a, int nb, hipStream_t st) {
    k_attn_prep<<<dim3(a.nh + 2 * a.nkv + 1, nb), a.hd, 0, st>>>(a);
    k_attn_part<<<dim3(a.nh, a.max_chunks, nb), ATTN_CHUNK, 0, st>>>(a);
    k_attn_combine<<<dim3(a.nh, nb), 256, 0, st>>>(a);
}

void launch_copy_f32(float* dst, const float* src, uint64_t n, hipStream_t st) {
    uint32_t grid = (uint32_t)std::min<uint64_t>((n + 255) / 256, 2048);
    if (n) k_copy_f32<<<grid, 256, 0, st>>>(dst, src, n);
}

void launch_zero_f32(float* dst, uint64_t n, hipStream_t st) {
    uint32_t grid = (uint32_t)std::min<uint64_t>((n + 255) / 256, 2048);
    if (n) k_zero_f32<<<grid, 256, 0, st>>>(dst, n);
}

}  // namespace chk
