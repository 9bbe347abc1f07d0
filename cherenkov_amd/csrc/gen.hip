// Synthetic weight generation on the device and the Q4 -> Q3/Q2 expert
// store repack.
//
// Generation follows include/cherenkov/synth.h element for element, so the
// HBM-resident store holds the same bytes the CPU oracle generates.
// The repack restates the reference's low-bit store builder
// (/root/reference/src/qwen4_exp/lowbit.rs:143-241: q2_slots, q3_slots,
// pack_matrix): one thread per 32-code chunk, codes dropped to their top 2
// or 3 bits and placed in the slots the decode kernels read.
#include "internal.h"

namespace chk {

__global__ void __launch_bounds__(256) k_gen_q4(uint32_t* w, uint16_t* s, uint16_t* b, uint64_t nwords, uint64_t ngroups,
                         uint64_t kw, uint64_t ks, uint64_t kb) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nwords; i += stride)
        w[i] = chk_q4_word(kw, i);
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < ngroups; i += stride) {
        s[i] = chk_normal_bf16(ks, i, CHK_SCALE_SIGMA);
        b[i] = chk_normal_bf16(kb, i, CHK_BIAS_SIGMA);
    }
}

__global__ void __launch_bounds__(256) k_gen_bf16(uint16_t* dst, uint64_t n, uint64_t seed, uint64_t id, uint32_t kind) {
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        dst[i] = chk_bf16_elem(seed, id, kind, i);
}

// All Q4 records of the routed-expert store: records [n_layers][E] of
// `stride` bytes, each gate/up/down in the pack.rs:351-393 field order.
struct RecGenArgs {
    uint8_t* base;
    uint64_t stride;
    uint64_t seed;
    uint32_t experts, layer0, n_layers;
    uint64_t off_w[3], off_s[3], off_b[3];
    uint64_t words[3], groups[3];
};

__global__ void __launch_bounds__(256) k_gen_records(RecGenArgs a) {
    // blockIdx.y = record within the launch, blockIdx.z = part
    uint32_t rec = blockIdx.y, part = blockIdx.z;
    uint32_t rl = a.layer0 + rec / a.experts, e = rec % a.experts;
    uint8_t* r = a.base + (uint64_t)(rl) * a.experts * a.stride + (uint64_t)e * a.stride;
    uint64_t id = chk_tensor_id(CHK_T_EXPERT, rl, e, part);
    uint64_t kw = chk_key(a.seed, id, CHK_STREAM_W), ks = chk_key(a.seed, id, CHK_STREAM_S),
             kb = chk_key(a.seed, id, CHK_STREAM_B);
    uint32_t* w = (uint32_t*)(r + a.off_w[part]);
    uint16_t* s = (uint16_t*)(r + a.off_s[part]);
    uint16_t* b = (uint16_t*)(r + a.off_b[part]);
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    uint64_t t0 = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (uint64_t i = t0; i < a.words[part]; i += stride) w[i] = chk_q4_word(kw, i);
    for (uint64_t i = t0; i < a.groups[part]; i += stride) {
        s[i] = chk_normal_bf16(ks, i, CHK_SCALE_SIGMA);
        b[i] = chk_normal_bf16(kb, i, CHK_BIAS_SIGMA);
    }
}

// Slot tables of lowbit.rs:143-184 for chunk position c (0..31).
CHK_DEV void slot_of(int c, int& t, int& p, int& byte) {
    t = c >> 4;
    int r = c & 15;
    bool even = (r & 1) == 0, low = r < 8;
    if (even && low) { p = 0; byte = r >> 1; }
    else if (even) { p = 1; byte = (r - 8) >> 1; }
    else if (low) { p = 2; byte = (r - 1) >> 1; }
    else { p = 3; byte = (r - 9) >> 1; }
}

__global__ void __launch_bounds__(256) k_repack_lowbit(const uint8_t* __restrict__ src, uint64_t src_stride, uint8_t* __restrict__ dst,
                                uint64_t dst_stride, uint32_t n_records, uint32_t bits, uint64_t mat_codes,
                                uint64_t src_w0, uint64_t src_w1, uint64_t src_w2, uint64_t dst_mat) {
    uint32_t rec = blockIdx.y, m = blockIdx.z;
    uint64_t src_off = m == 0 ? src_w0 : (m == 1 ? src_w1 : src_w2);
    const uint32_t* sw = (const uint32_t*)(src + (uint64_t)rec * src_stride + src_off);
    uint8_t* d = dst + (uint64_t)rec * dst_stride + (uint64_t)m * dst_mat;
    uint64_t chunks = mat_codes / 32;
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t ch = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; ch < chunks; ch += stride) {
        uint32_t q4w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) q4w[k] = sw[ch * 4 + k];
        if (bits == 2) {
            uint32_t pw0 = 0, pw1 = 0;
#pragma unroll
            for (int c = 0; c < 32; ++c) {
                int t, p, byte;
                slot_of(c, t, p, byte);
                uint32_t code = ((q4w[c >> 3] >> (4 * (c & 7))) & 15u) >> 2;
                uint32_t bitpos = 8 * byte + 2 * p;
                if (t == 0) pw0 |= code << bitpos;
                else pw1 |= code << bitpos;
            }
            uint32_t* o = (uint32_t*)(d + ch * 8);
            o[0] = pw0;
            o[1] = pw1;
        } else {
            uint32_t uw0 = 0, uw1 = 0, lb = 0;
#pragma unroll
            for (int c = 0; c < 32; ++c) {
                int t, j, byte;
                slot_of(c, t, j, byte);
                uint32_t v = ((q4w[c >> 3] >> (4 * (c & 7))) & 15u) >> 1;
                uint32_t up = 8 * byte + 2 * j, lo = 8 * byte + 4 * t + j;
                if (t == 0) uw0 |= (v >> 1) << up;
                else uw1 |= (v >> 1) << up;
                lb |= (v & 1u) << lo;
            }
            uint32_t* o = (uint32_t*)(d + ch * 12);
            o[0] = uw0;
            o[1] = uw1;
            o[2] = lb;
        }
    }
}

// Scale/bias blocks of a low-bit record are copied verbatim from Q4.
__global__ void __launch_bounds__(256) k_copy_scales(const uint8_t* __restrict__ src, uint64_t src_stride, uint8_t* __restrict__ dst,
                              uint64_t dst_stride, uint64_t src_off, uint64_t dst_off, uint64_t bytes) {
    uint32_t rec = blockIdx.y;
    const uint32_t* s = (const uint32_t*)(src + (uint64_t)rec * src_stride + src_off);
    uint32_t* d = (uint32_t*)(dst + (uint64_t)rec * dst_stride + dst_off);
    uint64_t n = bytes / 4, stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) d[i] = s[i];
}

// ------------------------------------------------------------- launchers

void gen_q4(uint32_t* w, uint16_t* s, uint16_t* b, uint32_t out, uint32_t in, uint64_t seed, uint64_t id,
            hipStream_t st) {
    uint64_t nw = (uint64_t)out * in / 8, ng = (uint64_t)out * in / 64;
    uint32_t grid = (uint32_t)std::min<uint64_t>((nw + 255) / 256, 8192);
    k_gen_q4<<<grid, 256, 0, st>>>(w, s, b, nw, ng, chk_key(seed, id, CHK_STREAM_W),
                                   chk_key(seed, id, CHK_STREAM_S), chk_key(seed, id, CHK_STREAM_B));
}

void gen_bf16(uint16_t* dst, uint64_t n, uint64_t seed, uint64_t id, uint32_t kind, hipStream_t st) {
    uint32_t grid = (uint32_t)std::min<uint64_t>((n + 255) / 256, 4096);
    k_gen_bf16<<<grid, 256, 0, st>>>(dst, n, seed, id, kind);
}

void gen_records(uint8_t* base, const RecordLayout& L, uint64_t seed, uint32_t experts, uint32_t layer0,
                 uint32_t n_layers, uint32_t hidden, uint32_t inter, hipStream_t st) {
    RecGenArgs a;
    a.base = base;
    a.stride = L.stride;
    a.seed = seed;
    a.experts = experts;
    a.layer0 = layer0;
    a.n_layers = n_layers;
    a.off_w[0] = L.gate_w; a.off_w[1] = L.up_w; a.off_w[2] = L.down_w;
    a.off_s[0] = L.gate_s; a.off_s[1] = L.up_s; a.off_s[2] = L.down_s;
    a.off_b[0] = L.gate_b; a.off_b[1] = L.up_b; a.off_b[2] = L.down_b;
    for (int p = 0; p < 3; ++p) {
        a.words[p] = (uint64_t)inter * hidden / 8;
        a.groups[p] = (uint64_t)inter * hidden / 64;
    }
    // one launch per layer keeps gridDim.y within limits
    for (uint32_t l = 0; l < n_layers; ++l) {
        a.layer0 = layer0 + l;
        dim3 grid((uint32_t)std::min<uint64_t>((a.words[0] + 255) / 256, 64), experts, 3);
        k_gen_records<<<grid, 256, 0, st>>>(a);
    }
}

void repack_lowbit(const uint8_t* q4, const RecordLayout& src, uint8_t* dst, const RecordLayout& lo,
                   uint32_t n_records, uint64_t mat_codes, hipStream_t st) {
    for (uint32_t r0 = 0; r0 < n_records; r0 += 65535) {
        uint32_t nr = std::min<uint32_t>(65535, n_records - r0);
        dim3 grid((uint32_t)std::min<uint64_t>((mat_codes / 32 + 255) / 256, 64), nr, 3);
        k_repack_lowbit<<<grid, 256, 0, st>>>(q4 + (uint64_t)r0 * src.stride, src.stride, dst + (uint64_t)r0 * lo.stride,
                                              lo.stride, nr, lo.bits, mat_codes, src.gate_w, src.up_w, src.down_w,
                                              lo.up_w - lo.gate_w);
        const uint64_t so[6] = {src.gate_s, src.gate_b, src.up_s, src.up_b, src.down_s, src.down_b};
        const uint64_t dof[6] = {lo.gate_s, lo.gate_b, lo.up_s, lo.up_b, lo.down_s, lo.down_b};
        const uint64_t sz[6] = {lo.scale_up, lo.scale_up, lo.scale_up, lo.scale_up, lo.scale_down, lo.scale_down};
        for (int i = 0; i < 6; ++i) {
            dim3 g2((uint32_t)std::min<uint64_t>((sz[i] / 4 + 255) / 256, 32), nr, 1);
            k_copy_scales<<<g2, 256, 0, st>>>(q4 + (uint64_t)r0 * src.stride, src.stride, dst + (uint64_t)r0 * lo.stride,
                                              lo.stride, so[i], dof[i], sz[i]);
        }
    }
}

}  // namespace chk
