// The PLE n-gram block (reference: CpuModel::ple, src/qwen4_exp/cpu.rs:
// 889-967; its GPU form gpu/ple.rs:48-164 with fn_ple_gate_b / fn_ple_conv_b,
// kernels/qwen4_exp/ple.metal) for decode rows and prefill chunks alike:
//
//   gather  e[r] = the 16 (heads) n-gram table rows of row r's token,
//           dequantised (Packed::ngram_row, packed.rs:233-256);
//   (key / value projections: the Q4 matvec or prefill GEMM of the caller)
//   gate    one workgroup per (row, stream): the stream's key and query
//           RMS, their dot, sigmoid(sign(dot) sqrt(max(|dot|, 1e-6))),
//           gated = s * value and its grouped RMSNorm gvn;
//   conv    one thread per (row, channel): the dilated causal depthwise
//           conv over gvn (taps at p - dilation * (K - 1 - k)), reading
//           positions inside the batch from this batch's gvn and older ones
//           from the ring, then hyper += gated + silu(acc);
//   ring    the batch's last min(rows, span) gvn rows into their ring slots
//           (p % span), first saving each slot's old contents when the
//           caller may roll rows back.
//
// The conv reads before the ring is written (separate launches), so rows of
// one batch never see a slot another row of the batch has overwritten.
#include "kernels_internal.h"

namespace chk {

namespace {

// Synthetic n-gram table (synth.h): row r = dim / 8 words, dim / group
// scales, dim / group biases.
__global__ void __launch_bounds__(256) k_ple_gen_table(uint8_t* __restrict__ table, uint64_t rows, uint32_t dim,
                                                       uint32_t group, uint64_t kw, uint64_t ks, uint64_t kb) {
    const uint64_t r = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (r >= rows) return;
    const uint32_t wpr = dim / 8, gpr = dim / group;
    uint8_t* rec = table + r * chk_ngram_row_bytes(dim, group);
    uint32_t* w = reinterpret_cast<uint32_t*>(rec);
    uint16_t* s = reinterpret_cast<uint16_t*>(rec + 4 * wpr);
    for (uint32_t j = 0; j < wpr; ++j) w[j] = chk_q4_word(kw, r * wpr + j);
    for (uint32_t g = 0; g < gpr; ++g) {
        s[g] = chk_normal_bf16(ks, r * gpr + g, CHK_SCALE_SIGMA);
        s[gpr + g] = chk_normal_bf16(kb, r * gpr + g, CHK_BIAS_SIGMA);
    }
}

// e[r][i] = scale * code + bias of element i % dim of table row
// ids[r][i / dim]; rounded mul then add, as ngram_row computes it.
__global__ void __launch_bounds__(256) k_ple_gather(const uint32_t* __restrict__ ids, uint32_t ids_stride,
                                                    uint32_t nids, const uint8_t* __restrict__ table,
                                                    uint64_t row_bytes, uint32_t dim, uint32_t group,
                                                    float* __restrict__ e) {
    const uint32_t r = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x, E = nids * dim;
    if (i >= E) return;
    const uint32_t j = i % dim, g = j / group, gpr = dim / group;
    const uint8_t* rec = table + (uint64_t)ids[(size_t)r * ids_stride + i / dim] * row_bytes;
    const uint32_t word = reinterpret_cast<const uint32_t*>(rec)[j / 8];
    const uint16_t* sb = reinterpret_cast<const uint16_t*>(rec + dim / 2);
    const float q = (float)((word >> (4 * (j % 8))) & 15u);
    e[(size_t)r * E + i] = __fadd_rn(__fmul_rn(bf16f(sb[g]), q), bf16f(sb[gpr + g]));
}

// Workgroup (stream g, row r).  keyn . query = inv_k inv_q sum(k wk x wq),
// and gated's mean square is s^2 mean(value^2), so one pass gathers the
// four sums and a second writes gated and gvn.
__global__ void __launch_bounds__(256) k_ple_gate(const float* __restrict__ key, const float* __restrict__ hyper,
                                                  uint64_t hyper_stride, const float* __restrict__ value,
                                                  const uint16_t* __restrict__ wk, const uint16_t* __restrict__ wq,
                                                  const uint16_t* __restrict__ wc, float* __restrict__ gated,
                                                  float* __restrict__ gvn, uint32_t H, uint32_t hc, float eps) {
    __shared__ float red[4][CHK_WG / 64];
    const uint32_t g = blockIdx.x, r = blockIdx.y, hh = H * hc;
    const float* k = key + (size_t)r * hh + (size_t)g * H;
    const float* x = hyper + (size_t)r * hyper_stride + (size_t)g * H;
    const float* v = value + (size_t)r * H;
    const uint16_t* wkg = wk + (size_t)g * H;
    const uint16_t* wqg = wq + (size_t)g * H;
    float skk = 0.0f, sxx = 0.0f, skx = 0.0f, svv = 0.0f;
    for (uint32_t i = threadIdx.x; i < H; i += CHK_WG) {
        const float kv = k[i], xv = x[i], vv = v[i];
        skk += kv * kv;
        sxx += xv * xv;
        skx += (kv * bf16f(wkg[i])) * (xv * bf16f(wqg[i]));
        svv += vv * vv;
    }
    skk = wave_sum(skk);
    sxx = wave_sum(sxx);
    skx = wave_sum(skx);
    svv = wave_sum(svv);
    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0) {
        red[0][w] = skk;
        red[1][w] = sxx;
        red[2][w] = skx;
        red[3][w] = svv;
    }
    __syncthreads();
    skk = sxx = skx = svv = 0.0f;
    for (int i = 0; i < CHK_WG / 64; ++i) {
        skk += red[0][i];
        sxx += red[1][i];
        skx += red[2][i];
        svv += red[3][i];
    }
    const float fH = (float)H;
    const float inv_k = 1.0f / sqrtf(skk / fH + eps), inv_q = 1.0f / sqrtf(sxx / fH + eps);
    const float dot = skx * inv_k * inv_q / sqrtf(fH);
    const float gate = sqrtf(fmaxf(fabsf(dot), 1e-6f)) * copysignf(1.0f, dot);
    const float s = sigmoidf_(gate);
    const float inv_c = 1.0f / sqrtf(s * s * svv / fH + eps);
    float* go = gated + (size_t)r * hh + (size_t)g * H;
    float* no = gvn + (size_t)r * hh + (size_t)g * H;
    const uint16_t* wcg = wc + (size_t)g * H;
    for (uint32_t i = threadIdx.x; i < H; i += CHK_WG) {
        const float gt = s * v[i];
        go[i] = gt;
        no[i] = gt * inv_c * bf16f(wcg[i]);
    }
}

// Thread (channel ch, row r) at position pos[r]; the batch starts at pos[0].
__global__ void __launch_bounds__(256) k_ple_conv(const float* __restrict__ gated, const float* __restrict__ gvn,
                                                  const uint16_t* __restrict__ conv, const float* __restrict__ ring,
                                                  float* __restrict__ hyper, uint64_t hyper_stride,
                                                  const uint32_t* __restrict__ pos, uint32_t hh, uint32_t K,
                                                  uint32_t dil, uint32_t span) {
    const uint32_t ch = blockIdx.x * 256 + threadIdx.x, r = blockIdx.y;
    if (ch >= hh) return;
    const uint32_t p = pos[r], p0 = pos[0];
    const uint16_t* w = conv + (size_t)ch * K;
    float acc = bf16f(w[K - 1]) * gvn[(size_t)r * hh + ch];
    for (uint32_t k = 0; k + 1 < K; ++k) {
        const uint32_t back = dil * (K - 1 - k);
        if (back <= p) {
            const uint32_t q = p - back;
            const float src = q >= p0 ? gvn[(size_t)(q - p0) * hh + ch] : ring[(size_t)(q % span) * hh + ch];
            acc += bf16f(w[k]) * src;
        }
    }
    float* hy = hyper + (size_t)r * hyper_stride + ch;
    *hy += gated[(size_t)r * hh + ch] + siluf_(acc);
}

// Block y = j of the batch's last nr rows (row rows - nr + j).
__global__ void __launch_bounds__(256) k_ple_ring(const float* __restrict__ gvn, float* __restrict__ ring,
                                                  float* __restrict__ backup, const uint32_t* __restrict__ pos,
                                                  uint32_t hh, uint32_t span, uint32_t rows, uint32_t nr) {
    const uint32_t ch = blockIdx.x * 256 + threadIdx.x, j = blockIdx.y, r = rows - nr + j;
    if (ch >= hh) return;
    float* slot = ring + (size_t)(pos[r] % span) * hh + ch;
    if (backup) backup[(size_t)j * hh + ch] = *slot;
    *slot = gvn[(size_t)r * hh + ch];
}

}  // namespace

void gen_ngram_table(uint8_t* table, uint64_t rows, uint32_t dim, uint32_t group, uint64_t seed, hipStream_t st) {
    const uint64_t id = chk_tensor_id(CHK_T_NGRAM_TABLE, 0, 0, 0);
    const uint32_t grid = (uint32_t)((rows + 255) / 256);
    k_ple_gen_table<<<grid, 256, 0, st>>>(table, rows, dim, group, chk_key(seed, id, CHK_STREAM_W),
                                          chk_key(seed, id, CHK_STREAM_S), chk_key(seed, id, CHK_STREAM_B));
}

void launch_ple_gather(const uint32_t* ids, uint32_t ids_stride, uint32_t nids, const uint8_t* table,
                       uint64_t row_bytes, uint32_t dim, uint32_t group, float* e, uint32_t rows, hipStream_t st) {
    const dim3 grid((nids * dim + 255) / 256, rows);
    k_ple_gather<<<grid, 256, 0, st>>>(ids, ids_stride, nids, table, row_bytes, dim, group, e);
}

void launch_ple_gate(const float* key, const float* hyper, uint64_t hyper_stride, const float* value,
                     const uint16_t* wk, const uint16_t* wq, const uint16_t* wc, float* gated, float* gvn, uint32_t H,
                     uint32_t hc, float eps, uint32_t rows, hipStream_t st) {
    k_ple_gate<<<dim3(hc, rows), CHK_WG, 0, st>>>(key, hyper, hyper_stride, value, wk, wq, wc, gated, gvn, H, hc, eps);
}

void launch_ple_conv(const float* gated, const float* gvn, const uint16_t* conv, const float* ring, float* hyper,
                     uint64_t hyper_stride, const uint32_t* pos, uint32_t hh, uint32_t K, uint32_t dil, uint32_t span,
                     uint32_t rows, hipStream_t st) {
    const dim3 grid((hh + 255) / 256, rows);
    k_ple_conv<<<grid, 256, 0, st>>>(gated, gvn, conv, ring, hyper, hyper_stride, pos, hh, K, dil, span);
}

void launch_ple_ring(const float* gvn, float* ring, float* backup, const uint32_t* pos, uint32_t hh, uint32_t span,
                     uint32_t rows, hipStream_t st) {
    const uint32_t nr = rows < span ? rows : span;
    const dim3 grid((hh + 255) / 256, nr);
    k_ple_ring<<<grid, 256, 0, st>>>(gvn, ring, backup, pos, hh, span, rows, nr);
}

}  // namespace chk
