// Prefill GEMMs on gfx950 MFMA: Y[t][n] = sum_k X[t][k] W[n][k] for an MLX
// affine Q4 (group 64) weight W [N][K] and activations X [T][K], with the
// reference's quantisation semantics (quant.rs:13-89: w = s q + b per group)
// kept exact: the MFMA multiplies the integer codes, and the group's scale
// and bias are applied to its partial sums in f32,
//   Y += s[n][g] * (sum_{k in g} q[n][k] x[t][k]) + b[n][g] * (sum_{k in g} x[t][k]).
//
// v_mfma_f32_16x16x32_f16 (A: 16 tokens x 32 k, B: 32 k x 16 outputs, D:
// 16 x 16 f32).  Lane l of B holds output column l % 16 and the 8 k
// values (l / 16) * 8 .. + 8, which is exactly one packed weight word.  The
// word unpacks the way the decode dot does (device.h q4_chunk_h): OR-ing
// the masked word into 1024.0|1024.0 and subtracting 1024 exactly gives the
// fp16 pairs (q0, q4), (16 q1, 16 q5), (q2, q6), (16 q3, 16 q7).  The
// k order inside each 8-block is arbitrary for a dot product as long as A
// uses the same one, so the prepared activations hold, per 8-block,
// x0, x4, x1/16, x5/16, x2, x6, x3/16, x7/16, split into hi and lo fp16
// planes (x = hi + lo, ~22 significant bits); each MFMA pair (hi, lo)
// multiplies exact small integers by exact fp16 values into f32.
//
// Reference counterpart: the prefill qmm GEMMs (gpu/prefill/projection.rs:8-108),
// which run on half operands.
#include <stdexcept>

#include "kernels_internal.h"

namespace chk {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------ activation prep
// X f32 [T][K] (row stride ldx) -> hi, lo fp16 [T][K] in the permuted
// 8-block order above, and xs f32 [T][K/64] = per-group sums of X.
// One thread per 8-block.
__global__ void __launch_bounds__(256) k_pf_xprep(const float* __restrict__ x, uint32_t ldx, uint32_t T, uint32_t K,
                                                  uint4* __restrict__ hi, uint4* __restrict__ lo,
                                                  float* __restrict__ xs) {
    const uint32_t blocks = K >> 3;
    const uint64_t i = (uint64_t)blockIdx.x * CHK_WG + threadIdx.x;
    const bool live = i < (uint64_t)T * blocks;
    const uint32_t t = live ? (uint32_t)(i / blocks) : 0, kb = live ? (uint32_t)(i % blocks) : 0;
    float v[8];
    const float4* p = reinterpret_cast<const float4*>(x + (size_t)t * ldx + kb * 8);
    const float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    // this 8-block's sum, then the 64-group sum over 8 neighbouring lanes
    float s = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    s += __shfl_xor(s, 4, 64);
    if (!live) return;
    const float o[8] = {v[0], v[4], v[1] * 0.0625f, v[5] * 0.0625f, v[2], v[6], v[3] * 0.0625f, v[7] * 0.0625f};
    h8 h, l;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const _Float16 hj = (_Float16)o[j];
        h[j] = hj;
        l[j] = (_Float16)(o[j] - (float)hj);
    }
    hi[i] = __builtin_bit_cast(uint4, h);
    lo[i] = __builtin_bit_cast(uint4, l);
    if ((kb & 7) == 0) xs[(size_t)t * (K >> 6) + (kb >> 3)] = s;
}

// --------------------------------------------------------------- GEMM
// A wave computes 64 tokens x 64 outputs (4 x 4 MFMA tiles); a workgroup's
// four waves cover 64 tokens x 256 outputs.  Grid (ceil(N / 256), ceil(T / 64)).
// Per 64-wide quant group: the group's partial sums accumulate from zero in
// acc_g (2 K-steps of 32, hi then lo), then fold into acc with the group's
// scale and bias.
struct PfGemmArgs {
    Q4Mat w;               // [N][K]
    const uint4* xhi;      // [T][K/8] prepared activations
    const uint4* xlo;
    const float* xs;       // [T][K/64]
    float* y;              // [T][ldy]
    uint32_t T, ldy;
    int accumulate;        // y += result instead of y = result
};

__global__ void __launch_bounds__(256) k_pf_gemm(PfGemmArgs a) {
    const int lane = threadIdx.x & 63, col = lane & 15, kq = lane >> 4;
    const uint32_t N = a.w.out, K = a.w.in, G = K >> 6, KB = K >> 3;
    const uint32_t n0 = blockIdx.x * 256 + wave_id() * 64, t0 = blockIdx.y * 64;
    if (n0 >= N) return;
    uint32_t nrow[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) nrow[j] = min(n0 + j * 16 + col, N - 1);
    uint32_t trow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) trow[i] = min(t0 + i * 16 + col, a.T - 1);
    const Q4Consts qk;
    f4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t g = 0; g < G; ++g) {
        f4 accg[4][4];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const uint32_t kb = g * 8 + s * 4 + kq;  // this lane's 8-block
            h8 bq[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t w = a.w.w[(size_t)nrow[j] * KB + kb], w8 = w >> 8;
                const h2 p0 = __builtin_bit_cast(h2, (w & qk.m1) | qk.magic) - qk.off;
                const h2 p1 = __builtin_bit_cast(h2, (w & qk.m2) | qk.magic) - qk.off;
                const h2 p2 = __builtin_bit_cast(h2, (w8 & qk.m1) | qk.magic) - qk.off;
                const h2 p3 = __builtin_bit_cast(h2, (w8 & qk.m2) | qk.magic) - qk.off;
                bq[j] = h8{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const h8 ah = __builtin_bit_cast(h8, a.xhi[(size_t)trow[i] * KB + kb]);
                const h8 al = __builtin_bit_cast(h8, a.xlo[(size_t)trow[i] * KB + kb]);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f4 c0 = s == 0 ? f4{0.0f, 0.0f, 0.0f, 0.0f} : accg[i][j];
                    accg[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bq[j], c0, 0, 0, 0);
                    accg[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bq[j], accg[i][j], 0, 0, 0);
                }
            }
        }
        // fold: D lane (col = output n0 + 16 j + col, rows t0 + 16 i + 4 kq + r)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float sc = bf16f(a.w.s[(size_t)nrow[j] * G + g]), bi = bf16f(a.w.b[(size_t)nrow[j] * G + g]);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t t = min(t0 + i * 16 + kq * 4 + r, a.T - 1);
                    acc[i][j][r] += sc * accg[i][j][r] + bi * a.xs[(size_t)t * G + g];
                }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t n = n0 + j * 16 + col;
            if (n >= N) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t t = t0 + i * 16 + kq * 4 + r;
                if (t < a.T) {
                    float* yp = a.y + (size_t)t * a.ldy + n;
                    *yp = a.accumulate ? *yp + acc[i][j][r] : acc[i][j][r];
                }
            }
        }
}

// -------------------------------------------------------------- launchers

void launch_pf_xprep(const float* x, uint32_t ldx, uint32_t T, uint32_t K, uint4* hi, uint4* lo, float* xs,
                     hipStream_t st) {
    const uint64_t n = (uint64_t)T * (K >> 3);
    if (!n) return;
    k_pf_xprep<<<(uint32_t)((n + CHK_WG - 1) / CHK_WG), CHK_WG, 0, st>>>(x, ldx, T, K, hi, lo, xs);
}

void launch_pf_gemm(const Q4Mat& w, const uint4* xhi, const uint4* xlo, const float* xs, float* y, uint32_t T,
                    uint32_t ldy, bool accumulate, hipStream_t st) {
    if (w.in % 64) throw std::runtime_error("prefill GEMM needs K a multiple of 64");
    if (!T) return;
    PfGemmArgs a{w, xhi, xlo, xs, y, T, ldy, accumulate ? 1 : 0};
    dim3 grid((w.out + 255) / 256, (T + 63) / 64);
    k_pf_gemm<<<grid, CHK_WG, 0, st>>>(a);
}

}  // namespace chk
