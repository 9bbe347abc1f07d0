// Prefill on gfx950: a chunk of T prompt tokens goes through the decoder
// one layer at a time, every projection as an MFMA GEMM over all T rows
// (prefill_chunk / pf_layer, src/qwen4_exp/gpu/prefill.rs:124-464).
//
// Q4 GEMMs: Y[t][n] = sum_k X[t][k] W[n][k] for an MLX affine Q4 (group 64)
// weight W [N][K] and activations X [T][K], with the reference's
// quantisation semantics (quant.rs:13-89: w = s q + b per group) kept
// exact: the MFMA multiplies the integer codes, and the group's scale and
// bias are applied to its partial sums in f32,
//   Y += s[n][g] * (sum_{k in g} q[n][k] x[t][k]) + b[n][g] * (sum_{k in g} x[t][k]).
//
// v_mfma_f32_16x16x32_f16 (A: 16 rows x 32 k, B: 32 k x 16 outputs, D:
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
// Reference counterparts: the prefill qmm GEMMs (gpu/prefill/projection.rs:8-108,
// half operands there), the grouped experts (gpu/prefill/experts.rs:29-345),
// the sequential scan (gpu/prefill/deltanet.rs:7-110).
#include <algorithm>
#include <cstdint>
#include <stdexcept>
#include <type_traits>

#include "kernels_internal.h"

namespace chk {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

CHK_DEV uint32_t f2bf_rne(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// ------------------------------------------------------ activation prep
// X f32 [T][K] (row stride ldx) -> hi, lo fp16 [T][K/8] uint4 in the
// permuted 8-block order above, xs f32 [T][K/64] = per-group sums of X, and
// optionally bf16 hi/lo planes in natural order (the router's operands).
// One thread per 8-block.  PP_DN_GATE prepares the DeltaNet output instead:
// x = y, and each value head is gated as rmsnorm(y_head) * w * sigmoid(z)
// (cpu.rs:814-826, eps 1e-6) before the split.
enum PfPrepMode { PP_PLAIN = 0, PP_DN_GATE = 1 };

template <int MODE, int HEAD_LANES>
__global__ void __launch_bounds__(256) k_pf_prep(PfPrepArgs a) {
    const uint32_t blocks = a.K >> 3;
    const uint64_t i = (uint64_t)blockIdx.x * CHK_WG + threadIdx.x;
    const bool live = i < (uint64_t)a.T * blocks;
    const uint32_t t = live ? (uint32_t)(i / blocks) : 0, kb = live ? (uint32_t)(i % blocks) : 0;
    float v[8];
    {
        const float4* p = reinterpret_cast<const float4*>(a.x + (size_t)t * a.ldx + kb * 8);
        const float4 u0 = p[0], u1 = p[1];
        v[0] = u0.x; v[1] = u0.y; v[2] = u0.z; v[3] = u0.w; v[4] = u1.x; v[5] = u1.y; v[6] = u1.z; v[7] = u1.w;
    }
    if (!live)
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = 0.0f;
    if (MODE == PP_DN_GATE) {
        float sq = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) sq += v[j] * v[j];
        sq = group_sum<HEAD_LANES>(sq);
        const float inv = 1.0f / sqrtf(sq / (float)a.dv + 1e-6f);
        const float4* zp = reinterpret_cast<const float4*>(a.z + (size_t)t * a.ldx + kb * 8);
        const float4 z0 = zp[0], z1 = zp[1];
        const float z[8] = {z0.x, z0.y, z0.z, z0.w, z1.x, z1.y, z1.z, z1.w};
        const uint32_t d0 = (kb * 8) % a.dv;
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = live ? v[j] * bf16f(a.norm[d0 + j]) * sigmoidf_(z[j]) * inv : 0.0f;
    }
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
    a.hi[i] = __builtin_bit_cast(uint4, h);
    a.lo[i] = __builtin_bit_cast(uint4, l);
    if ((kb & 7) == 0) a.xs[(size_t)t * (a.K >> 6) + (kb >> 3)] = s;
    if (a.bhi) {
        // three bf16 terms (x = hi + mid + lo, ~24 significant bits)
        uint32_t bh[8], bm[8], bl[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            bh[j] = f2bf_rne(v[j]);
            const float r1 = v[j] - __uint_as_float(bh[j] << 16);
            bm[j] = f2bf_rne(r1);
            bl[j] = f2bf_rne(r1 - __uint_as_float(bm[j] << 16));
        }
        a.bhi[i] = make_uint4(bh[0] | bh[1] << 16, bh[2] | bh[3] << 16, bh[4] | bh[5] << 16, bh[6] | bh[7] << 16);
        a.bmid[i] = make_uint4(bm[0] | bm[1] << 16, bm[2] | bm[3] << 16, bm[4] | bm[5] << 16, bm[6] | bm[7] << 16);
        a.blo[i] = make_uint4(bl[0] | bl[1] << 16, bl[2] | bl[3] << 16, bl[4] | bl[5] << 16, bl[6] | bl[7] << 16);
    }
}

// The GEMM epilogues' sigmoid and SiLU (T hc H sigmoids per
// hyper-connection read, T (k+1) I SiLUs per expert gate/up): e^-v as
// 2^(-v log2 e) on the transcendental unit and one hardware reciprocal, a
// few instructions against ~25 for 1 / (1 + expf(-v)).  Absolute error of
// the sigmoid below 3e-7 for |v| <= 16, exact limits 0 and 1 beyond.
CHK_DEV float sigmoid_hw(float v) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(v * -1.44269504088896341f));
}
CHK_DEV float silu_hw(float v) { return v * sigmoid_hw(v); }

// ----------------------------------------------- hyper-connection norm
// normed[t][g H + k] = hyper[t][g H + k] * inv[t][g] * w[g H + k] with
// inv = 1/sqrt(mean_k(hyper[t][g H + k]^2) + eps) per stream g (the
// grouped RMSNorm of gated_residual, cpu.rs:461-475), prepared as GEMM
// operands over K = hc H.  One workgroup per row; thread tau owns 8-blocks
// tau and tau + 256 of every stream (H <= 4096).
// With `part`, first the inject of the block before (cpu.rs:971-979) the
// out-projection left as nsplit K-chunk partials: hyper[t][g H + n] +=
// (sum_z part[z][t][n]) inj[t][g], written back to hyper.
// MK >= 0: instead the expert block before, left as its down rows (mc,
// k_pf_moe_combine's inputs and sums: the routed slots in rank order,
// then the gated shared slot; MK routed slots at compile time, 0: mc.topk
// at run time), injected the same way.
template <int MK>
__global__ void __launch_bounds__(256) k_pf_hc_prep(float* __restrict__ hyper, const uint16_t* __restrict__ norm,
                                                    uint32_t H, uint32_t hc, float eps, float* __restrict__ inv_out,
                                                    uint4* __restrict__ hi, uint4* __restrict__ lo,
                                                    float* __restrict__ xs, const float* __restrict__ part,
                                                    uint64_t pzs, uint32_t nsplit, const float* __restrict__ pinj,
                                                    PfCombine mc) {
    __shared__ float red[4][4];
    const uint32_t t = blockIdx.x, tau = threadIdx.x, bps = H >> 3, hh = H * hc;
    float* row = hyper + (size_t)t * hh;
    float pv[2][8];
    if constexpr (MK >= 0) {
        const uint32_t K = MK > 0 ? (uint32_t)MK : mc.topk, slots = K + 1;
        const uint32_t* pt = mc.pos + (size_t)t * slots;
        auto grow = [&](uint32_t r) {
            const uint32_t q = pt[r];
            return (size_t)(mc.goff[q >> 22] + (q & 0x3fffffu)) * H;
        };
        const float sgv = sigmoidf_(mc.sg[t]);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t kb = min(tau + 256 * j, bps - 1);
#pragma unroll
            for (int e = 0; e < 8; ++e) pv[j][e] = 0.0f;
            if (256 * j >= bps) continue;  // uniform
            auto add = [&](size_t ro, float w) {
                const float4* p = reinterpret_cast<const float4*>(mc.yd + ro + kb * 8);
                const float4 u0 = p[0], u1 = p[1];
                const float w8[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) pv[j][e] += w * w8[e];
            };
            if constexpr (MK > 0) {
                size_t ro[MK + 1];
#pragma unroll
                for (int r = 0; r <= MK; ++r) ro[r] = grow(r);
                float4 u[MK + 1][2];
#pragma unroll
                for (int r = 0; r <= MK; ++r) {
                    const float4* p = reinterpret_cast<const float4*>(mc.yd + ro[r] + kb * 8);
                    u[r][0] = p[0];
                    u[r][1] = p[1];
                }
#pragma unroll
                for (int r = 0; r <= MK; ++r) {
                    const float w = r < MK ? mc.wts[(size_t)t * MK + r] : sgv;
                    const float w8[8] = {u[r][0].x, u[r][0].y, u[r][0].z, u[r][0].w,
                                         u[r][1].x, u[r][1].y, u[r][1].z, u[r][1].w};
#pragma unroll
                    for (int e = 0; e < 8; ++e) pv[j][e] += w * w8[e];
                }
            } else {
                for (uint32_t r = 0; r < K; ++r) add(grow(r), mc.wts[(size_t)t * K + r]);
                add(grow(K), sgv);
            }
        }
        pinj = mc.inj;
    } else if (part) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t kb = min(tau + 256 * j, bps - 1);
#pragma unroll
            for (int e = 0; e < 8; ++e) pv[j][e] = 0.0f;
            for (uint32_t z = 0; z < nsplit; ++z) {
                const float4* p = reinterpret_cast<const float4*>(part + z * pzs + (size_t)t * H + kb * 8);
                const float4 u0 = p[0], u1 = p[1];
                const float w8[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) pv[j][e] += w8[e];
            }
        }
    }
    float v[4][2][8];
    float sq[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t kb = tau + 256 * j;
            const bool ok = (uint32_t)g < hc && kb < bps;
            float4* p = reinterpret_cast<float4*>(row + (size_t)(ok ? g : 0) * H + (ok ? kb : 0) * 8);
            float4 u0 = p[0], u1 = p[1];
            if ((MK >= 0 || part) && ok) {
                const float ij = pinj[(size_t)t * hc + g];
                u0 = make_float4(u0.x + pv[j][0] * ij, u0.y + pv[j][1] * ij, u0.z + pv[j][2] * ij, u0.w + pv[j][3] * ij);
                u1 = make_float4(u1.x + pv[j][4] * ij, u1.y + pv[j][5] * ij, u1.z + pv[j][6] * ij, u1.w + pv[j][7] * ij);
                p[0] = u0;
                p[1] = u1;
            }
            const float w8[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                v[g][j][e] = ok ? w8[e] : 0.0f;
                sq[g] += v[g][j][e] * v[g][j][e];
            }
        }
    // the four streams' sums of squares in one pass (one barrier)
#pragma unroll
    for (int g = 0; g < 4; ++g) sq[g] = wave_sum(sq[g]);
    if ((tau & 63) == 0)
#pragma unroll
        for (int g = 0; g < 4; ++g) red[tau >> 6][g] = sq[g];
    __syncthreads();
    float inv[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        if ((uint32_t)g >= hc) {
            inv[g] = 0.0f;
            continue;
        }
        inv[g] = 1.0f / sqrtf(((red[0][g] + red[1][g]) + (red[2][g] + red[3][g])) / (float)H + eps);
        if (tau == 0) inv_out[(size_t)t * hc + g] = inv[g];
    }
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t kb = tau + 256 * j;
            if ((uint32_t)g >= hc || 256 * j >= bps) continue;  // uniform
            const bool ok = kb < bps;
            float x[8];
            const uint4 nw = *reinterpret_cast<const uint4*>(norm + (size_t)g * H + min(kb, bps - 1) * 8);
            const uint32_t nn[4] = {nw.x, nw.y, nw.z, nw.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float wn = __uint_as_float(e & 1 ? nn[e >> 1] & 0xffff0000u : nn[e >> 1] << 16);
                x[e] = ok ? v[g][j][e] * inv[g] * wn : 0.0f;
            }
            float s = ((x[0] + x[1]) + (x[2] + x[3])) + ((x[4] + x[5]) + (x[6] + x[7]));
            s += __shfl_xor(s, 1, 64);
            s += __shfl_xor(s, 2, 64);
            s += __shfl_xor(s, 4, 64);
            if (!ok) continue;
            const float o[8] = {x[0], x[4], x[1] * 0.0625f, x[5] * 0.0625f, x[2], x[6], x[3] * 0.0625f, x[7] * 0.0625f};
            h8 h, l;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const _Float16 he = (_Float16)o[e];
                h[e] = he;
                l[e] = (_Float16)(o[e] - (float)he);
            }
            const size_t idx = (size_t)t * (hh >> 3) + (size_t)g * bps + kb;
            hi[idx] = __builtin_bit_cast(uint4, h);
            lo[idx] = __builtin_bit_cast(uint4, l);
            if ((kb & 7) == 0) xs[(size_t)t * (hh >> 6) + (size_t)g * (H >> 6) + (kb >> 3)] = s;
        }
}

// --------------------------------------------------------------- GEMM
// Tile: a workgroup of 4 waves covers 16 NI (64) rows x 256 / NMAT outputs
// of every matrix; wave w takes all rows and outputs 64 w / NMAT .. (four
// 16-wide MFMA tiles per 16 rows in all), so every unpacked weight word
// feeds NI x 2 MFMAs.  The A tile of each quant group (hi and lo planes)
// is staged through LDS once for the 4 waves, double-buffered with the
// next group's global loads; every wave streams its own weight words one
// group ahead.  Per group and 16-row slice the MFMA partial sums start from
// zero (two K-steps of 32, hi then lo) and fold into the accumulator with
// the group's scale.  Two workgroups share a CU.
//
// Rows: dense (row m of A and Y), or grouped: a tile list names (group,
// tile) and, per tile, the group's first row in grouped order (off) and
// its row count; Y row off + m, A row off + m, or, with a list,
// list[group][m] / div.  The routed-expert GEMMs group the (token, slot)
// entries e = t (k+1) + slot by expert: gate/up reads token t (list entry
// e, div k+1) and writes the entry's activation at its grouped position,
// down reads and writes grouped rows; group == X.experts is the shared
// expert.
//
// Epilogues: PE_STORE (concatenated segments, each with its own output),
// PE_HC_UP (the four 16-wide tiles of a wave are the hc streams of the same
// 16 outputs: mixed = (1/hc) sum_g sigmoid(v_g) normed_g, cpu.rs:477-491),
// PE_SILU_MUL (NMAT 2: silu(gate) * up, mlp, cpu.rs:981-992).
constexpr int PF_WG = 256;  // threads per GEMM workgroup
constexpr int PF_AROW = 9;  // uint4 per staged A row (8 + 1 pad: bank spread)

CHK_DEV h8 pf_unpack(uint32_t w, const Q4Consts& qk) {
    const uint32_t w8 = w >> 8;
    const h2 p0 = __builtin_bit_cast(h2, (w & qk.m1) | qk.magic) - qk.off;
    const h2 p1 = __builtin_bit_cast(h2, (w & qk.m2) | qk.magic) - qk.off;
    const h2 p2 = __builtin_bit_cast(h2, (w8 & qk.m1) | qk.magic) - qk.off;
    const h2 p3 = __builtin_bit_cast(h2, (w8 & qk.m2) | qk.magic) - qk.off;
    return h8{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

// SBL: the scales of the workgroup's 256 weight rows are staged through LDS
// in blocks of 8 groups (thread t loads row t's 8 scales with one 16-byte
// load per block and stores them as f32, group-major); the main loop then
// folds only s * partial, and the bias term sum_g b[n][g] xs[m][g] opens
// the accumulation as its own small MFMA contraction over the groups (bf16,
// with xs split into three bf16 terms so every product is exact).  Needs
// G % 8 == 0 and 16-byte aligned rows; otherwise each lane loads its scale
// and bias per group and folds both in the loop.  SBL launches also take
// the transposed tile.  NI: 16-row slices per tile (a tile computes only
// the slices that hold rows).
// BITS: the routed-expert records' precision.  Q3 / Q2 rows (lowbit.rs
// chunks of 32 codes in 3 / 2 words) load, per group and lane, the word of
// the lane's 16 inputs (and Q3's low-bit word) and expand it to the two
// Q4-order nibble words the unpack expects; their scale and bias carry the
// midpoint rule (step s, half s + b), folded per lane in f32, so such
// launches run without staged scales.
template <int NMAT, int EPI, bool SBL, int BITS = 4, int NI = 4>
__global__ void __launch_bounds__(PF_WG, 2) k_pf_gemm(PfGemmArgs ka) {
    // The arguments read through the kernarg segment's own (constant)
    // address space: every use is then a scalar load at its point of use
    // rather than a value held in SGPRs across the kernel (the kernel's
    // one argument sits at the segment's start).  Measured: expert down
    // GEMM -9%, dense in-projections -5%; the mix epilogue's GEMM runs
    // better on the by-value argument and keeps it.
#if defined(__HIP_DEVICE_COMPILE__)
    typedef std::conditional_t<EPI == PE_HC_UP, const PfGemmArgs,
                               const __attribute__((address_space(4))) PfGemmArgs>
        KArgs;
    KArgs* pa;
    if constexpr (EPI == PE_HC_UP) pa = &ka;
    else pa = (KArgs*)__builtin_amdgcn_kernarg_segment_ptr();
#else
    typedef const PfGemmArgs KArgs;  // (the host pass only parses the body)
    KArgs* pa = &ka;
#endif
    KArgs& a = *pa;
    static_assert(NI == 4 || SBL, "tiles of fewer than 64 rows take the transposed (staged-scale) form");
    constexpr int NJ = 4 / NMAT;       // 16-wide output tiles per matrix per wave
    constexpr uint32_t TR = 16 * NI;   // tile rows: NI 16-row slices per wave
    // SBL launches compute the transposed tile (weights as the MFMA's A
    // operand): a lane then holds 4 consecutive outputs of one row, so the
    // scales it folds are 4 consecutive staged rows and its results leave
    // as 16-byte stores straight from registers
    constexpr bool SW = SBL;
    __shared__ __align__(16) u32x4 sA[2][2][64 * PF_AROW];
    __shared__ __align__(16) float sX[2][64];
    __shared__ __align__(16) float sSB[SBL ? 2 : 1][SBL ? 8 * 256 : 1];  // [block][group % 8][local row]
    __shared__ uint32_t sRow[64];  // Y row of each tile row (staged epilogue)
    const int tid = threadIdx.x, lane = tid & 63, col = lane & 15, kq = lane >> 4;
    const uint32_t wn = wave_id();
    uint32_t bx = blockIdx.x, by = blockIdx.y;
    const bool grouped = a.tinfo != nullptr;
    if (grouped) {
        // XCD-aware order: workgroups are dealt to the 8 XCDs round-robin
        // by linear id, so linear ids L = 8 s + x map to items w = x C + s
        // % C of chunk s / C (C = 2 gridDim.x items: every column block of
        // two consecutive tiles).  Each chunk runs on one XCD: its tiles' A
        // rows come from HBM once for all column blocks, and an expert's
        // two tiles (the list starts them at even positions) share its
        // weights through that XCD's L2.  gridDim.y is a multiple of 16.
        const uint32_t C = 2 * gridDim.x, L = blockIdx.y * gridDim.x + blockIdx.x;
        const uint32_t sl = L >> 3, w = (sl / C) * 8 * C + (L & 7) * C + sl % C;
        bx = w % gridDim.x;
        by = w / gridDim.x;
    }
    // grouped: the tile's group, its first row in grouped order and the
    // group's row count come with the tile (one round trip)
    uint32_t grp = 0, mt = by, toff = 0, M = a.M;
    if (grouped) {
        if (by >= *a.ntiles) return;
        const uint32_t tv = a.tiles[by];
        const uint2 ti = a.tinfo[by];
        grp = tv >> 16;
        mt = tv & 0xffffu;
        toff = ti.x;
        M = ti.y;
    }
    const uint32_t m0 = mt * TR;
    if (m0 >= M) return;
    // 16-row slices holding rows (a grouped tile is often short: expert
    // row counts run from 1 to over 1000): the MFMAs, folds and bias terms
    // of the empty slices are skipped, a uniform branch per slice
    const uint32_t ni = min((uint32_t)NI, (M - m0 + 15) / 16);
    const uint32_t* list = a.list ? a.list + (size_t)grp * a.cap : nullptr;
    const uint32_t K = a.K, G = K >> 6, KB = K >> 3;
    // split K: this workgroup's groups [gb, ge)
    const uint32_t gc = G / gridDim.z, gb = blockIdx.z * gc, ge = gb + gc;

    // ---- weight rows as 32-bit element offsets from one workgroup-uniform
    // base per array (the record of a routed expert, else the lowest
    // segment matrix).  Local row lr = ((w NMAT + q) NJ + j) 16 + col of the
    // workgroup's 256 is matrix q, tile j of wave w.
    const bool expert = a.X.base && grp < a.X.experts;
    // a low-bit launch decodes the group's record at X.bits unless its kind
    // is 0, then from its 4-bit copy in X4 (workgroup-uniform)
    bool lowbit = BITS != 4 && expert;
    if (BITS != 4 && expert && a.kinds) lowbit = a.kinds[(size_t)a.record_layer * a.X.experts + grp] != 0;
    const ExpertsDev& XR = (BITS == 4 || lowbit) ? a.X : a.X4;
    constexpr uint32_t CW = BITS == 2 ? 2 : 3;  // words per 32-code low-bit chunk
    const uint8_t* rec = XR.base + ((size_t)a.record_layer * XR.experts + grp) * XR.stride;
    const uint32_t* wb = expert ? reinterpret_cast<const uint32_t*>(rec) : a.wbase;
    const uint16_t* sbase = expert ? reinterpret_cast<const uint16_t*>(rec) : a.sbase;
    auto out_of = [&](uint32_t wn_, int j, uint32_t col_) __attribute__((always_inline)) -> uint32_t {
        return EPI == PE_HC_UP ? bx * 64 + wn_ * 16 + col_ : bx * (256 / NMAT) + wn_ * (64 / NMAT) + j * 16 + col_;
    };
    auto row_of = [&](uint32_t wn_, int j, uint32_t col_) __attribute__((always_inline)) -> uint32_t {
        const uint32_t o = out_of(wn_, j, col_);
        return EPI == PE_HC_UP ? min((uint32_t)j, a.hc - 1) * a.H + min(o, a.H - 1) : min(o, a.N - 1);
    };
    // offsets (words, scales, biases) of row r of matrix q
    auto offs = [&](int q, uint32_t r, uint32_t& ow, uint32_t& os, uint32_t& ob) __attribute__((always_inline)) {
        if (expert) {
            const int part = EPI == PE_SILU_MUL ? q : 2;
            const uint64_t w0 = part == 0 ? XR.gate_w : part == 1 ? XR.up_w : XR.down_w;
            const uint64_t s0 = part == 0 ? XR.gate_s : part == 1 ? XR.up_s : XR.down_s;
            const uint64_t b0 = part == 0 ? XR.gate_b : part == 1 ? XR.up_b : XR.down_b;
            ow = (uint32_t)(w0 / 4) + r * (lowbit ? (K >> 5) * CW : KB);
            os = (uint32_t)(s0 / 2) + r * G;
            ob = (uint32_t)(b0 / 2) + r * G;
            return;
        }
        // concatenated segments along n (PE_STORE), else matrix q
        uint32_t mw = a.seg[q].wo, ms = a.seg[q].so, mb = a.seg[q].bo, rr = r;
        if (EPI == PE_STORE) {
#pragma unroll
            for (int sgi = 1; sgi < 4; ++sgi)
                if ((uint32_t)sgi < a.nseg && r >= a.seg[sgi].n0) {
                    mw = a.seg[sgi].wo;
                    ms = a.seg[sgi].so;
                    mb = a.seg[sgi].bo;
                    rr = r - a.seg[sgi].n0;
                }
        }
        ow = mw + rr * KB;
        os = ms + rr * G;
        ob = mb + rr * G;
    };
    uint32_t wo[NMAT][NJ], so[NMAT][NJ], bo[NMAT][NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const uint32_t r = row_of(wn, j, col);
#pragma unroll
        for (int q = 0; q < NMAT; ++q) offs(q, r, wo[q][j], so[q][j], bo[q][j]);
    }
    // scale loader (SBL): thread tid stages local row tid
    uint32_t ld_so = 0;
    if (SBL) {
        const uint32_t wn_ = (uint32_t)tid >> 6, rem = (uint32_t)tid & 63;
        const int q = (int)(rem / (NJ * 16)), j = (int)((rem >> 4) % NJ);
        uint32_t ow, ob;
        offs(q, row_of(wn_, j, rem & 15), ow, ld_so, ob);
    }

    // ---- A staging: thread tid loads 8-blocks 2 (tid % 4) + {0, 1} of row
    // tid / 4 (hi, lo planes) and the group sum of row tid % 64
    // (tiles under 64 rows: the threads past the tile re-read its last row,
    // into buffer rows nobody reads; no branch keeps the pipeline's
    // registers in one straight schedule)
    const uint32_t lrow = tid >> 2, lkb = (tid & 3) * 2;
    uint32_t arow_ld, arow_xs;
    {
        const uint32_t m = min(m0 + min(lrow, TR - 1), M - 1);
        arow_ld = list ? list[m] / a.div : toff + m;
        const uint32_t mx = min(m0 + (tid & 63), M - 1);
        arow_xs = list ? list[mx] / a.div : toff + mx;
        if (tid < 64) sRow[tid] = toff + mx;
    }
    const u32x4* ghi = reinterpret_cast<const u32x4*>(a.xhi) + (size_t)arow_ld * KB + lkb;
    const u32x4* glo = reinterpret_cast<const u32x4*>(a.xlo) + (size_t)arow_ld * KB + lkb;
    const float* gxs = a.xs + (size_t)arow_xs * G;
    // Software pipeline: the next group's A tile pieces and weight words
    // load while this group computes (register slot = group % 2, a
    // compile-time constant in the unrolled loop).  Every load is
    // unconditional (past the last group it re-reads the last one), so the
    // wait counters the compiler derives stay exact: a step waits only for
    // the loads it consumes.
    u32x4 rah0[2], rah1[2], ral0[2], ral1[2];
    float rx[2];
    u32x2 bw[2][NMAT][NJ];                         // words 2 kq, 2 kq + 1: K-steps 0, 1
    uint16_t bs[2][SBL ? 1 : NMAT][SBL ? 1 : NJ];  // per-lane scale, bias (not SBL)
    uint16_t bb[2][SBL ? 1 : NMAT][SBL ? 1 : NJ];
    u32x4 sreg_s;                                  // SBL: the next block's 8 scales
    auto fetch = [&](int slot, uint32_t g) __attribute__((always_inline)) {
        rah0[slot] = ghi[g * 8];
        rah1[slot] = ghi[g * 8 + 1];
        ral0[slot] = glo[g * 8];
        ral1[slot] = glo[g * 8 + 1];
        if (!SBL) rx[slot] = gxs[g];
#pragma unroll
        for (int q = 0; q < NMAT; ++q)
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                if (BITS == 4) {
                    bw[slot][q][j] = *reinterpret_cast<const u32x2*>(wb + wo[q][j] + g * 8 + kq * 2);
                } else {
                    // two word loads either way: a Q4 row's words 2 kq, + 1, or a
                    // low-bit row's word for inputs 16 (kq % 2) .. of chunk
                    // 2 g + kq / 2 and (Q3) that chunk's low-bit word
                    const uint32_t cb = wo[q][j] + (2 * g + (kq >> 1)) * CW;
                    const uint32_t i0 = lowbit ? cb + (kq & 1) : wo[q][j] + g * 8 + kq * 2;
                    const uint32_t i1 = lowbit ? (BITS == 3 ? cb + 2 : i0) : i0 + 1;
                    bw[slot][q][j] = u32x2{wb[i0], wb[i1]};
                }
                if (!SBL) {
                    bs[slot][SBL ? 0 : q][SBL ? 0 : j] = sbase[so[q][j] + g];
                    bb[slot][SBL ? 0 : q][SBL ? 0 : j] = sbase[bo[q][j] + g];
                }
            }
    };
    auto a_store = [&](int slot, uint32_t buf) __attribute__((always_inline)) {
        sA[buf][0][lrow * PF_AROW + lkb] = rah0[slot];
        sA[buf][0][lrow * PF_AROW + lkb + 1] = rah1[slot];
        sA[buf][1][lrow * PF_AROW + lkb] = ral0[slot];
        sA[buf][1][lrow * PF_AROW + lkb + 1] = ral1[slot];
        if (!SBL) sX[buf][tid & 63] = rx[slot];  // four identical writes per row: no branch
    };
    auto sb_fetch = [&](uint32_t g0) __attribute__((always_inline)) {
        sreg_s = *reinterpret_cast<const u32x4*>(sbase + ld_so + g0);
    };
    // low-bit records: the midpoint rule's step (w = (step q + half) s + b)
    // rides on the staged scale, exact as a power of two; half s joins the
    // bias contraction
    const float sstep = BITS != 4 && lowbit ? (BITS == 2 ? 4.0f : 2.0f) : 1.0f;
    auto sb_store = [&](uint32_t buf) __attribute__((always_inline)) {
        float* d = &sSB[buf][tid];
        const uint32_t sv[4] = {sreg_s.x, sreg_s.y, sreg_s.z, sreg_s.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            d[(2 * e) * 256] = __uint_as_float(sv[e] << 16) * sstep;
            d[(2 * e + 1) * 256] = __uint_as_float(sv[e] & 0xffff0000u) * sstep;
        }
    };

    f4 acc[NMAT][NI][NJ];
#pragma unroll
    for (int q = 0; q < NMAT; ++q)
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j) acc[q][i][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    const Q4Consts qk;

    // one quant group g; S = g % 8 under SBL (g % 2 otherwise): register slot
    // S % 2 and LDS buffer g % 2
    auto step = [&](auto sc_, uint32_t g) __attribute__((always_inline)) {
        constexpr int S = decltype(sc_)::value, P = S & 1;
        fetch(P ^ 1, min(g + 1, ge - 1));
        if (SBL && S == 0) sb_fetch(min(g + 8, ge - 8));
        // K-step s of lane quarter kq takes the group's word 2 kq + s (A
        // staged in the same 8-block order)
        h8 bq[NMAT][NJ][2];
#pragma unroll
        for (int q = 0; q < NMAT; ++q)
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                uint32_t w0 = bw[P][q][j].x, w1 = bw[P][q][j].y;
                if (BITS != 4 && lowbit) {
                    // the code word's 2-bit fields pp = 0, 2 of each byte are the
                    // nibbles of the lane's first Q4 word (mask 0x33), pp = 1, 3
                    // those of its second; Q3 codes take the low bit from the
                    // lo word (bit 8 byte + 4 (kq % 2) + pp) as 2 code + bit
                    constexpr uint32_t M = 0x33333333u;
                    const uint32_t c = bw[P][q][j].x, lo = bw[P][q][j].y, sh = 4 * (kq & 1);
                    w0 = c & M;
                    w1 = (c >> 2) & M;
                    if (BITS == 3) {
                        w0 = (w0 << 1) | ((lo >> sh) & 0x01010101u) | (((lo >> (sh + 2)) & 0x01010101u) << 4);
                        w1 = (w1 << 1) | ((lo >> (sh + 1)) & 0x01010101u) | (((lo >> (sh + 3)) & 0x01010101u) << 4);
                    }
                }
                bq[q][j][0] = pf_unpack(w0, qk);
                bq[q][j][1] = pf_unpack(w1, qk);
            }
        float sc[NMAT][NJ], bi[NMAT][NJ];
        float4 sc4[NMAT][NJ];  // SW: the scales of the lane's 4 outputs
#pragma unroll
        for (int q = 0; q < NMAT; ++q)
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                if (SBL) {
                    sc4[q][j] = *reinterpret_cast<const float4*>(
                        &sSB[((g - gb) >> 3) & 1][S * 256 + ((wn * NMAT + q) * NJ + j) * 16 + kq * 4]);
                    sc[q][j] = bi[q][j] = 0.0f;
                } else {
                    sc[q][j] = bf16f(bs[P][SBL ? 0 : q][SBL ? 0 : j]);
                    bi[q][j] = bf16f(bb[P][SBL ? 0 : q][SBL ? 0 : j]);
                    if (BITS != 4 && lowbit) {
                        // midpoint rule: w = (step q + half) s + b
                        bi[q][j] = fmaf(BITS == 2 ? 1.5f : 0.5f, sc[q][j], bi[q][j]);
                        sc[q][j] *= BITS == 2 ? 4.0f : 2.0f;
                    }
                }
            }
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            if ((uint32_t)i >= ni) break;
            f4 accg[NMAT][NJ];
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const uint32_t ai = (i * 16 + col) * PF_AROW + kq * 2 + s;
                const h8 ah = __builtin_bit_cast(h8, sA[P][0][ai]);
                const h8 al = __builtin_bit_cast(h8, sA[P][1][ai]);
#pragma unroll
                for (int q = 0; q < NMAT; ++q)
#pragma unroll
                    for (int j = 0; j < NJ; ++j) {
                        const f4 c0 = s == 0 ? f4{0.0f, 0.0f, 0.0f, 0.0f} : accg[q][j];
                        if (SW) {
                            accg[q][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bq[q][j][s], ah, c0, 0, 0, 0);
                            accg[q][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bq[q][j][s], al, accg[q][j], 0, 0, 0);
                        } else {
                            accg[q][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bq[q][j][s], c0, 0, 0, 0);
                            accg[q][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bq[q][j][s], accg[q][j], 0, 0, 0);
                        }
                    }
            }
            if (SBL) {
#pragma unroll
                for (int q = 0; q < NMAT; ++q)
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[q][i][j][r] = fmaf(sc4[q][j][r], accg[q][j][r], acc[q][i][j][r]);
            } else {
                const float4 xv = *reinterpret_cast<const float4*>(&sX[P][i * 16 + kq * 4]);
                const float xr[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
                for (int q = 0; q < NMAT; ++q)
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            acc[q][i][j][r] = fmaf(sc[q][j], accg[q][j][r], acc[q][i][j][r]);
                            acc[q][i][j][r] = fmaf(bi[q][j], xr[r], acc[q][i][j][r]);
                        }
            }
        }
        // A of group g + 1 into the other buffer (read by nobody since the
        // last barrier); the next scale block at the end of a block
        a_store(P ^ 1, P ^ 1);
        if (SBL && S == 7) sb_store((((g - gb) >> 3) + 1) & 1);
        __syncthreads();
    };

    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    // bias term (SBL): acc[n][m] = sum_{g in [gb, ge)} b[n][g] xs[m][g], a
    // small MFMA contraction over the groups (bf16, with xs split into three
    // bf16 terms so every product is exact), 32 groups per K-step: lane
    // (col, kq) takes groups k0 + 8 kq .. + 8 (whole 8-blocks: zero past
    // ge).  It opens the accumulation, its loads in flight with the first
    // group's, so its latency overlaps theirs rather than trailing the loop.
    auto bias_pass = [&](uint32_t k0) __attribute__((always_inline)) {
        const uint32_t kg = k0 + 8 * kq;
        const bool live = kg < ge;
        const uint32_t kc = live ? kg : gb;
        const bool lowb = BITS != 4 && lowbit;
        b8 bbv[NMAT][NJ];
        u32x4 ssv[BITS == 4 ? 1 : NMAT][BITS == 4 ? 1 : NJ];  // low-bit: the scales (half s term)
#pragma unroll
        for (int q = 0; q < NMAT; ++q)
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const u32x4 v = *reinterpret_cast<const u32x4*>(sbase + bo[q][j] + kc);
                bbv[q][j] = __builtin_bit_cast(b8, live ? v : u32x4{0u, 0u, 0u, 0u});
                if constexpr (BITS != 4) {
                    const u32x4 sv = lowb ? *reinterpret_cast<const u32x4*>(sbase + so[q][j] + kc) : u32x4{0u, 0u, 0u, 0u};
                    ssv[q][j] = live ? sv : u32x4{0u, 0u, 0u, 0u};
                }
            }
        float4 xg[NI][2];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            if ((uint32_t)i >= ni) break;
            const uint32_t m = min(m0 + i * 16 + col, M - 1);
            const uint32_t ar = list ? list[m] / a.div : toff + m;
            const float4* xp = reinterpret_cast<const float4*>(a.xs + (size_t)ar * G + kc);
            xg[i][0] = xp[0];
            xg[i][1] = xp[1];
        }
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            if ((uint32_t)i >= ni) break;
            const float4 x0 = xg[i][0], x1 = xg[i][1];
            const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            uint32_t hw[4], mw[4], lw[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                uint32_t h2_[2], m2_[2], l2_[2];
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const float xx = live ? xv[2 * e + u] : 0.0f;
                    h2_[u] = f2bf_rne(xx);
                    const float r1 = xx - __uint_as_float(h2_[u] << 16);
                    m2_[u] = f2bf_rne(r1);
                    l2_[u] = f2bf_rne(r1 - __uint_as_float(m2_[u] << 16));
                }
                hw[e] = h2_[0] | h2_[1] << 16;
                mw[e] = m2_[0] | m2_[1] << 16;
                lw[e] = l2_[0] | l2_[1] << 16;
            }
            const b8 xh = __builtin_bit_cast(b8, u32x4{hw[0], hw[1], hw[2], hw[3]});
            const b8 xm = __builtin_bit_cast(b8, u32x4{mw[0], mw[1], mw[2], mw[3]});
            const b8 xl = __builtin_bit_cast(b8, u32x4{lw[0], lw[1], lw[2], lw[3]});
#pragma unroll
            for (int q = 0; q < NMAT; ++q)
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    acc[q][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bbv[q][j], xl, acc[q][i][j], 0, 0, 0);
                    acc[q][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bbv[q][j], xm, acc[q][i][j], 0, 0, 0);
                    acc[q][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bbv[q][j], xh, acc[q][i][j], 0, 0, 0);
                    if constexpr (BITS != 4) {
                        if (lowb) {
                            // half s = s / 2 (Q3) or s + s / 2 (Q2), each exact in bf16
                            const uint32_t sw[4] = {ssv[q][j].x, ssv[q][j].y, ssv[q][j].z, ssv[q][j].w};
                            uint32_t hs[4];
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                hs[e] = f2bf_rne(__uint_as_float(sw[e] << 16) * 0.5f) |
                                        f2bf_rne(__uint_as_float(sw[e] & 0xffff0000u) * 0.5f) << 16;
                            const b8 sh = __builtin_bit_cast(b8, u32x4{hs[0], hs[1], hs[2], hs[3]});
                            acc[q][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sh, xl, acc[q][i][j], 0, 0, 0);
                            acc[q][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sh, xm, acc[q][i][j], 0, 0, 0);
                            acc[q][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sh, xh, acc[q][i][j], 0, 0, 0);
                            if (BITS == 2) {
                                const b8 sf = __builtin_bit_cast(b8, ssv[q][j]);
                                acc[q][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sf, xl, acc[q][i][j], 0, 0, 0);
                                acc[q][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sf, xm, acc[q][i][j], 0, 0, 0);
                                acc[q][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sf, xh, acc[q][i][j], 0, 0, 0);
                            }
                        }
                    }
                }
        }
    };
    fetch(0, gb);
    if (SBL) {
        sb_fetch(gb);
        for (uint32_t k0 = gb; k0 < ge; k0 += 32) bias_pass(k0);
        sb_store(0);
    }
    a_store(0, 0);
    __syncthreads();
    if (SBL) {
        for (uint32_t g = gb; g < ge; g += 8) {
            step(I0{}, g);
            step(I1{}, g + 1);
            step(std::integral_constant<int, 2>{}, g + 2);
            step(std::integral_constant<int, 3>{}, g + 3);
            step(std::integral_constant<int, 4>{}, g + 4);
            step(std::integral_constant<int, 5>{}, g + 5);
            step(std::integral_constant<int, 6>{}, g + 6);
            step(std::integral_constant<int, 7>{}, g + 7);
        }
    } else {
        uint32_t g = gb;
        for (; g + 2 <= ge; g += 2) {
            step(I0{}, g);
            step(I1{}, g + 1);
        }
        if (g < ge) step(I0{}, g);
    }

    // ---- epilogue, transposed tile (SW): lane (col, kq) of tile (i, j)
    // holds outputs tile base + 4 kq .. + 3 of row m0 + 16 i + col, which
    // leave as one 16-byte store (four scalar ones where rows or segments
    // are not 16-byte aligned)
    if constexpr (SW) {
        constexpr uint32_t NC = 256 / NMAT;
        uint32_t yrow[NI];
        bool mok[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            mok[i] = m0 + i * 16 + col < M;
            yrow[i] = sRow[i * 16 + col];
        }
        if (EPI == PE_HC_UP) {
            // the four tiles of a wave are the hc streams of the same outputs
            const uint32_t o4 = bx * 64 + wn * 16 + kq * 4;
            const bool ook = o4 < a.H;  // H % 4 == 0
            const uint32_t oc = ook ? o4 : 0;
            float nw[4][4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint2 q = (uint32_t)j < a.hc ? *reinterpret_cast<const uint2*>(a.norm + (size_t)j * a.H + oc)
                                                   : uint2{0u, 0u};
                nw[j][0] = __uint_as_float(q.x << 16);
                nw[j][1] = __uint_as_float(q.x & 0xffff0000u);
                nw[j][2] = __uint_as_float(q.y << 16);
                nw[j][3] = __uint_as_float(q.y & 0xffff0000u);
            }
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const uint32_t m = min(m0 + i * 16 + col, M - 1);
                const float* hy = a.hyper + (size_t)m * a.hc * a.H + oc;
                float4 hv[4];
                float iv[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const bool on = (uint32_t)j < a.hc;
                    hv[j] = on ? *reinterpret_cast<const float4*>(hy + (size_t)j * a.H) : make_float4(0.f, 0.f, 0.f, 0.f);
                    iv[j] = on ? a.inv[(size_t)m * a.hc + j] : 0.0f;
                }
                if (!mok[i] || !ook) continue;
                float sum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if ((uint32_t)j >= a.hc) continue;
                    const float hj[4] = {hv[j].x, hv[j].y, hv[j].z, hv[j].w};
#pragma unroll
                    for (int r = 0; r < 4; ++r) sum[r] += sigmoid_hw(acc[0][i][j][r]) * (hj[r] * iv[j] * nw[j][r]);
                }
                const float ih = (float)a.hc;
                *reinterpret_cast<float4*>(a.out + (size_t)m * a.H + o4) =
                    make_float4(sum[0] / ih, sum[1] / ih, sum[2] / ih, sum[3] / ih);
            }
        } else if (EPI == PE_SILU_MUL && a.phi) {
            // the activations leave as the down GEMM's operands (k_pf_prep's
            // planes, summed and split as it does): an 8-block's outputs sit
            // in lanes kq, kq + 1 (the even one writes it), a 64-group's in
            // waves 2 g, 2 g + 1 (its sum meets in LDS, the A buffers, free
            // after the main loop's last barrier)
            float* sG = reinterpret_cast<float*>(&sA[0][0][0]);  // [wave][slice][col]
            const uint32_t K8 = a.N >> 3, K64 = a.N >> 6;
            const uint32_t nw0 = bx * NC + wn * (NC / 4);  // the wave's first output
            const bool ev = (kq & 1) == 0;
            float X[NI];
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                float P[NJ];
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    float u[4], pv[4], v[8];
#pragma unroll
                    for (int r = 0; r < 4; ++r) u[r] = silu_hw(acc[0][i][j][r]) * acc[NMAT - 1][i][j][r];
#pragma unroll
                    for (int r = 0; r < 4; ++r) pv[r] = __shfl_xor(u[r], 16, 64);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        v[r] = ev ? u[r] : pv[r];
                        v[4 + r] = ev ? pv[r] : u[r];
                    }
                    float bs = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
                    bs += __shfl_xor(bs, 32, 64);
                    P[j] = bs;
                    if (ev && mok[i]) {
                        const float op[8] = {v[0], v[4], v[1] * 0.0625f, v[5] * 0.0625f,
                                             v[2], v[6], v[3] * 0.0625f, v[7] * 0.0625f};
                        h8 hh, hl;
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            const _Float16 he = (_Float16)op[e];
                            hh[e] = he;
                            hl[e] = (_Float16)(op[e] - (float)he);
                        }
                        const size_t bi = (size_t)yrow[i] * K8 + (nw0 + j * 16 + (kq >> 1) * 8) / 8;
                        a.phi[bi] = __builtin_bit_cast(uint4, hh);
                        a.plo[bi] = __builtin_bit_cast(uint4, hl);
                    }
                }
                X[i] = P[0] + P[NJ - 1];
            }
            __syncthreads();
            if (kq == 0)
#pragma unroll
                for (int i = 0; i < NI; ++i) sG[(wn * NI + i) * 16 + col] = X[i];
            __syncthreads();
            if (kq == 0 && (wn & 1) == 0)
#pragma unroll
                for (int i = 0; i < NI; ++i)
                    if (mok[i]) a.pxs[(size_t)yrow[i] * K64 + nw0 / 64] = X[i] + sG[((wn + 1) * NI + i) * 16 + col];
        } else {
            uint32_t n4[NJ];
            PfSeg sj[NJ];
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                n4[j] = bx * NC + wn * (64 / NMAT) + j * 16 + kq * 4;
                sj[j] = a.seg[0];
                if (EPI == PE_STORE) {
#pragma unroll
                    for (int sgi = 1; sgi < 4; ++sgi)
                        if ((uint32_t)sgi < a.nseg && n4[j] >= a.seg[sgi].n0) sj[j] = a.seg[sgi];
                }
            }
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const uint32_t m = m0 + i * 16 + col;
                if (!mok[i]) continue;
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    float u[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        u[r] = EPI == PE_SILU_MUL ? silu_hw(acc[0][i][j][r]) * acc[NMAT - 1][i][j][r] : acc[0][i][j][r];
                    float* dst = sj[j].y + (size_t)blockIdx.z * a.zstride + (size_t)yrow[i] * sj[j].ldy + (n4[j] - sj[j].n0);
                    if (a.vec4) {
                        if (n4[j] < a.N) *reinterpret_cast<float4*>(dst) = make_float4(u[0], u[1], u[2], u[3]);
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (n4[j] + r < a.N) dst[r] = u[r];
                    }
                }
            }
        }
    } else {
    // ---- epilogue: the tile leaves through LDS (the A staging buffers) in
        // two 32-row halves.  Each lane parks its accumulators (one value per
        // output: silu(gate) * up already formed for PE_SILU_MUL), then thread
        // t finishes column t (PE_HC_UP: output t % 64 of row t / 64 + 4 k), so
        // the per-output code is one loop body rather than one unrolled copy
        // per accumulator, and a wave's stores cover consecutive outputs.
        float* sO = reinterpret_cast<float*>(&sA[0][0][0]);
        constexpr uint32_t OS = 260;  // floats per staged row (256 + pad: the four kq rows of a write hit distinct banks)
        static_assert(32 * OS * sizeof(float) <= sizeof(sA), "a staged half fits the A buffers");
        constexpr uint32_t NC = 256 / NMAT;  // staged columns
        const uint32_t gcol = bx * NC + (uint32_t)tid % NC;  // PE_STORE / PE_SILU_MUL output column
        PfSeg sg = a.seg[0];
        if (EPI == PE_STORE) {
    #pragma unroll
            for (int sgi = 1; sgi < 4; ++sgi)
                if ((uint32_t)sgi < a.nseg && gcol >= a.seg[sgi].n0) sg = a.seg[sgi];
        }
        // the mix's stream values, norm weights and RMS factors for both
        // halves, requested before the first half is staged (their one
        // round trip overlaps the staging rather than following it)
        float4 mhv[2][4][2];
        uint4 mnq[4];
        float miv[2][4];
        if (EPI == PE_HC_UP && a.phi) {
            const uint32_t o = bx * 64 + 8 * ((uint32_t)tid & 7);
    #pragma unroll
            for (int j = 0; j < 4; ++j)
                mnq[j] = (uint32_t)j < a.hc ? *reinterpret_cast<const uint4*>(a.norm + (size_t)j * a.H + o)
                                            : make_uint4(0u, 0u, 0u, 0u);
    #pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t mc = min(m0 + 32 * h + ((uint32_t)tid >> 3), M - 1);
                const float* hy = a.hyper + (size_t)mc * a.hc * a.H + o;
    #pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const bool on = (uint32_t)j < a.hc;
                    mhv[h][j][0] = on ? *reinterpret_cast<const float4*>(hy + (size_t)j * a.H) : make_float4(0.f, 0.f, 0.f, 0.f);
                    mhv[h][j][1] = on ? *reinterpret_cast<const float4*>(hy + (size_t)j * a.H + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
                    miv[h][j] = on ? a.inv[(size_t)mc * a.hc + j] : 0.0f;
                }
            }
        }
    #pragma unroll
        for (int h = 0; h < 2; ++h) {
            __syncthreads();
    #pragma unroll
            for (int ii = 0; ii < 2; ++ii) {
                const int i = 2 * h + ii;
    #pragma unroll
                for (int j = 0; j < NJ; ++j)
    #pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float v = EPI == PE_SILU_MUL ? silu_hw(acc[0][i][j][r]) * acc[NMAT - 1][i][j][r] : acc[0][i][j][r];
                        sO[(ii * 16 + kq * 4 + r) * OS + wn * (64 / NMAT) + j * 16 + col] = v;
                    }
            }
            __syncthreads();
            const uint32_t mh = m0 + 32 * h;
            if (EPI == PE_HC_UP && a.phi) {
                // thread: 8-block tid % 8 (outputs 8 (tid % 8) .. + 7 of the
                // 64, one quant group of the next GEMM's K) of row tid / 8;
                // the mixed values leave as that GEMM's operands, summed and
                // split as k_pf_prep does (the row's eight threads are one
                // aligned lane group)
                const uint32_t rr = (uint32_t)tid >> 3, b8 = (uint32_t)tid & 7, ol = 8 * b8;
                const uint32_t o = bx * 64 + ol, sc0 = (ol >> 4) * 64 + (ol & 15);
                const uint32_t m = mh + rr;
                float4 uv[4][2];
                const auto& hv = mhv[h];
                const auto& nq = mnq;
                const auto& iv = miv[h];
    #pragma unroll
                for (int j = 0; j < 4; ++j) {
                    uv[j][0] = *reinterpret_cast<const float4*>(&sO[rr * OS + sc0 + j * 16]);
                    uv[j][1] = *reinterpret_cast<const float4*>(&sO[rr * OS + sc0 + j * 16 + 4]);
                }
                float v[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    #pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if ((uint32_t)j >= a.hc) continue;
                    const float hj[8] = {hv[j][0].x, hv[j][0].y, hv[j][0].z, hv[j][0].w,
                                         hv[j][1].x, hv[j][1].y, hv[j][1].z, hv[j][1].w};
                    const float uj[8] = {uv[j][0].x, uv[j][0].y, uv[j][0].z, uv[j][0].w,
                                         uv[j][1].x, uv[j][1].y, uv[j][1].z, uv[j][1].w};
                    const uint32_t nw[4] = {nq[j].x, nq[j].y, nq[j].z, nq[j].w};
    #pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float we = __uint_as_float(e & 1 ? nw[e >> 1] & 0xffff0000u : nw[e >> 1] << 16);
                        v[e] += sigmoid_hw(uj[e]) * (hj[e] * iv[j] * we);
                    }
                }
                // / hc: a product by the exact reciprocal for a power of two
                const float ih = (float)a.hc;
                if ((a.hc & (a.hc - 1)) == 0) {
                    const float rh = 1.0f / ih;
    #pragma unroll
                    for (int e = 0; e < 8; ++e) v[e] = v[e] * rh;
                } else {
    #pragma unroll
                    for (int e = 0; e < 8; ++e) v[e] = v[e] / ih;
                }
                float gs = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
                gs += __shfl_xor(gs, 1, 64);
                gs += __shfl_xor(gs, 2, 64);
                gs += __shfl_xor(gs, 4, 64);
                if (m < M) {
                    const float op[8] = {v[0], v[4], v[1] * 0.0625f, v[5] * 0.0625f, v[2], v[6], v[3] * 0.0625f, v[7] * 0.0625f};
                    h8 hh, hl;
    #pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const _Float16 he = (_Float16)op[e];
                        hh[e] = he;
                        hl[e] = (_Float16)(op[e] - (float)he);
                    }
                    const size_t bi = (size_t)m * (a.H >> 3) + (o >> 3);
                    a.phi[bi] = __builtin_bit_cast(uint4, hh);
                    a.plo[bi] = __builtin_bit_cast(uint4, hl);
                    if (b8 == 0) a.pxs[(size_t)m * (a.H >> 6) + bx] = gs;
                    if (a.pbhi) {
                        // three bf16 terms in natural order (the router's)
                        uint32_t bh[8], bm[8], bl[8];
    #pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            bh[e] = f2bf_rne(v[e]);
                            const float r1 = v[e] - __uint_as_float(bh[e] << 16);
                            bm[e] = f2bf_rne(r1);
                            bl[e] = f2bf_rne(r1 - __uint_as_float(bm[e] << 16));
                        }
                        a.pbhi[bi] = make_uint4(bh[0] | bh[1] << 16, bh[2] | bh[3] << 16, bh[4] | bh[5] << 16, bh[6] | bh[7] << 16);
                        a.pbmid[bi] = make_uint4(bm[0] | bm[1] << 16, bm[2] | bm[3] << 16, bm[4] | bm[5] << 16, bm[6] | bm[7] << 16);
                        a.pblo[bi] = make_uint4(bl[0] | bl[1] << 16, bl[2] | bl[3] << 16, bl[4] | bl[5] << 16, bl[6] | bl[7] << 16);
                    }
                }
            } else if (EPI == PE_HC_UP) {
                // thread: outputs 4 c4 .. + 3 of the 64, rows r0 + 16 k
                const uint32_t c4 = (uint32_t)tid & 15, r0 = (uint32_t)tid >> 4, ol = 4 * c4;
                const uint32_t o = bx * 64 + ol, sc0 = (ol >> 4) * 64 + (ol & 15);
                const bool ook = o < a.H;  // H % 4 == 0: the group is whole or out
                const uint32_t oc = ook ? o : 0;
                float nw[4][4];
    #pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint2 q = (uint32_t)j < a.hc ? *reinterpret_cast<const uint2*>(a.norm + (size_t)j * a.H + oc)
                                                       : uint2{0u, 0u};
                    nw[j][0] = __uint_as_float(q.x << 16);
                    nw[j][1] = __uint_as_float(q.x & 0xffff0000u);
                    nw[j][2] = __uint_as_float(q.y << 16);
                    nw[j][3] = __uint_as_float(q.y & 0xffff0000u);
                }
    #pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const uint32_t rr = r0 + 16 * k, m = mh + rr, mc = min(m, M - 1);
                    const float* hy = a.hyper + (size_t)mc * a.hc * a.H + oc;
                    float4 hv[4], uv[4];
                    float iv[4];
    #pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const bool on = (uint32_t)j < a.hc;
                        hv[j] = on ? *reinterpret_cast<const float4*>(hy + (size_t)j * a.H) : make_float4(0.f, 0.f, 0.f, 0.f);
                        iv[j] = on ? a.inv[(size_t)mc * a.hc + j] : 0.0f;
                        uv[j] = *reinterpret_cast<const float4*>(&sO[rr * OS + sc0 + j * 16]);
                    }
                    if (m >= M || !ook) continue;
                    float sum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    #pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        if ((uint32_t)j >= a.hc) continue;
                        const float hj[4] = {hv[j].x, hv[j].y, hv[j].z, hv[j].w};
                        const float uj[4] = {uv[j].x, uv[j].y, uv[j].z, uv[j].w};
    #pragma unroll
                        for (int e = 0; e < 4; ++e) sum[e] += sigmoid_hw(uj[e]) * (hj[e] * iv[j] * nw[j][e]);
                    }
                    const float ih = (float)a.hc;
                    *reinterpret_cast<float4*>(a.out + (size_t)m * a.H + o) =
                        make_float4(sum[0] / ih, sum[1] / ih, sum[2] / ih, sum[3] / ih);
                }
            } else if (a.vec4) {
                // thread: columns 4 c4 .. + 3, rows r0 + RPP k (16-byte
                // aligned rows and segments, N % 4 == 0: checked at launch)
                constexpr uint32_t G4 = NC / 4, RPP = 256 / G4, KB = 32 / RPP;
                const uint32_t c4 = (uint32_t)tid % G4, r0 = (uint32_t)tid / G4;
                const uint32_t n4 = bx * NC + 4 * c4;
                const bool nok = n4 < a.N;
                PfSeg s4 = a.seg[0];
                if (EPI == PE_STORE) {
    #pragma unroll
                    for (int sgi = 1; sgi < 4; ++sgi)
                        if ((uint32_t)sgi < a.nseg && n4 >= a.seg[sgi].n0) s4 = a.seg[sgi];
                }
                {
                    // one row per iteration, the next row's LDS read issued
                    // before this row's activation and store
                    float4 vn = *reinterpret_cast<const float4*>(&sO[r0 * OS + 4 * c4]);
                    uint32_t yn = sRow[32 * h + r0];
    #pragma unroll 1
                    for (uint32_t k = 0; k < KB; ++k) {
                        const uint32_t rr = r0 + RPP * k, m = mh + rr;
                        const float4 v = vn;
                        const uint32_t yr = yn;
                        if (k + 1 < KB) {
                            vn = *reinterpret_cast<const float4*>(&sO[(rr + RPP) * OS + 4 * c4]);
                            yn = sRow[32 * h + rr + RPP];
                        }
                        if (m >= M) break;
                        if (!nok) continue;
                        float u[4] = {v.x, v.y, v.z, v.w};
                        float* dst;
                        if (EPI == PE_SILU_MUL) {
                            dst = a.seg[0].y + (size_t)yr * a.seg[0].ldy + n4;
                        } else {
                            dst = s4.y + (size_t)blockIdx.z * a.zstride + (size_t)yr * s4.ldy + (n4 - s4.n0);
                        }
                        *reinterpret_cast<float4*>(dst) = make_float4(u[0], u[1], u[2], u[3]);
                    }
                }
            } else {
                // unaligned outputs (PE_STORE, PE_SILU_MUL): thread t takes
                // column t % NC, rows in batches of 8 whose reads are all
                // issued before the first store
                constexpr uint32_t RPP = 256 / NC;  // rows per pass
                constexpr int B = 8;
                const uint32_t lc = (uint32_t)tid % NC, r0 = (uint32_t)tid / NC;
                const bool nok = gcol < a.N;
    #pragma unroll 1
                for (uint32_t rb = 0; rb < 32; rb += B * RPP) {
                    float v[B];
                    uint32_t yr[B];
    #pragma unroll
                    for (int k = 0; k < B; ++k) {
                        const uint32_t rr = rb + r0 + k * RPP;
                        v[k] = sO[rr * OS + lc];
                        yr[k] = sRow[32 * h + rr];
                    }
    #pragma unroll
                    for (int k = 0; k < B; ++k) {
                        const uint32_t m = mh + rb + r0 + k * RPP;
                        if (m >= M || !nok) continue;
                        if (EPI == PE_SILU_MUL) {
                            a.seg[0].y[(size_t)yr[k] * a.seg[0].ldy + gcol] = v[k];
                        } else if (EPI == PE_STORE) {
                            const float u = v[k];
                            sg.y[(size_t)blockIdx.z * a.zstride + (size_t)yr[k] * sg.ldy + (gcol - sg.n0)] = u;
                        }
                    }
                }
            }
        }
    }
}

// Split-K hyper-connection read: the [down; inject] partials of the hc
// stream chunks summed in stream order, then d = silu(v / hc) and inj =
// 2 sigmoid(v / hc) (cpu.rs:493-500).
__global__ void __launch_bounds__(256) k_pf_hc_down_finish(const float* __restrict__ part, uint32_t nsplit,
                                                           uint64_t zstride, uint32_t T, uint32_t lowrank,
                                                           uint32_t hc, float alpha, float* __restrict__ d,
                                                           float* __restrict__ inj) {
    const uint32_t N = lowrank + hc;
    const uint64_t i = (uint64_t)blockIdx.x * CHK_WG + threadIdx.x;
    if (i >= (uint64_t)T * N) return;
    const uint32_t t = (uint32_t)(i / N), n = (uint32_t)(i % N);
    float v = 0.0f;
    for (uint32_t z = 0; z < nsplit; ++z) v += part[z * zstride + i];
    v *= alpha;
    if (n < lowrank) d[(size_t)t * lowrank + n] = siluf_(v);
    else inj[(size_t)t * hc + (n - lowrank)] = 2.0f * sigmoidf_(v);
}

// The same finisher with d staged straight into the up GEMM's operands
// (k_pf_prep's planes: fp16 hi / lo in the permuted 8-block order and the
// per-group sums, summed in k_pf_prep's order), so d itself is never
// written: thread i < T (lowrank / 8) takes 8-block i % (lowrank / 8) of
// row i / (lowrank / 8), the T hc threads after them the inject values.
// lowrank % 64 == 0 keeps every 64-group's eight threads in one aligned
// lane group.
__global__ void __launch_bounds__(256) k_pf_hc_down_finish_q(const float* __restrict__ part, uint32_t nsplit,
                                                             uint64_t zstride, uint32_t T, uint32_t lowrank,
                                                             uint32_t hc, float alpha, uint4* __restrict__ hi,
                                                             uint4* __restrict__ lo, float* __restrict__ xs,
                                                             float* __restrict__ inj) {
    const uint32_t N = lowrank + hc, blocks = lowrank >> 3;
    const uint64_t i = (uint64_t)blockIdx.x * CHK_WG + threadIdx.x, nb = (uint64_t)T * blocks;
    if (i >= nb) {
        const uint64_t j = i - nb;
        if (j >= (uint64_t)T * hc) return;
        const uint32_t t = (uint32_t)(j / hc), g = (uint32_t)(j % hc);
        float v = 0.0f;
        for (uint32_t z = 0; z < nsplit; ++z) v += part[z * zstride + (size_t)t * N + lowrank + g];
        v *= alpha;
        inj[(size_t)t * hc + g] = 2.0f * sigmoidf_(v);
        return;
    }
    const uint32_t t = (uint32_t)(i / blocks), kb = (uint32_t)(i % blocks);
    float v[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t z = 0; z < nsplit; ++z) {
        const float4* p = reinterpret_cast<const float4*>(part + z * zstride + (size_t)t * N + kb * 8);
        const float4 u0 = p[0], u1 = p[1];
        v[0] += u0.x; v[1] += u0.y; v[2] += u0.z; v[3] += u0.w;
        v[4] += u1.x; v[5] += u1.y; v[6] += u1.z; v[7] += u1.w;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = siluf_(v[j] * alpha);
    float s = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    s += __shfl_xor(s, 4, 64);
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
    if ((kb & 7) == 0) xs[(size_t)t * (lowrank >> 6) + (kb >> 3)] = s;
}

// ------------------------------------------------------------- router
// logits[t][e] = W_r[e] . x_t (bf16 [E][H], f32 sums) (moe, cpu.rs:506-508),
// on v_mfma_f32_16x16x32_bf16 with x split into three bf16 terms (natural k
// order): every product of bf16 values is exact in f32, so the logits keep
// f32-grade accuracy and the top-k cut sees what an f32 dot would.
// A workgroup covers 64 rows x 64 outputs, each wave one 16-output column
// tile over the 64 rows (E / 64 column blocks: one workgroup per CU at
// E = 512, T = 2048; the shared-expert gate logit is the routing wave's).  Per 64-wide k block the three x planes of the 64
// rows are staged through LDS once for the four waves (double-buffered;
// the next block's pieces and weight words load while this one computes).
constexpr int RT_AROW = 9;  // uint4 per staged row (8 + 1 pad)

template <int CT>
__global__ void __launch_bounds__(256) k_pf_router(const uint16_t* __restrict__ router,
                                                   const uint4* __restrict__ bhi, const uint4* __restrict__ bmid,
                                                   const uint4* __restrict__ blo, float* __restrict__ logits,
                                                   uint32_t T, uint32_t E, uint32_t H) {
    __shared__ __align__(16) u32x4 sA[2][3][64 * RT_AROW];
    const int tid = threadIdx.x, lane = tid & 63, col = lane & 15, kq = lane >> 4;
    const uint32_t m0 = blockIdx.y * 64, KB = H >> 3;
    // K chunk blockIdx.z: 64-wide blocks b0 .. NB - 1, partials at logits + z T E
    const uint32_t NBc = (H >> 6) / gridDim.z, b0 = blockIdx.z * NBc, NB = b0 + NBc;
    logits += (size_t)blockIdx.z * T * E;
    // wave w: CT 16-expert column tiles
    uint32_t nn[CT];
    const u32x4* bp[CT];
#pragma unroll
    for (int c = 0; c < CT; ++c) {
        nn[c] = (blockIdx.x * 4 + wave_id()) * 16 * CT + 16 * c + col;
        bp[c] = reinterpret_cast<const u32x4*>(router + (size_t)min(nn[c], E - 1) * H);
    }
    // staging: piece u of thread tid is plane u / 2, row (tid + 256 (u % 2)) / 8, 8-block tid % 8
    const uint32_t srow = (uint32_t)tid >> 3, skb = (uint32_t)tid & 7;
    size_t soff[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) soff[h] = (size_t)min(m0 + srow + 32 * h, T - 1) * KB + skb;
    // three register slots: block blk's loads are issued two blocks ahead
    // (slot blk % 3), so each step's wait covers two steps of latency
    u32x4 ra[3][6], rb[3][CT][2];
    auto fetch = [&](int slot, uint32_t blk) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < 6; ++u) {
            const u32x4* pl = reinterpret_cast<const u32x4*>(u < 2 ? bhi : u < 4 ? bmid : blo);
            ra[slot][u] = pl[soff[u & 1] + blk * 8];
        }
#pragma unroll
        for (int c = 0; c < CT; ++c) {
            rb[slot][c][0] = bp[c][blk * 8 + kq];
            rb[slot][c][1] = bp[c][blk * 8 + 4 + kq];
        }
    };
    auto store = [&](int slot, int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < 6; ++u) sA[buf][u >> 1][(srow + 32 * (u & 1)) * RT_AROW + skb] = ra[slot][u];
    };
    f4 acc[CT][4];
#pragma unroll
    for (int c = 0; c < CT; ++c)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[c][i] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    // block blk: registers slot P = (blk - b0) % 3, LDS buffer (blk - b0) % 2
    auto step = [&](auto sc_, uint32_t blk) __attribute__((always_inline)) {
        constexpr int P = decltype(sc_)::value;
        const uint32_t buf = (blk - b0) & 1;
        fetch((P + 2) % 3, min(blk + 2, NB - 1));
#pragma unroll
        for (int s = 0; s < 2; ++s) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t ai = (16 * i + col) * RT_AROW + 4 * s + kq;
                const b8 xh = __builtin_bit_cast(b8, sA[buf][0][ai]);
                const b8 xm = __builtin_bit_cast(b8, sA[buf][1][ai]);
                const b8 xl = __builtin_bit_cast(b8, sA[buf][2][ai]);
#pragma unroll
                for (int c = 0; c < CT; ++c) {
                    const b8 bq = __builtin_bit_cast(b8, rb[P][c][s]);
                    acc[c][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xl, bq, acc[c][i], 0, 0, 0);
                    acc[c][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xm, bq, acc[c][i], 0, 0, 0);
                    acc[c][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xh, bq, acc[c][i], 0, 0, 0);
                }
            }
        }
        store((P + 1) % 3, buf ^ 1);
        __syncthreads();
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    fetch(0, b0);
    fetch(1, min(b0 + 1, NB - 1));
    store(0, 0);
    __syncthreads();
    uint32_t blk = b0;
    for (; blk + 2 < NB; blk += 3) {
        step(I0{}, blk);
        step(I1{}, blk + 1);
        step(I2{}, blk + 2);
    }
    if (blk < NB) step(I0{}, blk);
    if (blk + 1 < NB) step(I1{}, blk + 1);
#pragma unroll
    for (int c = 0; c < CT; ++c)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const uint32_t m = m0 + i * 16 + kq * 4 + rr;
                if (m >= T) continue;
                if (nn[c] < E) logits[(size_t)m * E + nn[c]] = acc[c][i][rr];
            }
}

// ------------------------------------------------------------ routing
// One wave per token: softmax top-k (route_row) and the renormalised
// weights in rank order (cpu.rs:508-525); the last token's routing also
// goes to last_ids / last_wts (the layer's "last routes").
// Each entry t (k+1) + r also takes its place in its expert's group here
// (the grouping pass's list and pos, below): an atomic count per expert
// in gcnt, one 128-byte line each (PF_GCNT_STRIDE words apart; zero on
// entry; the grouping pass reads and clears them), so the entries'
// scattered stores are spread over the launch's workgroups.
// Places within a group come in arrival order, which only moves rows
// (every GEMM row is computed on its own).
template <int NZ>
__global__ void __launch_bounds__(256) k_pf_route(const float* __restrict__ logits, uint32_t T, uint32_t E,
                                                  uint32_t topk, int norm_topk, uint32_t* __restrict__ ids,
                                                  float* __restrict__ wts, uint32_t* __restrict__ last_ids,
                                                  float* __restrict__ last_wts, const uint16_t* __restrict__ shared_gate,
                                                  const uint4* __restrict__ bhi, const uint4* __restrict__ bmid,
                                                  const uint4* __restrict__ blo, float* __restrict__ sg, uint32_t H,
                                                  uint32_t* __restrict__ gcnt, uint32_t* __restrict__ list,
                                                  uint32_t* __restrict__ pos, uint32_t cap, uint32_t shared) {
    const int lane = threadIdx.x & 63;
    const uint32_t t = blockIdx.x * (CHK_WG >> 6) + wave_id();
    if (t >= T) return;
    // the shared-expert gate logit sg[t] = w_sg . x_t (cpu.rs:534-535) from
    // the same three bf16 terms of x, products exact in f32; its loads are
    // in flight beside the routing's
    const uint32_t KB = H >> 3;
    float sgs = 0.0f;
#pragma unroll 4
    for (uint32_t kb = lane; kb < KB; kb += 64) {
        const size_t xo = (size_t)t * KB + kb;
        const u32x4 w4 = reinterpret_cast<const u32x4*>(shared_gate)[kb];
        const u32x4 p4[3] = {__builtin_bit_cast(u32x4, bhi[xo]), __builtin_bit_cast(u32x4, bmid[xo]),
                             __builtin_bit_cast(u32x4, blo[xo])};
        const uint32_t wv[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float wl = __uint_as_float(wv[c] << 16), wh = __uint_as_float(wv[c] & 0xffff0000u);
#pragma unroll
            for (int u = 0; u < 3; ++u) {
                const uint32_t xv = c == 0 ? p4[u].x : c == 1 ? p4[u].y : c == 2 ? p4[u].z : p4[u].w;
                sgs = fmaf(wl, __uint_as_float(xv << 16), sgs);
                sgs = fmaf(wh, __uint_as_float(xv & 0xffff0000u), sgs);
            }
        }
    }
    uint32_t my_id;
    float my_p;
    route_row<NZ>(logits + (size_t)t * E, E, topk, lane, nullptr, my_id, my_p, (size_t)T * E);
    sgs = wave_sum_dpp(sgs);
    if (lane == 0) sg[t] = sgs;
    float topsum = 0.0f;
    for (uint32_t r = 0; r < topk; ++r) topsum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_p), (int)r));
    if ((uint32_t)lane < topk) {
        const float w = norm_topk ? my_p / topsum : my_p;
        ids[(size_t)t * topk + lane] = my_id;
        wts[(size_t)t * topk + lane] = w;
        if (t + 1 == T && last_ids) {
            last_ids[lane] = my_id;
            last_wts[lane] = w;
        }
        // route_row's ids are distinct and below E: a group holds at most
        // one entry per token, so p < T <= cap
        const uint32_t e = min(my_id, E - 1), slots = topk + 1;
        const uint32_t p = atomicAdd(&gcnt[(size_t)e * PF_GCNT_STRIDE], 1u);
        if (p < cap) {
            list[(size_t)e * cap + p] = t * slots + lane;
            pos[(size_t)t * slots + lane] = e << 22 | p;
        }
    }
    if (lane == 0) {
        // the shared slot: place t of group E
        if (shared) list[(size_t)E * cap + t] = t * (topk + 1) + topk;
        pos[(size_t)t * (topk + 1) + topk] = E << 22 | t;
    }
}

// Entries grouped by expert (the CSR lists of gpu/prefill/experts.rs:29-137):
// list[e][0..count[e]) holds the entries t (k+1) + slot routed to e (any
// order: every GEMM row is independent), list[E] every token's shared
// slot t (k+1) + k (both, and pos below, stored by the routing pass, which
// leaves the per-expert counts in gcnt; this pass clears them for the
// next layer), and tiles[] the (group, tr-row tile) pairs, *ntiles of
// them: first every group of two or more tiles, its count rounded up to
// even (the extra tile has no rows), so each starts at an even position
// (the GEMMs run tiles 2c and 2c + 1 on one XCD), then the one-tile groups.
// A second such list of 64-row tiles follows at tiles + pf_tile_bound(T,
// topk, E, tr), ntiles[1] of them (the gate/up and down GEMMs tile the same
// entries differently).
// Per tile also tinfo[] = (the group's first row in grouped order, its row
// count), per group goff[] = that first row, and per entry pos[] = its
// group << 22 | its place in the group (grouped row goff[group] + place;
// every token's shared slot is place t of group E, whose rows start where
// the routed entries end, at T k).
// With `act`, also the expert activity counters of `layer` (selected rows
// and selections, as the decode step's activity count does).  Without
// `shared`, group E gets no rows or tiles (a shared expert of another width
// runs as dense GEMMs of its own).  One workgroup.
constexpr uint32_t PG_WG = 1024;  // threads of the grouping workgroup (one group each)

__global__ void __launch_bounds__(PG_WG) k_pf_group(uint32_t* __restrict__ gcnt, uint32_t T, uint32_t E,
                                                    uint32_t cap, uint32_t* __restrict__ count,
                                                    uint32_t* __restrict__ tiles, uint32_t* __restrict__ ntiles,
                                                    uint2* __restrict__ tinfo, uint32_t* __restrict__ goff,
                                                    unsigned long long* __restrict__ act, uint32_t layer,
                                                    uint32_t tr, uint32_t topk, uint32_t shared) {
    __shared__ uint32_t cnt[PG_WG];
    __shared__ uint32_t offs[PG_WG];
    __shared__ unsigned long long wsum[PG_WG / 64];
    const uint32_t tau = threadIdx.x, lane = tau & 63, wv = tau >> 6;
    cnt[tau] = tau < E ? min(gcnt[(size_t)tau * PF_GCNT_STRIDE], cap) : tau == E && shared ? T : 0u;
    if (tau < E) gcnt[(size_t)tau * PF_GCNT_STRIDE] = 0;
    __syncthreads();
    const uint32_t e = tau;
    // grouped order: group e's rows start at the sum of the counts before it
    {
        const uint32_t c = e <= E ? cnt[e] : 0u;
        uint32_t incl = c;
        for (int d = 1; d < 64; d <<= 1) {
            const uint32_t o = __shfl_up(incl, d, 64);
            if ((int)lane >= d) incl += o;
        }
        if (lane == 63) wsum[wv] = incl;
        __syncthreads();
        uint32_t off = incl - c;
        for (uint32_t k = 0; k < wv; ++k) off += wsum[k];
        offs[e] = off;
        if (e <= E) goff[e] = off;
        __syncthreads();  // offs complete; wsum free again
    }
    // tiles per group (thread e takes group e): multi-tile counts in the
    // high half-word, single tiles in the low one, one workgroup prefix sum
    if (e <= E) count[e] = cnt[e];
    if (act && e < E && cnt[e]) {
        unsigned long long* ae = act + ((size_t)layer * E + e) * 2;
        ae[0] += cnt[e];
        ae[1] += 1;
    }
    // one tile list per tile height: tr-row tiles at tiles, 64-row tiles
    // at tiles + pf_tile_bound(T, topk, E, tr) (*ntiles, ntiles[1] of
    // them).  Tiles come in five classes, in this order: the tiles of the
    // longer groups, then the one-tile groups by their 16-row slices, most
    // first (the GEMMs deal workgroups in list order, so a launch ends on
    // its shortest ones); per group a count in the 12-bit field of its
    // class of one 64-bit workgroup prefix sum (the launcher keeps the
    // counts under 4096).
    const uint32_t trs[2] = {tr, 64u};
    uint32_t* dst = tiles;
    auto field = [](unsigned long long v, uint32_t k) { return (uint32_t)(v >> (12 * k)) & 0xfffu; };
    for (int h = 0; h < 2; ++h) {
        const uint32_t c = e <= E ? cnt[e] : 0u;
        const uint32_t nt0 = (c + trs[h] - 1) / trs[h];
        const uint32_t nt = nt0 > 1 ? (nt0 + 1) & ~1u : nt0;
        const uint32_t cls = nt > 1 ? 0u : 5u - min((c + 15) / 16, 4u);
        const unsigned long long packed = (unsigned long long)nt << (12 * cls);
        unsigned long long incl = packed;
        for (int d = 1; d < 64; d <<= 1) {
            const unsigned long long o = __shfl_up(incl, d, 64);
            if ((int)lane >= d) incl += o;
        }
        __syncthreads();  // the previous list's wsum reads are done
        if (lane == 63) wsum[wv] = incl;
        __syncthreads();
        unsigned long long off = incl - packed, all = 0;
        for (uint32_t k = 0; k < wv; ++k) off += wsum[k];
        for (uint32_t k = 0; k < PG_WG / 64; ++k) all += wsum[k];
        uint32_t start = field(off, cls), total = 0;
        for (uint32_t k = 0; k < 5; ++k) {
            if (k < cls) start += field(all, k);
            total += field(all, k);
        }
        uint2* tdst = tinfo + (dst - tiles);
        for (uint32_t q = 0; q < nt; ++q) {
            dst[start + q] = e << 16 | q;
            tdst[start + q] = make_uint2(offs[e], cnt[e]);
        }
        if (tau == PG_WG - 1) ntiles[h] = total;
        // bound of the first list, as pf_tile_bound computes it
        const uint32_t n = (T * topk + tr - 1) / tr + E + (T + tr - 1) / tr + 1 + (E + 1);
        dst = tiles + ((n + 15) & ~15u);
    }
}

// out[t][n] = sum_r w[t][r] yd[t][r][n] + sigmoid(sg[t]) yd[t][k][n]
// (cpu.rs:527-540), then hyper[t][g H + n] += out inj[t][g].  Slot r of
// token t is yd row goff[q >> 22] + (q & 0x3fffff), q = pos[t (k+1) + r]
// (the down GEMM's grouped order).
// K > 0: K routed slots known at compile time, a thread takes outputs
// 4 n .. + 3 with every slot's values in flight before the first is summed;
// K = 0: any topk, one output per thread.  Slots are summed in order either
// way.
template <int K>
__global__ void __launch_bounds__(256) k_pf_moe_combine(const float* __restrict__ yd, const uint32_t* __restrict__ goff,
                                                        const uint32_t* __restrict__ pos,
                                                        const float* __restrict__ wts,
                                                        const float* __restrict__ sg, const float* __restrict__ inj,
                                                        float* __restrict__ hyper, uint32_t H, uint32_t topk,
                                                        uint32_t hc) {
    const uint32_t t = blockIdx.y, slots = topk + 1;
    if constexpr (K == 0) {
        const uint32_t n = blockIdx.x * CHK_WG + threadIdx.x;
        if (n >= H) return;
        const uint32_t* pt = pos + (size_t)t * slots;
        auto row = [&](uint32_t r) { return (size_t)(goff[pt[r] >> 22] + (pt[r] & 0x3fffffu)); };
        float out = 0.0f;
        for (uint32_t r = 0; r < topk; ++r) out += wts[(size_t)t * topk + r] * yd[row(r) * H + n];
        out += sigmoidf_(sg[t]) * yd[row(topk) * H + n];
        float* hy = hyper + (size_t)t * hc * H + n;
        for (uint32_t g = 0; g < hc; ++g) hy[(size_t)g * H] += out * inj[(size_t)t * hc + g];
    } else {
        const uint32_t n = (blockIdx.x * CHK_WG + threadIdx.x) * 4;
        if (n >= H) return;
        uint32_t pr[K + 1];
#pragma unroll
        for (int r = 0; r <= K; ++r) pr[r] = pos[(size_t)t * slots + r];
#pragma unroll
        for (int r = 0; r <= K; ++r) pr[r] = goff[pr[r] >> 22] + (pr[r] & 0x3fffffu);
        float4 v[K + 1];
#pragma unroll
        for (int r = 0; r <= K; ++r) v[r] = *reinterpret_cast<const float4*>(yd + (size_t)pr[r] * H + n);
        float out[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int r = 0; r < K; ++r) {
            const float w = wts[(size_t)t * K + r];
            out[0] += w * v[r].x;
            out[1] += w * v[r].y;
            out[2] += w * v[r].z;
            out[3] += w * v[r].w;
        }
        const float sgv = sigmoidf_(sg[t]);
        out[0] += sgv * v[K].x;
        out[1] += sgv * v[K].y;
        out[2] += sgv * v[K].z;
        out[3] += sgv * v[K].w;
        float* hy = hyper + (size_t)t * hc * H + n;
        for (uint32_t g = 0; g < hc; ++g) {
            float4 h = *reinterpret_cast<const float4*>(hy + (size_t)g * H);
            const float ij = inj[(size_t)t * hc + g];
            h.x += out[0] * ij;
            h.y += out[1] * ij;
            h.z += out[2] * ij;
            h.w += out[3] * ij;
            *reinterpret_cast<float4*>(hy + (size_t)g * H) = h;
        }
    }
}

// ------------------------------------------------------------- embed
// embed.dequant_row replicated into the hc streams (cpu.rs:399-407), with
// explicitly rounded mul/add as on the decode path.
__global__ void __launch_bounds__(256) k_pf_embed(const uint32_t* __restrict__ tokens, Q4Mat emb,
                                                  float* __restrict__ hyper, uint32_t H, uint32_t hc) {
    const uint32_t t = blockIdx.y, i = blockIdx.x * CHK_WG + threadIdx.x;
    if (i >= H) return;
    const uint32_t tok = tokens[t];
    const uint32_t word = emb.w[(size_t)tok * (H / 8) + i / 8];
    const uint32_t g = i / 64;
    const float s = bf16f(emb.s[(size_t)tok * (H / 64) + g]), b = bf16f(emb.b[(size_t)tok * (H / 64) + g]);
    const float q = (float)((word >> (4 * (i % 8))) & 15u);
    const float e = __fadd_rn(__fmul_rn(s, q), b);
    for (uint32_t k = 0; k < hc; ++k) hyper[(size_t)t * hc * H + k * H + i] = e;
}

// ----------------------------------------------------------- DeltaNet
// Causal conv over time (cpu.rs:1067-1085) + silu for every channel, then
// the L2 norms of the q (times dk^-1/2) and k heads (eps 1e-6,
// cpu.rs:745-760).  Lane l of a workgroup owns four adjacent channels of
// one row (float4 loads of the row and of the rows before it), so a
// 128-channel head is a half wave; the window reaches into the layer's
// history for the first rows.
template <int CK>
__global__ void __launch_bounds__(256) k_pf_dn_conv(PfDnArgs a) {
    // CK > 0: the kernel width at compile time (its taps load as whole
    // words), else a.ck
    const uint32_t ck = CK > 0 ? (uint32_t)CK : a.ck, km1 = ck - 1;
    const uint32_t t = blockIdx.y, c0 = (blockIdx.x * CHK_WG + threadIdx.x) * 4;
    const bool live = c0 < a.conv_dim;
    const uint32_t cc = live ? c0 : 0;
    // taps of the four channels: w[e][j] = conv_w[(cc + e) ck + j]
    float w[4][CK > 0 ? CK : 9];
    if constexpr (CK == 4) {
        const uint4* wp = reinterpret_cast<const uint4*>(a.conv_w + (size_t)cc * 4);
        const uint4 w0 = wp[0], w1 = wp[1];
        const uint32_t ww[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t word = ww[(e * 4 + j) >> 1];
                w[e][j] = __uint_as_float((j & 1) ? word & 0xffff0000u : word << 16);
            }
    } else {
        for (int e = 0; e < 4; ++e)
            for (uint32_t j = 0; j < ck; ++j) w[e][j] = bf16f(a.conv_w[(size_t)(cc + e) * ck + j]);
    }
    const float4 cur = *reinterpret_cast<const float4*>(a.raw + (size_t)t * a.ld_raw + cc);
    float o[4] = {w[0][km1] * cur.x, w[1][km1] * cur.y, w[2][km1] * cur.z, w[3][km1] * cur.w};
#pragma unroll
    for (uint32_t j = 0; j < km1; ++j) {
        const int tau = (int)t - (int)km1 + (int)j;
        float x[4];
        if (tau >= 0) {
            const float4 v = *reinterpret_cast<const float4*>(a.raw + (size_t)tau * a.ld_raw + cc);
            x[0] = v.x;
            x[1] = v.y;
            x[2] = v.z;
            x[3] = v.w;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] = a.hist[(size_t)(cc + e) * km1 + (tau + (int)km1)];
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] += w[e][j] * x[e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = siluf_(o[e]);
    // q and k heads: 128 channels = the 32 lanes of a half wave
    const float sq = group_sum<32>((o[0] * o[0] + o[1] * o[1]) + (o[2] * o[2] + o[3] * o[3]));
    if (c0 < 2 * a.qk_dim) {
        float inv = 1.0f / sqrtf(sq + 1e-6f);
        if (c0 < a.qk_dim) inv *= a.qscale;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] *= inv;
    }
    if (live) *reinterpret_cast<float4*>(a.conv + (size_t)t * a.conv_dim + c0) = make_float4(o[0], o[1], o[2], o[3]);
}

// The new conv history (the last ck-1 raw inputs, reaching into the old
// history when T < ck-1) and the per-row decay / beta of every value head:
// g = -exp(A_log) softplus(a + dt_bias), decay = e^g, beta = sigmoid(b)
// (cpu.rs:775-777).  Runs after k_pf_dn_conv, which reads the old history.
__global__ void __launch_bounds__(256) k_pf_dn_misc(PfDnArgs a) {
    const uint32_t i = blockIdx.x * CHK_WG + threadIdx.x, km1 = a.ck - 1;
    if (i < a.conv_dim) {
        float nh[8];
#pragma unroll
        for (uint32_t h = 0; h < 8; ++h) {
            if (h >= km1) break;
            const int tau = (int)a.T - (int)km1 + (int)h;
            nh[h] = tau >= 0 ? a.raw[(size_t)tau * a.ld_raw + i] : a.hist[(size_t)i * km1 + (tau + (int)km1)];
        }
#pragma unroll
        for (uint32_t h = 0; h < 8; ++h) {
            if (h >= km1) break;
            a.hist[(size_t)i * km1 + h] = nh[h];
        }
        return;
    }
    const uint32_t j = i - a.conv_dim;
    if (j >= a.T * a.nv) return;
    const uint32_t t = j / a.nv, hv = j % a.nv;
    float av = 0.0f, bv = 0.0f;
    for (uint32_t z = 0; z < a.ab_split; ++z) {
        const size_t o = z * a.ab_zstride + (size_t)t * a.ld_ab + hv;
        av += a.a_raw[o];
        bv += a.b_raw[o];
    }
    const float gg = -expf(bf16f(a.a_log[hv])) * softplusf_(av + bf16f(a.dt_bias[hv]));
    a.decay[(size_t)t * a.nv + hv] = expf(gg);
    a.beta[(size_t)t * a.nv + hv] = sigmoidf_(bv);
}

// The gated delta rule over the chunk's rows in order (cpu.rs:745-812; the
// reference prefill runs the same sequential recurrence, deltanet.rs:80-95).
// One wave per (value head, 4 value columns): lane (c, p) holds keys
// 8p..8p+7 of column c of the head's fp32 state (kept transposed, [dv][dk])
// in VGPRs.  With S the state before row t, the row needs three 16-lane
// dot products that do not depend on each other, so they reduce together:
//   sk = S^T k, sq = S^T q, kq = k . q;
//   delta = beta (v - decay sk), y = decay sq + delta kq,
//   S <- decay S + k delta^T.
// The q, k, v, decay, beta of row t + PF_SCAN_AHEAD load while row t
// computes.
constexpr int PF_SCAN_AHEAD = 16;

__global__ void __launch_bounds__(64) k_pf_dn_scan(PfDnArgs a) {
    constexpr int DK = 128, KPL = 8, D = PF_SCAN_AHEAD;
    const int lane = threadIdx.x, c = lane >> 4, p = lane & 15;
    const uint32_t blocks = a.dv / 4;
    const uint32_t hv = blockIdx.x / blocks, iv = (blockIdx.x % blocks) * 4 + c;
    const uint32_t hk = hv / (a.nv / a.nk);
    float S[KPL];
    float* sp = a.state + ((size_t)hv * a.dv + iv) * DK + p * KPL;
    {
        const float4 s0 = *reinterpret_cast<const float4*>(sp), s1 = *reinterpret_cast<const float4*>(sp + 4);
        S[0] = s0.x; S[1] = s0.y; S[2] = s0.z; S[3] = s0.w; S[4] = s1.x; S[5] = s1.y; S[6] = s1.z; S[7] = s1.w;
    }
    const float* qb = a.conv + hk * DK + p * KPL;
    const float* kb = a.conv + a.qk_dim + hk * DK + p * KPL;
    const float* vb = a.conv + 2 * a.qk_dim + hv * a.dv + iv;
    float Q[D][KPL], Kk[D][KPL], V[D], DC[D], BT[D];
    auto load = [&](int d, uint32_t t) __attribute__((always_inline)) {
        const uint32_t tt = min(t, a.T - 1);
        const size_t ro = (size_t)tt * a.conv_dim;
        const float4 q0 = *reinterpret_cast<const float4*>(qb + ro), q1 = *reinterpret_cast<const float4*>(qb + ro + 4);
        const float4 k0 = *reinterpret_cast<const float4*>(kb + ro), k1 = *reinterpret_cast<const float4*>(kb + ro + 4);
        Q[d][0] = q0.x; Q[d][1] = q0.y; Q[d][2] = q0.z; Q[d][3] = q0.w;
        Q[d][4] = q1.x; Q[d][5] = q1.y; Q[d][6] = q1.z; Q[d][7] = q1.w;
        Kk[d][0] = k0.x; Kk[d][1] = k0.y; Kk[d][2] = k0.z; Kk[d][3] = k0.w;
        Kk[d][4] = k1.x; Kk[d][5] = k1.y; Kk[d][6] = k1.z; Kk[d][7] = k1.w;
        V[d] = vb[ro];
        DC[d] = a.decay[(size_t)tt * a.nv + hv];
        BT[d] = a.beta[(size_t)tt * a.nv + hv];
    };
#pragma unroll
    for (int d = 0; d < D; ++d) load(d, d);
    float* yout = a.y + hv * a.dv + iv;
    for (uint32_t t0 = 0; t0 < a.T; t0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const uint32_t t = t0 + d;
            if (t >= a.T) break;
            float sk = 0.0f, sq = 0.0f, kq = 0.0f;
#pragma unroll
            for (int j = 0; j < KPL; ++j) {
                sk += S[j] * Kk[d][j];
                sq += S[j] * Q[d][j];
                kq += Kk[d][j] * Q[d][j];
            }
            sk = group_sum<16>(sk);
            sq = group_sum<16>(sq);
            kq = group_sum<16>(kq);
            const float dec = DC[d];
            const float delta = BT[d] * (V[d] - dec * sk);
            const float y = dec * sq + delta * kq;
#pragma unroll
            for (int j = 0; j < KPL; ++j) S[j] = dec * S[j] + Kk[d][j] * delta;
            if (p == 0) yout[(size_t)t * a.v_dim] = y;
            load(d, t + D);
        }
    }
    *reinterpret_cast<float4*>(sp) = make_float4(S[0], S[1], S[2], S[3]);
    *reinterpret_cast<float4*>(sp + 4) = make_float4(S[4], S[5], S[6], S[7]);
}

// -------------------------------------------------------------- launchers

void launch_pf_prep(const PfPrepArgs& a, hipStream_t st) {
    const uint64_t n = (uint64_t)a.T * (a.K >> 3);
    if (!n) return;
    if (a.K % 64) throw std::runtime_error("prefill operands need K a multiple of 64");
    const uint32_t grid = (uint32_t)((n + CHK_WG - 1) / CHK_WG);
    if (!a.z) {
        k_pf_prep<PP_PLAIN, 1><<<grid, CHK_WG, 0, st>>>(a);
        return;
    }
    switch (a.dv) {
    case 64: k_pf_prep<PP_DN_GATE, 8><<<grid, CHK_WG, 0, st>>>(a); break;
    case 128: k_pf_prep<PP_DN_GATE, 16><<<grid, CHK_WG, 0, st>>>(a); break;
    case 256: k_pf_prep<PP_DN_GATE, 32><<<grid, CHK_WG, 0, st>>>(a); break;
    default: throw std::runtime_error("prefill gated norm needs a value head dim of 64, 128 or 256");
    }
}

void launch_pf_xprep(const float* x, uint32_t ldx, uint32_t T, uint32_t K, uint4* hi, uint4* lo, float* xs,
                     hipStream_t st) {
    PfPrepArgs a{};
    a.x = x;
    a.ldx = ldx;
    a.T = T;
    a.K = K;
    a.hi = hi;
    a.lo = lo;
    a.xs = xs;
    launch_pf_prep(a, st);
}

void launch_pf_hc_prep(float* hyper, const uint16_t* norm, uint32_t H, uint32_t hc, float eps, float* inv,
                       uint4* hi, uint4* lo, float* xs, uint32_t T, const float* part, uint64_t pzs, uint32_t nsplit,
                       const float* pinj, hipStream_t st, const PfCombine& mc) {
    if (H > 4096 || hc > 4 || H % 64) throw std::runtime_error("prefill hyper-connection norm needs hidden <= 4096, hc <= 4");
    if (part && (!nsplit || pzs % 4 || (uintptr_t)part % 16 || !pinj))
        throw std::runtime_error("pending inject needs 16-byte aligned partials");
    if (mc.yd) {
        if (part) throw std::runtime_error("prefill hyper-connection norm: one pending inject at a time");
        if ((uintptr_t)mc.yd % 16 || !mc.inj || !mc.topk) throw std::runtime_error("pending combine needs 16-byte rows");
        if (!T) return;
        if (mc.topk == 10) k_pf_hc_prep<10><<<T, CHK_WG, 0, st>>>(hyper, norm, H, hc, eps, inv, hi, lo, xs, part, pzs, nsplit, pinj, mc);
        else k_pf_hc_prep<0><<<T, CHK_WG, 0, st>>>(hyper, norm, H, hc, eps, inv, hi, lo, xs, part, pzs, nsplit, pinj, mc);
        return;
    }
    if (T) k_pf_hc_prep<-1><<<T, CHK_WG, 0, st>>>(hyper, norm, H, hc, eps, inv, hi, lo, xs, part, pzs, nsplit, pinj, mc);
}

// The launch form of a GEMM: 32-bit element offsets of the dense matrices
// from their lowest base, and whether its scales can be staged (whole
// blocks of 8 groups on 16-byte aligned rows).
static bool pf_gemm_prepare(PfGemmArgs& a, int epi) {
    const int nm = std::max<int>(a.nseg, epi == PE_SILU_MUL ? 2 : 1);
    uintptr_t wmin = UINTPTR_MAX, smin = UINTPTR_MAX;
    for (int q = 0; q < nm; ++q) {
        wmin = std::min(wmin, (uintptr_t)a.seg[q].m.w);
        smin = std::min({smin, (uintptr_t)a.seg[q].m.s, (uintptr_t)a.seg[q].m.b});
    }
    a.wbase = (const uint32_t*)wmin;
    a.sbase = (const uint16_t*)smin;
    for (int q = 0; q < nm; ++q) {
        const uint64_t w = ((uintptr_t)a.seg[q].m.w - wmin) / 4, s = ((uintptr_t)a.seg[q].m.s - smin) / 2,
                       b = ((uintptr_t)a.seg[q].m.b - smin) / 2;
        const uint64_t rows = a.seg[q].m.out;
        if (w + rows * (a.K / 8) > UINT32_MAX || std::max(s, b) + rows * (a.K / 64) > UINT32_MAX)
            throw std::runtime_error("prefill GEMM weights span more than 32-bit offsets reach");
        a.seg[q].wo = (uint32_t)w;
        a.seg[q].so = (uint32_t)s;
        a.seg[q].bo = (uint32_t)b;
    }
    const uint32_t ksplit = std::max<uint32_t>(1, a.ksplit);
    bool sbl = (a.K / 64 / ksplit) % 8 == 0 && smin % 16 == 0;
    for (int q = 0; q < nm; ++q) sbl = sbl && a.seg[q].so % 8 == 0 && a.seg[q].bo % 8 == 0;
    auto aligned = [](const ExpertsDev& X) {
        return (uintptr_t)X.base % 16 == 0 && X.stride % 16 == 0 && X.gate_s % 16 == 0 && X.gate_b % 16 == 0 &&
               X.up_s % 16 == 0 && X.up_b % 16 == 0 && X.down_s % 16 == 0 && X.down_b % 16 == 0;
    };
    if (a.X.base) sbl = sbl && aligned(a.X) && (a.X.bits == 4 || (a.X4.base && aligned(a.X4)));
    return sbl;
}


bool launch_pf_gemm_args(const PfGemmArgs& args, int epi, uint32_t grid_y, hipStream_t st) {
    if (args.K % 64 || !args.K) throw std::runtime_error("prefill GEMM needs K a multiple of 64");
    if (!grid_y) return true;
    PfGemmArgs a = args;
    const bool sbl = pf_gemm_prepare(a, epi);
    // the epilogue writes the next GEMM's operands (phi) where it can: the
    // mix in its staged form, gate/up in its transposed (staged-scale)
    // form; else its f32 rows, and the caller stages them
    if (a.phi && epi == PE_SILU_MUL && (!sbl || a.N % 64 || (uintptr_t)a.phi % 16 || (uintptr_t)a.plo % 16 || !a.pxs))
        a.phi = nullptr;
    if (a.phi && epi == PE_HC_UP && sbl) a.phi = nullptr;
    const bool fused = !args.phi || a.phi;
    const uint32_t ksplit = std::max<uint32_t>(1, a.ksplit);
    if ((a.K / 64) % ksplit || (ksplit > 1 && epi != PE_STORE))
        throw std::runtime_error("split K needs whole groups per chunk and a plain store");
    if (epi == PE_HC_UP && a.hc > 4) throw std::runtime_error("prefill mix needs hc <= 4");
    // 16-byte output stores: N, every output row and every segment start on
    // a 4-float boundary.  The hc-stream mix epilogue has only that form.
    bool v4 = a.N % 4 == 0 && (ksplit == 1 || a.zstride % 4 == 0);
    for (uint32_t q = 0; q < (epi == PE_STORE ? a.nseg : 1u); ++q)
        v4 = v4 && (uintptr_t)a.seg[q].y % 16 == 0 && a.seg[q].ldy % 4 == 0 && a.seg[q].n0 % 4 == 0;
    if (epi == PE_HC_UP) {
        v4 = a.H % 4 == 0 && a.N % 4 == 0 && (uintptr_t)a.hyper % 16 == 0 &&
             (uintptr_t)a.out % 16 == 0 && (uintptr_t)a.norm % 8 == 0;
        if (!v4) throw std::runtime_error("prefill hyper-connection GEMMs need 16-byte aligned streams");
        if (a.phi && (a.H % 64 || (uintptr_t)a.norm % 16 || !a.plo || !a.pxs || (a.pbhi && (!a.pbmid || !a.pblo))))
            throw std::runtime_error("prefill mix into operands needs hidden % 64 == 0 and 16-byte aligned norms");
    }
    a.vec4 = v4 ? 1u : 0u;
#define PF_GEMM(NM, E, GX)                                                             \
    do {                                                                               \
        if (sbl) k_pf_gemm<NM, E, true><<<dim3(GX, grid_y, ksplit), PF_WG, 0, st>>>(a); \
        else k_pf_gemm<NM, E, false><<<dim3(GX, grid_y, ksplit), PF_WG, 0, st>>>(a);    \
    } while (0)
    const uint32_t xbits = a.X.base ? a.X.bits : 4;
    if (xbits != 4) {
        // grouped expert GEMMs over Q3 / Q2 records (scales staged where
        // the groups come in blocks of 8, else folded per lane)
        if (epi != PE_STORE && epi != PE_SILU_MUL) throw std::runtime_error("low-bit records: gate/up and down only");
        const uint32_t gx = epi == PE_STORE ? (a.N + 255) / 256 : (a.N + 127) / 128;
        const dim3 grid(gx, grid_y, ksplit);
#define PF_LB(B, S)                                                                       \
    do {                                                                                  \
        if (epi == PE_STORE) k_pf_gemm<1, PE_STORE, S, B><<<grid, PF_WG, 0, st>>>(a);     \
        else k_pf_gemm<2, PE_SILU_MUL, S, B><<<grid, PF_WG, 0, st>>>(a);                  \
    } while (0)
        if (xbits == 3 && sbl) PF_LB(3, true);
        else if (xbits == 3) PF_LB(3, false);
        else if (xbits == 2 && sbl) PF_LB(2, true);
        else if (xbits == 2) PF_LB(2, false);
        else throw std::runtime_error("expert records of 4, 3 or 2 bits");
#undef PF_LB
        return fused;
    }
    switch (epi) {
    case PE_STORE: PF_GEMM(1, PE_STORE, (a.N + 255) / 256); break;
    case PE_HC_UP: PF_GEMM(1, PE_HC_UP, (a.H + 63) / 64); break;
    default: PF_GEMM(2, PE_SILU_MUL, (a.N + 127) / 128); break;
    }
#undef PF_GEMM
    return fused;
}

void launch_pf_gemm(const Q4Mat& w, const uint4* xhi, const uint4* xlo, const float* xs, float* y, uint32_t T,
                    uint32_t ldy, hipStream_t st) {
    PfGemmArgs a{};
    a.seg[0] = PfSeg{w, y, ldy, 0};
    a.nseg = 1;
    a.N = w.out;
    a.K = w.in;
    a.M = T;
    a.xhi = xhi;
    a.xlo = xlo;
    a.xs = xs;
    launch_pf_gemm_args(a, PE_STORE, (T + 63) / 64, st);
}

void launch_pf_hc_down_finish(const float* part, uint32_t nsplit, uint32_t T, uint32_t lowrank, uint32_t hc,
                              float alpha, float* d, float* inj, uint4* hi, uint4* lo, float* xs, hipStream_t st) {
    const uint64_t n = (uint64_t)T * (lowrank + hc);
    if (!n) return;
    if (lowrank % 64 == 0 && (lowrank + hc) % 4 == 0) {
        // d staged straight into the up GEMM's operands
        const uint64_t m = (uint64_t)T * (lowrank / 8 + hc);
        k_pf_hc_down_finish_q<<<(uint32_t)((m + CHK_WG - 1) / CHK_WG), CHK_WG, 0, st>>>(part, nsplit, n, T, lowrank, hc, alpha,
                                                                                    hi, lo, xs, inj);
        return;
    }
    k_pf_hc_down_finish<<<(uint32_t)((n + CHK_WG - 1) / CHK_WG), CHK_WG, 0, st>>>(part, nsplit, n, T, lowrank, hc, alpha, d, inj);
    launch_pf_xprep(d, lowrank, T, lowrank, hi, lo, xs, st);
}

// The router's grid: x = column blocks of 64 PF_ROUTER_CT experts, z = K
// chunks.  Wide blocks (the x planes are re-read once per column block)
// with PF_ROUTER_CHUNKS chunks where every chunk keeps whole 64-wide
// blocks, at least three (the staging runs two blocks ahead), E % 4 == 0
// (16-byte partials) and E fills the blocks; else 64-expert blocks over
// the whole K.
dim3 pf_router_plan(uint32_t T, uint32_t E, uint32_t H) {
    const uint32_t NB = H / 64;
    if (NB % PF_ROUTER_CHUNKS == 0 && NB / PF_ROUTER_CHUNKS >= 3 && E % 4 == 0 && E % (64 * PF_ROUTER_CT) == 0)
        return dim3(E / (64 * PF_ROUTER_CT), (T + 63) / 64, PF_ROUTER_CHUNKS);
    return dim3((E + 63) / 64, (T + 63) / 64, 1);
}

void launch_pf_router(const uint16_t* router, const uint4* bhi, const uint4* bmid, const uint4* blo, float* logits,
                      uint32_t T, uint32_t E, uint32_t H, hipStream_t st) {
    if (H % 64) throw std::runtime_error("router width must be a multiple of 64");
    if (!T) return;
    const dim3 g = pf_router_plan(T, E, H);
    if (g.z > 1) k_pf_router<PF_ROUTER_CT><<<g, CHK_WG, 0, st>>>(router, bhi, bmid, blo, logits, T, E, H);
    else k_pf_router<1><<<g, CHK_WG, 0, st>>>(router, bhi, bmid, blo, logits, T, E, H);
}

void launch_pf_route(const float* logits, uint32_t T, uint32_t E, uint32_t topk, int norm_topk, uint32_t* ids,
                     float* wts, uint32_t* last_ids, float* last_wts, const uint16_t* shared_gate, const uint4* bhi,
                     const uint4* bmid, const uint4* blo, float* sg, uint32_t H, uint32_t* gcnt, uint32_t* list,
                     uint32_t* pos, uint32_t cap, bool shared, hipStream_t st) {
    if (H % 8 || (uintptr_t)shared_gate % 16) throw std::runtime_error("shared gate needs 16-byte rows");
    if (E > 512 || topk > 64 || topk >= E) throw std::runtime_error("prefill routing: at most 512 experts");
    if (T > cap || (uint64_t)T * (topk + 1) >= (1u << 22)) throw std::runtime_error("prefill grouping: too many entries");
    if (!T) return;
    // the router's K-chunk partials, summed in chunk order
    const uint32_t nz = pf_router_plan(T, E, H).z;
    if (nz == PF_ROUTER_CHUNKS)
        k_pf_route<PF_ROUTER_CHUNKS><<<(T + 3) / 4, CHK_WG, 0, st>>>(logits, T, E, topk, norm_topk, ids, wts, last_ids,
                                                                     last_wts, shared_gate, bhi, bmid, blo, sg, H,
                                                                     gcnt, list, pos, cap, shared ? 1u : 0u);
    else
        k_pf_route<1><<<(T + 3) / 4, CHK_WG, 0, st>>>(logits, T, E, topk, norm_topk, ids, wts, last_ids, last_wts,
                                                      shared_gate, bhi, bmid, blo, sg, H, gcnt, list, pos, cap,
                                                      shared ? 1u : 0u);
}

void launch_pf_group(uint32_t* gcnt, uint32_t T, uint32_t topk, uint32_t E, uint32_t cap, uint32_t* count,
                     uint32_t* tiles, uint32_t* ntiles, uint2* tinfo, uint32_t* goff, uint64_t* act, uint32_t layer,
                     uint32_t tr, bool shared, hipStream_t st) {
    if (E + 1 > PG_WG) throw std::runtime_error("prefill grouping supports at most 1023 experts");
    if (T > cap || (uint64_t)T * (topk + 1) >= (1u << 22)) throw std::runtime_error("prefill grouping: too many entries");
    if (tr != 48 && tr != 64) throw std::runtime_error("prefill grouping: tiles of 48 or 64 rows");
    if (pf_tile_bound(T, topk, E, tr) >= 0x1000u || pf_tile_bound(T, topk, E, 64) >= 0x1000u)
        throw std::runtime_error("prefill grouping: too many tiles");
    k_pf_group<<<1, PG_WG, 0, st>>>(gcnt, T, E, cap, count, tiles, ntiles, tinfo, goff,
                                    reinterpret_cast<unsigned long long*>(act), layer, tr, topk, shared ? 1u : 0u);
}

// Tiles of a grouped GEMM: every group's rows in tr-row tiles, one more
// per group for the even rounding, the grid rounded up to 16 tiles.
uint32_t pf_tile_bound(uint32_t T, uint32_t topk, uint32_t E, uint32_t tr) {
    const uint32_t n = (T * topk + tr - 1) / tr + E + (T + tr - 1) / tr + 1 + (E + 1);
    return (n + 15) & ~15u;
}

void launch_pf_moe_combine(const float* yd, const uint32_t* goff, const uint32_t* pos, const float* wts, const float* sg,
                           const float* inj, float* hyper, uint32_t T, uint32_t H, uint32_t topk, uint32_t hc,
                           hipStream_t st) {
    if (!T) return;
    if (topk == 10 && H % 4 == 0)
        k_pf_moe_combine<10><<<dim3((H / 4 + 255) / 256, T), CHK_WG, 0, st>>>(yd, goff, pos, wts, sg, inj, hyper, H, topk, hc);
    else
        k_pf_moe_combine<0><<<dim3((H + 255) / 256, T), CHK_WG, 0, st>>>(yd, goff, pos, wts, sg, inj, hyper, H, topk, hc);
}

void launch_pf_embed(const uint32_t* tokens, const Q4Mat& emb, float* hyper, uint32_t H, uint32_t hc, uint32_t T,
                     hipStream_t st) {
    if (T) k_pf_embed<<<dim3((H + 255) / 256, T), CHK_WG, 0, st>>>(tokens, emb, hyper, H, hc);
}

void launch_pf_dn_scan(const PfDnArgs& a, float* work, hipStream_t st) {
    if (!a.T) return;
    if (a.dv % 4 || a.qk_dim != a.nk * 128) throw std::runtime_error("scan needs key head dim 128, value head dim a multiple of 4");
    if (work && dc_supported(a.nk, a.nv, a.qk_dim / a.nk, a.dv)) launch_dc_scan(a, work, st);
    else k_pf_dn_scan<<<a.nv * (a.dv / 4), 64, 0, st>>>(a);
}

void launch_pf_dn(const PfDnArgs& a, float* work, hipStream_t st) {
    if (!a.T) return;
    if (a.ck < 2 || a.ck > 9) throw std::runtime_error("conv kernel 2..=9");
    if (a.dv % 4) throw std::runtime_error("value head dim must be a multiple of 4");
    if (a.conv_dim % 128 || a.qk_dim % 128 || a.ld_raw % 4)
        throw std::runtime_error("prefill conv needs whole 128-channel heads");
    const dim3 grid((a.conv_dim + 4 * CHK_WG - 1) / (4 * CHK_WG), a.T);
    if (a.ck == 4 && (uintptr_t)a.conv_w % 16 == 0) k_pf_dn_conv<4><<<grid, CHK_WG, 0, st>>>(a);
    else k_pf_dn_conv<0><<<grid, CHK_WG, 0, st>>>(a);
    const uint32_t n = a.conv_dim + a.T * a.nv;
    k_pf_dn_misc<<<(n + CHK_WG - 1) / CHK_WG, CHK_WG, 0, st>>>(a);
    launch_pf_dn_scan(a, work, st);
}

}  // namespace chk

namespace chk {

// ------------------------------------------------- causal flash attention
// Prefill attention (the reference's GEMM attention, gpu/prefill/attention.rs,
// with the decode semantics of cpu.rs:589-634 over the engine's q8 KV rule):
// for every prompt row r at position pos0 + r and query head h,
//   o = softmax_t(scale q . k_t) . v_t over t <= pos0 + r, times sigmoid(gate).
//
// Work: per kv head, (16-row block, 32-token tile) steps; row block rb
// needs tiles 0 .. (pos0 + 16 rb + 15) / 32, so late blocks hold up to
// twice the average.  A plan (pf_flash_plan, on the host) deals the steps
// to the workgroups in equal shares: row blocks in zigzag order (first,
// last, second, ...), the sequence cut into W equal ranges, so a workgroup
// runs a few segments (row block, tile range); a row block cut between
// workgroups leaves unnormalised partials (m, l, o) that k_pf_flash_merge
// joins.  Within a segment, wave w serves the kv head's query head w
// (GQA: the group's waves share every staged K/V tile).  Per
// 32-token tile the workgroup dequantises K and V (int8 x fp16 scale,
// exact in f32) into LDS as fp16 hi + lo planes (V transposed), then each
// wave runs S = Q K^T and O += P V on v_mfma_f32_16x16x32_f16 with three
// passes (hi.hi + hi.lo + lo.hi, ~22-bit operands) and an online softmax in
// f32.  Layouts (16x16x32): A lane l = row l%16, k (l/16)*8..+8; B lane l =
// column l%16, k (l/16)*8..+8; D lane l = column l%16, rows 4(l/16)..+4.
constexpr int FA_TOK = 32;    // tokens per staged tile
constexpr int FA_ROWS = 16;   // query rows per workgroup

struct PfFlashArgs {
    const float* q_ready;  // [T][nh][hd] normed, roped queries
    const float* q_raw;    // [T][nh][2 hd] (the gate is each head's second half)
    KvDev kv;
    float* out;            // [T][nh * hd]
    uint32_t T, pos0, nh, nkv;
    float scale;
    const uint4* seg;      // [W][FA_MAXSEG] the plan's segments (pf_flash_plan)
    float* part;           // [nkv][nslots][FA_ROWS][G][2 + hd] partials of split row blocks
    uint32_t nslots;
};

CHK_DEV h8 split_hi(const float (&v)[8], h8& lo) {
    h8 hi;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        hi[j] = (_Float16)v[j];
        lo[j] = (_Float16)(v[j] - (float)hi[j]);
    }
    return hi;
}

template <int HD, int G>
__global__ void __launch_bounds__(64 * G) k_pf_flash(PfFlashArgs a) {
    constexpr int KS = HD / 32;          // dim steps of 32
    constexpr int DT = HD / 16;          // 16-dim output tiles
    constexpr int KP = HD + 8;           // padded K row (halves)
    constexpr int VP = FA_TOK + 8;       // padded V^T row (halves)
    constexpr int PP = FA_TOK + 8;       // padded P row (halves)
    __shared__ __align__(16) _Float16 kh[FA_TOK][KP], kl[FA_TOK][KP];
    __shared__ __align__(16) _Float16 vh[HD][VP], vl[HD][VP];
    __shared__ __align__(16) _Float16 ph[G][FA_ROWS][PP], pl[G][FA_ROWS][PP];
    constexpr uint32_t nthr = 64 * G;
    constexpr int IPT = (FA_TOK * HD / 16 + nthr - 1) / nthr;  // staging items per thread
    const uint32_t tid = threadIdx.x, lane = tid & 63, w = wave_id();
    const uint32_t col = lane & 15, kq = lane >> 4;
    const uint32_t hk = blockIdx.y, h = hk * G + w;
    const uint32_t kv_row = a.nkv * HD, last_tok = a.pos0 + a.T - 1;
    const uint4* segs = a.seg + (size_t)blockIdx.x * FA_MAXSEG;
    for (uint32_t sgi = 0; sgi < FA_MAXSEG; ++sgi) {
    const uint4 sg = segs[sgi];  // (row block, first tile, end tile, slot or ~0: the whole block)
    if (sg.x == ~0u) break;
    if (sgi) __syncthreads();  // every wave is done with the previous segment's tiles
    const uint32_t rb = sg.x, ta = sg.y, tb = sg.z;
    const uint32_t r0 = rb * FA_ROWS;
    // this wave's queries as A operands
    h8 qh[KS], ql[KS];
    {
        const uint32_t r = min(r0 + col, a.T - 1);
        const float* qp = a.q_ready + ((size_t)r * a.nh + h) * HD;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const float4 v0 = *reinterpret_cast<const float4*>(qp + s * 32 + kq * 8);
            const float4 v1 = *reinterpret_cast<const float4*>(qp + s * 32 + kq * 8 + 4);
            const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
            qh[s] = split_hi(v, ql[s]);
        }
    }
    // positions of the 4 rows this lane holds in D layout (rows past T
    // repeat the last row; they are never written)
    uint32_t qpos[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) qpos[i] = a.pos0 + min(r0 + kq * 4 + i, a.T - 1);
    f4 o[DT];
#pragma unroll
    for (int d = 0; d < DT; ++d) o[d] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    float m[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        m[i] = -INFINITY;
        l[i] = 0.0f;
    }
    // Staging: K as (token tid % 32, 16 dims), V as (token pair tid % 16,
    // 8 dims) so that the transposed V writes are whole dwords in
    // consecutive banks; a tile's raw bytes are loaded one tile ahead.
    uint4 kraw[IPT];
    uint2 vraw[IPT][2];
    uint16_t ksc[IPT], vsc[IPT][2];
    auto load_raw = [&](uint32_t t0) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < IPT; ++r) {
            const uint32_t i = tid + r * nthr;
            kraw[r] = make_uint4(0, 0, 0, 0);
            vraw[r][0] = vraw[r][1] = make_uint2(0, 0);
            ksc[r] = vsc[r][0] = vsc[r][1] = 0;
            if (i >= (uint32_t)(FA_TOK * HD / 16)) continue;
            const uint32_t kt = t0 + i % FA_TOK, kd = (i / FA_TOK) * 16;
            if (kt <= last_tok) {
                kraw[r] = *reinterpret_cast<const uint4*>(a.kv.k + (size_t)kt * kv_row + hk * HD + kd);
                ksc[r] = a.kv.ks[(size_t)kt * (kv_row / 32) + (hk * HD + kd) / 32];
            }
            const uint32_t vt = t0 + 2 * (i % (FA_TOK / 2)), vd = (i / (FA_TOK / 2)) * 8;
#pragma unroll
            for (int e = 0; e < 2; ++e)
                if (vt + e <= last_tok) {
                    vraw[r][e] = *reinterpret_cast<const uint2*>(a.kv.v + (size_t)(vt + e) * kv_row + hk * HD + vd);
                    vsc[r][e] = a.kv.vs[(size_t)(vt + e) * (kv_row / 32) + (hk * HD + vd) / 32];
                }
        }
    };
    auto store_tile = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < IPT; ++r) {
            const uint32_t i = tid + r * nthr;
            if (i >= (uint32_t)(FA_TOK * HD / 16)) continue;
            const uint32_t kt = i % FA_TOK, kd = (i / FA_TOK) * 16;
            const float kscale = __half2float(__ushort_as_half(ksc[r]));
            const uint32_t kwv[4] = {kraw[r].x, kraw[r].y, kraw[r].z, kraw[r].w};
#pragma unroll
            for (int hlf = 0; hlf < 2; ++hlf) {
                float kv8[8];
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    kv8[j] = (float)(int8_t)(kwv[hlf * 2 + j / 4] >> (8 * (j % 4))) * kscale;
                h8 lo8;
                const h8 hi8 = split_hi(kv8, lo8);
                *reinterpret_cast<h8*>(&kh[kt][kd + hlf * 8]) = hi8;
                *reinterpret_cast<h8*>(&kl[kt][kd + hlf * 8]) = lo8;
            }
            const uint32_t vt = 2 * (i % (FA_TOK / 2)), vd = (i / (FA_TOK / 2)) * 8;
            const float vs0 = __half2float(__ushort_as_half(vsc[r][0])), vs1 = __half2float(__ushort_as_half(vsc[r][1]));
            const uint32_t v0[2] = {vraw[r][0].x, vraw[r][0].y}, v1[2] = {vraw[r][1].x, vraw[r][1].y};
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float x0 = (float)(int8_t)(v0[j / 4] >> (8 * (j % 4))) * vs0;
                const float x1 = (float)(int8_t)(v1[j / 4] >> (8 * (j % 4))) * vs1;
                const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1;
                typedef _Float16 hh2 __attribute__((ext_vector_type(2)));
                *reinterpret_cast<hh2*>(&vh[vd + j][vt]) = hh2{h0, h1};
                *reinterpret_cast<hh2*>(&vl[vd + j][vt]) = hh2{(_Float16)(x0 - (float)h0), (_Float16)(x1 - (float)h1)};
            }
        }
    };
    load_raw(ta * FA_TOK);
    store_tile();
    __syncthreads();
    for (uint32_t tile = ta; tile < tb; ++tile) {
        const uint32_t t0 = tile * FA_TOK;
        if (tile + 1 < tb) load_raw(t0 + FA_TOK);
        // ---- S = Q K^T for 2 token tiles
        f4 s[2];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            s[tt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const h8 bh = *reinterpret_cast<const h8*>(&kh[tt * 16 + col][ks * 32 + kq * 8]);
                const h8 bl = *reinterpret_cast<const h8*>(&kl[tt * 16 + col][ks * 32 + kq * 8]);
                s[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ql[ks], bh, s[tt], 0, 0, 0);
                s[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh[ks], bl, s[tt], 0, 0, 0);
                s[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh[ks], bh, s[tt], 0, 0, 0);
            }
        }
        // ---- online softmax over the tile (rows kq*4 + i, tokens col, 16 + col)
        float p[2][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float mx = -INFINITY;
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                const uint32_t t = t0 + tt * 16 + col;
                const float v = t <= qpos[i] ? s[tt][i] * a.scale : -INFINITY;
                p[tt][i] = v;
                mx = fmaxf(mx, v);
            }
            mx = group_max<16>(mx);
            const float mn = fmaxf(m[i], mx);
            const float corr = m[i] == -INFINITY ? 0.0f : expf(m[i] - mn);
            float rs = 0.0f;
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                const float e = p[tt][i] == -INFINITY ? 0.0f : expf(p[tt][i] - mn);
                p[tt][i] = e;
                rs += e;
            }
            rs = group_sum<16>(rs);
            l[i] = l[i] * corr + rs;
            m[i] = mn;
#pragma unroll
            for (int d = 0; d < DT; ++d) o[d][i] *= corr;
        }
        // ---- P to this wave's LDS rows (hi, lo), read back as A operands:
        // LDS instructions of one wave complete in order, so only the
        // compiler has to be kept from reordering them
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const _Float16 hi = (_Float16)p[tt][i];
                ph[w][kq * 4 + i][tt * 16 + col] = hi;
                pl[w][kq * 4 + i][tt * 16 + col] = (_Float16)(p[tt][i] - (float)hi);
            }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const h8 pah = *reinterpret_cast<const h8*>(&ph[w][col][kq * 8]);
        const h8 pal = *reinterpret_cast<const h8*>(&pl[w][col][kq * 8]);
#pragma unroll
        for (int d = 0; d < DT; ++d) {
            const h8 bh = *reinterpret_cast<const h8*>(&vh[d * 16 + col][kq * 8]);
            const h8 bl = *reinterpret_cast<const h8*>(&vl[d * 16 + col][kq * 8]);
            o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pal, bh, o[d], 0, 0, 0);
            o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pah, bl, o[d], 0, 0, 0);
            o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pah, bh, o[d], 0, 0, 0);
        }
        if (tile + 1 < tb) {
            __syncthreads();  // every wave is done with this tile's K and V
            store_tile();
            __syncthreads();
        }
    }
    if (sg.w == ~0u) {
        // ---- o / l times the per-dim sigmoid gate (cpu.rs:629-633)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t r = r0 + kq * 4 + i;
            if (r >= a.T) continue;
            const float inv = 1.0f / l[i];
            const float* gp = a.q_raw + ((size_t)r * a.nh + h) * 2 * HD + HD;
            float* op = a.out + (size_t)r * a.nh * HD + (size_t)h * HD;
#pragma unroll
            for (int d = 0; d < DT; ++d) {
                const uint32_t dd = d * 16 + col;
                op[dd] = o[d][i] * inv * sigmoidf_(gp[dd]);
            }
        }
    } else {
        // ---- a piece of a split row block: (m, l, unnormalised o) per row
        float* pp = a.part + ((size_t)hk * a.nslots + sg.w) * FA_ROWS * G * (2 + HD);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float* q = pp + ((size_t)(kq * 4 + i) * G + w) * (2 + HD);
            if (col == 0) {
                q[0] = m[i];
                q[1] = l[i];
            }
#pragma unroll
            for (int d = 0; d < DT; ++d) q[2 + d * 16 + col] = o[d][i];
        }
    }
    }
}

// Joins the pieces of the row blocks a flash plan split: per row, head and
// dim, o = sum_k o_k e^(m_k - M) / sum_k l_k e^(m_k - M) with M = max_k m_k
// (a piece whose tokens a row cannot see holds m = -inf, l = 0), times the
// sigmoid gate.  Workgroup (entry, row) of kv head blockIdx.z; thread d
// takes dims d, d + 256 of every head, all loads issued before the sums.
template <int G, int HD>
__global__ void __launch_bounds__(256) k_pf_flash_merge(PfFlashArgs a, const uint4* __restrict__ merge) {
    constexpr int DPT = (HD + CHK_WG - 1) / CHK_WG;
    const uint4 me = merge[blockIdx.x];  // (row block, first slot, pieces, 0)
    const uint32_t row = blockIdx.y, hk = blockIdx.z, r = me.x * FA_ROWS + row, np = me.z;
    if (r >= a.T) return;
    const float* __restrict__ part = a.part;
    const float* __restrict__ qraw = a.q_raw;
    float* __restrict__ outp = a.out;
    const size_t ps = (size_t)FA_ROWS * G * (2 + HD);  // floats per slot
    const float* p0 = part + ((size_t)hk * a.nslots + me.y) * ps + (size_t)row * G * (2 + HD);
    float mk[G][FA_MAXP], lk[G][FA_MAXP], ok[G][FA_MAXP][DPT], gate[G][DPT];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float* q = p0 + (size_t)g * (2 + HD);
#pragma unroll
        for (int k = 0; k < FA_MAXP; ++k) {
            const bool on = (uint32_t)k < np;
            mk[g][k] = on ? q[k * ps] : -INFINITY;
            lk[g][k] = on ? q[k * ps + 1] : 0.0f;
#pragma unroll
            for (int j = 0; j < DPT; ++j) {
                const uint32_t d = threadIdx.x + j * CHK_WG;
                ok[g][k][j] = on && d < (uint32_t)HD ? q[k * ps + 2 + d] : 0.0f;
            }
        }
#pragma unroll
        for (int j = 0; j < DPT; ++j) {
            const uint32_t d = min(threadIdx.x + j * CHK_WG, (uint32_t)HD - 1);
            gate[g][j] = qraw[((size_t)r * a.nh + hk * G + g) * 2 * HD + HD + d];
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float M = -INFINITY;
#pragma unroll
        for (int k = 0; k < FA_MAXP; ++k) M = fmaxf(M, mk[g][k]);
        float e[FA_MAXP], L = 0.0f;
#pragma unroll
        for (int k = 0; k < FA_MAXP; ++k) {
            e[k] = mk[g][k] == -INFINITY ? 0.0f : expf(mk[g][k] - M);
            L += lk[g][k] * e[k];
        }
        const float inv = 1.0f / L;
#pragma unroll
        for (int j = 0; j < DPT; ++j) {
            const uint32_t d = threadIdx.x + j * CHK_WG;
            if (d >= (uint32_t)HD) continue;
            float O = 0.0f;
#pragma unroll
            for (int k = 0; k < FA_MAXP; ++k) O += ok[g][k][j] * e[k];
            outp[(size_t)r * a.nh * HD + (size_t)(hk * G + g) * HD + d] = O * inv * sigmoidf_(gate[g][j]);
        }
    }
}

// Deals every kv head's (row block, tile) steps to max_wg workgroups in
// equal shares (see k_pf_flash); one whole row block per workgroup, heavy
// ones first, where the blocks' work is within 15% of even or a share
// would need more than FA_MAXSEG segments.
PfFlashPlan pf_flash_plan(uint32_t T, uint32_t pos0, uint32_t max_wg) {
    PfFlashPlan p;
    const uint32_t R = (T + FA_ROWS - 1) / FA_ROWS;
    std::vector<uint32_t> tiles(R);
    uint64_t total = 0;
    uint32_t most = 0;
    for (uint32_t rb = 0; rb < R; ++rb) {
        tiles[rb] = (pos0 + std::min(rb * FA_ROWS + FA_ROWS - 1, T - 1)) / FA_TOK + 1;
        total += tiles[rb];
        most = std::max(most, tiles[rb]);
    }
    const uint32_t W = std::max<uint32_t>(1, std::min(R, max_wg));
    auto whole = [&]() {
        p = PfFlashPlan{};
        p.W = R;
        p.seg.assign((size_t)R * FA_MAXSEG, make_uint4(~0u, 0, 0, 0));
        for (uint32_t x = 0; x < R; ++x) {
            const uint32_t rb = R - 1 - x;
            p.seg[(size_t)x * FA_MAXSEG] = make_uint4(rb, 0, tiles[rb], ~0u);
        }
        return p;
    };
    if ((double)most <= 1.15 * (double)total / W) return whole();
    p.W = W;
    p.seg.assign((size_t)W * FA_MAXSEG, make_uint4(~0u, 0, 0, 0));
    std::vector<uint32_t> order;
    for (uint32_t i = 0, j = R; i < j;) {
        order.push_back(i++);
        if (i < j) order.push_back(--j);
    }
    uint64_t start = 0;
    std::vector<uint32_t> nseg(W, 0);
    for (uint32_t rb : order) {
        const uint64_t end = start + tiles[rb];
        // workgroups whose range [k total / W, (k + 1) total / W) meets [start, end)
        uint32_t k = (uint32_t)(start * W / total);
        while (k > 0 && k * total / W > start) --k;
        while (k + 1 < W && (k + 1) * total / W <= start) ++k;  // the range holding tile `start`
        const bool split = (k + 1) * total / W < end;
        uint32_t pieces = 0;
        const uint32_t first_slot = p.nslots;
        for (; k < W && k * total / W < end; ++k) {
            const uint64_t lo = std::max<uint64_t>(start, k * total / W), hi = std::min<uint64_t>(end, (k + 1) * total / W);
            if (lo >= hi) continue;
            if (nseg[k] == FA_MAXSEG) return whole();
            const uint32_t slot = split ? p.nslots++ : ~0u;
            p.seg[(size_t)k * FA_MAXSEG + nseg[k]++] = make_uint4(rb, (uint32_t)(lo - start), (uint32_t)(hi - start), slot);
            ++pieces;
        }
        if (split) {
            if (pieces > FA_MAXP) return whole();
            p.merge.push_back(make_uint4(rb, first_slot, pieces, 0));
        }
        start = end;
    }
    return p;
}

void launch_pf_flash(const float* q_ready, const float* q_raw, const KvDev& kv, float* out, uint32_t T, uint32_t pos0,
                     uint32_t nh, uint32_t nkv, uint32_t hd, float scale, const PfFlashLaunch& plan, hipStream_t st) {
    if (nkv == 0 || nh % nkv || nh / nkv > 8 || (hd != 128 && hd != 256))
        throw std::runtime_error("flash prefill takes head_dim 128 or 256 and up to 8 query heads per kv head");
    if (!T) return;
    if (!plan.seg || !plan.W || (plan.nmerge && (!plan.merge || !plan.part)))
        throw std::runtime_error("flash prefill needs its plan");
    PfFlashArgs a{q_ready, q_raw, kv, out, T, pos0, nh, nkv, scale, plan.seg, plan.part, plan.nslots};
    const dim3 grid(plan.W, nkv);
    const dim3 mgrid(plan.nmerge, FA_ROWS, nkv);
#define CHK_FA(HDV)                                                                                      \
    switch (nh / nkv) {                                                                                  \
    case 1: k_pf_flash<HDV, 1><<<grid, 64, 0, st>>>(a); break;                                           \
    case 2: k_pf_flash<HDV, 2><<<grid, 128, 0, st>>>(a); break;                                          \
    case 3: case 4: k_pf_flash<HDV, 4><<<grid, 256, 0, st>>>(a); break;                                  \
    default: k_pf_flash<HDV, 8><<<grid, 512, 0, st>>>(a); break;                                         \
    }                                                                                                    \
    if (plan.nmerge) switch (nh / nkv) {                                                                 \
        case 1: k_pf_flash_merge<1, HDV><<<mgrid, CHK_WG, 0, st>>>(a, plan.merge); break;                \
        case 2: k_pf_flash_merge<2, HDV><<<mgrid, CHK_WG, 0, st>>>(a, plan.merge); break;                \
        case 3: case 4: k_pf_flash_merge<4, HDV><<<mgrid, CHK_WG, 0, st>>>(a, plan.merge); break;        \
        default: k_pf_flash_merge<8, HDV><<<mgrid, CHK_WG, 0, st>>>(a, plan.merge); break;               \
        }
    if (nh / nkv != 1 && nh / nkv != 2 && nh / nkv != 4 && nh / nkv != 8)
        throw std::runtime_error("flash prefill takes 1, 2, 4 or 8 query heads per kv head");
    if (hd == 256) {
        CHK_FA(256)
    } else {
        CHK_FA(128)
    }
#undef CHK_FA
}

}  // namespace chk
