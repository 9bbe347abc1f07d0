// Gated attention decode over the int8 (q8) KV cache.
//
// Reference semantics: attention (cpu.rs:544-641) with the engine's q8 KV
// rule (kv_append_q8, kernels/common/attention.metal:187-234): per 32-lane
// block d = amax/127, q = rint(v/d) clamped to +-127 (0 when d = 0), d kept
// as fp16, dequantised as q * fp16(d).  The split-T flash-decode shape
// (partials (m, l, o) per chunk, then an LSE merge with the sigmoid output
// gate) replaces attn_part2_q8/attn_combine (attention.metal:138-310).
#include <stdexcept>

#include "kernels_internal.h"

namespace chk {

// rms_norm then rope_partial at position `pos` of one vector held one
// element per thread (d < n live), as cpu.rs:575-587 and 676-681 apply them
// to q/k heads and to the indexer's query heads.
CHK_DEV float norm_rope(float x, bool live, uint32_t d, uint32_t n, const uint16_t* w, float eps, uint32_t rot,
                        float theta, uint32_t pos, float* red, float* sx) {
    // the norm weight (raw bf16 in a 32-bit register) and the rotation
    // are fetched and computed ahead of the reduction, not after it
    const uint32_t wv = w[min(d, n - 1)];
    const uint32_t half = rot / 2, j = d < half ? d : d - half;
    float sn = 0.0f, cs = 1.0f;
    if (d < rot) {
        const float inv_freq = powf(theta, -(2.0f * (float)j) / (float)rot);
        const float ang = (float)pos * inv_freq;
        sn = sinf(ang);
        cs = cosf(ang);
    }
    const float ss = block_sum(live ? x * x : 0.0f, red);
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
    if (live) {
        x = x * inv * __uint_as_float(wv << 16);
        sx[d] = x;
    }
    __syncthreads();
    if (d < rot) {
        const float av = sx[j], bv = sx[j + half];
        x = d < half ? av * cs - bv * sn : bv * cs + av * sn;
    }
    return x;
}

// The step batch's form of k_attn_prep below (the same items and the same
// arithmetic, sums in the same order): one CHK_WG-thread
// workgroup per (row, item), thread d < hd owning dim d, which gives a
// decode step's single row the shortest path (a wave per 64 dims).
__global__ void __launch_bounds__(256) k_attn_prep_wg(AttnArgs a) {
    __shared__ float red[8];
    __shared__ float sx[512];
    const uint32_t b = blockIdx.y, item = blockIdx.x, d = threadIdx.x, hd = a.hd;
    const bool live = d < hd;
    const uint32_t pos = a.pos[b];
    const KvDev& kv = a.kv[a.one_kv ? 0 : b];
    if (item == a.nh + 2 * a.nkv) {
        if (d < a.ihd) kv.index_k[(size_t)pos * a.ihd + d] = a.idx_raw[(size_t)b * (a.inh + 1) * a.ihd + a.inh * a.ihd + d];
        return;
    }
    if (item > a.nh + 2 * a.nkv) {
        // select_tokens' query heads (cpu.rs:676-681): index_q_norm, rope at pos
        const uint32_t h = item - (a.nh + 2 * a.nkv + 1);
        const bool il = d < a.ihd;
        const float x0 = il ? a.idx_raw[(size_t)b * (a.inh + 1) * a.ihd + h * a.ihd + d] : 0.0f;
        const float x = norm_rope(x0, il, d, a.ihd, a.iq_norm, a.eps, a.rot, a.theta, pos, red, sx);
        if (il) a.iq_ready[((size_t)b * a.inh + h) * a.ihd + d] = x;
        return;
    }
    const bool is_q = item < a.nh, is_k = !is_q && item < a.nh + a.nkv;
    float x = 0.0f;
    if (live) {
        if (is_q) x = a.q_raw[(size_t)b * a.nh * 2 * hd + item * 2 * hd + d];
        else if (is_k) x = a.k_raw[(size_t)b * a.nkv * hd + (item - a.nh) * hd + d];
        else x = a.v_raw[(size_t)b * a.nkv * hd + (item - a.nh - a.nkv) * hd + d];
    }
    if (is_q || is_k)
        // nn::rms_norm (nn.rs:6-15) then rope_partial (cpu.rs:1051-1063)
        x = norm_rope(x, live, d, hd, is_q ? a.q_norm : a.k_norm, a.eps, a.rot, a.theta, pos, red, sx);
    if (is_q) {
        if (live) a.q_ready[((size_t)b * a.nh + item) * hd + d] = x;
        return;
    }
    // q8: 32-lane blocks are half-waves (dims past hd hold 0 and write nothing)
    float amax = group_max<32>(fabsf(x));
    float dq = amax / 127.0f;
    float qv = dq > 0.0f ? rintf(x / dq) : 0.0f;
    qv = fminf(fmaxf(qv, -127.0f), 127.0f);
    if (!live) return;
    const uint32_t kvh = is_k ? item - a.nh : item - a.nh - a.nkv;
    const uint32_t kv_row = a.nkv * hd;
    int8_t* plane = is_k ? kv.k : kv.v;
    uint16_t* sc = is_k ? kv.ks : kv.vs;
    plane[(size_t)pos * kv_row + kvh * hd + d] = (int8_t)qv;
    if ((d & 31) == 0) sc[(size_t)pos * (kv_row / 32) + (kvh * hd + d) / 32] = __half_as_ushort(__float2half_rn(dq));
}


// rms_norm then rope_partial at position `pos` of one vector of n <= 256
// dims held by a wave, lane l holding dims l + 64 i in x[i] (0 past n), as
// cpu.rs:575-587 and 676-681 apply them to q/k heads and to the indexer's
// query heads.  The sum of squares is summed per 64-dim slab, slabs in
// order; a rotated dim's partner (d -+ rot / 2) comes by a lane permute.
CHK_DEV void wave_norm_rope(float (&x)[4], uint32_t n, const uint16_t* __restrict__ w, float eps, uint32_t rot,
                            float theta, uint32_t pos, uint32_t lane) {
    uint32_t wv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) wv[i] = w[min(64 * i + lane, n - 1)];
    // the rotations, computed ahead of the reduction
    const uint32_t half = rot / 2;
    float sn[4], cs[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t d = 64 * i + lane, j = d < half ? d : d - half;
        sn[i] = 0.0f;
        cs[i] = 1.0f;
        if (64 * i < rot && d < rot) {
            const float inv_freq = powf(theta, -(2.0f * (float)j) / (float)rot);
            const float ang = (float)pos * inv_freq;
            sn[i] = sinf(ang);
            cs[i] = cosf(ang);
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) ss += wave_sum(64 * i + lane < n ? x[i] * x[i] : 0.0f);
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (64 * i + lane < n) x[i] = x[i] * inv * __uint_as_float(wv[i] << 16);
    float y[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        y[i] = x[i];
        if (64 * i >= rot) continue;  // uniform
        const uint32_t d = 64 * i + lane, p = d < half ? d + half : d - half;
        const int lp = (int)(p & 63u);
        // every lane takes part in the permutes; only d < rot uses them
        float xp = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (64 * q >= rot) break;  // uniform: partners lie below rot
            const float v = __shfl(x[q], lp, 64);
            if ((p >> 6) == (uint32_t)q) xp = v;
        }
        if (d < rot) {
            const float av = d < half ? x[i] : xp, bv = d < half ? xp : x[i];
            y[i] = d < half ? av * cs[i] - bv * sn[i] : bv * cs[i] + av * sn[i];
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = y[i];
}

// Per head: q RMSNorm + partial RoPE -> q_ready; k RMSNorm + RoPE -> q8 K
// row; v -> q8 V row; the raw indexer key -> index cache; with QSA the
// indexer's query heads, normed and roped -> iq_ready.  One wave per (row,
// item), four items per workgroup: items [0, nh) q heads, [nh, nh + nkv) k
// heads, [nh + nkv, nh + 2 nkv) v heads, nh + 2 nkv the index key, then inh
// index query heads.  Lane l holds dims l + 64 i, so a q8 block of 32 dims
// is a half-wave.
__global__ void __launch_bounds__(256) k_attn_prep(AttnArgs a) {
    const uint32_t b = blockIdx.y, lane = threadIdx.x & 63, hd = a.hd;
    const uint32_t item = blockIdx.x * (CHK_WG >> 6) + wave_id();
    const uint32_t nkey = a.nh + 2 * a.nkv;
    if (item > nkey + (a.qsa ? a.inh : 0)) return;
    const uint32_t pos = a.pos[b];
    const KvDev& kv = a.kv[a.one_kv ? 0 : b];
    const size_t irow = (size_t)b * (a.inh + 1) * a.ihd;
    float x[4];
    if (item == nkey) {
        for (uint32_t d = lane; d < a.ihd; d += 64) kv.index_k[(size_t)pos * a.ihd + d] = a.idx_raw[irow + a.inh * a.ihd + d];
        return;
    }
    if (item > nkey) {
        // select_tokens' query heads (cpu.rs:676-681): index_q_norm, rope at pos
        const uint32_t h = item - (nkey + 1);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t d = 64 * i + lane;
            x[i] = d < a.ihd ? a.idx_raw[irow + h * a.ihd + d] : 0.0f;
        }
        wave_norm_rope(x, a.ihd, a.iq_norm, a.eps, a.rot, a.theta, pos, lane);
        float* dst = a.iq_ready + ((size_t)b * a.inh + h) * a.ihd;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (64 * i + lane < a.ihd) dst[64 * i + lane] = x[i];
        return;
    }
    const bool is_q = item < a.nh, is_k = !is_q && item < a.nh + a.nkv;
    const float* src = is_q   ? a.q_raw + (size_t)b * a.nh * 2 * hd + item * 2 * hd
                       : is_k ? a.k_raw + (size_t)b * a.nkv * hd + (item - a.nh) * hd
                              : a.v_raw + (size_t)b * a.nkv * hd + (item - a.nh - a.nkv) * hd;
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = 64 * i + lane < hd ? src[64 * i + lane] : 0.0f;
    if (is_q || is_k)
        // nn::rms_norm (nn.rs:6-15) then rope_partial (cpu.rs:1051-1063)
        wave_norm_rope(x, hd, is_q ? a.q_norm : a.k_norm, a.eps, a.rot, a.theta, pos, lane);
    if (is_q) {
        float* dst = a.q_ready + ((size_t)b * a.nh + item) * hd;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (64 * i + lane < hd) dst[64 * i + lane] = x[i];
        return;
    }
    const uint32_t kvh = is_k ? item - a.nh : item - a.nh - a.nkv;
    const uint32_t kv_row = a.nkv * hd;
    int8_t* plane = is_k ? kv.k : kv.v;
    uint16_t* sc = is_k ? kv.ks : kv.vs;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (64 * i >= hd) break;  // uniform; hd is a multiple of 64
        // q8 over the half-wave's 32 dims
        const float amax = group_max<32>(fabsf(x[i]));
        const float dq = amax / 127.0f;
        float qv = dq > 0.0f ? rintf(x[i] / dq) : 0.0f;
        qv = fminf(fmaxf(qv, -127.0f), 127.0f);
        const uint32_t d = 64 * i + lane;
        plane[(size_t)pos * kv_row + kvh * hd + d] = (int8_t)qv;
        if ((d & 31) == 0) sc[(size_t)pos * (kv_row / 32) + (kvh * hd + d) / 32] = __half_as_ushort(__float2half_rn(dq));
    }
}


// ---------------------------------------------------------------- QSA
// select_tokens (cpu.rs:643-719) for rows whose complete blocks exceed the
// budget: blocks of `ratio` tokens, scored by sum_h relu(q_h . key_b) /
// sqrt(ihd) against the block's pooled key (mean of its index keys,
// index_k_norm, rope at the block's first position); the top kblk blocks
// (ties: lowest block) plus the incomplete tail stay visible.
//
// Row b's sequence started this batch at position pos0: rows of one
// sequence are consecutive positions (decode verify rows, prefill rows).
CHK_DEV uint32_t qsa_pos0(const AttnArgs& a, uint32_t b) {
    return (a.one_kv || a.kv[b].index_k == a.kv[0].index_k) ? a.pos[0] : a.pos[b];
}

// Is row b past the budget (selective), and how many complete blocks has it?
CHK_DEV bool qsa_selective(const AttnArgs& a, uint32_t b, uint32_t& nblk) {
    nblk = (a.pos[b] + 1) / a.ratio;
    return a.qsa && nblk > a.kblk;
}

// Block keys and block scores.  A wave takes QSA_BPW blocks of one row;
// lane l holds dims l + 64 i.  A block whose last token arrived in this
// batch gets its key computed here (from the index keys k_attn_prep just
// appended) and cached in block_k; older blocks read the cache.  Rows that
// are still dense only complete keys.
constexpr uint32_t QSA_BPW = 8;
constexpr uint32_t QSA_BPG = QSA_BPW * (CHK_WG / 64);

// The pooled key of block blk (cpu.rs:687-697): mean of its `ratio` index
// keys, rms_norm(index_k_norm), rope at blk * ratio; lane l ends with dims
// l + 64 i in x[i], and the key is stored in block_k.
template <int DPL>
CHK_DEV void qsa_block_key(const AttnArgs& a, const KvDev& kv, uint32_t blk, uint32_t lane, float (&x)[DPL]) {
    const uint32_t half = a.rot / 2;
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < DPL; ++i) {
        const uint32_t d = lane + 64 * i;
        float p = 0.0f;
        for (uint32_t tk = blk * a.ratio; tk < (blk + 1) * a.ratio; ++tk) p += kv.index_k[(size_t)tk * a.ihd + d];
        x[i] = p / (float)a.ratio;
        ss += x[i] * x[i];
    }
    const float inv = 1.0f / sqrtf(wave_sum(ss) / (float)a.ihd + a.eps);
#pragma unroll
    for (int i = 0; i < DPL; ++i) x[i] = x[i] * inv * bf16f(a.ik_norm[lane + 64 * i]);
    // rot <= 64: pair (j, j + half) sits in lanes (l, l ^ half) of slot 0
    const float other = __shfl_xor(x[0], (int)half, 64);
    if (lane < a.rot) {
        const uint32_t jj = lane < half ? lane : lane - half;
        const float inv_freq = powf(a.theta, -(2.0f * (float)jj) / (float)a.rot);
        const float ang = (float)(blk * a.ratio) * inv_freq;
        const float sn = sinf(ang), cs = cosf(ang);
        x[0] = lane < half ? x[0] * cs - other * sn : x[0] * cs + other * sn;
    }
#pragma unroll
    for (int i = 0; i < DPL; ++i) kv.block_k[(size_t)blk * a.ihd + lane + 64 * i] = x[i];
}

// Block keys of blocks [blk0, blk1) (their index keys all appended): a
// prefill chunk's completed blocks, one wave per block.
template <int DPL>
__global__ void __launch_bounds__(256) k_qsa_block_keys(AttnArgs a, uint32_t blk0, uint32_t blk1) {
    const uint32_t blk = blk0 + blockIdx.x * (CHK_WG / 64) + wave_id(), lane = threadIdx.x & 63;
    if (blk >= blk1) return;
    float x[DPL];
    qsa_block_key<DPL>(a, a.kv[0], blk, lane, x);
}

template <int DPL>
__global__ void __launch_bounds__(256) k_qsa_score(AttnArgs a) {
    __shared__ float sq[8 * 256];
    const uint32_t b = blockIdx.y, t = threadIdx.x, lane = t & 63, w = wave_id();
    const KvDev& kv = a.kv[a.one_kv ? 0 : b];
    uint32_t nblk;
    const bool sel = qsa_selective(a, b, nblk);
    const uint32_t pos0 = qsa_pos0(a, b);
    if (sel)
        for (uint32_t i = t; i < a.inh * a.ihd; i += CHK_WG) sq[i] = a.iq_ready[(size_t)b * a.inh * a.ihd + i];
    __syncthreads();
    for (uint32_t j = 0; j < QSA_BPW; ++j) {
        const uint32_t blk = blockIdx.x * QSA_BPG + w * QSA_BPW + j;
        if (blk >= nblk) break;
        const bool fresh = (blk + 1) * a.ratio - 1 >= pos0;
        if (!fresh && !sel) continue;
        float x[DPL];
        if (fresh) {
            qsa_block_key<DPL>(a, kv, blk, lane, x);
        } else {
#pragma unroll
            for (int i = 0; i < DPL; ++i) x[i] = kv.block_k[(size_t)blk * a.ihd + lane + 64 * i];
        }
        if (!sel) continue;
        float s = 0.0f;
        for (uint32_t h = 0; h < a.inh; ++h) {
            float dot = 0.0f;
#pragma unroll
            for (int i = 0; i < DPL; ++i) dot += sq[h * a.ihd + lane + 64 * i] * x[i];
            s += fmaxf(wave_sum(dot), 0.0f);
        }
        if (lane == 0) a.bscore[(size_t)b * a.max_blocks + blk] = s / sqrtf((float)a.ihd);
    }
}

// The top kblk of a row's nblk block scores by (score desc, block asc):
// scores are >= 0, so their bit patterns order like the floats.  A radix
// select over four 8-bit digits finds the kblk-th largest key K and how
// many blocks equal to K to keep; an ordered count over the blocks then
// keeps the lowest-indexed of those.  One 1024-thread workgroup per row;
// vmask gets one bit per selected complete block.
constexpr uint32_t QSA_SEL_WG = 1024;
constexpr uint32_t QSA_MAX_WORDS = 2048;  // 65536 blocks

__global__ void __launch_bounds__(1024) k_qsa_select(AttnArgs a) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t s_key, s_need;
    __shared__ uint32_t wsum[QSA_SEL_WG / 64];
    __shared__ uint32_t mask[QSA_MAX_WORDS];
    const uint32_t b = blockIdx.x, t = threadIdx.x, lane = t & 63, w = t >> 6;
    uint32_t nblk;
    if (!qsa_selective(a, b, nblk)) return;
    const uint32_t* key = reinterpret_cast<const uint32_t*>(a.bscore + (size_t)b * a.max_blocks);
    uint32_t prefix = 0, pmask = 0, need = a.kblk;
    for (int shift = 24; shift >= 0; shift -= 8) {
        if (t < 256) hist[t] = 0;
        __syncthreads();
        for (uint32_t i = t; i < nblk; i += QSA_SEL_WG) {
            const uint32_t k = key[i];
            if ((k & pmask) == prefix) atomicAdd(&hist[(k >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (w == 0) {
            // lane l owns digits 255 - 4l .. 252 - 4l; find the digit where
            // the count from the top reaches `need`
            uint32_t c[4], tot = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                c[i] = hist[255 - 4 * lane - i];
                tot += c[i];
            }
            uint32_t incl = tot;  // inclusive prefix over lanes 0..l (from the top digit down)
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t v = __shfl_up(incl, o, 64);
                if (lane >= (uint32_t)o) incl += v;
            }
            const uint32_t above = incl - tot;
            if (above < need && need <= incl) {
                uint32_t cum = above;
                int i = 0;
                for (; i < 3; ++i) {
                    if (cum + c[i] >= need) break;
                    cum += c[i];
                }
                s_key = prefix | ((255u - 4u * lane - (uint32_t)i) << shift);
                s_need = need - cum;
            }
        }
        __syncthreads();
        prefix = s_key;
        need = s_need;
        pmask |= 255u << shift;
        __syncthreads();
    }
    // keep key > K, and the first `need` blocks (by index) with key == K
    const uint32_t words = (nblk + 31) / 32;
    for (uint32_t i = t; i < words; i += QSA_SEL_WG) mask[i] = 0u;
    const uint32_t seg = (nblk + QSA_SEL_WG - 1) / QSA_SEL_WG;
    const uint32_t lo = min(t * seg, nblk), hi = min(lo + seg, nblk);
    uint32_t eq = 0;
    for (uint32_t i = lo; i < hi; ++i) eq += key[i] == prefix;
    // exclusive count of equal keys before this thread's segment
    uint32_t incl = eq;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t v = __shfl_up(incl, o, 64);
        if (lane >= (uint32_t)o) incl += v;
    }
    if (lane == 63) wsum[w] = incl;
    __syncthreads();
    uint32_t before = incl - eq;
    for (uint32_t k = 0; k < w; ++k) before += wsum[k];
    for (uint32_t i = lo; i < hi; ++i) {
        const uint32_t k = key[i];
        bool keep = k > prefix;
        if (k == prefix) {
            keep = before < need;
            ++before;
        }
        if (keep) atomicOr(&mask[i >> 5], 1u << (i & 31));
    }
    __syncthreads();
    for (uint32_t i = t; i < words; i += QSA_SEL_WG) a.vmask[(size_t)b * a.mask_words + i] = mask[i];
}

CHK_DEV float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }

// Partials over one chunk of ATTN_CHUNK tokens for (row b, kv head hk):
// the G = nh / nkv query heads that share the kv head are served from one
// read of the chunk's K and V.  Every K and V load of the workgroup is
// issued before any arithmetic, so the kernel pays one memory latency.
//
// Scores: 4 threads per token, each a quarter of the head dims (HD / 4,
// i.e. HD / 128 q8 blocks of 32).  P.V: lanes own 4 consecutive dims (one
// u32 of int8 values), NS = 256 / (HD / 4) token slots stride the chunk,
// and the slots are summed through LDS.
template <int G, int HD>
__global__ void __launch_bounds__(256) k_attn_part(AttnArgs a) {
    constexpr int CH = ATTN_CHUNK;          // tokens per chunk (64)
    constexpr int DPT = HD / 4;             // score dims per thread
    constexpr int KB = DPT / 32;            // q8 blocks per thread
    constexpr int QP = HD + 16;             // padded q row (bank spread)
    constexpr int LPV = HD / 4;             // P.V lanes per token
    constexpr int NS = 256 / LPV;           // P.V token slots
    constexpr int TPS = CH / NS;            // tokens per slot
    static_assert(CH * 4 == 256, "one thread quarter per token");
    __shared__ __align__(16) float sq[G][QP];
    __shared__ float sp[G][CH];
    __shared__ float sml[G][2];
    __shared__ __align__(16) float so[NS][G][HD];
    // x = (kv head, slice of G of its query heads): a kv head's query heads
    // may be split over several workgroups for parallelism.  Workgroups are
    // dealt to the 8 XCDs round-robin by linear id; the ids are remapped so
    // that the gridDim.x workgroups of one (chunk, row) sit 8 apart, on one
    // XCD, and the kv heads' chunks come from HBM once into that XCD's L2
    // (the ids past the last whole span of 8 gridDim.x keep their places).
    uint32_t x = blockIdx.x, yz = blockIdx.z * gridDim.y + blockIdx.y;
    const uint32_t split = (a.nh / a.nkv) / G;
    const uint32_t hk = x / split, h0 = hk * (a.nh / a.nkv) + (x % split) * G;
    const uint32_t c = yz % gridDim.y, b = yz / gridDim.y, t = threadIdx.x;
    const uint32_t T = a.pos[b] + 1;  // causal: rows see positions <= their own
    const uint32_t t0 = c * CH;
    if (t0 >= T) return;
    // QSA: past the budget only the selected complete blocks and the tail
    uint32_t nblk;
    const bool sel = qsa_selective(a, b, nblk);
    const KvDev& kv = a.kv[a.one_kv ? 0 : b];
    const uint32_t kv_row = a.nkv * HD, n = min((uint32_t)CH, T - t0);

    // ---- issue: q of the G heads first (written by the previous kernel;
    // loads return in issue order, so behind the cache rows its LDS
    // staging would wait for all of them), then K quarter-rows, V u32
    // lanes and their fp16 scales (raw, one per 32-bit register)
    constexpr uint32_t QI = (G * HD + 255) / 256;
    float qreg[QI];
#pragma unroll
    for (uint32_t j = 0; j < QI; ++j) {
        const uint32_t i = min(t + 256 * j, (uint32_t)(G * HD) - 1);
        qreg[j] = a.q_ready[((size_t)b * a.nh + h0 + i / HD) * HD + i % HD];
    }
    asm volatile("" ::: "memory");  // compiler-only: the cache loads stay behind q
    const uint32_t tk = t >> 2, qq = t & 3;
    const uint32_t ktok = t0 + min(tk, n - 1);
    uint4 kw[KB][2];
    uint32_t ksc[KB];
#pragma unroll
    for (int k = 0; k < KB; ++k) {
        const uint32_t d0 = qq * DPT + k * 32;
        const uint4* kp = reinterpret_cast<const uint4*>(kv.k + (size_t)ktok * kv_row + hk * HD + d0);
        kw[k][0] = kp[0];
        kw[k][1] = kp[1];
        ksc[k] = kv.ks[(size_t)ktok * (kv_row / 32) + (hk * HD + d0) / 32];
    }
    const uint32_t slot = t / LPV, vl = t % LPV;
    uint32_t vw[TPS];
    uint32_t vsc[TPS];
#pragma unroll
    for (int i = 0; i < TPS; ++i) {
        const uint32_t vt = t0 + min(slot + (uint32_t)(i * NS), n - 1);
        vw[i] = *reinterpret_cast<const uint32_t*>(kv.v + (size_t)vt * kv_row + hk * HD + vl * 4);
        vsc[i] = kv.vs[(size_t)vt * (kv_row / 32) + (hk * HD + vl * 4) / 32];
    }
    // q of the G heads into LDS
#pragma unroll
    for (uint32_t j = 0; j < QI; ++j) asm volatile("" : "+v"(qreg[j])::"memory");
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (uint32_t j = 0; j < QI; ++j) {
        const uint32_t i = t + 256 * j;
        if (i < (uint32_t)(G * HD)) {
            const uint32_t g = i / HD, d = i % HD;
            sq[g][(d / DPT) * (DPT + 4) + d % DPT] = qreg[j];
        }
    }
    __syncthreads();

    // ---- scores: s[g][tk] = scale * sum_blocks fp16(ks) * (q . k_int8)
    float kf[KB][32];
#pragma unroll
    for (int k = 0; k < KB; ++k) {
        const uint32_t w[8] = {kw[k][0].x, kw[k][0].y, kw[k][0].z, kw[k][0].w,
                               kw[k][1].x, kw[k][1].y, kw[k][1].z, kw[k][1].w};
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) kf[k][j * 4 + e] = (float)(int8_t)(w[j] >> (8 * e));
    }
    bool vis = true;
    if (sel) {
        const uint32_t tok = t0 + tk, blk = tok / a.ratio;
        vis = blk >= nblk || ((a.vmask[(size_t)b * a.mask_words + (blk >> 5)] >> (blk & 31)) & 1u);
    }
#pragma unroll 1
    for (int g = 0; g < G; ++g) {
        float v = 0.0f;
#pragma unroll
        for (int k = 0; k < KB; ++k) {
            const float4* qp = reinterpret_cast<const float4*>(&sq[g][qq * (DPT + 4) + k * 32]);
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float4 qv = qp[j];
                acc += qv.x * kf[k][4 * j] + qv.y * kf[k][4 * j + 1] + qv.z * kf[k][4 * j + 2] + qv.w * kf[k][4 * j + 3];
            }
            v += acc * h2f(ksc[k]);
        }
        v += __shfl_xor(v, 1);
        v += __shfl_xor(v, 2);
        if (qq == 0) sp[g][tk] = tk < n && vis ? v * a.scale : -INFINITY;
    }
    __syncthreads();

    // ---- per-head chunk softmax numerators: wave w takes heads w, w + 4, ...
    const uint32_t wv = t >> 6, lane = t & 63;
    for (uint32_t g = wv; g < (uint32_t)G; g += 4) {
        const float s = sp[g][lane];
        const float m = wave_max(s);
        // a chunk may hold no visible token (QSA): then m = -inf and p = 0
        const float p = lane < n && s != -INFINITY ? expf(s - m) : 0.0f;
        sp[g][lane] = p;
        const float l = wave_sum(p);
        if (lane == 0) {
            sml[g][0] = m;
            sml[g][1] = l;
        }
    }
    __syncthreads();

    // ---- P.V over this slot's tokens
    float o[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) o[g][e] = 0.0f;
#pragma unroll
    for (int i = 0; i < TPS; ++i) {
        const uint32_t j = slot + i * NS;
        const float ds = h2f(vsc[i]);
        float vf[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) vf[e] = (float)(int8_t)(vw[i] >> (8 * e)) * ds;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float p = sp[g][j];  // 0 past the chunk's valid tokens
#pragma unroll
            for (int e = 0; e < 4; ++e) o[g][e] += p * vf[e];
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
        *reinterpret_cast<float4*>(&so[slot][g][vl * 4]) = make_float4(o[g][0], o[g][1], o[g][2], o[g][3]);
    __syncthreads();
    for (uint32_t i = t; i < (uint32_t)(G * HD); i += 256) {
        const uint32_t g = i / HD, d = i % HD;
        float acc = 0.0f;
#pragma unroll
        for (int s2 = 0; s2 < NS; ++s2) acc += so[s2][g][d];
        float* part = a.part + (((size_t)b * a.nh + h0 + g) * a.max_chunks + c) * (HD + 2);
        part[2 + d] = acc;
        if (d == 0) {
            part[0] = sml[g][0];
            part[1] = sml[g][1];
        }
    }
}

// LSE merge of the chunk partials and the per-dim sigmoid gate
// (cpu.rs:629-633: the gate is the second half of each head's q_proj rows).
// COMBINE_SPLIT workgroups per head each own hd / COMBINE_SPLIT dims; every
// one forms the chunk weights exp(m_c - M) in LDS, then its waves sum
// interleaved chunks for its dims (8 loads in flight) and meet in LDS.
constexpr uint32_t COMBINE_SPLIT = 4;

__global__ void __launch_bounds__(256) k_attn_combine(AttnArgs a) {
    __shared__ float red[8];
    __shared__ float sw[MAX_ATTN_CHUNKS];
    __shared__ float acc_s[4][64];
    const uint32_t h = blockIdx.x / COMBINE_SPLIT, ds = blockIdx.x % COMBINE_SPLIT, b = blockIdx.y, hd = a.hd,
                   t = threadIdx.x;
    const uint32_t T = a.pos[b] + 1, nc = (T + ATTN_CHUNK - 1) / ATTN_CHUNK;
    const float* part = a.part + ((size_t)b * a.nh + h) * a.max_chunks * (hd + 2);
    const uint32_t per = hd / COMBINE_SPLIT;  // dims of this workgroup (<= 64)
    const uint32_t dl = t & 63, cg = t >> 6;
    const uint32_t d = ds * per + dl;
    const float* pd = part + 2 + d;
    // The first chunk's (max, sum) of this thread, the first 32 chunks'
    // partial outputs of its dimension and the gate load together, ahead
    // of any use (branch-free, clamped): one round trip instead of one
    // per pass.  Longer contexts continue in the loops below.
    const uint32_t tc = min(t, nc - 1), dc = min(d, hd - 1);
    const float m0 = part[(size_t)tc * (hd + 2)], l0 = part[(size_t)tc * (hd + 2) + 1];
    float v0[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v0[k] = part[2 + dc + (size_t)min(cg + 4 * k, nc - 1) * (hd + 2)];
    const float gate = a.q_raw[(size_t)b * a.nh * 2 * hd + h * 2 * hd + hd + dc];
    asm volatile("" ::: "memory");  // compiler-only: later loads stay behind these
    float m = t < nc ? m0 : -INFINITY;
    for (uint32_t c = t + CHK_WG; c < nc; c += CHK_WG) m = fmaxf(m, part[(size_t)c * (hd + 2)]);
    const float M = block_max(m, red);
    float l = 0.0f;
    if (t < nc) {
        const float w = expf(m0 - M);
        sw[t] = w;
        l += l0 * w;
    }
    for (uint32_t c = t + CHK_WG; c < nc; c += CHK_WG) {
        const float w = expf(part[(size_t)c * (hd + 2)] - M);
        sw[c] = w;
        l += part[(size_t)c * (hd + 2) + 1] * w;
    }
    const float L = block_sum(l, red);  // its barriers also publish sw
    float o = 0.0f;
    if (dl < per) {
        uint32_t c = cg;
        if (c + 28 < nc) {
#pragma unroll
            for (int k = 0; k < 8; ++k) o += v0[k] * sw[c + 4 * k];
            c += 32;
        }
        // long contexts: 32 loads in flight per round trip (the same
        // ascending chunk order as the 8-wide rounds)
        for (; c + 124 < nc; c += 128) {
            float v[32];
#pragma unroll
            for (int k = 0; k < 32; ++k) v[k] = pd[(size_t)(c + 4 * k) * (hd + 2)];
#pragma unroll
            for (int k = 0; k < 32; ++k) o += v[k] * sw[c + 4 * k];
        }
        for (; c + 28 < nc; c += 32) {
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = pd[(size_t)(c + 4 * k) * (hd + 2)];
#pragma unroll
            for (int k = 0; k < 8; ++k) o += v[k] * sw[c + 4 * k];
        }
        for (; c < nc; c += 4) o += pd[(size_t)c * (hd + 2)] * sw[c];
    }
    acc_s[cg][dl] = o;
    __syncthreads();
    if (cg == 0 && dl < per) {
        const float ot = (acc_s[0][dl] + acc_s[1][dl]) + (acc_s[2][dl] + acc_s[3][dl]);
        a.out[(size_t)b * a.nh * hd + h * hd + d] = ot / L * sigmoidf_(gate);
    }
}

__global__ void __launch_bounds__(256) k_copy_f32(float* __restrict__ dst, const float* __restrict__ src, uint64_t n) {
    uint64_t stride = (uint64_t)gridDim.x * CHK_WG;
    for (uint64_t i = (uint64_t)blockIdx.x * CHK_WG + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

__global__ void __launch_bounds__(256) k_zero_f32(float* __restrict__ dst, uint64_t n) {
    uint64_t stride = (uint64_t)gridDim.x * CHK_WG;
    for (uint64_t i = (uint64_t)blockIdx.x * CHK_WG + threadIdx.x; i < n; i += stride) dst[i] = 0.0f;
}

__global__ void __launch_bounds__(256) k_fill_u8(uint8_t* __restrict__ dst, uint8_t v, uint64_t n) {
    uint64_t stride = (uint64_t)gridDim.x * CHK_WG;
    for (uint64_t i = (uint64_t)blockIdx.x * CHK_WG + threadIdx.x; i < n; i += stride) dst[i] = v;
}

// Positions come from device memory and the chunk grid covers the whole
// context capacity (chunks past a row's length exit at once), so the
// launch is the same every step and can live in a captured graph.
bool attn_shape_ok(uint32_t nh, uint32_t nkv, uint32_t hd) {
    if (nkv == 0 || nh % nkv || (hd != 128 && hd != 256)) return false;
    const uint32_t g = nh / nkv;
    return g == 1 || g == 2 || g == 4 || g == 8 || g == 12;
}

void launch_attn_core(const AttnArgs& a, int nb, hipStream_t st) {
    const uint32_t g = a.nh / a.nkv, gw = g < 4 ? g : 4;
    if (g % gw) throw std::runtime_error("query heads per kv head must be 1, 2, 4, 8 or 12");
    if (a.hd % COMBINE_SPLIT || a.hd / COMBINE_SPLIT > 64) throw std::runtime_error("head_dim 128 or 256");
    const dim3 grid(a.nkv * (g / gw), a.max_chunks, nb);
// query heads per partial workgroup: at most 4 (a kv head with 8 or 12
// query heads is split over 2 or 3 workgroups that read the same chunk)
#define CHK_ATTN_G(HDV)                                                              \
    switch (gw) {                                                                    \
    case 1: k_attn_part<1, HDV><<<grid, 256, 0, st>>>(a); break;                     \
    case 2: k_attn_part<2, HDV><<<grid, 256, 0, st>>>(a); break;                     \
    default: k_attn_part<4, HDV><<<grid, 256, 0, st>>>(a); break;                    \
    }
    if (a.hd == 128) {
        CHK_ATTN_G(128)
    } else {
        CHK_ATTN_G(256)
    }
#undef CHK_ATTN_G
    k_attn_combine<<<dim3(a.nh * COMBINE_SPLIT, nb), 256, 0, st>>>(a);
}

void launch_attn_prep(const AttnArgs& a, int nb, hipStream_t st) {
    if (nb > MAX_NB && !a.one_kv) throw std::runtime_error("rows beyond the step batch must share one sequence");
    if (a.hd > 256 || a.hd % 64 || a.ihd > 256 || a.rot > a.hd || (a.qsa && a.rot > a.ihd))
        throw std::runtime_error("attention heads of at most 256 dims (a multiple of 64), rotation within the head");
    const uint32_t items = a.nh + 2 * a.nkv + 1 + (a.qsa ? a.inh : 0);
    // a step batch: a workgroup per item (latency); prefill rows: a wave per
    // item (four per workgroup)
    if (nb <= MAX_NB) k_attn_prep_wg<<<dim3(items, nb), CHK_WG, 0, st>>>(a);
    else k_attn_prep<<<dim3((items + 3) / 4, nb), CHK_WG, 0, st>>>(a);
}

// Block keys, scores and selection; a no-op for rows still within the budget
// (their block keys are still cached as blocks complete).
void launch_qsa(const AttnArgs& a, int nb, hipStream_t st) {
    if (!a.qsa) return;
    // DPL = ihd / 64 dims per lane: 1, 2 or 4 (no 3-dim instantiation)
    if ((a.ihd != 64 && a.ihd != 128 && a.ihd != 256) || a.rot > 64 || a.rot > a.ihd || (a.rot & (a.rot - 1)) ||
        a.rot < 2 ||
        a.inh * a.ihd > 8 * 256 ||
        a.mask_words > QSA_MAX_WORDS || !a.iq_ready || !a.bscore || !a.vmask || !a.kv[0].block_k)
        throw std::runtime_error("QSA indexer shape not supported");
    const dim3 grid((a.max_blocks + QSA_BPG - 1) / QSA_BPG, nb);
    switch (a.ihd / 64) {
    case 1: k_qsa_score<1><<<grid, CHK_WG, 0, st>>>(a); break;
    case 2: k_qsa_score<2><<<grid, CHK_WG, 0, st>>>(a); break;
    default: k_qsa_score<4><<<grid, CHK_WG, 0, st>>>(a); break;
    }
    k_qsa_select<<<nb, QSA_SEL_WG, 0, st>>>(a);
}

void launch_qsa_block_keys(const AttnArgs& a, uint32_t blk0, uint32_t blk1, hipStream_t st) {
    if (blk1 <= blk0) return;
    if ((a.ihd != 64 && a.ihd != 128 && a.ihd != 256) || a.rot > 64 || !a.kv[0].block_k)
        throw std::runtime_error("QSA indexer shape not supported");
    const uint32_t grid = (blk1 - blk0 + CHK_WG / 64 - 1) / (CHK_WG / 64);
    switch (a.ihd / 64) {
    case 1: k_qsa_block_keys<1><<<grid, CHK_WG, 0, st>>>(a, blk0, blk1); break;
    case 2: k_qsa_block_keys<2><<<grid, CHK_WG, 0, st>>>(a, blk0, blk1); break;
    default: k_qsa_block_keys<4><<<grid, CHK_WG, 0, st>>>(a, blk0, blk1); break;
    }
}

void launch_qsa_select(const AttnArgs& a, int nb, hipStream_t st) {
    if (a.mask_words > QSA_MAX_WORDS) throw std::runtime_error("more QSA blocks than one selection workgroup holds");
    k_qsa_select<<<nb, QSA_SEL_WG, 0, st>>>(a);
}

void launch_attn(const AttnArgs& a, int nb, hipStream_t st) {
    launch_attn_prep(a, nb, st);
    launch_qsa(a, nb, st);
    launch_attn_core(a, nb, st);
}

void launch_copy_f32(float* dst, const float* src, uint64_t n, hipStream_t st) {
    uint32_t grid = (uint32_t)std::min<uint64_t>((n + 255) / 256, 2048);
    if (n) k_copy_f32<<<grid, 256, 0, st>>>(dst, src, n);
}

void launch_zero_f32(float* dst, uint64_t n, hipStream_t st) {
    uint32_t grid = (uint32_t)std::min<uint64_t>((n + 255) / 256, 2048);
    if (n) k_zero_f32<<<grid, 256, 0, st>>>(dst, n);
}

void launch_fill_u8(uint8_t* dst, uint8_t v, uint64_t n, hipStream_t st) {
    uint32_t grid = (uint32_t)std::min<uint64_t>((n + 255) / 256, 2048);
    if (n) k_fill_u8<<<grid, 256, 0, st>>>(dst, v, n);
}

}  // namespace chk
