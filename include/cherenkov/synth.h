/* Seeded synthetic weights for qwen4_exp-shaped models.
 *
 * No checkpoint is available, so every weight is a pure function of
 * (seed, tensor id, element index).  The same header is compiled by g++ for
 * the CPU oracle and by hipcc for the device generator, so host and device
 * produce identical bytes: only integer arithmetic and single IEEE float
 * multiplies/adds (no contraction) are used.
 *
 * Distributions (the tiny-model config prescribes the quantised ones):
 *   Q4 weight words: 8 uniform nibbles per u32;
 *   Q4 scales  ~ N(0, 0.02) in bf16, Q4 biases ~ N(0, 0.01) in bf16;
 *   router / shared-expert gate vectors ~ N(0, 0.02) bf16;
 *   RMSNorm weights (plain convention) ~ U(0.9, 1.1) bf16;
 *   MTP enorm / hnorm ((1 + w) convention) ~ U(-0.1, 0.1) bf16;
 *   DeltaNet conv1d ~ U(-0.5, 0.5), A_log ~ U(-2, 0.5), dt_bias ~ U(-1, 1).
 * "N(0, s)" is the Irwin-Hall sum of four 16-bit uniforms, centred and
 * scaled to unit variance (support +-3.46 s): exact integer arithmetic plus
 * two rounded float multiplies, hence bit-reproducible everywhere.
 *
 * The element hash is SplitMix64 (Steele, Lea, Flood 2014): the tensor key
 * mixes (seed, tensor id) and element i draws mix64(key + i * golden).
 */
#ifndef CHERENKOV_SYNTH_H
#define CHERENKOV_SYNTH_H

#include <stdint.h>

#if defined(__HIPCC__)
#define CHK_HD __host__ __device__
#else
#define CHK_HD
#endif

#define CHK_GOLDEN 0x9E3779B97F4A7C15ull

/* Tensor kinds.  A tensor id is kind | slot << 8 | expert << 24 | part << 48,
 * where slot is the decoder layer (num_hidden_layers for the MTP layer), and
 * for routed experts `expert` is the expert index and `part` the projection
 * (0 gate, 1 up, 2 down).  Each quantised linear draws three streams
 * (words, scales, biases) from ids with `stream` 0, 1, 2 in bits 56..59. */
enum ChkTensorKind {
    CHK_T_EMBED = 1,
    CHK_T_LM_HEAD,
    CHK_T_HC_NORM,   /* slot: layer; part: 0 attn hc, 1 mlp hc, 2 final, 3 mtp mixer */
    CHK_T_HC_DOWN,
    CHK_T_HC_UP,
    CHK_T_HC_INJECT,
    CHK_T_DN_QKV,
    CHK_T_DN_Z,
    CHK_T_DN_A,
    CHK_T_DN_B,
    CHK_T_DN_CONV,
    CHK_T_DN_ALOG,
    CHK_T_DN_DTBIAS,
    CHK_T_DN_NORM,
    CHK_T_DN_OUT,
    CHK_T_AT_Q,
    CHK_T_AT_K,
    CHK_T_AT_V,
    CHK_T_AT_O,
    CHK_T_AT_QNORM,
    CHK_T_AT_KNORM,
    CHK_T_AT_IDX,
    CHK_T_AT_IDX_QNORM,
    CHK_T_AT_IDX_KNORM,
    CHK_T_MOE_ROUTER,
    CHK_T_MOE_SHARED_GATE,
    CHK_T_MOE_SH_GATE_PROJ,
    CHK_T_MOE_SH_UP,
    CHK_T_MOE_SH_DOWN,
    CHK_T_EXPERT,
    CHK_T_MTP_ENORM,
    CHK_T_MTP_HNORM,
    CHK_T_MTP_FC_E,
    CHK_T_MTP_FC_H,
    /* PLE n-gram block (slot: its decoder layer) */
    CHK_T_PLE_KEY,
    CHK_T_PLE_VALUE,
    CHK_T_PLE_NORM_KEY,
    CHK_T_PLE_NORM_QUERY,
    CHK_T_PLE_NORM_CONV,
    CHK_T_PLE_CONV,
    CHK_T_NGRAM_TABLE, /* rows of (words | scales | biases), ngram.bin layout */
    CHK_T_NGRAM_MULT   /* per-order hash multipliers */
};

enum { CHK_HC_ATTN = 0, CHK_HC_MLP = 1, CHK_HC_FINAL = 2, CHK_HC_MTP = 3 };
enum { CHK_STREAM_W = 0, CHK_STREAM_S = 1, CHK_STREAM_B = 2 };

static inline CHK_HD uint64_t chk_tensor_id(uint32_t kind, uint32_t slot, uint32_t expert,
                                            uint32_t part) {
    return (uint64_t)kind | ((uint64_t)slot << 8) | ((uint64_t)expert << 24) |
           ((uint64_t)part << 48);
}

static inline CHK_HD uint64_t chk_mix64(uint64_t z) {
    z += CHK_GOLDEN;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline CHK_HD uint64_t chk_key(uint64_t seed, uint64_t tensor_id, uint32_t stream) {
    return chk_mix64(seed ^ chk_mix64(tensor_id | ((uint64_t)stream << 56)));
}

static inline CHK_HD uint64_t chk_draw(uint64_t key, uint64_t index) {
    return chk_mix64(key + index * CHK_GOLDEN);
}

static inline CHK_HD uint32_t chk_f32_bits(float f) {
    uint32_t u;
    __builtin_memcpy(&u, &f, 4);
    return u;
}

/* bf16 round-to-nearest-even (the `half` crate's from_f32 rule). */
static inline CHK_HD uint16_t chk_f32_to_bf16(float f) {
    uint32_t u = chk_f32_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static inline CHK_HD float chk_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    __builtin_memcpy(&f, &u, 4);
    return f;
}

/* One u32 of eight uniform 4-bit codes. */
static inline CHK_HD uint32_t chk_q4_word(uint64_t key, uint64_t index) {
    return (uint32_t)(chk_draw(key, index) >> 32);
}

/* Irwin-Hall(4) unit normal, exact up to the final rounded multiply. */
static inline CHK_HD float chk_unit_normal(uint64_t h) {
#ifdef __clang__
#pragma clang fp contract(off)
#endif
    int32_t s = (int32_t)(h & 0xffffu) + (int32_t)((h >> 16) & 0xffffu) +
                (int32_t)((h >> 32) & 0xffffu) + (int32_t)((h >> 48) & 0xffffu);
    /* mean 4 * 65535 / 2, sd 65536 / sqrt(3) */
    return (float)(s - 131070) * 2.6428e-5f;
}

static inline CHK_HD uint16_t chk_normal_bf16(uint64_t key, uint64_t index, float sigma) {
#ifdef __clang__
#pragma clang fp contract(off)
#endif
    float z = chk_unit_normal(chk_draw(key, index));
    return chk_f32_to_bf16(z * sigma);
}

static inline CHK_HD uint16_t chk_uniform_bf16(uint64_t key, uint64_t index, float lo, float hi) {
#ifdef __clang__
#pragma clang fp contract(off)
#endif
    float u = (float)(uint32_t)(chk_draw(key, index) >> 40) * 5.9604645e-8f; /* 2^-24 */
    float span = hi - lo;
    float v = span * u;
    return chk_f32_to_bf16(lo + v);
}

/* Distribution of each bf16 (non-quantised) tensor kind. */
typedef struct ChkDist {
    int uniform; /* 1: U(a, b); 0: N(0, a) */
    float a, b;
} ChkDist;

static inline CHK_HD ChkDist chk_dist(uint32_t kind) {
    ChkDist d;
    d.uniform = 1;
    d.a = 0.9f;
    d.b = 1.1f;
    switch (kind) {
    case CHK_T_MOE_ROUTER:
    case CHK_T_MOE_SHARED_GATE:
        d.uniform = 0; d.a = 0.02f; d.b = 0.0f; break;
    case CHK_T_MTP_ENORM:
    case CHK_T_MTP_HNORM:
        d.a = -0.1f; d.b = 0.1f; break;
    case CHK_T_DN_CONV:
    case CHK_T_PLE_CONV:
        d.a = -0.5f; d.b = 0.5f; break;
    case CHK_T_DN_ALOG:
        d.a = -2.0f; d.b = 0.5f; break;
    case CHK_T_DN_DTBIAS:
        d.a = -1.0f; d.b = 1.0f; break;
    default:
        break; /* RMSNorm weights: U(0.9, 1.1) */
    }
    return d;
}

static inline CHK_HD uint16_t chk_bf16_elem(uint64_t seed, uint64_t tensor_id, uint32_t kind,
                                            uint64_t index) {
    ChkDist d = chk_dist(kind);
    uint64_t key = chk_key(seed, tensor_id, CHK_STREAM_W);
    return d.uniform ? chk_uniform_bf16(key, index, d.a, d.b) : chk_normal_bf16(key, index, d.a);
}

#define CHK_SCALE_SIGMA 0.02f
#define CHK_BIAS_SIGMA 0.01f

/* Synthetic n-gram table (PLE): head h of the table has
 * ngram_head_rows - h rows, heads laid out back to back (head_offsets the
 * running sums); a row holds dim / 8 words of 4-bit codes, then dim / group
 * bf16 scales, then as many biases (manifest.rs:42-55).  Word j of row r is
 * element r * dim / 8 + j of the table's word stream; scale / bias g of row
 * r element r * dim / group + g of its stream.  The hash multipliers are
 * positive odd 63-bit integers. */
static inline CHK_HD uint64_t chk_ngram_head_size(uint32_t head_rows, uint32_t h) {
    return (uint64_t)(head_rows - h);
}

static inline CHK_HD int64_t chk_ngram_multiplier(uint64_t seed, uint32_t k) {
    uint64_t key = chk_key(seed, chk_tensor_id(CHK_T_NGRAM_MULT, 0, 0, 0), CHK_STREAM_W);
    return (int64_t)((chk_draw(key, k) >> 1) | 1u);
}

static inline CHK_HD uint64_t chk_ngram_row_bytes(uint32_t dim, uint32_t group) {
    return (uint64_t)dim / 2 + 4ull * (dim / group);
}

#endif
