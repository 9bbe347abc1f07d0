// Internal declarations shared by the engine and the kernel translation
// units (not part of the public C ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <string>

#include "cherenkov/synth.h"
#include "cherenkov/types.h"
#include "device.h"

namespace chk {

// last error message of the calling thread (chk_last_error)
extern thread_local std::string g_err;

constexpr int MAX_NB = 4;    // rows per step: one token + up to 3 drafts (gpu.rs:68)
constexpr int MAX_SNAP = 3;  // rollback planes (gpu.rs:70)
constexpr int ATTN_CHUNK = 64;  // tokens per attention partial
constexpr int MAX_ATTN_CHUNKS = 4096;  // context capacity / ATTN_CHUNK (256k tokens)

// Byte layout of one routed-expert record (manifest.rs:21-40 fields).
struct RecordLayout {
    uint32_t bits;
    uint64_t stride, bytes, mat;
    uint64_t gate_w, up_w, down_w, gate_s, gate_b, up_s, up_b, down_s, down_b;
    uint64_t scale_up, scale_down;
};

// Q4 record: pack.rs:351-393 order; Q3/Q2 record: lowbit.rs:81-115.
RecordLayout record_layout(uint32_t bits, uint32_t hidden, uint32_t inter);

struct HcDev {
    const uint16_t* norm;
    Q4Mat down, up, inject;
    int has_inject;
};

struct DnDev {
    Q4Mat qkv, z, a, b, out;
    const uint16_t *conv, *a_log, *dt_bias, *norm;
};

struct AtDev {
    Q4Mat q, k, v, o, idx;
    const uint16_t *q_norm, *k_norm, *idx_q_norm, *idx_k_norm;
};

struct MoeDev {
    const uint16_t* router;
    const uint16_t* shared_gate;
    Q4Mat sh_gate, sh_up, sh_down;
    uint32_t record_layer;
};

// Routed-expert store as seen by the decode kernels.
struct ExpertsDev {
    const uint8_t* base;
    uint64_t stride;
    uint32_t bits, experts;
    uint64_t gate_w, up_w, down_w, gate_s, gate_b, up_s, up_b, down_s, down_b;
};

// Model dimensions the kernels need.
struct Dims {
    uint32_t H, hc, hh, lowrank;
    uint32_t nk, nv, dk, dv, qk_dim, v_dim, conv_dim, ck;
    uint32_t nh, nkv, hd, rot, kv_row;
    uint32_t inh, ihd, idx_out;
    uint32_t ratio, kblk, max_blocks, mask_words;  // QSA blocks (cpu.rs:650-653)
    int qsa;                                       // some context can pass the budget
    uint32_t E, topk, I, SI;
    uint32_t V;
    float eps, theta, attn_scale, qscale;
    int norm_topk;
};

// Per-attention-layer q8 KV cache: int8 planes [max_t][kv_row] and fp16
// scale planes [max_t][kv_row / 32] per side (attention.metal:187-190).
struct KvDev {
    int8_t* k;
    int8_t* v;
    uint16_t* ks;
    uint16_t* vs;
    float* index_k;  // [max_t][ihd]
    float* block_k;  // [max_t / ratio][ihd] QSA block keys: pooled, normed, roped (null while dense)
};

// ----------------------------------------------------------- launchers
void gen_q4(uint32_t* w, uint16_t* s, uint16_t* b, uint32_t out, uint32_t in, uint64_t seed, uint64_t id,
            hipStream_t st);
void gen_bf16(uint16_t* dst, uint64_t n, uint64_t seed, uint64_t id, uint32_t kind, hipStream_t st);
void gen_records(uint8_t* base, const RecordLayout& L, uint64_t seed, uint32_t experts, uint32_t layer0,
                 uint32_t n_layers, uint32_t hidden, uint32_t inter, hipStream_t st);
void repack_lowbit(const uint8_t* q4, const RecordLayout& src, uint8_t* dst, const RecordLayout& lo,
                   uint32_t n_records, uint64_t mat_codes, hipStream_t st);

}  // namespace chk
