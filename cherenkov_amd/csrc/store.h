// The packed-store format of the reference (manifest.json + dense.bin +
// experts.bin beside config.json; src/qwen4_exp/manifest.rs:7-110,
// packed.rs:66-231, pack.rs:351-393) as read by this engine: a minimal JSON
// reader, the store's manifest, the text config, and the reference's
// tensor names for each weight this engine holds.
#pragma once

#include <stdint.h>

#include <map>
#include <memory>
#include <string>
#include <vector>

#include "cherenkov/types.h"

namespace chk {

// ----------------------------------------------------------------- JSON
struct Json {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;

    const Json* get(const std::string& k) const;  // object member or null
    const Json& at(const std::string& k) const;   // throws when absent
    double number() const;
    uint64_t u64() const;
    const std::string& string() const;
};
Json parse_json(const std::string& text);

// ------------------------------------------------------------- manifest
struct DenseEntry {
    std::string dtype;
    std::vector<uint64_t> shape;
    uint64_t offset = 0, nbytes = 0;
};

// ExpertLayout (manifest.rs:18-41)
struct StoreExperts {
    uint64_t layers = 0, experts = 0, inter = 0, hidden = 0, group = 0, record_bytes = 0, record_stride = 0;
    std::vector<std::string> layer_prefixes;
    uint64_t gate_w = 0, up_w = 0, down_w = 0, gate_s = 0, gate_b = 0, up_s = 0, up_b = 0, down_s = 0, down_b = 0;
};

// NgramLayout (manifest.rs:42-55): ngram.bin rows of weight | scales | biases
struct StoreNgram {
    uint64_t rows = 0, row_bytes = 0, dim = 0, group = 0, weight_bytes = 0, scale_bytes = 0;
};

struct Store {
    std::string dir;
    ChkConfig cfg{};
    std::map<std::string, DenseEntry> dense;
    StoreExperts experts;
    StoreNgram ngram;
    const DenseEntry& entry(const std::string& name) const;
};

// Manifest::load + Qwen4ExpConfig::load + the checks Packed::open and
// Gpu::load make (version 1, group 64, layer types, record count).
std::unique_ptr<Store> open_store(const std::string& dir);

// The reference's name of a weight of this engine (tensor kind, decoder
// layer `slot` (num_hidden_layers: the MTP layer), part; synth.h ids).
// Q4 linears name the prefix of their .weight / .scales / .biases.
std::string tensor_name(const ChkConfig& c, uint32_t kind, uint32_t slot, uint32_t part);

}  // namespace chk
