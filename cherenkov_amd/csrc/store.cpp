// Reading the reference's packed store: JSON, manifest, text config and
// tensor names (see store.h).
#include "store.h"

#include <sys/stat.h>

#include <cstring>

#include <cmath>
#include <cstdio>
#include <fstream>
#include <sstream>
#include <stdexcept>

#include "cherenkov/synth.h"

namespace chk {

static void fail(const std::string& msg) { throw std::runtime_error(msg); }

// ------------------------------------------------------------------ JSON
// A recursive-descent reader of RFC 8259 JSON (no comments, no trailing
// commas); numbers as doubles, strings with the standard escapes.
namespace {
struct Reader {
    const std::string& t;
    size_t i = 0;
    explicit Reader(const std::string& s) : t(s) {}
    void ws() {
        while (i < t.size() && (t[i] == ' ' || t[i] == '\n' || t[i] == '\r' || t[i] == '\t')) ++i;
    }
    char peek() {
        ws();
        if (i >= t.size()) fail("JSON: unexpected end");
        return t[i];
    }
    void expect(char c) {
        if (peek() != c) fail(std::string("JSON: expected '") + c + "' at byte " + std::to_string(i));
        ++i;
    }
    bool literal(const char* w) {
        const size_t n = strlen(w);
        if (t.compare(i, n, w) == 0) {
            i += n;
            return true;
        }
        return false;
    }
    static void utf8(std::string& out, uint32_t cp) {
        if (cp < 0x80) out += (char)cp;
        else if (cp < 0x800) {
            out += (char)(0xC0 | (cp >> 6));
            out += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            out += (char)(0xE0 | (cp >> 12));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
        } else {
            out += (char)(0xF0 | (cp >> 18));
            out += (char)(0x80 | ((cp >> 12) & 0x3F));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
        }
    }
    uint32_t hex4() {
        if (i + 4 > t.size()) fail("JSON: short \\u escape");
        uint32_t v = 0;
        for (int k = 0; k < 4; ++k) {
            const char c = t[i++];
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else fail("JSON: bad \\u escape");
        }
        return v;
    }
    std::string str() {
        expect('"');
        std::string out;
        while (true) {
            if (i >= t.size()) fail("JSON: unterminated string");
            const char c = t[i++];
            if (c == '"') break;
            if (c != '\\') {
                out += c;
                continue;
            }
            if (i >= t.size()) fail("JSON: unterminated escape");
            const char e = t[i++];
            switch (e) {
            case '"': out += '"'; break;
            case '\\': out += '\\'; break;
            case '/': out += '/'; break;
            case 'b': out += '\b'; break;
            case 'f': out += '\f'; break;
            case 'n': out += '\n'; break;
            case 'r': out += '\r'; break;
            case 't': out += '\t'; break;
            case 'u': {
                uint32_t cp = hex4();
                if (cp >= 0xD800 && cp < 0xDC00 && i + 1 < t.size() && t[i] == '\\' && t[i + 1] == 'u') {
                    i += 2;
                    const uint32_t lo = hex4();
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                }
                utf8(out, cp);
                break;
            }
            default: fail("JSON: bad escape");
            }
        }
        return out;
    }
    Json value() {
        Json v;
        const char c = peek();
        if (c == '{') {
            ++i;
            v.kind = Json::OBJ;
            if (peek() == '}') {
                ++i;
                return v;
            }
            while (true) {
                std::string k = str();
                expect(':');
                v.obj.emplace_back(std::move(k), value());
                if (peek() == ',') {
                    ++i;
                    continue;
                }
                expect('}');
                return v;
            }
        }
        if (c == '[') {
            ++i;
            v.kind = Json::ARR;
            if (peek() == ']') {
                ++i;
                return v;
            }
            while (true) {
                v.arr.push_back(value());
                if (peek() == ',') {
                    ++i;
                    continue;
                }
                expect(']');
                return v;
            }
        }
        if (c == '"') {
            v.kind = Json::STR;
            v.str = str();
            return v;
        }
        if (literal("true")) {
            v.kind = Json::BOOL;
            v.b = true;
            return v;
        }
        if (literal("false")) {
            v.kind = Json::BOOL;
            return v;
        }
        if (literal("null")) return v;
        const size_t s = i;
        if (t[i] == '-') ++i;
        while (i < t.size() && (isdigit((unsigned char)t[i]) || t[i] == '.' || t[i] == 'e' || t[i] == 'E' ||
                                t[i] == '+' || t[i] == '-'))
            ++i;
        if (s == i) fail("JSON: unexpected character at byte " + std::to_string(i));
        v.kind = Json::NUM;
        v.num = std::stod(t.substr(s, i - s));
        return v;
    }
};
}  // namespace

Json parse_json(const std::string& text) {
    Reader r(text);
    Json v = r.value();
    r.ws();
    if (r.i != text.size()) fail("JSON: trailing data");
    return v;
}

const Json* Json::get(const std::string& k) const {
    if (kind != OBJ) return nullptr;
    for (const auto& kv : obj)
        if (kv.first == k) return &kv.second;
    return nullptr;
}
const Json& Json::at(const std::string& k) const {
    const Json* v = get(k);
    if (!v) fail("missing field \"" + k + "\"");
    return *v;
}
double Json::number() const {
    if (kind == BOOL) return b ? 1.0 : 0.0;
    if (kind != NUM) fail("expected a number");
    return num;
}
uint64_t Json::u64() const {
    const double v = number();
    if (v < 0 || v != std::floor(v)) fail("expected a non-negative integer");
    // every integer up to 2^53 is exact in the double it was parsed into;
    // above that the value is not the manifest's and the cast may overflow
    if (v > 9007199254740992.0) fail("integer above 2^53");
    return (uint64_t)v;
}
const std::string& Json::string() const {
    if (kind != STR) fail("expected a string");
    return str;
}

// ---------------------------------------------------------------- store
static bool is_file(const std::string& p) {
    struct stat st;
    return stat(p.c_str(), &st) == 0 && S_ISREG(st.st_mode);
}

static std::string read_text(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) fail("reading " + path);
    std::ostringstream ss;
    ss << f.rdbuf();
    return ss.str();
}

const DenseEntry& Store::entry(const std::string& name) const {
    auto it = dense.find(name);
    if (it == dense.end()) fail("dense tensor \"" + name + "\" not in manifest");
    return it->second;
}

static uint32_t u32f(const Json& j, const char* k) {
    const uint64_t v = j.at(k).u64();
    if (v > 0xffffffffu) fail(std::string(k) + " out of range");
    return (uint32_t)v;
}
static uint32_t u32d(const Json& j, const char* k, uint32_t dflt) { return j.get(k) ? u32f(j, k) : dflt; }

// Qwen4ExpConfig::load (config.rs:93-122) into ChkConfig: layer_types
// becomes the attention interval (layer l is attention iff
// (l + 1) % interval == 0, checked), ple_layer_ids' first id is kept
// (1-based, 0 = none).
static ChkConfig read_config(const std::string& path) {
    const Json root = parse_json(read_text(path));
    const std::string& mt = root.at("model_type").string();
    if (mt != "qwen4_exp" && mt != "qwen4_exp_text") fail("unsupported model_type " + mt + "; expected qwen4_exp");
    const Json& t = root.get("text_config") ? root.at("text_config") : root;
    if (!t.get("model_type") || t.at("model_type").string() != "qwen4_exp_text")
        fail("expected qwen4_exp_text configuration");
    ChkConfig c{};
    c.hidden_size = u32f(t, "hidden_size");
    c.num_hidden_layers = u32f(t, "num_hidden_layers");
    c.vocab_size = u32f(t, "vocab_size");
    c.num_attention_heads = u32f(t, "num_attention_heads");
    c.num_key_value_heads = u32f(t, "num_key_value_heads");
    c.head_dim = u32f(t, "head_dim");
    c.linear_num_key_heads = u32f(t, "linear_num_key_heads");
    c.linear_num_value_heads = u32f(t, "linear_num_value_heads");
    c.linear_key_head_dim = u32f(t, "linear_key_head_dim");
    c.linear_value_head_dim = u32f(t, "linear_value_head_dim");
    c.linear_conv_kernel_dim = u32f(t, "linear_conv_kernel_dim");
    c.hc_count = u32d(t, "hc_count", 4);
    c.hc_lowrank = u32d(t, "hc_lowrank", 320);
    c.num_experts = u32f(t, "num_experts");
    c.num_experts_per_tok = u32f(t, "num_experts_per_tok");
    c.moe_intermediate_size = u32f(t, "moe_intermediate_size");
    c.shared_expert_intermediate_size = u32f(t, "shared_expert_intermediate_size");
    c.norm_topk_prob = t.get("norm_topk_prob") ? (t.at("norm_topk_prob").number() != 0 ? 1u : 0u) : 1u;
    c.indexer_n_heads = u32f(t, "indexer_n_heads");
    c.indexer_head_dim = u32f(t, "indexer_head_dim");
    c.indexer_budget = u32f(t, "indexer_budget");
    c.indexer_compress_ratio = u32f(t, "indexer_compress_ratio");
    c.mtp_num_hidden_layers = u32d(t, "mtp_num_hidden_layers", 0);
    c.eos_token_id = u32f(t, "eos_token_id");
    c.rms_norm_eps = t.at("rms_norm_eps").number();
    c.partial_rotary_factor = t.at("partial_rotary_factor").number();
    c.rope_theta = t.at("rope_parameters").at("rope_theta").number();
    c.seed = 0;
    const std::string gate = t.get("output_gate_type") ? t.at("output_gate_type").string() : "silu";
    if (gate != "sigmoid") fail("output_gate_type must be sigmoid (gpu/load.rs:49-52)");
    if (const Json* ple = t.get("ple_layer_ids"); ple && ple->kind == Json::ARR && !ple->arr.empty())
        c.ple_layer = (uint32_t)ple->arr[0].u64();
    // config.rs:36-43 (ple_embed_dim has no default there)
    c.ple_embed_dim = u32f(t, "ple_embed_dim");
    c.ple_conv_kernel_size = u32d(t, "ple_conv_kernel_size", 4);
    c.ngram_size = u32d(t, "ngram_size", 3);
    c.heads_per_ngram = u32d(t, "heads_per_ngram", 8);
    const Json& lt = t.at("layer_types");
    if (lt.kind != Json::ARR || lt.arr.size() != c.num_hidden_layers) fail("layer_types length mismatch");
    uint32_t interval = 0;
    for (uint32_t l = 0; l < c.num_hidden_layers; ++l)
        if (lt.arr[l].string() != "linear_attention") {
            interval = l + 1;
            break;
        }
    if (!interval) interval = c.num_hidden_layers + 1;  // every layer linear
    for (uint32_t l = 0; l < c.num_hidden_layers; ++l) {
        const bool linear = lt.arr[l].string() == "linear_attention";
        if (linear != ((l + 1) % interval != 0))
            fail("layer_types must repeat (linear_attention x k, then full attention): layer " + std::to_string(l));
    }
    c.full_attention_interval = interval;
    if (c.hc_count <= 1) fail("hc_count must exceed 1");
    return c;
}

std::unique_ptr<Store> open_store(const std::string& model_dir) {
    auto S = std::make_unique<Store>();
    // Packed::open (packed.rs:66-100): the packed files live in the model
    // directory or its packed/ subdirectory; config.json beside them wins
    S->dir = is_file(model_dir + "/manifest.json") ? model_dir : model_dir + "/packed";
    const std::string cfg_path =
        is_file(S->dir + "/config.json") ? S->dir + "/config.json" : model_dir + "/config.json";
    S->cfg = read_config(cfg_path);
    const Json m = parse_json(read_text(S->dir + "/manifest.json"));
    if (m.at("version").u64() != 1)
        fail("unsupported packed layout version " + std::to_string(m.at("version").u64()));
    for (const Json& e : m.at("dense").arr) {
        DenseEntry d;
        d.dtype = e.at("dtype").string();
        for (const Json& x : e.at("shape").arr) d.shape.push_back(x.u64());
        d.offset = e.at("offset").u64();
        d.nbytes = e.at("nbytes").u64();
        S->dense[e.at("name").string()] = d;
    }
    const Json& x = m.at("experts");
    StoreExperts& X = S->experts;
    X.layers = x.at("layers").u64();
    X.experts = x.at("experts").u64();
    X.inter = x.at("inter").u64();
    X.hidden = x.at("hidden").u64();
    X.group = x.at("group").u64();
    X.record_bytes = x.at("record_bytes").u64();
    X.record_stride = x.at("record_stride").u64();
    for (const Json& p : x.at("layer_prefixes").arr) X.layer_prefixes.push_back(p.string());
    X.gate_w = x.at("gate_w").u64();
    X.up_w = x.at("up_w").u64();
    X.down_w = x.at("down_w").u64();
    X.gate_s = x.at("gate_s").u64();
    X.gate_b = x.at("gate_b").u64();
    X.up_s = x.at("up_s").u64();
    X.up_b = x.at("up_b").u64();
    X.down_s = x.at("down_s").u64();
    X.down_b = x.at("down_b").u64();
    // ExpertLayout::validate_dimensions (manifest.rs:95-110) and Packed::open
    if (X.layers == 0 || X.experts == 0) fail("expert layer dimensions must be nonzero");
    if (X.layer_prefixes.size() != X.layers) fail("expert layer count does not match layer prefixes");
    if (X.group != 64) fail("expert group size must be 64");
    if (X.record_bytes == 0 || X.record_stride == 0) fail("expert record size must be nonzero");
    if (X.record_bytes > X.record_stride) fail("expert record larger than its stride");
    uint64_t span = 0;
    if (__builtin_mul_overflow(X.layers, X.experts, &span) || __builtin_mul_overflow(span, X.record_stride, &span) ||
        span > (1ull << 62))
        fail("expert records exceed the addressable file size");
    const ChkConfig& c = S->cfg;
    if (X.experts != c.num_experts || X.inter != c.moe_intermediate_size || X.hidden != c.hidden_size)
        fail("expert layout does not match config.json");
    const uint64_t codes = X.inter * X.hidden;
    const uint64_t sc_up = X.inter * (X.hidden / 64) * 2, sc_down = X.hidden * (X.inter / 64) * 2;
    const std::pair<uint64_t, uint64_t> fields[] = {{X.gate_w, codes / 2}, {X.up_w, codes / 2},
                                                    {X.down_w, codes / 2}, {X.gate_s, sc_up},
                                                    {X.gate_b, sc_up},     {X.up_s, sc_up},
                                                    {X.up_b, sc_up},       {X.down_s, sc_down},
                                                    {X.down_b, sc_down}};
    for (const auto& f : fields)
        if (f.first > X.record_bytes || f.second > X.record_bytes - f.first)
            fail("expert record field outside the record");
    // NgramLayout, read when the config has a PLE layer; the row group
    // reaches the config (ngram rows are not necessarily groups of 64)
    if (const Json* n = m.get("ngram"); n && c.ple_layer) {
        StoreNgram& N = S->ngram;
        N.rows = n->at("rows").u64();
        N.row_bytes = n->at("row_bytes").u64();
        N.dim = n->at("dim").u64();
        N.group = n->at("group").u64();
        N.weight_bytes = n->at("weight_bytes").u64();
        N.scale_bytes = n->at("scale_bytes").u64();
        if (N.group == 0 || N.dim % 8 || N.dim % N.group || N.weight_bytes != N.dim / 2 ||
            N.scale_bytes != N.dim / N.group * 2 || N.row_bytes != N.weight_bytes + 2 * N.scale_bytes)
            fail("n-gram row layout is inconsistent");
        S->cfg.ngram_group = (uint32_t)N.group;
    } else if (c.ple_layer) {
        fail("manifest has no n-gram layout");
    }
    // the record layers the engine reads: each main layer, then the MTP layer
    for (uint32_t l = 0; l < c.num_hidden_layers; ++l)
        if (l >= X.layers || X.layer_prefixes[l] != "language_model.model.layers." + std::to_string(l) + ".mlp.switch_mlp")
            fail("no expert records for layer " + std::to_string(l));
    if (c.mtp_num_hidden_layers > 0) {
        bool found = false;
        for (const auto& p : X.layer_prefixes) found |= p == "mtp.layers.0.mlp.switch_mlp";
        if (!found) fail("no expert records for mtp.layers.0.mlp.switch_mlp");
    }
    return S;
}

// ------------------------------------------------------------ tensor names
// cpu.rs:143-272 and gpu/load.rs name every weight by these prefixes.
std::string tensor_name(const ChkConfig& c, uint32_t kind, uint32_t slot, uint32_t part) {
    const std::string m = "language_model.model";
    const bool mtp = slot == c.num_hidden_layers;
    const std::string lp = mtp ? std::string("mtp.layers.0") : m + ".layers." + std::to_string(slot);
    auto hc = [&](const char* leaf) {
        std::string p;
        switch (part) {
        case CHK_HC_ATTN: p = lp + ".attn_hyper_connection"; break;
        case CHK_HC_MLP: p = lp + ".mlp_hyper_connection"; break;
        case CHK_HC_FINAL: p = m + ".hyper_connection_mixer"; break;
        default: p = "mtp.hyper_connection_mixer"; break;
        }
        return p + leaf;
    };
    switch (kind) {
    case CHK_T_EMBED: return m + ".embed_tokens";
    case CHK_T_LM_HEAD: return "language_model.lm_head";
    case CHK_T_HC_NORM: return hc(".hc_norm.weight");
    case CHK_T_HC_DOWN: return hc(".input_mix_weight_down");
    case CHK_T_HC_UP: return hc(".input_mix_weight_up");
    case CHK_T_HC_INJECT: return hc(".block_inject_weight");
    case CHK_T_DN_QKV: return lp + ".linear_attn.in_proj_qkv";
    case CHK_T_DN_Z: return lp + ".linear_attn.in_proj_z";
    case CHK_T_DN_A: return lp + ".linear_attn.in_proj_a";
    case CHK_T_DN_B: return lp + ".linear_attn.in_proj_b";
    case CHK_T_DN_CONV: return lp + ".linear_attn.conv1d.weight";
    case CHK_T_DN_ALOG: return lp + ".linear_attn.A_log";
    case CHK_T_DN_DTBIAS: return lp + ".linear_attn.dt_bias";
    case CHK_T_DN_NORM: return lp + ".linear_attn.norm.weight";
    case CHK_T_DN_OUT: return lp + ".linear_attn.out_proj";
    case CHK_T_AT_Q: return lp + ".self_attn.q_proj";
    case CHK_T_AT_K: return lp + ".self_attn.k_proj";
    case CHK_T_AT_V: return lp + ".self_attn.v_proj";
    case CHK_T_AT_O: return lp + ".self_attn.o_proj";
    case CHK_T_AT_QNORM: return lp + ".self_attn.q_norm.weight";
    case CHK_T_AT_KNORM: return lp + ".self_attn.k_norm.weight";
    case CHK_T_AT_IDX: return lp + ".self_attn.indexer.index_qk_proj";
    case CHK_T_AT_IDX_QNORM: return lp + ".self_attn.indexer.q_layernorm.weight";
    case CHK_T_AT_IDX_KNORM: return lp + ".self_attn.indexer.k_layernorm.weight";
    case CHK_T_MOE_ROUTER: return lp + ".mlp.gate.weight";
    case CHK_T_MOE_SHARED_GATE: return lp + ".mlp.shared_expert_gate.weight";
    case CHK_T_MOE_SH_GATE_PROJ: return lp + ".mlp.shared_expert.gate_proj";
    case CHK_T_MOE_SH_UP: return lp + ".mlp.shared_expert.up_proj";
    case CHK_T_MOE_SH_DOWN: return lp + ".mlp.shared_expert.down_proj";
    case CHK_T_MTP_ENORM: return "mtp.pre_fc_norm_embedding.weight";
    case CHK_T_MTP_HNORM: return "mtp.pre_fc_norm_hidden.weight";
    case CHK_T_MTP_FC_E: return "mtp.fc_embedding";
    case CHK_T_MTP_FC_H: return "mtp.fc_hidden";
    case CHK_T_PLE_KEY: return lp + ".ple.key_proj";
    case CHK_T_PLE_VALUE: return lp + ".ple.value_proj";
    case CHK_T_PLE_NORM_KEY: return lp + ".ple.norm_key.weight";
    case CHK_T_PLE_NORM_QUERY: return lp + ".ple.norm_query.weight";
    case CHK_T_PLE_NORM_CONV: return lp + ".ple.norm_conv.weight";
    case CHK_T_PLE_CONV: return lp + ".ple.conv1d.weight";
    case CHK_T_NGRAM_MULT: return lp + ".ple.ple_embedding";  // prefix of the hash metadata
    default: fail("no store name for tensor kind " + std::to_string(kind));
    }
    return "";
}

}  // namespace chk
