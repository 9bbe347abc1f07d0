// The request sampler of the reference (src/sampling.rs:98-226): presence
// and frequency penalties, temperature, top-k, nucleus (top-p) and a
// seeded random stream, on host f64 arithmetic in the reference's order.
//
// The random stream restates the crates the reference pins (Cargo.lock):
//   rand 0.9.5        StdRng = ChaCha12Rng; random::<f64>() takes the top
//                     53 bits of next_u64() times 2^-53;
//   rand_chacha 0.9.0 ChaCha with 12 rounds, 64-bit block counter in words
//                     12-13, stream id 0 in words 14-15, the keystream's
//                     words in order (four blocks per refill);
//   rand_core 0.9.5   seed_from_u64: the 32-byte key filled with PCG32
//                     outputs (state advanced before each output),
//                     little-endian; next_u64 = two u32 results, low first.
// Unseeded requests draw their key from std::random_device (the
// reference's from_os_rng).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "cherenkov/engine.h"

namespace chk {
extern thread_local std::string g_err;
}

namespace {

// --------------------------------------------------------------- PCG32
// O'Neill's PCG32 (XSH-RR 64/32): a 64-bit LCG and its output permutation.
constexpr uint64_t kPcgMul = 6364136223846793005ull;
constexpr uint64_t kPcgInc = 11634580027462260723ull;  // rand_core's stream
inline uint64_t pcg_step(uint64_t state, uint64_t inc) { return state * kPcgMul + inc; }
inline uint32_t pcg_output(uint64_t state) {
    const uint32_t xorshifted = (uint32_t)(((state >> 18) ^ state) >> 27);
    const uint32_t rot = (uint32_t)(state >> 59);
    return (xorshifted >> rot) | (xorshifted << ((32 - rot) & 31));
}

// ------------------------------------------------------------ ChaCha12
struct ChaCha12 {
    uint32_t key[8];
    uint64_t counter = 0;  // next block
    uint32_t buf[64];
    uint32_t index = 64;   // next unread word of buf

    static uint32_t rotl(uint32_t v, int n) { return (v << n) | (v >> (32 - n)); }
    static void qr(uint32_t& a, uint32_t& b, uint32_t& c, uint32_t& d) {
        a += b; d ^= a; d = rotl(d, 16);
        c += d; b ^= c; b = rotl(b, 12);
        a += b; d ^= a; d = rotl(d, 8);
        c += d; b ^= c; b = rotl(b, 7);
    }
    // one 16-word block of `rounds` rounds from the 16-word input state
    static void block(const uint32_t in[16], int rounds, uint32_t out[16]) {
        uint32_t x[16];
        memcpy(x, in, sizeof(x));
        for (int i = 0; i < rounds; i += 2) {
            qr(x[0], x[4], x[8], x[12]);
            qr(x[1], x[5], x[9], x[13]);
            qr(x[2], x[6], x[10], x[14]);
            qr(x[3], x[7], x[11], x[15]);
            qr(x[0], x[5], x[10], x[15]);
            qr(x[1], x[6], x[11], x[12]);
            qr(x[2], x[7], x[8], x[13]);
            qr(x[3], x[4], x[9], x[14]);
        }
        for (int i = 0; i < 16; ++i) out[i] = x[i] + in[i];
    }
    void refill() {
        for (int b = 0; b < 4; ++b) {
            uint32_t st[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u};
            for (int i = 0; i < 8; ++i) st[4 + i] = key[i];
            st[12] = (uint32_t)counter;
            st[13] = (uint32_t)(counter >> 32);
            st[14] = 0;
            st[15] = 0;
            block(st, 12, buf + 16 * b);
            ++counter;
        }
        index = 0;
    }
    // rand_core's BlockRng::next_u64: low word first (across a refill the
    // low word is the buffer's last, the high word the new buffer's first)
    uint64_t next_u64() {
        if (index < 63) {
            const uint64_t lo = buf[index], hi = buf[index + 1];
            index += 2;
            return (hi << 32) | lo;
        }
        if (index >= 64) {
            refill();
            const uint64_t lo = buf[0], hi = buf[1];
            index = 2;
            return (hi << 32) | lo;
        }
        const uint64_t lo = buf[63];
        refill();
        const uint64_t hi = buf[0];
        index = 1;
        return (hi << 32) | lo;
    }
    double next_f64() { return (double)(next_u64() >> 11) * (1.0 / 9007199254740992.0); }

    void seed_bytes(const uint8_t s[32]) {
        for (int i = 0; i < 8; ++i)
            key[i] = (uint32_t)s[4 * i] | (uint32_t)s[4 * i + 1] << 8 | (uint32_t)s[4 * i + 2] << 16 |
                     (uint32_t)s[4 * i + 3] << 24;
        counter = 0;
        index = 64;
    }
    // rand_core::SeedableRng::seed_from_u64: each 4 key bytes are the PCG32
    // output of the state after one LCG step (the step comes first)
    void seed_u64(uint64_t state) {
        uint8_t s[32];
        for (int i = 0; i < 8; ++i) {
            state = pcg_step(state, kPcgInc);
            const uint32_t x = pcg_output(state);
            memcpy(s + 4 * i, &x, 4);  // little-endian host
        }
        seed_bytes(s);
    }
};

// IEEE 754 totalOrder key of a double (Rust's f64::total_cmp): the bits
// as a signed integer, with the magnitude bits flipped for negatives, so
// -0.0 orders below +0.0 and -inf below every finite value.
inline int64_t total_key(double v) {
    int64_t b;
    memcpy(&b, &v, 8);
    return b ^ (int64_t)((uint64_t)(b >> 63) >> 1);
}

// rank (sampling.rs:211-213): larger weight first, then the lower id
inline bool rank_less(const std::pair<uint32_t, double>& a, const std::pair<uint32_t, double>& b) {
    const int64_t ka = total_key(a.second), kb = total_key(b.second);
    if (ka != kb) return ka > kb;
    return a.first < b.first;
}

}  // namespace

struct ChkSampler {
    ChkSampling o{};
    ChaCha12 rng;
    std::vector<uint32_t> counts;
    std::vector<std::pair<uint32_t, double>> cand;

    // Sampling::validate (sampling.rs:46-68)
    static void validate(const ChkSampling& s) {
        if (!(std::isfinite(s.temperature) && s.temperature >= 0.0 && s.temperature <= 2.0))
            throw std::runtime_error("temperature must be finite and in 0..2");
        if (!(std::isfinite(s.top_p) && s.top_p > 0.0 && s.top_p <= 1.0))
            throw std::runtime_error("top_p must be finite and in (0, 1]");
        if (s.top_k > 1000000) throw std::runtime_error("top_k must be 0..1000000");
        if (!(std::isfinite(s.presence_penalty) && s.presence_penalty >= -2.0 && s.presence_penalty <= 2.0))
            throw std::runtime_error("presence_penalty must be finite and in -2..2");
        if (!(std::isfinite(s.frequency_penalty) && s.frequency_penalty >= -2.0 && s.frequency_penalty <= 2.0))
            throw std::runtime_error("frequency_penalty must be finite and in -2..2");
    }

    // Sampler::new (sampling.rs:114-134)
    ChkSampler(const ChkSampling& s, const uint32_t* prompt, uint32_t n, uint32_t vocab) : o(s), counts(vocab, 0) {
        validate(s);
        if (s.has_seed) {
            rng.seed_u64(s.seed);
        } else {
            std::random_device rd;
            uint8_t k[32];
            for (int i = 0; i < 8; ++i) {
                const uint32_t v = rd();
                memcpy(k + 4 * i, &v, 4);
            }
            rng.seed_bytes(k);
        }
        cand.reserve(vocab);
        for (uint32_t i = 0; i < n; ++i) accept(prompt[i]);
    }

    // Sampler::accept (sampling.rs:136-144)
    void accept(uint32_t token) {
        if (token >= counts.size()) throw std::runtime_error("token exceeds vocabulary");
        if (counts[token] != 0xffffffffu) ++counts[token];
    }

    // Sampler::sample (sampling.rs:146-209)
    uint32_t sample(const float* logits, uint32_t n) {
        if (n != counts.size()) throw std::runtime_error("logit vocabulary mismatch");
        cand.clear();
        for (uint32_t id = 0; id < n; ++id) {
            const float l = logits[id];
            if (std::isnan(l) || l == INFINITY) throw std::runtime_error("non-finite model logits");
            const uint32_t c = counts[id];
            const double penalty = o.frequency_penalty * (double)c + (c > 0 ? o.presence_penalty : 0.0);
            cand.push_back({id, (double)l - penalty});
        }
        if (cand.empty()) throw std::runtime_error("empty vocabulary");
        std::pair<uint32_t, double> best = cand[0];
        for (const auto& c : cand)
            if (rank_less(c, best)) best = c;
        if (!std::isfinite(best.second)) throw std::runtime_error("no finite candidate logits");
        if (o.temperature == 0.0) return best.first;
        const uint32_t k = o.top_k;
        if (k > 0 && k < cand.size()) {
            // the reference keeps select_nth_unstable's (unspecified) order
            // of the k best; this keeps std::nth_element's
            std::nth_element(cand.begin(), cand.begin() + k, cand.end(), rank_less);
            cand.resize(k);
        }
        if (o.top_p < 1.0) std::sort(cand.begin(), cand.end(), rank_less);
        double total = 0.0;
        for (auto& c : cand) {
            c.second = std::exp((c.second - best.second) / o.temperature);
            total += c.second;
        }
        // nucleus (sampling.rs:215-227)
        const double threshold = total * o.top_p;
        size_t keep = cand.size();
        double mass = 0.0;
        for (size_t i = 0; i < cand.size(); ++i) {
            mass += cand[i].second;
            if (mass >= threshold) {
                keep = i + 1;
                break;
            }
        }
        const double draw = rng.next_f64() * mass;
        double cumulative = 0.0;
        for (size_t i = 0; i < keep; ++i) {
            cumulative += cand[i].second;
            if (draw < cumulative) return cand[i].first;
        }
        return cand[keep - 1].first;
    }
};

extern "C" {

int chk_sampling_validate(const ChkSampling* s) {
    try {
        ChkSampler::validate(*s);
        return 0;
    } catch (const std::exception& e) {
        chk::g_err = e.what();
        return -1;
    }
}

int chk_sampling_greedy(const ChkSampling* s) {
    return s->temperature == 0.0 && s->presence_penalty == 0.0 && s->frequency_penalty == 0.0 ? 1 : 0;
}

int chk_sampler_new(const ChkSampling* s, const uint32_t* prompt, uint32_t n, uint32_t vocab, ChkSampler** out) {
    *out = nullptr;
    try {
        *out = new ChkSampler(*s, prompt, n, vocab);
        return 0;
    } catch (const std::exception& e) {
        chk::g_err = e.what();
        return -1;
    }
}

void chk_sampler_free(ChkSampler* s) { delete s; }

int chk_sampler_accept(ChkSampler* s, uint32_t token) {
    try {
        s->accept(token);
        return 0;
    } catch (const std::exception& e) {
        chk::g_err = e.what();
        return -1;
    }
}

int chk_sampler_sample(ChkSampler* s, const float* logits, uint32_t n, uint32_t* token) {
    try {
        *token = s->sample(logits, n);
        return 0;
    } catch (const std::exception& e) {
        chk::g_err = e.what();
        return -1;
    }
}

// The sampler's random stream alone (test support for the restatement):
// n next_u64 draws of StdRng::from_seed(seed32), or of
// StdRng::seed_from_u64(seed) when seed32 is NULL.
int chk_rng_u64(const uint8_t* seed32, uint64_t seed, uint64_t* out, uint32_t n) {
    ChaCha12 r;
    if (seed32)
        r.seed_bytes(seed32);
    else
        r.seed_u64(seed);
    for (uint32_t i = 0; i < n; ++i) out[i] = r.next_u64();
    return 0;
}

// PCG32 as its reference generator runs it (pcg32_srandom_r /
// pcg32_random_r: the output comes from the state before each step), on
// the step and output functions the seeding uses (test support).
void chk_pcg32(uint64_t init_state, uint64_t init_seq, uint32_t* out, uint32_t n) {
    const uint64_t inc = (init_seq << 1) | 1u;
    uint64_t state = pcg_step(0, inc);
    state += init_state;
    state = pcg_step(state, inc);
    for (uint32_t i = 0; i < n; ++i) {
        out[i] = pcg_output(state);
        state = pcg_step(state, inc);
    }
}

// The ChaCha block function with `rounds` rounds on a caller's 16-word
// input state (test support: RFC 8439 vectors pin the core).
void chk_chacha_block(const uint32_t* in, int rounds, uint32_t* out) { ChaCha12::block(in, rounds, out); }

}  // extern "C"
