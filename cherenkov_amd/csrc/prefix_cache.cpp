// Bounded LRU checkpoints of whole sequence state and the resumable prompt
// cursor over them: the reference's PrefixCache / Prefill
// (/root/reference/src/prefix_cache.rs:12-335) over the engine ABI.
//
// An entry is a device checkpoint (chk_save_prefix) of a prompt prefix
// with what decode needs to resume from it (the greedy next token, MTP
// drafts, the last row's logits).  A request restores the longest entry
// its prompt extends (the MTP cache's last row depends on the token after
// the prefix, so an entry made while drafting is reused only for the same
// continuation), then prefills the rest chunk by chunk, storing an entry
// at each stable boundary it crosses.  Entries are evicted oldest first
// to stay within the byte capacity and entry count, and after an idle
// time.
#include <algorithm>
#include <chrono>
#include <cstdlib>
#include <deque>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "cherenkov/engine.h"

namespace chk {
extern thread_local std::string g_err;
}

namespace {

using Clock = std::chrono::steady_clock;

void check(int rc) {
    if (rc != 0) throw std::runtime_error(chk_last_error());
}

// PrefillResume (runner.rs:450-454)
struct Resume {
    uint32_t next = 0;
    std::vector<uint32_t> drafts;
    bool has_logits = false;
    std::vector<float> logits;
};

struct Entry {
    std::vector<uint32_t> tokens;
    bool has_following = false;
    uint32_t following = 0;
    bool complete = false;
    Resume seed;
    bool drafting = false;
    ChkPrefixState* state = nullptr;
    uint64_t bytes = 0;
    Clock::time_point touched;
};

// matches (prefix_cache.rs:35-45)
bool matches(const uint32_t* tokens, uint32_t nt, bool has_following, uint32_t following, bool complete,
             const uint32_t* request, uint32_t nr) {
    if (nr < nt || !std::equal(tokens, tokens + nt, request)) return false;
    if (nr == nt) return complete;
    return !has_following || request[nt] == following;
}

// chunk_len (prefix_cache.rs:256-266): balance a boundary's chunks
uint32_t chunk_len(uint32_t remaining, uint32_t capacity, uint32_t quantum) {
    const uint32_t size = std::min(capacity, quantum);
    if (remaining == 0 || size == 0) throw std::runtime_error("prefill chunk requires tokens and capacity");
    const uint32_t chunks = (remaining + size - 1) / size;
    return (remaining + chunks - 1) / chunks;
}

// pacing_sample (prefix_cache.rs:251-253)
bool pacing_sample(uint32_t remaining, uint32_t capacity, uint32_t quantum, bool engine) {
    return engine && remaining >= quantum && capacity >= quantum;
}

uint32_t env_u32(const char* name, uint32_t dflt) {
    const char* v = std::getenv(name);
    if (!v || !*v) return dflt;
    char* end = nullptr;
    const unsigned long x = std::strtoul(v, &end, 10);
    return (end && *end == '\0') ? (uint32_t)x : dflt;
}

const float* copy_logits(ChkEngine* e, const float* p, std::vector<float>& out) {
    if (!p) throw std::runtime_error(chk_last_error());
    out.assign(p, p + chk_vocab_size(e));
    return p;
}

// prefill_rows (prefix_cache.rs:268-330): one chunk, engine or row path
Resume prefill_rows(ChkEngine* e, const uint32_t* rows, uint32_t n, bool has_following, uint32_t following,
                    uint32_t drafts, bool engine) {
    const bool last = !has_following;
    Resume seed;
    if (engine) {
        uint32_t next = 0, draft = 0;
        check(chk_prefill_chunk(e, rows, n, has_following ? following : CHK_NO_TOKEN, 0, &next, &draft));
        seed.next = next;
        seed.has_logits = true;
        copy_logits(e, chk_logits(e), seed.logits);
        if (drafts == 0 || !last) return seed;
        seed.drafts.push_back(draft);
        if (drafts >= 2) {
            uint32_t d2 = 0;
            check(chk_mtp_chain(e, draft, &d2));
            seed.drafts.push_back(d2);
        }
        return seed;
    }
    std::vector<uint32_t> result(n);
    check(chk_step_rows(e, rows, n, 0, 0, result.data()));
    check(chk_commit(e, n));
    seed.next = result[n - 1];
    seed.has_logits = true;
    copy_logits(e, chk_logits_row(e, n - 1), seed.logits);
    if (drafts == 0) return seed;
    std::vector<uint32_t> next(rows + 1, rows + n);
    next.push_back(has_following ? following : seed.next);
    const uint32_t chain = last ? drafts : 1;
    std::vector<uint32_t> d(std::max<uint32_t>(chain, 1));
    uint32_t nd = 0;
    check(chk_mtp_draft(e, next.data(), (uint32_t)next.size(), chain, d.data(), &nd));
    seed.drafts.assign(d.begin(), d.begin() + nd);
    return seed;
}

}  // namespace

struct ChkPrefixCache {
    std::deque<Entry> entries;
    uint64_t capacity = 0, used = 0, evictions = 0, max_entries = 0;
    bool has_idle = false;
    Clock::duration idle{};

    ~ChkPrefixCache() {
        for (Entry& x : entries) chk_prefix_free(x.state);
    }

    void evict_oldest() {
        if (entries.empty()) return;
        used -= entries.front().bytes;
        chk_prefix_free(entries.front().state);
        entries.pop_front();
        ++evictions;
    }

    // PrefixCache::expire (prefix_cache.rs:64-75)
    void expire() {
        if (!has_idle) return;
        while (!entries.empty() && Clock::now() - entries.front().touched >= idle) evict_oldest();
    }

    // PrefixCache::store (prefix_cache.rs:81-121)
    void store(ChkEngine* e, const uint32_t* ids, uint32_t n_ids, const Resume& seed, bool drafting) {
        const uint32_t pos = chk_pos(e);
        const uint64_t bytes = chk_prefix_state_bytes(e) + (uint64_t)pos * 4 + sizeof(Entry) +
                               seed.drafts.size() * 4 + seed.logits.size() * 4;
        if (bytes > capacity || pos == 0) return;
        for (auto it = entries.begin(); it != entries.end(); ++it) {
            if (it->drafting == drafting && it->tokens.size() == pos && std::equal(ids, ids + pos, it->tokens.begin())) {
                used -= it->bytes;
                chk_prefix_free(it->state);
                entries.erase(it);
                break;
            }
        }
        // evict before copying state: allocation peaks stay within the budget
        while (used + bytes > capacity || entries.size() >= max_entries) {
            if (entries.empty()) return;
            evict_oldest();
        }
        Entry x;
        x.tokens.assign(ids, ids + pos);
        x.has_following = drafting;
        x.following = pos < n_ids ? ids[pos] : seed.next;
        x.complete = pos == n_ids;
        x.seed = seed;
        x.drafting = drafting;
        check(chk_save_prefix(e, &x.state));
        x.bytes = bytes;
        x.touched = Clock::now();
        entries.push_back(std::move(x));
        used += bytes;
    }
};

struct ChkPrefill {
    uint32_t cached = 0;
    std::vector<uint32_t> boundaries;
    Resume seed;
};

extern "C" {

int chk_prefix_matches(const uint32_t* tokens, uint32_t n_tokens, int has_following, uint32_t following,
                       int complete, const uint32_t* request, uint32_t n_request) {
    return matches(tokens, n_tokens, has_following != 0, following, complete != 0, request, n_request) ? 1 : 0;
}

int chk_prefill_chunk_len(uint32_t remaining, uint32_t capacity, uint32_t quantum, uint32_t* out) {
    try {
        *out = chunk_len(remaining, capacity, quantum);
        return 0;
    } catch (const std::exception& x) {
        chk::g_err = x.what();
        return -1;
    }
}

int chk_prefill_pacing_sample(uint32_t remaining, uint32_t capacity, uint32_t quantum, int engine) {
    return pacing_sample(remaining, capacity, quantum, engine != 0) ? 1 : 0;
}

int chk_prefix_cache_new(uint64_t capacity, uint64_t max_entries, uint64_t idle_seconds, ChkPrefixCache** out) {
    *out = nullptr;
    try {
        auto c = std::make_unique<ChkPrefixCache>();
        c->capacity = capacity;
        c->max_entries = max_entries;
        c->has_idle = idle_seconds > 0;
        c->idle = std::chrono::seconds(idle_seconds);
        *out = c.release();
        return 0;
    } catch (const std::exception& x) {
        chk::g_err = x.what();
        return -1;
    }
}

void chk_prefix_cache_free(ChkPrefixCache* c) { delete c; }

void chk_prefix_cache_expire(ChkPrefixCache* c) { c->expire(); }

void chk_prefix_cache_stats(const ChkPrefixCache* c, uint64_t* entries, uint64_t* used, uint64_t* evictions) {
    *entries = c->entries.size();
    *used = c->used;
    *evictions = c->evictions;
}

// PrefixCache::begin (prefix_cache.rs:123-181)
int chk_prefix_cache_begin(ChkPrefixCache* c, ChkEngine* e, const uint32_t* ids, uint32_t n,
                           const uint32_t* stable_boundaries, uint32_t n_boundaries, uint32_t effective_drafts,
                           ChkPrefill** out) {
    *out = nullptr;
    try {
        c->expire();
        const bool drafting = effective_drafts > 0;
        auto p = std::make_unique<ChkPrefill>();
        int best = -1;
        size_t best_len = 0;
        for (size_t i = 0; i < c->entries.size(); ++i) {
            const Entry& x = c->entries[i];
            if (x.drafting != drafting ||
                !matches(x.tokens.data(), (uint32_t)x.tokens.size(), x.has_following, x.following, x.complete, ids, n))
                continue;
            // max_by_key keeps the last of equal lengths
            if (best < 0 || x.tokens.size() >= best_len) {
                best = (int)i;
                best_len = x.tokens.size();
            }
        }
        if (best >= 0) {
            Entry x = std::move(c->entries[(size_t)best]);
            c->entries.erase(c->entries.begin() + best);
            x.touched = Clock::now();
            const int rc = chk_restore_prefix(e, x.state);
            if (rc != 0) {
                // the entry leaves the cache on a failed restore, as the
                // reference's `?` drops the removed entry
                c->used -= x.bytes;
                chk_prefix_free(x.state);
                throw std::runtime_error(chk_last_error());
            }
            p->cached = (uint32_t)x.tokens.size();
            p->seed = x.seed;
            p->seed.has_logits = true;
            c->entries.push_back(std::move(x));
        }
        p->boundaries.push_back(n);
        if (c->capacity > 0) {
            for (uint32_t i = 0; i < n_boundaries; ++i)
                if (stable_boundaries[i] > p->cached && stable_boundaries[i] < n)
                    p->boundaries.push_back(stable_boundaries[i]);
            if (n > 1) p->boundaries.push_back(n - 1);
        }
        std::sort(p->boundaries.begin(), p->boundaries.end());
        p->boundaries.erase(std::unique(p->boundaries.begin(), p->boundaries.end()), p->boundaries.end());
        *out = p.release();
        return 0;
    } catch (const std::exception& x) {
        chk::g_err = x.what();
        return -1;
    }
}

void chk_prefill_free(ChkPrefill* p) { delete p; }

uint32_t chk_prefill_cached(const ChkPrefill* p) { return p->cached; }

// Prefill::advance (prefix_cache.rs:197-249): at most one chunk toward the
// next boundary past the engine's position (CHERENKOV_PREFILL_MIN,
// CHERENKOV_PREFILL_CHUNK and CHERENKOV_ROWS_MAX as in the reference).
// *pacing_tokens = 0 when the chunk is no pacing sample.
int chk_prefill_advance(ChkPrefill* p, ChkPrefixCache* c, ChkEngine* e, const uint32_t* ids, uint32_t n,
                        uint32_t effective_drafts, uint32_t quantum, int* done, uint32_t* pacing_tokens) {
    try {
        *pacing_tokens = 0;
        const uint32_t pos = chk_pos(e);
        auto it = std::find_if(p->boundaries.begin(), p->boundaries.end(), [&](uint32_t b) { return b > pos; });
        if (it == p->boundaries.end()) {
            *done = 1;
            return 0;
        }
        const uint32_t end = *it;
        if (end > n) throw std::runtime_error("prefill boundary beyond the prompt");
        const uint32_t remaining = end - pos;
        const bool engine = remaining >= env_u32("CHERENKOV_PREFILL_MIN", 64);
        uint32_t capacity = 0;
        if (engine) {
            uint32_t fit = 0;
            check(chk_prefill_rows_fit(e, 0, &fit));
            capacity = std::min(env_u32("CHERENKOV_PREFILL_CHUNK", fit), fit);
        } else {
            capacity = std::clamp<uint32_t>(env_u32("CHERENKOV_ROWS_MAX", 4), 1, 4);
            capacity = std::min(capacity, chk_trunk_rows(e));
        }
        const uint32_t rows = chunk_len(remaining, capacity, quantum);
        const bool has_following = pos + rows < n;
        p->seed = prefill_rows(e, ids + pos, rows, has_following, has_following ? ids[pos + rows] : 0,
                               effective_drafts, engine);
        if (chk_pos(e) == end || engine) c->store(e, ids, n, p->seed, effective_drafts > 0);
        chk_prefill_release(e);
        *done = chk_pos(e) == n ? 1 : 0;
        if (pacing_sample(remaining, capacity, quantum, engine)) *pacing_tokens = rows;
        return 0;
    } catch (const std::exception& x) {
        chk::g_err = x.what();
        return -1;
    }
}

// The resume point after the last advance (or the restored entry):
// next token, drafts (up to `cap`), and the logits row (vocab floats; NULL
// when none).
uint32_t chk_prefill_next(const ChkPrefill* p) { return p->seed.next; }
uint32_t chk_prefill_drafts(const ChkPrefill* p, uint32_t* out, uint32_t cap) {
    const uint32_t n = (uint32_t)p->seed.drafts.size();
    for (uint32_t i = 0; i < n && i < cap; ++i) out[i] = p->seed.drafts[i];
    return n;
}
const float* chk_prefill_logits(const ChkPrefill* p) {
    return p->seed.has_logits && !p->seed.logits.empty() ? p->seed.logits.data() : nullptr;
}

}  // extern "C"
