// Decode loop: the reference runner's `Decode` (/root/reference/
// src/runner/decode.rs:6-171) over the engine ABI.  Rows are the current
// token plus the MTP drafts; the longest prefix of drafts that matches the
// trunk's own greedy predictions is accepted, the step is committed to
// that length (rolling the recurrent state back), and new drafts are
// chained from the MTP head (one after a rejection, else n_draft).  With
// non-greedy sampling options there are no drafts: each step runs the
// current token alone and the request's sampler draws the next one from
// that row's logits.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "cherenkov/engine.h"

namespace {
thread_local std::string g_runner_err;
}

struct ChkDecode {
    ChkEngine* e = nullptr;
    uint32_t cur = 0;
    std::vector<uint32_t> drafts;
    uint32_t n_draft = 0;
    bool use_eos = true;
    std::vector<uint32_t> eos;  // the stop ids (the reference's [im_end, endoftext])
    uint32_t limit = 0;
    std::vector<uint32_t> tokens;
    int finish = 0;  // 0 running, 1 stop, 2 length
    uint32_t steps = 0, accepted = 0;
    ChkSampler* sampler = nullptr;  // owned; null when greedy

    ~ChkDecode() { chk_sampler_free(sampler); }

    bool is_eos(uint32_t t) const { return use_eos && std::find(eos.begin(), eos.end(), t) != eos.end(); }

    static void check(int rc) {
        if (rc != 0) throw std::runtime_error(chk_last_error());
    }

    // Decode::emit (decode.rs:76-84)
    void emit(uint32_t t, std::vector<uint32_t>& emitted) {
        tokens.push_back(t);
        if (sampler) check(chk_sampler_accept(sampler, t));
        emitted.push_back(t);
    }

    // Decode::step (decode.rs:88-171)
    void step(std::vector<uint32_t>& emitted) {
        emitted.clear();
        if (finish) return;
        if (is_eos(cur)) {
            finish = 1;
            return;
        }
        if (tokens.size() >= limit) {
            finish = 2;
            return;
        }
        std::vector<uint32_t> rows{cur};
        uint32_t remaining = limit - (uint32_t)tokens.size() - 1;
        for (uint32_t i = 0; i < std::min<uint32_t>(n_draft, remaining) && i < drafts.size(); ++i)
            rows.push_back(drafts[i]);
        emit(cur, emitted);
        std::vector<uint32_t> result(rows.size());
        check(chk_step_rows(e, rows.data(), (uint32_t)rows.size(), rows.size() > 1, n_draft > 0, result.data()));
        uint32_t n = 1;
        while (n < rows.size() && result[n - 1] == rows[n] && !is_eos(rows[n])) ++n;
        check(chk_commit(e, n));
        steps += 1;
        accepted += n - 1;
        std::vector<uint32_t> next(rows.begin() + 1, rows.begin() + n);
        next.push_back(result[n - 1]);
        if (n_draft > 0) {
            uint32_t chain = (n_draft >= 2 && n < rows.size()) ? 1 : n_draft;
            std::vector<uint32_t> d(std::max<uint32_t>(chain, 1));
            uint32_t nd = 0;
            check(chk_mtp_draft(e, next.data(), (uint32_t)next.size(), chain, d.data(), &nd));
            drafts.assign(d.begin(), d.begin() + nd);
        }
        for (uint32_t i = 1; i < n; ++i) emit(rows[i], emitted);
        if (tokens.size() == limit) {
            finish = 2;
            return;
        }
        if (sampler) {
            const float* l = chk_logits_row(e, n - 1);
            if (!l) throw std::runtime_error(chk_last_error());
            check(chk_sampler_sample(sampler, l, chk_vocab_size(e), &cur));
        } else {
            cur = result[n - 1];
        }
    }
};

extern "C" {

// Decode::new (decode.rs:28-71) for the greedy sampler: `next` is the
// prefill's greedy token, drafts its MTP drafts; n_draft = effective
// drafts; `limit` output tokens; EOS (the config's eos_token_id) ends
// generation unless no_eos.
int chk_decode_new(ChkEngine* e, uint32_t next, const uint32_t* drafts, uint32_t n_drafts, uint32_t n_draft,
                   uint32_t limit, uint32_t no_eos, ChkDecode** out) {
    ChkSampling greedy{};
    greedy.top_p = 1.0;
    return chk_decode_new_sampling(e, &greedy, nullptr, 0, nullptr, next, drafts, n_drafts, n_draft, limit, no_eos,
                                   out);
}

// Decode::new with the request's sampling options: greedy options keep the
// prefill's token and drafts; otherwise the sampler (counts from the
// prompt) draws the first token from the prompt's final logits and the
// effective draft count is 0 (options.rs:165-171).
int chk_decode_new_sampling(ChkEngine* e, const ChkSampling* sampling, const uint32_t* prompt, uint32_t n_prompt,
                            const float* final_logits, uint32_t next, const uint32_t* drafts, uint32_t n_drafts,
                            uint32_t n_draft, uint32_t limit, uint32_t no_eos, ChkDecode** out) {
    *out = nullptr;
    try {
        std::unique_ptr<ChkDecode> d(new ChkDecode());
        d->e = e;
        d->limit = limit;
        d->use_eos = no_eos == 0;
        d->eos.assign(1, chk_eos_token(e));
        if (chk_sampling_greedy(sampling)) {
            ChkDecode::check(chk_sampling_validate(sampling));
            d->cur = next;
            d->drafts.assign(drafts, drafts + n_drafts);
            d->n_draft = n_draft;
        } else {
            const uint32_t vocab = final_logits ? chk_vocab_size(e) : 0;
            ChkDecode::check(chk_sampler_new(sampling, prompt, n_prompt, vocab, &d->sampler));
            if (!final_logits) throw std::runtime_error("sampling needs final prompt logits");
            ChkDecode::check(chk_sampler_sample(d->sampler, final_logits, vocab, &d->cur));
            d->n_draft = 0;
        }
        *out = d.release();
        return 0;
    } catch (const std::exception& ex) {
        g_runner_err = ex.what();
        return -1;
    }
}

void chk_decode_free(ChkDecode* d) { delete d; }

// The stop ids: the reference stops on the tokenizer's [im_end, endoftext]
// (decode.rs:64); the engine has no tokenizer, so the caller that owns it
// passes them.  Until called, the config's eos_token_id alone.
int chk_decode_set_eos(ChkDecode* d, const uint32_t* ids, uint32_t n) {
    if (n < 1 || n > 16) {
        g_runner_err = "EOS ids must be 1..=16";
        return -1;
    }
    d->eos.assign(ids, ids + n);
    return 0;
}

// One Decode::step; writes the tokens emitted by this step (at most 4).
int chk_decode_step(ChkDecode* d, uint32_t* emitted, uint32_t* n_emitted) {
    try {
        std::vector<uint32_t> em;
        d->step(em);
        for (size_t i = 0; i < em.size(); ++i) emitted[i] = em[i];
        *n_emitted = (uint32_t)em.size();
        return 0;
    } catch (const std::exception& ex) {
        g_runner_err = ex.what();
        *n_emitted = 0;
        return -1;
    }
}

int chk_decode_finished(ChkDecode* d) { return d->finish; }

const char* chk_decode_error(void) { return g_runner_err.c_str(); }

int chk_decode_stats(ChkDecode* d, uint32_t* steps, uint32_t* accepted) {
    *steps = d->steps;
    *accepted = d->accepted;
    return 0;
}

}  // extern "C"
