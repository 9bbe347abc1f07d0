"""Non-greedy decoding on the GPU: the native runner with a request's
sampling options (decode.rs:28-171 with sampling.rs).

The runner's sampled tokens must equal the reference loop replayed by hand
over the engine ABI (one row per step, commit 1, sample from that row's
logits with a sampler of the same seed and counts), and the logits each
draw sees must match the CPU oracle's to the float bar.
"""

from __future__ import annotations

import numpy as np
import pytest

from cherenkov_amd import presets
from cherenkov_amd.engine import Decode, Engine
from cherenkov_amd.sampling import Sampler, Sampling
from oracle.oracle import OracleModel
from tests.gpu_util import assert_close

pytestmark = pytest.mark.gpu


def test_sampled_decode_follows_the_reference_loop(have_gpu):
    cfg = presets.tiny(seed=5)
    rng = np.random.default_rng(5)
    prompt = rng.integers(0, cfg.vocab_size, size=12).tolist()
    opts = Sampling(temperature=0.9, top_p=0.95, top_k=40, seed=1234, presence_penalty=0.4, frequency_penalty=0.1)
    limit = 24
    eng = Engine(cfg, experts=4, drafts=2, max_t=256)
    try:
        nxt, dr = eng.prefill_chunk(prompt)
        d = Decode(eng, nxt, [dr], 2, limit=limit, no_eos=True, sampling=opts, prompt=prompt,
                   final_logits=eng.logits())
        got = d.run()
        steps, acc = d.stats()
        print(f"sampled: {got}", flush=True)
        assert (steps, acc) == (limit, 0)  # no drafts when not greedy

        eng.reset()
        eng.prefill_chunk(prompt)
        st = OracleModel(cfg).new_state()
        for t in prompt[:-1]:
            st.forward_token(t)
        ref = st.forward_token(prompt[-1])
        logits = eng.logits()
        assert_close(logits, ref, "prompt logits")
        s = Sampler(opts, prompt, cfg.vocab_size)
        cur = s.sample(logits)
        want = []
        while True:
            want.append(cur)
            s.accept(cur)
            if len(want) == limit:
                break
            eng.step_rows([cur])
            eng.commit(1)
            logits = eng.logits_row(0)
            assert_close(logits, st.forward_token(cur), f"step {len(want)} logits")
            cur = s.sample(logits)
        assert got == want
    finally:
        eng.close()


def test_greedy_options_keep_speculative_decoding(have_gpu):
    """Sampling() is greedy: the runner keeps its drafts and emits the
    tokens of the plain greedy loop."""
    cfg = presets.tiny(seed=99)
    cfg.vocab_size = 16
    prompt = np.random.default_rng(99).integers(0, cfg.vocab_size, size=8).tolist()
    eng = Engine(cfg, experts=4, drafts=2, max_t=256)
    try:
        nxt, dr = eng.prefill_chunk(prompt)
        plain = Decode(eng, nxt, [dr], 2, limit=32, no_eos=True).run()
        eng.reset()
        nxt, dr = eng.prefill_chunk(prompt)
        d = Decode(eng, nxt, [dr], 2, limit=32, no_eos=True, sampling=Sampling(top_k=3, seed=7), prompt=prompt,
                   final_logits=eng.logits())
        assert d.run() == plain
        assert d.stats()[1] > 0
    finally:
        eng.close()


def test_sampled_decode_needs_final_logits(have_gpu):
    """Without final logits the reference sizes the sampler's counts to a
    vocabulary of 0 (decode.rs:38-44), so a prompt token fails first; an
    empty prompt reaches the missing-logits error."""
    cfg = presets.tiny(seed=5)
    eng = Engine(cfg, experts=4, drafts=0, max_t=64)
    try:
        nxt, _ = eng.prefill_chunk([1, 2, 3])
        opts = Sampling(temperature=1.0, seed=1)
        with pytest.raises(Exception, match="token exceeds vocabulary"):
            Decode(eng, nxt, [], 0, limit=4, sampling=opts, prompt=[1, 2, 3])
        with pytest.raises(Exception, match="sampling needs final prompt logits"):
            Decode(eng, nxt, [], 0, limit=4, sampling=opts, prompt=[])
    finally:
        eng.close()
