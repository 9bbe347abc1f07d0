"""The request sampler without a GPU (native sampler.cpp through the C ABI).

The first four tests restate the reference's own unit tests of the sampler
(/root/reference/tests/unit/sampling.rs:3-110).  The random stream is pinned
by published vectors: RFC 8439 and the zero-key ChaCha20/12/8 keystreams for
the block function, the PCG32 reference generator's first outputs for
seed_from_u64's generator, and rand's StdRng value-stability vector
(rand/src/rngs/std.rs test_stdrng_construction) for from_seed + next_u64.
The rest checks what the mathematics fixes: the drawn distribution against
the softmax of the penalised logits, and the rank order's tie-breaks.
"""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from cherenkov_amd import abi

pytestmark = pytest.mark.skipif(not abi.LIB_PATH.exists(), reason="libcherenkov.so not built")

from cherenkov_amd.abi import EngineError  # noqa: E402
from cherenkov_amd.sampling import Sampler, Sampling, rng_u64  # noqa: E402

NEG_INF = float("-inf")


# ----------------------------------------------------- reference unit tests
def test_greedy_ties_and_penalties_are_explicit():
    """sampling.rs test greedy_ties_and_penalties_are_explicit."""
    s = Sampler(Sampling(), [], 3)
    assert s.sample([1.0, 1.0, 0.0]) == 0
    s = Sampler(Sampling(presence_penalty=1.0, frequency_penalty=0.5), [0, 0], 3)
    assert s.sample([2.0, 1.0, 0.0]) == 1
    s.accept(1)
    assert s.sample([2.0, 1.0, 0.1]) == 2


def test_top_k_and_nucleus_keep_the_boundary_token():
    """sampling.rs test top_k_and_nucleus_keep_the_boundary_token; the
    nucleus cut itself (nucleus([.5,.3,.2], .6) == (2, .8)) is checked
    through the sampler: top_p .6 over those probabilities keeps tokens 0
    and 1, drawn .5/.8 and .3/.8 of the time."""
    opts = Sampling(temperature=1.0, top_k=1, seed=1)
    s = Sampler(opts, [], 3)
    for _ in range(50):
        assert s.sample([0.0, 5.0, 2.0]) == 1
    s = Sampler(Sampling(temperature=1.0, top_k=0, top_p=0.1, seed=1), [], 3)
    for _ in range(50):
        assert s.sample([0.0, 5.0, 2.0]) == 1

    s = Sampler(Sampling(temperature=1.0, top_p=0.6, seed=3), [], 3)
    logits = np.log(np.array([0.5, 0.3, 0.2], dtype=np.float32))
    counts = np.bincount([s.sample(logits) for _ in range(20000)], minlength=3)
    assert counts[2] == 0
    assert abs(counts[0] / 20000 - 0.5 / 0.8) < 0.02


def test_distribution_and_seed_are_independent_of_other_requests():
    """sampling.rs test distribution_and_seed_are_independent_of_other_requests."""
    opts = Sampling(temperature=1.0, seed=42)
    a = Sampler(opts, [], 2)
    b = Sampler(opts, [], 2)
    unrelated = Sampler(Sampling(temperature=1.0, seed=8), [], 2)
    logits = np.log(np.array([0.25, 0.75], dtype=np.float32))
    counts = [0, 0]
    for _ in range(20000):
        t = a.sample(logits)
        unrelated.sample([0.0, 0.0])
        assert t == b.sample(logits)
        counts[t] += 1
    assert abs(counts[0] / 20000 - 0.25) < 0.02


@pytest.mark.parametrize("value", [{"top_p": 0}, {"temperature": -1}, {"top_k": -1}, {"seed": "wrong"}])
def test_rejects_invalid_parameters(value):
    """sampling.rs test rejects_invalid_parameters_and_logits (requests)."""
    with pytest.raises(EngineError):
        Sampling.from_request(value, Sampling())


def test_rejects_invalid_logits():
    """sampling.rs test rejects_invalid_parameters_and_logits (logits)."""
    s = Sampler(Sampling(), [], 2)
    with pytest.raises(EngineError, match="non-finite model logits"):
        s.sample([float("nan"), 0.0])
    with pytest.raises(EngineError, match="no finite candidate logits"):
        s.sample([NEG_INF, NEG_INF])
    assert s.sample([NEG_INF, 0.0]) == 1


# ------------------------------------------------------- options and errors
def test_from_request_merges_over_defaults_and_validates():
    d = Sampling(temperature=0.7, top_k=40)
    got = Sampling.from_request({"top_p": 0.9, "seed": 5, "temperature": None}, d)
    assert got == Sampling(temperature=0.7, top_p=0.9, top_k=40, seed=5)
    assert Sampling.from_request({"temperature": 1}, Sampling()).temperature == 1.0
    for bad in ({"temperature": 2.5}, {"top_p": 1.5}, {"top_k": 1_000_001}, {"presence_penalty": -2.1},
                {"frequency_penalty": 3}, {"top_k": 1.0}, {"temperature": True}):
        with pytest.raises(EngineError):
            Sampling.from_request(bad, Sampling())
    for edge in ({"temperature": 2}, {"top_p": 1}, {"top_k": 1_000_000}, {"presence_penalty": -2},
                 {"frequency_penalty": 2}):
        Sampling.from_request(edge, Sampling())


def test_greedy_means_no_temperature_and_no_penalties():
    assert Sampling().greedy()
    assert Sampling(top_k=5, top_p=0.5, seed=1).greedy()
    assert not Sampling(temperature=0.1).greedy()
    assert not Sampling(presence_penalty=0.1).greedy()
    assert not Sampling(frequency_penalty=-0.1).greedy()


def test_sampler_errors():
    with pytest.raises(EngineError, match="token exceeds vocabulary"):
        Sampler(Sampling(), [3], 3)
    s = Sampler(Sampling(), [], 3)
    with pytest.raises(EngineError, match="token exceeds vocabulary"):
        s.accept(3)
    with pytest.raises(EngineError, match="logit vocabulary mismatch"):
        s.sample([0.0, 1.0])
    with pytest.raises(EngineError, match="non-finite model logits"):
        s.sample([0.0, float("inf"), 1.0])
    with pytest.raises(EngineError, match="temperature"):
        Sampler(Sampling(temperature=float("nan")), [], 3)


# ------------------------------------------------ rank order and penalties
def test_rank_prefers_the_larger_weight_then_the_lower_id():
    s = Sampler(Sampling(), [], 4)
    assert s.sample([0.0, 3.0, 3.0, 1.0]) == 1
    # total order: +0.0 ranks above -0.0 (f64::total_cmp), so id 1 wins
    assert s.sample([-0.0, 0.0, NEG_INF, NEG_INF]) == 1
    assert s.sample([0.0, -0.0, NEG_INF, NEG_INF]) == 0


def test_penalties_follow_counts():
    """adjusted = logit - (frequency * count + presence * [count > 0]),
    counts from the prompt plus every accepted token."""
    s = Sampler(Sampling(frequency_penalty=1.0), [2, 2, 2], 3)  # 5 - 3 = 2 < 2.5
    assert s.sample([0.0, 2.5, 5.0]) == 1
    s = Sampler(Sampling(presence_penalty=-2.0), [0], 3)  # a negative penalty promotes
    assert s.sample([1.0, 2.5, 0.0]) == 0
    s = Sampler(Sampling(frequency_penalty=0.25), [], 3)
    for _ in range(4):
        s.accept(1)  # 2.0 - 1.0 = 1.0 < 1.5
    assert s.sample([0.0, 2.0, 1.5]) == 2


def test_draws_follow_the_softmax_of_the_penalised_logits():
    """Empirical frequencies match softmax((logit - penalty) / T) within a
    6-sigma binomial band; top_k keeps exactly the k best."""
    rng = np.random.default_rng(7)
    logits = rng.normal(0.0, 1.5, 8).astype(np.float32)
    prompt = [3, 3, 5]
    opts = Sampling(temperature=0.8, seed=11, presence_penalty=0.3, frequency_penalty=0.2)
    s = Sampler(opts, prompt, 8)
    counts = np.bincount(prompt, minlength=8).astype(np.float64)
    adj = logits.astype(np.float64) - (0.2 * counts + 0.3 * (counts > 0))
    p = np.exp((adj - adj.max()) / 0.8)
    p /= p.sum()
    n = 40000
    got = np.bincount([s.sample(logits) for _ in range(n)], minlength=8) / n
    assert np.all(np.abs(got - p) <= 6 * np.sqrt(p * (1 - p) / n) + 1e-9)

    s = Sampler(Sampling(temperature=1.0, top_k=3, seed=12), [], 8)
    drawn = {s.sample(logits) for _ in range(2000)}
    assert drawn == set(np.argsort(-logits.astype(np.float64), kind="stable")[:3].tolist())


def test_seeded_streams_repeat_and_unseeded_streams_differ():
    opts = Sampling(temperature=1.5, seed=2024)
    logits = np.zeros(64, dtype=np.float32)
    s1, s2 = Sampler(opts, [], 64), Sampler(opts, [], 64)
    assert [s1.sample(logits) for _ in range(200)] == [s2.sample(logits) for _ in range(200)]
    u1, u2 = Sampler(Sampling(temperature=1.5), [], 64), Sampler(Sampling(temperature=1.5), [], 64)
    assert [u1.sample(logits) for _ in range(200)] != [u2.sample(logits) for _ in range(200)]


# ---------------------------------------------------------- random stream
def _block(state: list[int], rounds: int) -> list[int]:
    i = (C.c_uint32 * 16)(*state)
    o = (C.c_uint32 * 16)()
    abi.lib().chk_chacha_block(i, rounds, o)
    return list(o)


SIGMA = [0x61707865, 0x3320646E, 0x79622D32, 0x6B206574]


def test_chacha_block_rfc8439():
    """RFC 8439 section 2.3.2: key 00..1f, counter 1, nonce
    000000090000004a00000000, 20 rounds."""
    key = bytes(range(32))
    kw = [int.from_bytes(key[4 * i:4 * i + 4], "little") for i in range(8)]
    nonce = bytes.fromhex("000000090000004a00000000")
    nw = [int.from_bytes(nonce[4 * i:4 * i + 4], "little") for i in range(3)]
    out = _block(SIGMA + kw + [1] + nw, 20)
    assert out == [0xE4E7F110, 0x15593BD1, 0x1FDD0F50, 0xC47120A3, 0xC7F4D1C7, 0x0368C033, 0x9AAA2204, 0x4E6CD4C3,
                   0x466482D2, 0x09AA9F07, 0x05D7C214, 0xA2028BD9, 0xD19C12B5, 0xB94E16DE, 0xE883D0CB, 0x4E3C50A2]


@pytest.mark.parametrize("rounds,first32", [
    (20, "76b8e0ada0f13d90405d6ae55386bd28bdd219b8a08ded1aa836efcc8b770dc7"),
    (12, "9bf49a6a0755f953811fce125f2683d50429c3bb49e074147e0089a52eae155f"),
    (8, "3e00ef2f895f40d67f5bb8e81f09a5a12c840ec3ce9a7f3b181be188ef711a1e"),
])
def test_chacha_zero_key_keystreams(rounds, first32):
    """The first 32 keystream bytes of ChaCha20/12/8 under the all-zero key
    and nonce (RFC 8439 appendix A.1 for 20 rounds; the published
    reduced-round test vectors for 12 and 8)."""
    out = _block(SIGMA + [0] * 12, rounds)
    assert b"".join(w.to_bytes(4, "little") for w in out)[:32].hex() == first32


def test_pcg32_reference_outputs():
    """pcg32_srandom_r(42, 54) then pcg32_random_r: the PCG reference
    generator's first outputs (its pcg32-demo)."""
    out = (C.c_uint32 * 6)()
    abi.lib().chk_pcg32(42, 54, out, 6)
    assert list(out) == [0xA15C02B7, 0x7B47F409, 0xBA1D3330, 0x83D2F293, 0xBFA4784B, 0xCBED606E]


def test_stdrng_from_seed_value_stability():
    """rand's StdRng value-stability vector: from_seed of the bytes below
    gives next_u64 = 10719222850664546238; a second StdRng seeded by 32
    bytes filled from the first (words 2..9 of its stream) gives
    14064965282130556830."""
    seed = bytes([1, 0, 0, 0, 23, 0, 0, 0, 200, 1, 0, 0, 210, 30, 0, 0] + [0] * 16)
    d = rng_u64(5, seed32=seed)
    assert d[0] == 10719222850664546238
    words = []
    for v in d[1:5]:
        words += [v & 0xFFFFFFFF, v >> 32]
    seed2 = b"".join(w.to_bytes(4, "little") for w in words)
    assert rng_u64(1, seed32=seed2)[0] == 14064965282130556830


def test_seed_from_u64_is_from_seed_of_pcg32_words():
    """seed_from_u64(s) = from_seed(eight PCG32 outputs, each taken after a
    step from s, little-endian).  The PCG32 reference generator emits the
    output of its state before each step and, seeded with (s - INC, INC >> 1),
    starts from the state one step after s, so it yields the same words."""
    inc = 11634580027462260723
    for s in (0, 1, 42, 2**64 - 1):
        out = (C.c_uint32 * 8)()
        abi.lib().chk_pcg32((s - inc) % 2**64, inc >> 1, out, 8)
        seed32 = b"".join(int(w).to_bytes(4, "little") for w in out)
        assert rng_u64(70, seed=s) == rng_u64(70, seed32=seed32)


def test_stream_crosses_block_refills():
    """64 words per refill: the 33rd next_u64 starts the second refill,
    whose first block is block counter 4 of the same key."""
    seed = bytes(range(32))
    d = rng_u64(40, seed32=seed)
    kw = [int.from_bytes(seed[4 * i:4 * i + 4], "little") for i in range(8)]
    blk4 = _block(SIGMA + kw + [4, 0, 0, 0], 12)
    assert d[32] == blk4[0] | blk4[1] << 32
    blk0 = _block(SIGMA + kw + [0, 0, 0, 0], 12)
    assert d[0] == blk0[0] | blk0[1] << 32
