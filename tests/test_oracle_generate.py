"""Known answers for the oracle's generate_native_core (src/nn/llm/forward.rs:215-330).

The loop around the model is pinned here by hand-worked token streams: a stub
whose forward_core replays scripted logits stands in for the model, so each
expected sequence follows from the reference's rules alone:
  - penalty (:243-260): for every generated id (EOS ids removed), a negative
    logit is multiplied by the penalty and a positive one divided, only when
    penalty > 1.0;
  - greedy argmax (:262-271): strict '>', so the first maximum wins;
  - EOS (:300-302): the token is emitted and generation stops;
  - loop detector (:305-318): after each token, for w = 2..=48, stop when the
    last three w-long chunks are equal.
Each case is chosen so that a plausible slip (penalty sign rule swapped, '>='
in the argmax, detector bounds off by one, EOS not emitted) changes the
expected stream.

The multinomial branch (:272-297) draws from thread_rng upstream, so no token
stream is fixed there; what it does fix is pinned instead: the distribution
(a chi-square test of seeded draws against softmax(l / T) in float64, which a
temperature applied the wrong way or a dropped 1/T fails), the near-greedy
limit (T just above 1e-5 with a clear maximum always picks it), and the order
of the penalty before the draw.
"""
import numpy as np
import pytest

from oracle import oracle as O


class _Stub:
    """forward_core(tid) -> logits from `table(tid, step)`; counts the prompt too."""

    def __init__(self, table):
        self.table = table
        self.calls = []

    def clear_cache_core(self):
        self.calls.clear()

    def forward_core(self, tid, clear_cache=False):
        self.calls.append(int(tid))
        return np.asarray(self.table(int(tid), len(self.calls)), dtype=np.float32)


def _gen(table, prompt, max_new, penalty=1.0, eos=(), temperature=0.0):
    stub = _Stub(table)
    out = O.GenomicLLM.generate_native_core(stub, list(prompt), max_new, temperature, penalty, list(eos))
    return out, stub.calls


def test_penalty_divides_positive_logit():
    # logits fixed at [2.0, 1.5, -3, -3]; penalty 1.5
    # step 1: 0; step 2: 2/1.5 = 1.333 < 1.5 -> 1; then 1.333 > 1.0 -> 0 forever;
    # the detector (w = 2) first sees three equal chunks [0,0][0,0][0,0] at 8
    # tokens (at 7 the oldest chunk is [1,0]).
    out, calls = _gen(lambda t, n: [2.0, 1.5, -3.0, -3.0], [3], 50, penalty=1.5)
    assert out == [0, 1, 0, 0, 0, 0, 0, 0]
    # the prompt and every token except the last are fed back
    assert calls == [3, 0, 1, 0, 0, 0, 0, 0]


def test_penalty_multiplies_negative_logit():
    # [-1.0, -1.2, -5, -5]: -1.0 * 1.5 = -1.5 < -1.2 -> 1; then -1.5 > -1.8 -> 0
    out, _ = _gen(lambda t, n: [-1.0, -1.2, -5.0, -5.0], [2], 50, penalty=1.5)
    assert out == [0, 1, 0, 0, 0, 0, 0, 0]


def test_penalty_off_at_one_and_below():
    for p in (1.0, 0.5):
        out, _ = _gen(lambda t, n: [2.0, 1.5, -3.0], [1], 50, penalty=p)
        assert out == [0] * 6  # constant stream: w = 2 fires at 6


def test_penalty_rounding_is_float32():
    # 1.0 / 1.1 rounds in float32 to 0.90909094; a competitor at 0.90909094
    # ties and loses to the lower index, at 0.9090910 (next float) it wins.
    a = np.float32(np.float32(1.0) / np.float32(1.1))
    for comp, want in ((a, 0), (np.nextafter(a, np.float32(2)), 1)):
        out, _ = _gen(lambda t, n, c=comp: [1.0, c, -9.0], [2], 2, penalty=1.1)
        assert out[1] == want


def test_argmax_first_maximum():
    out, _ = _gen(lambda t, n: [1.0, 3.0, 3.0, -np.inf], [0], 1)
    assert out == [1]
    out, _ = _gen(lambda t, n: [np.nan, 2.0, np.nan, 2.0], [0], 1)
    assert out == [1]
    out, _ = _gen(lambda t, n: [np.nan, -np.inf], [0], 1)
    assert out == [0]


@pytest.mark.parametrize("w", [2, 3, 17, 48])
def test_detector_fires_at_three_periods(w):
    # input t -> next token (t + 1) % w: the stream 0, 1, ..., w-1, 0, ... has
    # period w and no shorter one, so it stops at exactly 3w tokens
    def table(t, n):
        v = np.full(64, -1.0, dtype=np.float32)
        v[(t + 1) % w] = 1.0
        return v
    out, _ = _gen(table, [w - 1], 400)
    assert len(out) == 3 * w
    assert out == [i % w for i in range(3 * w)]


def test_detector_ignores_period_49():
    def table(t, n):
        v = np.full(64, -1.0, dtype=np.float32)
        v[(t + 1) % 49] = 1.0
        return v
    out, _ = _gen(table, [48], 200)
    assert len(out) == 200  # 49 > 48 and 98 > 48: never fires; max_new ends it


def test_detector_constant_stream_and_max_new():
    out, _ = _gen(lambda t, n: [0.0, 5.0], [0], 100)
    assert out == [1] * 6
    out, _ = _gen(lambda t, n: [0.0, 5.0], [0], 4)
    assert out == [1] * 4
    out, calls = _gen(lambda t, n: [0.0, 5.0], [0, 1, 0], 0)
    assert out == [] and calls == [0, 1, 0]


def test_eos_is_emitted_and_stops():
    # stream 0,1,2,3,... with EOS 4: the EOS token is the last one returned and
    # is not fed back (no forward after it)
    def table(t, n):
        v = np.zeros(16, dtype=np.float32)
        v[(t + 1) % 16] = 1.0
        return v
    out, calls = _gen(table, [15], 50, eos=[4, 9])
    assert out == [0, 1, 2, 3, 4]
    assert calls == [15, 0, 1, 2, 3]


def test_eos_ids_not_penalised():
    # The reference drops EOS ids from the penalty's seen-set (:250-252).  A
    # generated EOS ends the loop at once, so no later step can see it there:
    # the removal leaves no trace in the output, and the stream equals the one
    # without it.  Penalty with an EOS id that is never generated changes nothing.
    base, _ = _gen(lambda t, n: [2.0, 1.5, -3.0, -3.0], [3], 50, penalty=1.5)
    with_eos, _ = _gen(lambda t, n: [2.0, 1.5, -3.0, -3.0], [3], 50, penalty=1.5, eos=[3])
    assert base == with_eos == [0, 1, 0, 0, 0, 0, 0, 0]


def test_empty_prompt_error():
    with pytest.raises(ValueError, match="Prompt tokens cannot be empty"):
        _gen(lambda t, n: [1.0], [], 3)


def test_penalty_three_way_cycle():
    # [3.0, 2.9, 2.8, -1], penalty 1.25: 0; then 2.4 < 2.9 -> 1; then 2.4, 2.32,
    # 2.8 -> 2; then all seen (2.4, 2.32, 2.24) -> 0 forever: [0,1,2,0,0,...],
    # whose last three 2-chunks are first equal at 9 tokens.
    out, _ = _gen(lambda t, n: [3.0, 2.9, 2.8, -1.0], [3], 50, penalty=1.25)
    assert out == [0, 1, 2, 0, 0, 0, 0, 0, 0]


# ---- the multinomial branch (forward.rs:272-297) ---------------------------

_LOGITS = np.array([1.2, -0.4, 2.0, 0.3, 1.9, -2.5, 0.0, 1.1, 0.8, -1.0, 2.2, 0.5], np.float32)


def _chi2(counts, p):
    exp = p * counts.sum()
    return float(((counts - exp) ** 2 / exp).sum())


def test_sampler_distribution_chi_square():
    T, N = 0.7, 20000
    rng = O.SplitMixDraws(12345)
    counts = np.bincount([O.sample_next(_LOGITS, T, rng) for _ in range(N)], minlength=_LOGITS.size)
    l64 = _LOGITS.astype(np.float64)
    p = np.exp((l64 - l64.max()) / T)
    p /= p.sum()
    # 11 degrees of freedom: the 0.999 quantile is 31.26
    assert _chi2(counts, p) < 31.26
    # the test tells the distribution apart from plausible slips
    for wrong in (np.exp((l64 - l64.max()) * T), np.exp(l64 - l64.max())):
        assert _chi2(counts, wrong / wrong.sum()) > 200.0


def test_sampler_numpy_generator_draws():
    # a numpy Generator stands in for thread_rng with the same 24-bit draws
    rng = np.random.default_rng(3)
    counts = np.bincount([O.sample_next(_LOGITS, 1.3, rng) for _ in range(20000)], minlength=_LOGITS.size)
    l64 = _LOGITS.astype(np.float64)
    p = np.exp((l64 - l64.max()) / 1.3)
    assert _chi2(counts, p / p.sum()) < 31.26


def test_sampler_draw_stream():
    # the device library's splitmix stream: state += golden gamma, 24 bits of mix(state)
    d = O.SplitMixDraws(0)
    u = [d() for _ in range(3)]
    st, M = 0, (1 << 64) - 1
    for k in range(3):
        st = (st + 0x9E3779B97F4A7C15) & M
        z = st
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
        z ^= z >> 31
        assert u[k] == np.float32((z >> 40) / 2.0 ** 24)
    assert all(0.0 <= v < 1.0 for v in u)


def test_sampler_near_greedy_limit():
    # T just above the greedy threshold: exp((l - max) / T) underflows to 0 for
    # every logit a clear margin below the maximum, so the maximum is always drawn
    rng = O.SplitMixDraws(7)
    picks = {O.sample_next(_LOGITS, 1.1e-5, rng) for _ in range(2000)}
    assert picks == {int(np.argmax(_LOGITS))}
    # at T = 1e-5 the loop takes the greedy branch and needs no rng at all
    out, _ = _gen(lambda t, n: _LOGITS, [1], 3, temperature=1e-5)
    assert out == [10, 10, 10]


def test_sampler_penalty_applies_before_the_draw():
    # near-greedy sampling with a penalty: 2.2 / 1.5 = 1.467 drops below 2.0,
    # so the second token is 2; a penalty applied after the draw would give 10
    # again.  Then 2.0 / 1.5 = 1.333 and 1.467 -> 1.9 (index 4) wins.
    rng = O.SplitMixDraws(1)
    stub = _Stub(lambda t, n: _LOGITS)
    out = O.GenomicLLM.generate_native_core(stub, [0], 3, 2e-5, 1.5, [], rng=rng)
    assert out == [10, 2, 4]


def test_sampler_needs_an_rng():
    with pytest.raises(ValueError, match="rng"):
        _gen(lambda t, n: _LOGITS, [1], 2, temperature=0.7)


def test_signed_zero_maximum_ties():
    # -0.0 and +0.0 compare equal under the strict '>', so the first one wins
    assert O.argmax_first(np.array([-1.0, -0.0, 0.0, -2.0], np.float32)) == 1
    out, _ = _gen(lambda t, n: [-1.0, -0.0, 0.0, -2.0], [3], 2)
    assert out == [1, 1]
