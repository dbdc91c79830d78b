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
expected stream.  The multinomial branch (thread_rng upstream) stays unpinned.
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
