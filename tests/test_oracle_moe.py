"""The MoE routing restated in the oracle, pinned by what the mathematics fixes.

No reference function routes tokens (the reference has no MoE), so the routing
semantics are parity unpinned; what is checked here is that the oracle computes
the semantics it states: its logits are the reference dot_product, its top-2
agrees with a float64 softmax wherever there is no near-tie, ties go to the lower
expert id, and the weights are the renormalised pair.
"""
import numpy as np


def test_moe_route_against_float64_softmax():
    from oracle import oracle as O
    rng = np.random.default_rng(3)
    T, h, E = 64, 96, 6
    x = rng.standard_normal((T, h)).astype(np.float32)
    router = (0.3 * rng.standard_normal((E, h))).astype(np.float32)
    idx, w = O.moe_route(x, router)
    l64 = x.astype(np.float64) @ router.astype(np.float64).T
    p64 = np.exp(l64 - l64.max(axis=1, keepdims=True))
    p64 /= p64.sum(axis=1, keepdims=True)
    order = np.argsort(-p64, axis=1, kind="stable")
    for t in range(T):
        srt = np.sort(p64[t])[::-1]
        if srt[0] - srt[1] > 1e-5 and srt[1] - srt[2] > 1e-5:
            assert list(idx[t]) == list(order[t, :2])
        a, b = idx[t]
        ref = p64[t, [a, b]] / (p64[t, a] + p64[t, b])
        assert np.allclose(w[t], ref, rtol=2e-6, atol=1e-7)
        assert abs(float(w[t, 0]) + float(w[t, 1]) - 1.0) < 3e-7
        assert w[t, 0] >= w[t, 1]


def test_moe_route_ties_and_logits():
    from oracle import oracle as O
    h, E = 32, 4
    x = np.ones((1, h), np.float32)
    router = np.zeros((E, h), np.float32)  # all logits equal: experts 0 and 1, weights 1/2
    idx, w = O.moe_route(x, router)
    assert list(idx[0]) == [0, 1] and list(w[0]) == [0.5, 0.5]
    router[2] = 1.0 / 32  # expert 2 first; experts 0, 1, 3 tie for second: the lowest id
    idx, w = O.moe_route(x, router)
    assert list(idx[0]) == [2, 0]
    # the logits are the reference dot_product (a single exact case)
    assert O.dot_f32(x[0], router[2]) == 1.0
