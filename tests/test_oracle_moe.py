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


def _random_q4_0(rng, n, k):
    """n rows of k/32 Q4_0Blocks: codes uniform in 0..15, f16 scale in
    [0.01, 0.05), min = -7.5 * scale (a centred affine grid)."""
    nb = n * k // 32
    scale = rng.uniform(0.01, 0.05, nb).astype(np.float16)
    mn = (np.float32(-7.5) * scale.astype(np.float32)).astype(np.float16)
    codes = rng.integers(0, 16, (nb, 32)).astype(np.uint8)
    blk = np.zeros((nb, 20), np.uint8)
    blk[:, 0:2] = scale.view(np.uint8).reshape(nb, 2)
    blk[:, 2:4] = mn.view(np.uint8).reshape(nb, 2)
    blk[:, 4:] = codes[:, 0::2] | (codes[:, 1::2] << 4)
    return blk.reshape(-1)


def _moe_f64(x, idx, w, gate_up, down, ffn):
    """The MoE layer composed in float64 from the exactly dequantised experts:
    y_t = w_a FFN_a(x_t) + w_b FFN_b(x_t), FFN_e(x) = D_e (silu(g) * u) with
    [g; u] = GU_e x and silu taken on the gate clamped to [-64, 64]
    (activation.rs:35-51: sigma of the clamped gate times the raw gate)."""
    from oracle import oracle as O
    h = x.shape[1]
    GU = [O.q4_0_dequant(b).astype(np.float64).reshape(2 * ffn, h) for b in gate_up]
    D = [O.q4_0_dequant(b).astype(np.float64).reshape(h, ffn) for b in down]
    y = np.zeros(x.shape, np.float64)
    for t in range(x.shape[0]):
        for k in range(2):
            e = int(idx[t, k])
            gu = GU[e] @ x[t].astype(np.float64)
            g, u = gu[:ffn], gu[ffn:]
            sig = 1.0 / (1.0 + np.exp(-np.clip(g, -64.0, 64.0)))
            y[t] += float(w[t, k]) * (D[e] @ (g * sig * u))
    return y


def _rel(got, ref):
    from conftest import floored_rel_err
    return floored_rel_err(got, ref)


def test_moe_ffn_against_float64_composition(monkeypatch):
    """The oracle's expert dispatch and combine against a float64 composition of
    the same routing; a swapped pair of routing weights, a wrong expert for the
    second slot, or gate and up exchanged in the oracle each leave the bound."""
    from oracle import oracle as O
    rng = np.random.default_rng(11)
    T, h, ffn, E = 10, 64, 96, 4
    x = rng.standard_normal((T, h)).astype(np.float32)
    router = (0.3 * rng.standard_normal((E, h))).astype(np.float32)
    gate_up = [_random_q4_0(rng, 2 * ffn, h) for _ in range(E)]
    down = [_random_q4_0(rng, h, ffn) for _ in range(E)]
    y, idx, w = O.moe_ffn(x, router, gate_up, down, ffn)
    assert not np.array_equal(w[:, 0], w[:, 1])  # the swap below changes something
    ref = _moe_f64(x, idx, w, gate_up, down, ffn)
    err = _rel(y, ref)
    assert err < 1e-4, err  # float32 rounding of two chained products and the combine

    route = O.moe_route
    # slip 1: the routing weights swapped between the two experts
    monkeypatch.setattr(O, "moe_route", lambda x_, r_: (route(x_, r_)[0], route(x_, r_)[1][:, ::-1].copy()))
    assert _rel(O.moe_ffn(x, router, gate_up, down, ffn)[0], ref) > 1e-2
    # slip 2: the second slot takes the next expert
    monkeypatch.setattr(O, "moe_route", lambda x_, r_: (np.stack([route(x_, r_)[0][:, 0],
                                                                  (route(x_, r_)[0][:, 1] + 1) % E], 1),
                                                        route(x_, r_)[1]))
    assert _rel(O.moe_ffn(x, router, gate_up, down, ffn)[0], ref) > 1e-2
    monkeypatch.setattr(O, "moe_route", route)
    # slip 3: gate and up exchanged
    sw = O.swiglu_balanced
    monkeypatch.setattr(O, "swiglu_balanced", lambda g, u: sw(u, g))
    assert _rel(O.moe_ffn(x, router, gate_up, down, ffn)[0], ref) > 1e-2
