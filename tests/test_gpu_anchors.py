"""GPU parity of sparse f16 anchors (GenomicLinear::new, src/nn/linear/init.rs:61-107;
compute_single_row, src/nn/linear/forward.rs:103-112) against the CPU oracle.

Every body tensor of these synthetic models carries a "GAJE" anchor buffer in
one of the three forms the writer produces (n+1 row pointers with columns past
in_features and an inverted row range; genomize_4bit_core's two pointers; none),
over Q4_0, LUT-4bit and 2-bit rows, fused and split tensors.  The device adds
each row's anchors after the row dot and before the bias, in the reference
order, so the logits must equal the oracle's bit for bit.
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TINY = dict(n_embd=128, n_head=4, n_head_kv=2, n_blocks=2, ffn=256, vocab_size=1000, eps=1e-6,
            rope_base=1e4, arch_family=1, qkv_bias=1, tied_embeddings=0)


@pytest.fixture(scope="module")
def hip():
    import gaje_hip
    if gaje_hip.ops.device_count() < 1:
        pytest.fail("no HIP device visible")
    return gaje_hip


@pytest.fixture(scope="module")
def O():
    from oracle import oracle
    return oracle


def _write(hip, path, **kw):
    if not os.path.exists(path):
        hip.synth.write_flat(str(path), **kw)
    return str(path)


def same_bits(a, b) -> bool:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _stream(hip, O, path, n, seed):
    toks = [int(t) for t in np.random.default_rng(seed).integers(0, TINY["vocab_size"], n)]
    g = hip.load_genomic_auto(path)
    r = O.load_genomic(path)
    g.set_k_wta_ratio(0.0)
    r.set_k_wta_ratio(0.0)
    for i, t in enumerate(toks):
        gl, rl = g.forward(t, i == 0), r.forward_core(t, i == 0)
        assert same_bits(gl, rl), f"logits differ at token {i}"
    out = g.decode_greedy(toks[-1], 6)
    tok = toks[-1]
    for i in range(6):
        tok = O.argmax_first(r.forward_core(tok))
        assert int(out[i]) == tok, f"greedy token {i}"
    g.close()


@pytest.mark.parametrize("form", [1, 2, 3])
@pytest.mark.parametrize("fmt,fused", [(1, True), (1, False), (2, True), (4, True)])
def test_anchored_model_stream(hip, O, tmp_models, form, fmt, fused):
    p = _write(hip, tmp_models / f"anc_{form}_{fmt}_{int(fused)}.flat", seed=30 + form, body_format=fmt,
               fused=fused, anchors=form, **TINY)
    _stream(hip, O, p, 7, form + 10 * fmt)


def test_anchored_benchmark_shape(hip, O, tmp_models):
    """Qwen2-0.5B block shapes (the split QKV/o/down kernels and the row-per-lane gate_up), 2 blocks."""
    p = _write(hip, tmp_models / "anc_c2_2blk.flat", preset="qwen2-0.5b", seed=2, n_blocks=2, vocab_size=2048,
               anchors=1)
    toks = [int(t) for t in np.random.default_rng(3).integers(0, 2048, 4)]
    g = hip.load_genomic_auto(p)
    r = O.load_genomic(p)
    g.set_k_wta_ratio(0.0)
    r.set_k_wta_ratio(0.0)
    for i, t in enumerate(toks):
        assert same_bits(g.forward(t, i == 0), r.forward_core(t, i == 0)), f"token {i}"
    g.close()


def test_anchored_batch(hip, O, tmp_models):
    p = _write(hip, tmp_models / "anc_1_1_1.flat", seed=31, body_format=1, fused=True, anchors=1, **TINY)
    rng = np.random.default_rng(5)
    prompts = [[int(t) for t in rng.integers(0, TINY["vocab_size"], 6)] for _ in range(3)]
    g = hip.load_genomic_auto(p)
    g.set_k_wta_ratio(0.0)
    b = hip.GenomicBatch(g, 3, 64)
    logits = b.feed(np.array(prompts, np.uint32), want_logits=True)
    for s, pr in enumerate(prompts):
        r = O.load_genomic(p)
        r.set_k_wta_ratio(0.0)
        last = None
        for i, t in enumerate(pr):
            last = r.forward_core(t, i == 0)
        assert same_bits(logits[s], last), f"sequence {s}"
    b.close()
    g.close()


def test_anchored_prefill_mfma_unsupported(hip, tmp_models):
    from gaje_hip._lib import GajeError
    p = _write(hip, tmp_models / "anc_1_1_1.flat", seed=31, body_format=1, fused=True, anchors=1, **TINY)
    g = hip.load_genomic_auto(p)
    with pytest.raises(GajeError):
        g.prefill_mfma([1, 2, 3])
    g.close()
