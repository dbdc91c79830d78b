"""GPU parity of the 2-bit (Genomic2Bit) path against the oracle.

The matvec follows genomic_dot_product's x86 AVX2 branch (genomic.rs:17-144)
over the row slicing of linear/forward.rs:33-57, and the embedding rows
get_row_core (forward.rs:210-237), so the bar is bit-for-bit equality with the
oracle for the operator, for every centroid-table form, and for whole models
with 2-bit bodies.
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


def same_bits(a, b) -> bool:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _gemv(hip, codes, cent, n, k, x, bias=None, modulation=None):
    D = hip.ops.DeviceBuffer
    y = D(n * 4)
    cb = D.from_array(cent) if cent is not None and cent.size else None
    hip.ops.bit2_gemv(D.from_array(codes), cb, 0 if cent is None else cent.size, D.from_array(x), y, n, k,
                      modulation=modulation, bias=D.from_array(bias) if bias is not None and bias.size else None,
                      bias_len=0 if bias is None else bias.size)
    return y.read(np.float32)


@pytest.mark.parametrize("n,k", [(4864, 896), (896, 4864), (1152, 896), (17, 1536), (5, 32), (9, 96),
                                 (300, 8192), (131, 256)])
def test_2bit_gemv_per_row_tables(hip, O, n, k):
    codes, cent = hip.synth.bit2_tensor(3, f"g2.{n}.{k}", n, k)
    x = hip.synth.normal(4, f"x2.{k}", k)
    bias = hip.synth.normal(5, f"b2.{n}", n // 2, 0.0, 0.02)
    got = _gemv(hip, codes, cent, n, k, x, bias)
    L = O.GenomicLinear(codes, b"", cent, n, k, bias, 2)
    assert same_bits(got, L.forward_core(x))


@pytest.mark.parametrize("form", ["shared", "column", "partial", "none"])
def test_2bit_gemv_table_forms(hip, O, form):
    n, k = 203, 640
    nb = k // 32
    codes, cent = hip.synth.bit2_tensor(6, "g2.forms", n, k)
    x = hip.synth.normal(7, "x2.forms", k)
    table = {"shared": cent[:4], "column": cent[:nb * 4], "partial": cent[:int(70.5 * nb * 4)],
             "none": np.zeros(0, np.float32)}[form]
    got = _gemv(hip, codes, table, n, k, x)
    L = O.GenomicLinear(codes, b"", table, n, k, None, 2)
    assert same_bits(got, L.forward_core(x))


def test_2bit_gemv_modulation(hip, O):
    n, k = 97, 512
    codes, cent = hip.synth.bit2_tensor(8, "g2.mod", n, k)
    x = hip.synth.normal(9, "x2.mod", k)
    m = np.array([0.75, 1.5, -0.5, 2.25], np.float32)
    got = _gemv(hip, codes, cent, n, k, x, modulation=m)
    nb = k // 32
    ref = np.array([O.dot_2bit(codes[i * nb * 8:(i + 1) * nb * 8], x, cent[i * nb * 4:(i + 1) * nb * 4], m)
                    for i in range(n)], np.float32)
    assert same_bits(got, ref)


def _write(hip, path, **kw):
    if not os.path.exists(path):
        hip.synth.write_flat(str(path), **kw)
    return str(path)


@pytest.mark.parametrize("fused", [True, False])
def test_2bit_model_stream(hip, O, tmp_models, fused):
    p = _write(hip, tmp_models / f"tiny_2bit_{int(fused)}.flat", seed=9, body_format=hip.synth.BIT2,
               fused=fused, **TINY)
    g = hip.load_genomic_auto(p)
    r = O.load_genomic(p)
    assert g.info["body_format"] == 4
    g.set_k_wta_ratio(0.0)
    r.set_k_wta_ratio(0.0)
    toks = [int(t) for t in np.random.default_rng(4).integers(0, TINY["vocab_size"], 14)]
    for i, t in enumerate(toks):
        gl, gh = g.forward_with_hidden(t, i == 0)
        rl, rh = r.forward_with_hidden_core(t, i == 0)
        assert same_bits(gh, rh), f"h_norm differs at token {i}"
        assert same_bits(gl, rl), f"logits differ at token {i}"
    out = g.decode_greedy(toks[-1], 10)
    tok = toks[-1]
    for i in range(10):
        tok = O.argmax_first(r.forward_core(tok))
        assert int(out[i]) == tok
    g.close()


@pytest.mark.parametrize("tables,tied", [(0, 0), (1, 1), (2, 0), (3, 0), (3, 1)])
def test_2bit_embeddings_and_table_forms(hip, O, tmp_models, tables, tied):
    """token_embd / lm_head as 2-bit too, with each centroid-table form on every tensor
    (form 3 leaves rows past the first half without tables, and row 500 with its
    first block's only)."""
    kw = dict(TINY)
    kw.update(tied_embeddings=tied)
    p = _write(hip, tmp_models / f"tiny_2bit_e{tables}_{tied}.flat", seed=13, body_format=hip.synth.BIT2,
               quant_embed=2, g2_tables=tables, **kw)
    g = hip.load_genomic_auto(p)
    r = O.load_genomic(p)
    assert r.embeddings.kind == O.KIND_2BIT and r.lm_head.kind == O.KIND_2BIT
    g.set_k_wta_ratio(0.0)
    r.set_k_wta_ratio(0.0)
    for i, t in enumerate([0, 499, 500, 501, 999, 250, 750]):
        gl, gh = g.forward_with_hidden(t, i == 0)
        rl, rh = r.forward_with_hidden_core(t, i == 0)
        assert same_bits(gh, rh), f"h_norm differs at token {i}"
        assert same_bits(gl, rl), f"logits differ at token {i}"
    g.close()


def test_2bit_model_kwta_on(hip, O, tmp_models):
    """The default K-WTA ratio (0.5 on the logits) over a 2-bit body."""
    p = _write(hip, tmp_models / "tiny_2bit_1.flat", seed=9, body_format=hip.synth.BIT2, fused=True, **TINY)
    g = hip.load_genomic_auto(p)
    r = O.load_genomic(p)
    for i, t in enumerate([5, 17, 999, 3]):
        assert same_bits(g.forward(t, i == 0), r.forward_core(t, i == 0)), f"token {i}"
    g.close()


def test_2bit_benchmark_shape(hip, O, tmp_models):
    """Qwen2-0.5B shapes with a 2-bit body (24 blocks), three tokens."""
    p = _write(hip, tmp_models / "qwen2-0.5b_2bit.flat", preset="qwen2-0.5b", seed=1, body_format=hip.synth.BIT2)
    g = hip.load_genomic_auto(p)
    r = O.load_genomic(p)
    g.set_k_wta_ratio(0.0)
    r.set_k_wta_ratio(0.0)
    for i, t in enumerate([11, 2024, 151000]):
        assert same_bits(g.forward(t, i == 0), r.forward_core(t, i == 0)), f"token {i}"
    g.close()


def test_2bit_body_refused_by_matrix_paths(hip, tmp_models):
    from gaje_hip._lib import GajeError
    p = _write(hip, tmp_models / "tiny_2bit_1.flat", seed=9, body_format=hip.synth.BIT2, fused=True, **TINY)
    g = hip.load_genomic_auto(p)
    with pytest.raises(GajeError):
        g.prefill_mfma(np.arange(8, dtype=np.uint32))
    with pytest.raises(Exception):
        hip.GenomicBatch(g, 2, 64)
    g.close()
