"""GPU parity of the Q8_0 path (token_embd / lm_head with --quant-embed) against the oracle.

Q8_0 rows follow genomic_dot_product_q8_0_avx2's order (genomic.rs:377-448) and
the embedding rows dequantize_weight (blocks.rs:43-49), so the bar is bit-for-bit
equality with the oracle, for the operators and for whole models.
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q8_TAIL_PAD = 4096
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


def _q8_rows(O, n, k, seed):
    w = (0.05 * np.random.default_rng(seed).standard_normal(n * k)).astype(np.float32)
    return O.q8_0_quantize(w)


def pack_q8_0_numpy(blocks, n, k):
    """Tiles of 8 rows; per group of four blocks the 8 rows' codes (chain l's 16
    bytes at 16l: dword b = block 4g+b, byte c = element 8c+l), then the 8 rows'
    four f16 scales; missing rows and blocks are zero."""
    nb = k // 32
    G = (nb + 3) // 4
    T = (n + 7) // 8
    b = np.zeros((8 * T, 4 * G, 34), np.uint8)
    b[:n, :nb] = np.asarray(blocks, np.uint8).reshape(n, nb, 34)
    q = b[:, :, 2:].reshape(T, 8, G, 4, 4, 8)            # [tile][row][g][block][c][l]
    codes = q.transpose(0, 2, 1, 5, 3, 4).reshape(T, G * 1024)
    sc = b[:, :, :2].reshape(T, 8, G, 8).transpose(0, 2, 1, 3).reshape(T, G * 64)
    return np.concatenate([codes, sc], axis=1).reshape(-1)


@pytest.mark.parametrize("n,k", [(3, 896), (5, 32), (4, 96), (7, 576), (17, 1536), (16, 224)])
def test_q8_0_pack_layout(hip, O, n, k):
    blocks = _q8_rows(O, n, k, 1)
    packed = hip.ops.q8_0_upload(blocks, n, k)
    ref = pack_q8_0_numpy(blocks, n, k)
    got = packed.read(np.uint8)
    assert packed.nbytes == hip.ops.q8_0_packed_bytes(n, k) == ref.size + Q8_TAIL_PAD
    assert np.array_equal(got[:ref.size], ref)
    assert not got[ref.size:].any()


@pytest.mark.parametrize("n,k", [(151936, 896), (4864, 896), (963, 576), (17, 1536), (64, 8960), (5, 32),
                                 (9, 96), (11, 160), (300, 8192)])
def test_q8_0_gemv(hip, O, n, k):
    blocks = _q8_rows(O, n, k, n + k)
    x = hip.synth.normal(12, f"x8.{k}", k)
    bias = hip.synth.normal(13, f"b8.{n}", n // 2, 0.0, 0.02)
    y = hip.ops.DeviceBuffer(n * 4)
    hip.ops.q8_0_gemv(hip.ops.q8_0_upload(blocks, n, k), hip.ops.DeviceBuffer.from_array(x), y, n, k,
                      bias=hip.ops.DeviceBuffer.from_array(bias) if bias.size else None, bias_len=bias.size)
    got = y.read(np.float32)
    L = O.GenomicLinear(blocks, b"", None, n, k, bias, 8)
    assert same_bits(got, L.forward_core(x))


@pytest.mark.parametrize("n,k", [(151936, 896), (65547, 896), (70001, 1024), (20000, 512), (16400, 128)])
def test_q8_0_gemv_long_no_bias(hip, O, n, k):
    """Long Q8_0 matrices without a bias take the LDS-staged kernel (16-row
    super-tiles): a partial last tile, an odd tile count (the last super-tile
    half past the rows), K = 1024 (8 groups) and one-group rows; bit for bit."""
    blocks = _q8_rows(O, n, k, n + 2 * k)
    x = hip.synth.normal(14, f"x8l.{k}", k)
    y = hip.ops.DeviceBuffer(n * 4)
    hip.ops.q8_0_gemv(hip.ops.q8_0_upload(blocks, n, k), hip.ops.DeviceBuffer.from_array(x), y, n, k)
    got = y.read(np.float32)
    L = O.GenomicLinear(blocks, b"", None, n, k, None, 8)
    assert same_bits(got, L.forward_core(x))


def test_q8_0_dequant_every_code_and_edge_scale(hip, O):
    codes = np.arange(256, dtype=np.uint8)
    scales = np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0x7BFF, 0xBC00, 0xFBFF, 0x2E66, 0x7C00, 0xFC00],
                      np.uint16)
    blocks = []
    for s in scales:
        for part in range(8):
            b = np.zeros(34, np.uint8)
            b[0:2] = np.frombuffer(np.uint16(s).tobytes(), np.uint8)
            b[2:] = codes[32 * part:32 * part + 32]
            blocks.append(b)
    blocks = np.concatenate(blocks)
    nb = blocks.size // 34
    out = hip.ops.DeviceBuffer(nb * 32 * 4)
    hip.ops.q8_0_dequant(hip.ops.DeviceBuffer.from_array(blocks), out, nb)
    got = out.read(np.float32)
    ref = O.q8_0_dequant(blocks)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def _write(hip, path, **kw):
    if not os.path.exists(path):
        hip.synth.write_flat(str(path), **kw)
    return str(path)


@pytest.mark.parametrize("tied", [0, 1])
def test_q8_0_embeddings_model_stream(hip, O, tmp_models, tied):
    kw = dict(TINY)
    kw.update(tied_embeddings=tied, quant_embed=1)
    p = _write(hip, tmp_models / f"tiny_q8_{tied}.flat", seed=7, **kw)
    g = hip.load_genomic_auto(p)
    r = O.load_genomic(p)
    assert r.embeddings.kind == O.KIND_Q8_0 and r.lm_head.kind == O.KIND_Q8_0
    g.set_k_wta_ratio(0.0)
    r.set_k_wta_ratio(0.0)
    toks = [int(t) for t in np.random.default_rng(3).integers(0, TINY["vocab_size"], 12)]
    for i, t in enumerate(toks):
        gl, gh = g.forward_with_hidden(t, i == 0)
        rl, rh = r.forward_with_hidden_core(t, i == 0)
        assert same_bits(gh, rh), f"h_norm differs at token {i}"
        assert same_bits(gl, rl), f"logits differ at token {i}"
    # greedy decode continuing both caches (first fed token: toks[-1] again)
    out = g.decode_greedy(toks[-1], 10)
    tok = toks[-1]
    for i in range(10):
        tok = O.argmax_first(r.forward_core(tok))
        assert int(out[i]) == tok
    g.close()


def test_q8_0_benchmark_shape(hip, O, tmp_models):
    """Qwen2-0.5B shape with Q8_0 token_embd / lm_head (151936 x 896): three tokens' logits, then
    three greedy tokens through the lm_head's device argmax."""
    p = _write(hip, tmp_models / "qwen2-0.5b_q8.flat", preset="qwen2-0.5b", seed=0, quant_embed=1)
    g = hip.load_genomic_auto(p)
    r = O.load_genomic(p)
    g.set_k_wta_ratio(0.0)
    r.set_k_wta_ratio(0.0)
    for i, t in enumerate([11, 2024, 151000]):
        assert same_bits(g.forward(t, i == 0), r.forward_core(t, i == 0)), f"token {i}"
    # the lm_head's device argmax (greedy decode), continuing both caches
    out = g.decode_greedy(151000, 3)
    tok = 151000
    for i in range(3):
        tok = O.argmax_first(r.forward_core(tok))
        assert int(out[i]) == tok, f"greedy token {i}"
    g.close()
