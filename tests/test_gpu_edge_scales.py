"""Q4_0 matvecs on edge-case f16 scales and mins.

quantize_q4_0_native stores (max - min) / 15 as an f16 (src/compute/
quantize/python.rs:179-220), so any block whose range is below ~9e-4 gets a
subnormal scale, and flat blocks a zero one.  Q4_0Block::dequantize_weight
(src/io/header/blocks.rs:18-30) and the AVX2 row dot (genomic.rs:298-316)
read both halves exactly.  Every Q4_0 matvec form here dequantises through
v_fma_mix_f32 reading the f16 scale and min, so each form is fed the f16 edge
set (+-0, the smallest and largest subnormal, 1, -1, the largest normal and
two ordinary values) and held to the oracle bit for bit:
  - the chain-fed kernel (few rows: the model's qkv / o / down shapes),
  - the split kernel (up to 4096 rows),
  - the LDS-staged kernel, few tiles (C0) and streams,
  - the row-per-lane kernel, short and long rows,
  - the model's own modes (QKV with RoPE, residual, SwiGLU) through a decode
    and the batched matvecs through a two-sequence batch, on a model whose
    blocks carry subnormal and signed-zero scales and mins,
and the block-scaled MFMA product is held to its 2e-3 floored tolerance.
"""
import os

import numpy as np
import pytest

from conftest import floored_rel_err

pytestmark = pytest.mark.gpu

EDGE = np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x3C00, 0x7BFF, 0xBC00, 0x2E66, 0x1400], np.uint16)
SUBNORMAL = np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x0200, 0x8155], np.uint16)


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


def edge_blocks(n, k, seed, halves=EDGE):
    """[n][k/32] Q4_0 blocks with uniform random codes and (scale, min) pairs
    walking every pair of `halves`, offset per row so that each chain, lane and
    block position meets every pair."""
    rng = np.random.default_rng(seed)
    nb = k // 32
    b = np.zeros((n, nb, 20), np.uint8)
    b[:, :, 4:] = rng.integers(0, 256, (n, nb, 16), dtype=np.uint8)
    m = halves.size
    idx = (np.arange(n)[:, None] * 7 + np.arange(nb)[None, :]) % (m * m)
    sc, mn = halves[idx // m], halves[idx % m]
    b[:, :, 0:2] = sc[..., None].view(np.uint8).reshape(n, nb, 2)
    b[:, :, 2:4] = mn[..., None].view(np.uint8).reshape(n, nb, 2)
    return b.reshape(-1)


def _run(hip, O, n, k, bias, seed, native=False):
    blocks = edge_blocks(n, k, seed)
    x = hip.synth.normal(seed, f"edge.x.{k}", k)
    b = hip.synth.normal(seed, f"edge.b.{n}", n, 0.0, 0.02) if bias else None
    y = hip.ops.DeviceBuffer(n * 4)
    kw = dict(bias=hip.ops.DeviceBuffer.from_array(b) if bias else None, bias_len=n if bias else 0)
    if native:
        hip.ops.q4_0_gemv_blocks(hip.ops.DeviceBuffer.from_array(blocks), hip.ops.DeviceBuffer.from_array(x), y, n, k,
                                 **kw)
    else:
        hip.ops.q4_0_gemv(hip.ops.q4_0_upload(blocks, n, k), hip.ops.DeviceBuffer.from_array(x), y, n, k, **kw)
    got = y.read(np.float32)
    ref = O.GenomicLinear(blocks, b"", None, n, k, b, 4).forward_core(x)
    return got, ref


@pytest.mark.parametrize("n,k,bias,form", [
    (1152, 896, True, "chain, qkv shape"),
    (896, 4864, True, "chain, down shape (long rows)"),
    (3000, 896, True, "split"),
    (4864, 896, False, "LDS-staged, few tiles (C0)"),
    (20000, 896, False, "LDS-staged stream"),
    (9000, 896, True, "row per lane, short rows"),
    (5000, 4864, True, "row per lane, long rows"),
    (7, 160, False, "partial groups"),
])
def test_q4_0_gemv_edge_scales(hip, O, n, k, bias, form):
    got, ref = _run(hip, O, n, k, bias, 100 + n % 97)
    assert np.isfinite(ref).all()
    assert same_bits(got, ref), form


@pytest.mark.parametrize("n,k", [(896, 576), (300, 4864)])
def test_q4_0_gemv_blocks_edge_scales(hip, O, n, k):
    """The same scale/min set through the matvec on unpacked Q4_0Block rows."""
    got, ref = _run(hip, O, n, k, True, 300 + n % 89, native=True)
    assert np.isfinite(ref).all()
    assert same_bits(got, ref)


def _scale_blocks_in_file(path, out, every=3):
    """A copy of a flat file in which every `every`-th Q4_0 block of each body
    tensor takes a subnormal / signed-zero (scale, min) pair."""
    from oracle.flat import FlatFile
    ff = FlatFile(path)
    data = bytearray(open(path, "rb").read())
    m = SUBNORMAL.size
    for name, e in ff.tensors.items():
        if e["bit_depth"] != 4 or e["c_len"] != 0 or e["dna_len"] == 0:
            continue
        off = ff.weights_offset + e["dna_off"]
        nblk = e["dna_len"] // 20
        blk = np.frombuffer(bytes(data[off:off + nblk * 20]), np.uint8).reshape(nblk, 20).copy()
        sel = np.arange(0, nblk, every)
        pair = (sel // every) % (m * m)
        blk[sel, 0:2] = SUBNORMAL[pair // m][:, None].view(np.uint8).reshape(-1, 2)
        blk[sel, 2:4] = SUBNORMAL[pair % m][:, None].view(np.uint8).reshape(-1, 2)
        data[off:off + nblk * 20] = blk.tobytes()
    open(out, "wb").write(bytes(data))
    return out


def test_model_modes_and_batch_on_subnormal_scales(hip, O, tmp_models):
    """The decode step's matvec modes and the batched matvecs, bit for bit."""
    raw = str(tmp_models / "edge_raw.flat")
    hip.synth.write_flat(raw, n_embd=128, n_head=4, n_head_kv=2, n_blocks=2, ffn=256, vocab_size=1000, eps=1e-6,
                         rope_base=1e4, arch_family=1, qkv_bias=1, tied_embeddings=0, seed=19)
    path = _scale_blocks_in_file(raw, str(tmp_models / "edge.flat"))
    prompts = [[5, 17, 999, 0, 64, 3], [250, 7, 7, 1, 998, 42]]  # equal lengths: the batch returns the last step's logits
    g = hip.load_genomic_auto(path)
    g.set_k_wta_ratio(0.0)
    refs = []
    for p in prompts:
        r = O.load_genomic(path)
        r.set_k_wta_ratio(0.0)
        for i, t in enumerate(p):
            rl = r.forward_core(t, i == 0)
            assert same_bits(g.forward(t, i == 0), rl), f"decode token {i}"
        refs.append(rl)
    ids = np.array(prompts, np.uint32)
    b = hip.GenomicBatch(g, 2, ids.shape[1] + 4)
    logits = b.feed(ids, want_logits=True)
    for s in range(2):
        assert same_bits(logits[s], refs[s]), f"batched sequence {s}"
    b.close()
    g.close()


@pytest.mark.parametrize("halves,name", [(EDGE, "edge"), (SUBNORMAL, "subnormal")])
def test_block_scaled_product_edge_scales(hip, O, halves, name):
    """The MFMA product at its 2e-3 floored tolerance, per output row group so
    that rows of tiny scale are not judged against the largest ones."""
    m, n, k = 64, 512, 1536
    blocks = edge_blocks(n, k, 7, halves)
    X = hip.synth.normal(8, f"edge.X.{name}", m * k).reshape(m, k)
    Y = hip.ops.DeviceBuffer(m * n * 4)
    ws = hip.ops.DeviceBuffer(hip.ops.q4_0_gemm_mfma_workspace(m, n, k))
    hip.ops.q4_0_gemm_mfma(hip.ops.q4_0_upload(blocks, n, k), hip.ops.DeviceBuffer.from_array(X), Y, m, n, k, ws)
    got = Y.read(np.float32).reshape(m, n)
    L = O.GenomicLinear(blocks, b"", None, n, k, None, 4)
    worst = 0.0
    for r in range(0, m, 9):
        ref = L.forward_core(X[r])
        for c in range(0, n, 64):
            worst = max(worst, floored_rel_err(got[r, c:c + 64], ref[c:c + 64]))
    print(f"block-scaled product, {name} scales: worst floored rel err {worst:.2e}")
    assert worst < 2e-3
