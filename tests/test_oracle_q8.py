"""The oracle's Q8_0 restatement against the reference's own known answer and
against what mathematics fixes, on the CPU.

  Q8_0 writer + dequant   header/tests.rs:121-165: weights i*0.1 - 1.6 quantised
                          by quantize_q8_0_native's rule come back within
                          scale/2 + 1e-5
  dequant                 closed form f32(q) * f32(scale) (exact) over all 256
                          codes and f16 edge scales (subnormal, -0, inf)
  dot                     fp64 dot within Higham's bound; the scalar factored form
                          (genomic.rs:338-372) within its own bound; reading the
                          codes as unsigned (a plausible slip) leaves the bound
  linear / get_row        GenomicLinear with bit_depth 8 selects GenomicQ8_0
                          (init.rs:40-45): rows are the per-row dot, get_row_core
                          is the dequantised row (forward.rs:271-281)
"""
import numpy as np
import pytest

from oracle import oracle as O

U = 2.0 ** -24


def gamma(n):
    return n * U / (1 - n * U)


def test_q8_0_block_quantize_dequantize_kat():
    w = (np.arange(32, dtype=np.float32) * np.float32(0.1) - np.float32(1.6)).astype(np.float32)
    blk = O.q8_0_quantize(w)
    assert blk.size == 34
    scale = float(blk[0:2].copy().view(np.float16)[0])
    d = O.q8_0_dequant(blk)
    assert np.all(np.abs(w - d) <= scale / 2 + 1e-5)
    # the writer's rule itself: scale = max|w| / 127 (f16), q = round(w / scale) half away
    assert np.float16(np.float32(1.6) / np.float32(127)) == np.float16(scale)
    q = blk[2:].view(np.int8)
    inv = np.float32(1.0) / (np.float32(1.6) / np.float32(127))
    ref = np.clip(np.sign(w * inv) * np.floor(np.abs(w * inv) + 0.5), -128, 127).astype(np.int8)
    assert np.array_equal(q, ref)
    # scale <= 1e-7: all codes 0
    tiny = O.q8_0_quantize(np.full(32, 1e-6, np.float32))
    assert not tiny[2:].any()


F16_EDGES = np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0x7BFF, 0xBC00, 0xFBFF,
                      0x2E66, 0x1400, 0x7C00, 0xFC00, 0x3555, 0xC1A3], np.uint16)


def test_q8_0_dequant_closed_form_every_code():
    codes = np.arange(256, dtype=np.uint8)
    blocks, expect = [], []
    rng = np.random.default_rng(9)
    scales = np.concatenate([F16_EDGES, rng.integers(0, 0xFC00, 30, dtype=np.uint16)])
    for s in scales:
        sf = np.uint16(s).view(np.float16).astype(np.float32)
        for part in range(8):
            b = np.zeros(34, np.uint8)
            b[0:2] = np.frombuffer(np.uint16(s).tobytes(), np.uint8)
            b[2:] = codes[32 * part:32 * part + 32]
            blocks.append(b)
            with np.errstate(invalid="ignore", over="ignore"):
                expect.append((b[2:].view(np.int8).astype(np.float32) * sf).astype(np.float32))
    got = O.q8_0_dequant(np.concatenate(blocks))
    ref = np.concatenate(expect)
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all()
    # the product is exact: an 8-bit integer times an 11-bit significand fits f32
    finite = np.isfinite(ref)
    q64 = np.concatenate([b[2:].view(np.int8).astype(np.float64) for b in blocks])
    s64 = np.repeat([np.uint16(s).view(np.float16).astype(np.float64) for s in scales], 256)
    assert np.array_equal(ref[finite].astype(np.float64), (q64 * s64)[finite])


def _q8_rows(n, k, seed):
    rng = np.random.default_rng(seed)
    w = (0.05 * rng.standard_normal(n * k)).astype(np.float32)
    return O.q8_0_quantize(w).reshape(n, k // 32 * 34)


@pytest.mark.parametrize("k", [32, 896, 1536])
def test_dot_q8_0_within_higham_bound(k):
    rows = _q8_rows(5, k, k)
    x = np.random.default_rng(k + 1).standard_normal(k).astype(np.float32)
    for r in range(rows.shape[0]):
        d = O.q8_0_dequant(rows[r]).astype(np.float64)
        ref = float(np.dot(d, x.astype(np.float64)))
        s = float(np.abs(d * x).sum())
        assert abs(O.dot_q8_0(rows[r], x) - ref) <= gamma(k // 8 + 4) * s + 1e-6
        assert abs(O.dot_q8_0(rows[r], x, scalar=True) - ref) <= gamma(k + 4) * s + 1e-6
    # codes read as unsigned: far outside the bound
    bad = rows[0].reshape(-1, 34).copy()
    d = O.q8_0_dequant(rows[0]).astype(np.float64)
    ref = float(np.dot(d, x.astype(np.float64)))
    sc = bad[:, 0:2].copy().view(np.float16).astype(np.float64)
    du = (bad[:, 2:].astype(np.float64) * sc).reshape(-1)
    assert abs(float(np.dot(du, x)) - ref) > 100 * (gamma(k // 8 + 4) * float(np.abs(d * x).sum()) + 1e-6)


def test_q8_0_linear_and_get_row():
    n, k = 7, 96
    rows = _q8_rows(n, k, 3)
    L = O.GenomicLinear(rows.reshape(-1), b"", None, n, k, None, 8)
    assert L.kind == O.KIND_Q8_0
    x = np.random.default_rng(4).standard_normal(k).astype(np.float32)
    out = L.forward_core(x)
    for r in range(n):
        assert out[r] == np.float32(O.dot_q8_0(rows[r], x))
        assert np.array_equal(L.get_row_core(r), O.q8_0_dequant(rows[r]))
    assert np.array_equal(L.get_row_core(n + 2), O.q8_0_dequant(rows[2]))  # idx % out_features
