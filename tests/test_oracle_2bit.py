"""The oracle's 2-bit (Genomic2Bit) restatement against the reference's own known
answers and against what mathematics fixes, on the CPU.

  mapping KAT        tests/unit/test_kernels.py:12-38: quantize_embedding with
                     thresholds [0.1, 0.2, 0.3] puts w = 1.0 in code 10, which the
                     row dot maps to the fourth centroid: y == 42.0 exactly, and
                     equal to dequantize_embedding(...) . x
  row dot vs rows    tests/unit/test_kernels.py:41-59: forward equals get_row . x
                     within atol 1e-5 (64 x 128, random codes and centroids)
  dot                fp64 dot of the dequantised row within Higham's bound, for
                     the AVX2-branch order and for the scalar order; a Gray-order
                     slip (10 -> c2, 11 -> c3) leaves the bound
  modulation         factors multiply centroids index-aligned (c_k * m_k) before
                     the Gray reordering
  centroid tables    4 floats (one table), n_blocks * 4 (per block column), per
                     (row, block), and rows past the stored ones reading the
                     table's start block by block (forward.rs:40-45)
  flush              |sum| < 1e-5 returns +0
"""
import numpy as np
import pytest

from oracle import oracle as O


def _rand_row(rng, nb):
    codes = rng.integers(0, 256, nb * 8, dtype=np.uint8)
    cent = np.sort(rng.normal(0, 0.05, (nb, 4)).astype(np.float32), axis=1)
    # Gray order of the table: c0 < c1 < c2 < c3 are codes 00, 01, 11, 10
    return codes, cent


def _dequant_row(codes, cent):
    nb = cent.shape[0]
    return np.concatenate([O.dequantize_embedding(codes[8 * b:8 * b + 8], 32, cent[b]) for b in range(nb)])


def test_mapping_kat():
    w = np.zeros(32, np.float32)
    w[0] = 1.0
    x = np.zeros(32, np.float32)
    x[0] = 1.0
    dna = O.quantize_embedding(w, [0.1, 0.2, 0.3])
    assert dna[0] >> 6 == 0b10 and not any(dna[1:]) and dna[0] & 0x3F == 0
    c = np.array([1.0, 2.0, 3.0, 42.0], np.float32)
    L = O.GenomicLinear(np.frombuffer(dna, np.uint8), b"", c, 1, 32, None, 2)
    y = L.forward_core(x)[0]
    assert y == np.dot(O.dequantize_embedding(dna, 32, c), x) == 42.0
    assert np.array_equal(L.get_row_core(0), O.dequantize_embedding(dna, 32, c))


def test_quantize_thresholds_default():
    v = np.array([-1.0, -0.43, -0.1, 0.0, 0.2, 0.43, 0.5, 0.42], np.float32)
    b = O.quantize_embedding(v)
    codes = [(b[i // 4] >> (6 - 2 * (i % 4))) & 3 for i in range(8)]
    assert codes == [0b00, 0b01, 0b01, 0b11, 0b11, 0b10, 0b10, 0b11]


def test_forward_vs_get_row_dot():
    rng = np.random.default_rng(0)
    n, k = 64, 128
    nb = k // 32
    codes = rng.integers(0, 256, n * nb * 8, dtype=np.uint8)
    cent = rng.normal(0, 0.02, n * nb * 4).astype(np.float32)
    L = O.GenomicLinear(codes, b"", cent, n, k, None, 2)
    x = rng.normal(0, 1.0, k).astype(np.float32)
    y = L.forward_core(x)
    W = np.stack([L.get_row_core(i) for i in range(n)])
    assert np.allclose(y, W @ x, atol=1e-5)


@pytest.mark.parametrize("nb", [1, 4, 28, 48])
def test_dot_within_higham_bound(nb):
    rng = np.random.default_rng(nb)
    u = 2.0 ** -24
    for trial in range(20):
        codes, cent = _rand_row(rng, nb)
        x = rng.normal(0, 1, nb * 32).astype(np.float32)
        w = _dequant_row(codes, cent)
        exact = float(np.dot(w.astype(np.float64), x.astype(np.float64)))
        bound = 1.01 * (nb * 32) * u * float(np.abs(w.astype(np.float64) * x).sum()) + 1e-5
        for scalar in (False, True):
            got = O.dot_2bit(codes, x, cent.reshape(-1), scalar=scalar)
            assert abs(got - exact) <= bound, (trial, scalar)
        # a slip in the Gray order (code 10 -> c2, 11 -> c3) leaves the bound
        swapped = cent[:, [0, 1, 3, 2]]
        slip = O.dot_2bit(codes, x, swapped.reshape(-1))
        if trial == 0:
            assert abs(slip - exact) > 100 * bound


def test_avx2_order_differs_from_scalar_order_somewhere():
    # the two restated orders are different summations of the same products
    rng = np.random.default_rng(5)
    diffs = 0
    for _ in range(200):
        codes, cent = _rand_row(rng, 28)
        x = rng.normal(0, 1, 896).astype(np.float32)
        diffs += O.dot_2bit(codes, x, cent.reshape(-1)) != O.dot_2bit(codes, x, cent.reshape(-1), scalar=True)
    assert diffs > 50


def test_modulation_index_aligned():
    rng = np.random.default_rng(7)
    codes, cent = _rand_row(rng, 8)
    x = rng.normal(0, 1, 256).astype(np.float32)
    m = np.array([0.5, 1.25, 3.0, -2.0], np.float32)
    pre = (cent * m).astype(np.float32)
    assert O.dot_2bit(codes, x, cent.reshape(-1), m) == O.dot_2bit(codes, x, pre.reshape(-1))
    assert O.dot_2bit(codes, x, cent.reshape(-1), np.ones(4, np.float32)) == O.dot_2bit(codes, x, cent.reshape(-1))


def test_centroid_table_forms():
    rng = np.random.default_rng(11)
    n, k = 6, 96
    nb = k // 32
    codes = rng.integers(0, 256, n * nb * 8, dtype=np.uint8)
    x = rng.normal(0, 1, k).astype(np.float32)
    one = rng.normal(0, 0.1, 4).astype(np.float32)
    col = rng.normal(0, 0.1, nb * 4).astype(np.float32)
    own = rng.normal(0, 0.1, n * nb * 4).astype(np.float32)
    for table, per_row in ((one, lambda i: np.tile(one, nb)), (col, lambda i: col),
                           (own, lambda i: own[i * nb * 4:(i + 1) * nb * 4])):
        L = O.GenomicLinear(codes, b"", table, n, k, None, 2)
        y = L.forward_core(x)
        for i in range(n):
            assert y[i] == O.dot_2bit(codes[i * nb * 8:(i + 1) * nb * 8], x, per_row(i))
            assert np.array_equal(L.get_row_core(i),
                                  _dequant_row(codes[i * nb * 8:(i + 1) * nb * 8], per_row(i).reshape(nb, 4)))
    # a table covering the first 2.5 rows: rows 0-1 own; the row dot of rows 2-5
    # reads the table's start block by block, get_row uses each block's own
    # entries where they exist and the first four otherwise
    part = own[: int(2.5 * nb * 4)]
    L = O.GenomicLinear(codes, b"", part, n, k, None, 2)
    y = L.forward_core(x)
    for i in range(n):
        base = part[i * nb * 4:(i + 1) * nb * 4] if i < 2 else part[:nb * 4]
        assert y[i] == O.dot_2bit(codes[i * nb * 8:(i + 1) * nb * 8], x, base)
    r2 = L.get_row_core(2)
    for b in range(nb):
        off = (2 * nb + b) * 4
        c = part[off:off + 4] if off + 4 <= part.size else part[:4]
        assert np.array_equal(r2[32 * b:32 * b + 32], O.dequantize_embedding(codes[2 * nb * 8 + 8 * b:][:8], 32, c))
    with pytest.raises(ValueError):
        O.GenomicLinear(codes, b"", own[:6], n, k, None, 2)


def test_flush_below_1e5():
    codes = np.full(8, 0b01010101, np.uint8)  # every weight c1
    cent = np.array([0.0, 1e-7, 0.0, 0.0], np.float32)
    x = np.ones(32, np.float32)
    got = O.dot_2bit(codes, x, cent)
    assert got == 0.0 and not np.signbit(got)  # 32e-7 < 1e-5
    cent[1] = 1e-6
    assert O.dot_2bit(codes, x, cent) == pytest.approx(3.2e-5, rel=1e-5)
