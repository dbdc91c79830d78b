"""Sparse f16 anchors in the oracle, pinned by the closed form of compute_single_row.

GenomicLinear::new parses a "GAJE" buffer (src/nn/linear/init.rs:61-107):
count, u32 flat indices, f16 values, then either out_features + 1 u64 row
pointers or, when the buffer is too short for them, pointers derived from
flat_index / in_features.  compute_single_row (src/nn/linear/forward.rs:103-112)
adds x[index % in_features] * value for k in [ptr[i], ptr[i+1]) when
ptr[i] < ptr[i+1] <= count, after the row dot and before the bias.

Checked here against a float64 composition, row = dequant(row) . x +
sum_k x[col_k] value_k (+ bias), within the dot's Higham bound: every pointer
form, columns past in_features, an inverted row range, genomize_4bit_core's
two-pointer buffer (src/compute/quantize/genomize.rs:367-381), and Q4_0, LUT-4bit
and 2-bit rows.  Slips (no modulo on the column, the fallback rows taken from the
column instead of the row, the inverted range kept) leave the bound.
"""
import struct

import numpy as np
import pytest

from oracle import oracle as O

F16 = np.float16


def _buf(idx, vals, ptrs=None):
    idx = np.asarray(idx, np.uint32)
    vals = np.asarray(vals, np.float32).astype(F16)
    b = b"GAJE" + struct.pack("<I", idx.size) + idx.astype("<u4").tobytes() + vals.view("<u2").tobytes()
    if ptrs is not None:
        b += np.asarray(ptrs, "<u8").tobytes()
    return b


def _q4_0(rng, n, k):
    nb = n * k // 32
    scale = rng.uniform(0.01, 0.05, nb).astype(F16)
    mn = (np.float32(-7.5) * scale.astype(np.float32)).astype(F16)
    codes = rng.integers(0, 16, (nb, 32)).astype(np.uint8)
    blk = np.zeros((nb, 20), np.uint8)
    blk[:, 0:2] = scale.view(np.uint8).reshape(nb, 2)
    blk[:, 2:4] = mn.view(np.uint8).reshape(nb, 2)
    blk[:, 4:] = codes[:, 0::2] | (codes[:, 1::2] << 4)
    return blk.reshape(-1)


def _dense_q4_0(blocks, n, k):
    return O.q4_0_dequant(blocks).astype(np.float64).reshape(n, k)


def _expected(W, x, rows_anchors, bias=None):
    """float64 rows and their error bounds: rows_anchors[r] = [(col, value), ...]."""
    x64 = x.astype(np.float64)
    y = W @ x64
    bound = 1.2e-7 * (W.shape[1] + 8) * (np.abs(W) @ np.abs(x64))
    for r, an in enumerate(rows_anchors):
        for col, v in an:
            y[r] += x64[col] * float(np.float32(F16(v)))
            bound[r] += 1.2e-7 * abs(y[r]) + 1.2e-7 * abs(x64[col] * float(v))
    if bias is not None:
        y += bias
    return y, bound + 1e-6  # the reference flushes |dot| < 1e-6 to 0 before the anchors


def _check(out, ref, bound):
    assert np.all(np.abs(out.astype(np.float64) - ref) <= bound), np.max(np.abs(out - ref) - bound)


def _miss(out, ref, bound):
    return bool(np.any(np.abs(out.astype(np.float64) - ref) > bound))


N, K = 5, 64


@pytest.fixture(scope="module")
def layer():
    rng = np.random.default_rng(21)
    blocks = _q4_0(rng, N, K)
    x = rng.standard_normal(K).astype(np.float32)
    return blocks, x, _dense_q4_0(blocks, N, K)


def test_row_pointer_form(layer):
    blocks, x, W = layer
    # row 0: two anchors (one with a flat index past the tensor), row 1: none,
    # row 2: one, row 3: three (unsorted columns), row 4: one at column 0
    idx = [0 * K + 5, 7 * K + 9, 2 * K + 63, 3 * K + 40, 3 * K + 1, 99 * K + 17, 4 * K]
    vals = [0.5, -0.25, 1.5, -2.0, 0.125, 0.75, 3.0]
    ptrs = [0, 2, 2, 3, 6, 7]
    L = O.GenomicLinear(blocks, _buf(idx, vals, ptrs), None, N, K, None, 4)
    out = L.forward_core(x)
    rows = [[(5, 0.5), (9, -0.25)], [], [(63, 1.5)], [(40, -2.0), (1, 0.125), (17, 0.75)], [(0, 3.0)]]
    ref, bound = _expected(W, x, rows)
    _check(out, ref, bound)
    # slip: the flat index used as the column (out of range -> dropped)
    slip = [[(5, 0.5)], [], [], [], []]
    assert _miss(out, *_expected(W, x, slip))


def test_inverted_range_is_skipped(layer):
    blocks, x, W = layer
    idx = [0 * K + 3, 1 * K + 4, 1 * K + 8, 2 * K + 12]
    vals = [1.0, 2.0, -1.0, 0.5]
    # row 1's range [2, 1) is inverted: it adds nothing; row 2 takes [1, 4)
    ptrs = [0, 2, 1, 4, 4, 4]
    L = O.GenomicLinear(blocks, _buf(idx, vals, ptrs), None, N, K, None, 4)
    out = L.forward_core(x)
    rows = [[(3, 1.0), (4, 2.0)], [], [(4, 2.0), (8, -1.0), (12, 0.5)], [], []]
    ref, bound = _expected(W, x, rows)
    _check(out, ref, bound)
    kept = [[(3, 1.0), (4, 2.0)], [(4, 2.0)], [(4, 2.0), (8, -1.0), (12, 0.5)], [], []]
    assert _miss(out, *_expected(W, x, kept))
    # a range ending past count is skipped too
    L = O.GenomicLinear(blocks, _buf(idx, vals, [0, 2, 2, 9, 9, 9]), None, N, K, None, 4)
    out = L.forward_core(x)
    _check(out, *_expected(W, x, [[(3, 1.0), (4, 2.0)], [], [], [], []]))


@pytest.mark.parametrize("form", ["genomize", "none"])
def test_fallback_rows_from_flat_index(layer, form):
    blocks, x, W = layer
    idx = [0 * K + 2, 0 * K + 60, 2 * K + 7, 4 * K + 31, 4 * K + 32]
    vals = [0.5, -1.5, 2.5, 0.25, -0.75]
    ptrs = [0, len(idx)] if form == "genomize" else None  # genomize_4bit_core's {0, count}
    L = O.GenomicLinear(blocks, _buf(idx, vals, ptrs), None, N, K, None, 4)
    out = L.forward_core(x)
    rows = [[(2, 0.5), (60, -1.5)], [], [(7, 2.5)], [], [(31, 0.25), (32, -0.75)]]
    ref, bound = _expected(W, x, rows)
    _check(out, ref, bound)
    # slip: the two pointers read as a one-row CSR (every anchor on row 0)
    allrow0 = [[(2, 0.5), (60, -1.5), (7, 2.5), (31, 0.25), (32, -0.75)], [], [], [], []]
    assert _miss(out, *_expected(W, x, allrow0))


def test_genomize_single_row_uses_its_pointers():
    # out_features = 1: {0, count} is a complete pointer array, flat indices of
    # any size then wrap modulo in_features
    rng = np.random.default_rng(5)
    blocks = _q4_0(rng, 1, K)
    x = rng.standard_normal(K).astype(np.float32)
    W = _dense_q4_0(blocks, 1, K)
    L = O.GenomicLinear(blocks, _buf([3, K + 3, 5 * K + 10], [1.0, 1.0, -2.0], [0, 3]), None, 1, K, None, 4)
    out = L.forward_core(x)
    _check(out, *_expected(W, x, [[(3, 1.0), (3, 1.0), (10, -2.0)]]))


def test_anchors_then_bias(layer):
    blocks, x, W = layer
    bias = np.linspace(-0.3, 0.3, N).astype(np.float32)
    L = O.GenomicLinear(blocks, _buf([K + 1], [4.0], [0, 0, 1, 1, 1, 1]), None, N, K, bias, 4)
    out = L.forward_core(x)
    _check(out, *_expected(W, x, [[], [(1, 4.0)], [], [], []], bias.astype(np.float64)))
    # no "GAJE" magic: no anchors
    L = O.GenomicLinear(blocks, b"XXXX" + _buf([K + 1], [4.0], [0, 0, 1, 1, 1, 1])[4:], None, N, K, None, 4)
    _check(L.forward_core(x), *_expected(W, x, [[]] * N))


def test_lut_and_2bit_rows():
    rng = np.random.default_rng(8)
    nb = K // 32
    anchors = _buf([0 * K + 1, 1 * K + 33, 1 * K + 2], [0.5, -1.0, 2.0], [0, 1, 3])
    rows = [[(1, 0.5)], [(33, -1.0), (2, 2.0)]]
    x = rng.standard_normal(K).astype(np.float32)
    # LUT-4bit: high nibble = even element, per-(row, block) 16-entry tables
    codes = rng.integers(0, 16, (2, K)).astype(np.uint8)
    lut = rng.standard_normal((2, nb, 16)).astype(np.float32)
    packed = (codes[:, 0::2] << 4) | codes[:, 1::2]
    W = np.array([[lut[r, c // 32, codes[r, c]] for c in range(K)] for r in range(2)], np.float64)
    L = O.GenomicLinear(packed.reshape(-1), anchors, lut.reshape(-1), 2, K, None, 4)
    _check(L.forward_core(x), *_expected(W, x, rows))
    # 2-bit: MSB-first codes, 00/01/10/11 -> centroids 0/1/3/2
    c2 = rng.integers(0, 4, (2, K)).astype(np.uint8)
    cent = rng.standard_normal((2, nb, 4)).astype(np.float32)
    b2 = (c2[:, 0::4] << 6) | (c2[:, 1::4] << 4) | (c2[:, 2::4] << 2) | c2[:, 3::4]
    sel = np.array([0, 1, 3, 2])
    W2 = np.array([[cent[r, c // 32, sel[c2[r, c]]] for c in range(K)] for r in range(2)], np.float64)
    L2 = O.GenomicLinear(b2.reshape(-1), anchors, cent.reshape(-1), 2, K, None, 2)
    _check(L2.forward_core(x), *_expected(W2, x, rows))


@pytest.mark.parametrize("form", [1, 2, 3])
def test_synthetic_file_anchors(tmp_models, form):
    """The writer's anchor buffers load into the oracle as their documented rows."""
    import gaje_hip
    from oracle.flat import FlatFile
    p = str(tmp_models / f"anchors_{form}.flat")
    gaje_hip.synth.write_flat(p, n_embd=64, n_head=2, n_head_kv=1, n_blocks=1, ffn=96, vocab_size=50,
                              eps=1e-6, rope_base=1e4, arch_family=1, qkv_bias=1, tied_embeddings=0,
                              seed=4, anchors=form)
    ff = FlatFile(p)
    e = ff.tensors["blk.0.ffn_down"]
    assert e["anc_len"] > 8
    buf = bytes(ff.get_slice(e["anc_off"], e["anc_len"]))
    n, k = e["out_features"], e["in_features"]
    cnt = struct.unpack_from("<I", buf, 4)[0]
    idx = np.frombuffer(buf, "<u4", cnt, 8)
    val = np.frombuffer(buf, "<u2", cnt, 8 + 4 * cnt).view(F16)
    rows = [[] for _ in range(n)]
    if form == 1:
        ptr = np.frombuffer(buf, "<u8", n + 1, 8 + 6 * cnt).astype(np.int64)
        assert ptr[2] == ptr[1] - 1  # the inverted range of row 1
        for r in range(n):
            if ptr[r] < ptr[r + 1] <= cnt:
                rows[r] = [(int(idx[j]) % k, float(val[j])) for j in range(ptr[r], ptr[r + 1])]
        assert any(int(i) >= n * k for i in idx)  # columns placed only by the modulo
    else:
        for j in range(cnt):
            rows[int(idx[j]) // k].append((int(idx[j]) % k, float(val[j])))
    r = O.load_genomic(p)
    L = r.blocks[0].w_down
    x = np.random.default_rng(1).standard_normal(k).astype(np.float32)
    W = _dense_q4_0(np.array(ff.get_slice(e["dna_off"], e["dna_len"])), n, k)
    _check(L.forward_core(x), *_expected(W, x, rows))
    assert sum(len(a) for a in rows) > 0
