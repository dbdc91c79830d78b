"""GPU parity of the MFMA Q4_0 matrix product (prompt prefill, batched rows).

The reference has no matrix product: each activation row goes through
GenomicLinear::forward_core (linear/forward.rs:119-132), one AVX2 dot per weight
row (genomic.rs:263-336).  The MFMA path computes the same dot products with
f16 hi/lo operand pairs and fp32 accumulation, so it is held to the tolerance
stated for the prefill path: floored max relative error <= 2e-3 against the
oracle (conftest.floored_rel_err, tau = 1e-3 max|ref|).  A second bound pins
the arithmetic itself: against an fp64 product of the dequantised weights the
normwise error must be below 2e-6 of max|ref|, which single-f16 operands
(about 1e-3) would miss by orders of magnitude.
"""
import numpy as np
import pytest

from conftest import floored_rel_err

pytestmark = pytest.mark.gpu

PREFILL_TOL = 2e-3
FP32_LEVEL = 2e-6


@pytest.fixture(scope="module")
def hip():
    import gaje_hip
    from gaje_hip import ops
    if ops.device_count() < 1:
        pytest.fail("no HIP device visible")
    return gaje_hip


@pytest.fixture(scope="module")
def O():
    from oracle import oracle
    return oracle


def _run(hip, blocks, X, n, k, bias=None):
    m = X.shape[0]
    packed = hip.ops.q4_0_upload(blocks, n, k)
    ws = hip.ops.DeviceBuffer(max(hip.ops.q4_0_gemm_mfma_workspace(m, n, k), 1))
    Xd = hip.ops.DeviceBuffer.from_array(np.ascontiguousarray(X, np.float32))
    Y = hip.ops.DeviceBuffer(max(m * n * 4, 4))
    bd = hip.ops.DeviceBuffer.from_array(bias) if bias is not None and bias.size else None
    hip.ops.q4_0_gemm_mfma(packed, Xd, Y, m, n, k, ws, bias=bd, bias_len=0 if bd is None else bias.size)
    hip.ops.synchronize()
    return Y.read(np.float32, m * n).reshape(m, n)


def _oracle(O, blocks, X, n, k, bias=None):
    L = O.GenomicLinear(blocks, b"", None, n, k, bias, 4)
    return np.stack([L.forward_core(X[i]) for i in range(X.shape[0])])


def _exact(O, blocks, X, n, k, bias=None):
    """fp64 product of the dequantised weights with the reference's row epilogue:
    |dot| < 1e-6 -> 0, then + bias.  Returns (Y, mask of outputs whose dot is not
    within 1% of the flush threshold, where either side may round across it)."""
    W = O.q4_0_dequant(blocks).reshape(n, k).astype(np.float64)
    D = np.asarray(X, np.float64) @ W.T
    a = np.abs(D)
    Y = np.where(a < 1e-6, 0.0, D)
    if bias is not None and bias.size:
        Y[:, :bias.size] += bias
    return Y, (a < 0.99e-6) | (a > 1.01e-6)


def _check(got, ref, exact_mask, label):
    exact, mask = exact_mask
    err = floored_rel_err(got, ref)
    norm = float(np.max(np.abs(got - exact) * mask) / max(np.max(np.abs(exact)), 1e-30))
    print(f"{label}: floored err vs oracle {err:.3e}, normwise vs fp64 {norm:.3e}")
    assert err <= PREFILL_TOL
    assert norm <= FP32_LEVEL


@pytest.mark.parametrize("m,n,k", [(512, 2048, 1536), (512, 1536, 8960), (64, 4864, 896), (17, 200, 576),
                                   (1, 128, 32), (300, 1000, 96), (130, 257, 160), (256, 17920, 1536),
                                   (129, 129, 4096), (40, 33, 15360)])
def test_q4_0_gemm_mfma(hip, O, m, n, k):
    blocks = hip.synth.q4_0_tensor(21, f"gemm.{n}.{k}", n, k)
    X = hip.synth.normal(22, f"gemm.x.{m}.{k}", m * k).reshape(m, k)
    bias = hip.synth.normal(23, f"gemm.b.{n}", n - n // 3, 0.0, 0.02)  # rows past its length get none
    got = _run(hip, blocks, X, n, k, bias)
    _check(got, _oracle(O, blocks, X, n, k, bias), _exact(O, blocks, X, n, k, bias), f"gemm m={m} n={n} k={k}")


def test_q4_0_gemm_mfma_row_scales(hip, O):
    # rows of very different magnitude, and weight rows whose scales and mins span
    # f16's range: the per-row power-of-two scaling keeps every row at fp32 accuracy
    m, n, k = 48, 96, 256
    rng = np.random.default_rng(7)
    X = rng.standard_normal((m, k)).astype(np.float32)
    X *= (10.0 ** rng.uniform(-20, 20, size=(m, 1))).astype(np.float32)
    X[5] = 0.0
    nb = k // 32
    blk = np.zeros((n, nb, 20), np.uint8)
    row_mag = 10.0 ** rng.uniform(-6, 3, size=(n, 1))
    scale = (row_mag * rng.uniform(0.5, 1.5, size=(n, nb))).astype(np.float16)
    mn = (-7.5 * row_mag * rng.uniform(0.5, 1.5, size=(n, nb))).astype(np.float16)
    blk[:, :, 0:2] = scale.view(np.uint8).reshape(n, nb, 2)
    blk[:, :, 2:4] = mn.view(np.uint8).reshape(n, nb, 2)
    blk[:, :, 4:] = rng.integers(0, 256, size=(n, nb, 16), dtype=np.uint8)
    blk[3] = 0  # an all-zero weight row
    blocks = blk.reshape(-1)
    got = _run(hip, blocks, X, n, k)
    ref = _oracle(O, blocks, X, n, k)
    exact = _exact(O, blocks, X, n, k)
    assert np.all(np.isfinite(got))
    # rows differ by up to 1e40 in magnitude, so each row is held to the bars on its own
    for i in range(m):
        if not np.any(ref[i]):
            assert not np.any(got[i])
            continue
        _check(got[i], ref[i], (exact[0][i], exact[1][i]), f"row {i}")


def test_q4_0_gemm_mfma_edges(hip, O):
    from gaje_hip._lib import GajeError
    n, k = 64, 64
    blocks = hip.synth.q4_0_tensor(24, "gemm.edge", n, k)
    packed = hip.ops.q4_0_upload(blocks, n, k)
    assert hip.ops.q4_0_gemm_mfma_workspace(0, n, k) == 0
    assert hip.ops.q4_0_gemm_mfma_workspace(4, n, 48) == -1
    Y = hip.ops.DeviceBuffer(4)
    X = hip.ops.DeviceBuffer(4)
    ws = hip.ops.DeviceBuffer(4)
    hip.ops.q4_0_gemm_mfma(packed, X, Y, 0, n, k, ws)  # m = 0: nothing to do
    need = hip.ops.q4_0_gemm_mfma_workspace(8, n, k)
    X = hip.ops.DeviceBuffer(8 * k * 4)
    Y = hip.ops.DeviceBuffer(8 * n * 4)
    small = hip.ops.DeviceBuffer(need - 256)
    with pytest.raises(GajeError):
        hip.ops.q4_0_gemm_mfma(packed, X, Y, 8, n, k, small)
