"""gaje_hip_q4_0_gemm_mfma_noalloc (no counterpart in the reference): the MFMA product
with its workspace in the library's own device scratch, called through the C ABI, equal
bit for bit to gaje_hip_q4_0_gemm_mfma with a caller workspace, on two calls in a row
(the second smaller, so stale scratch from the first is in place), and a product whose
workspace exceeds the scratch refused without a launch."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _run(hip, fn, m, n, k, seed):
    from gaje_hip._lib import check, lib
    blocks = hip.synth.q4_0_tensor(seed, f"noalloc.{n}.{k}", n, k)
    W = hip.ops.q4_0_upload(blocks, n, k)
    X = hip.ops.DeviceBuffer.from_array(hip.synth.normal(seed + 1, f"noalloc.x.{m}.{k}", m * k))
    bias = hip.ops.DeviceBuffer.from_array(hip.synth.normal(seed + 2, f"noalloc.b.{n}", n, 0.0, 0.02))
    Y = hip.ops.DeviceBuffer(m * n * 4)
    if fn == "noalloc":
        check(lib().gaje_hip_q4_0_gemm_mfma_noalloc(W.ptr, X.ptr, bias.ptr, n, Y.ptr, m, n, k, None))
    else:
        ws = hip.ops.DeviceBuffer(max(hip.ops.q4_0_gemm_mfma_workspace(m, n, k), 1))
        check(lib().gaje_hip_q4_0_gemm_mfma(W.ptr, X.ptr, bias.ptr, n, Y.ptr, m, n, k, ws.ptr, ws.nbytes, None))
    hip.ops.synchronize()
    return Y.read(np.float32)


def test_noalloc_matches_workspace_entry_point():
    import gaje_hip as hip
    if hip.ops.device_count() < 1:
        pytest.fail("no HIP device visible")
    # split-K partials in use (few output tiles), then a smaller product
    for m, n, k in ((64, 512, 4096), (40, 256, 2048)):
        a = _run(hip, "noalloc", m, n, k, 31)
        b = _run(hip, "workspace", m, n, k, 31)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (m, n, k)
        assert np.all(np.isfinite(a))


def test_noalloc_rejects_beyond_scratch():
    import gaje_hip as hip
    from gaje_hip._lib import GajeError, check, lib
    if hip.ops.device_count() < 1:
        pytest.fail("no HIP device visible")
    m, n, k = 4096, 1536, 8960
    assert hip.ops.q4_0_gemm_mfma_workspace(m, n, k) > (64 << 20)
    with pytest.raises(GajeError, match="scratch"):
        check(lib().gaje_hip_q4_0_gemm_mfma_noalloc(None, None, None, 0, None, m, n, k, None))


def test_noalloc_empty_products_match():
    """m == 0 or n == 0: both entry points return OK without a launch."""
    import gaje_hip as hip
    from gaje_hip._lib import check, lib
    if hip.ops.device_count() < 1:
        pytest.fail("no HIP device visible")
    k = 512
    W = hip.ops.q4_0_upload(hip.synth.q4_0_tensor(5, "noalloc.empty", 4, k), 4, k)
    X = hip.ops.DeviceBuffer.from_array(np.zeros(16 * k, np.float32))
    Y = hip.ops.DeviceBuffer(256)
    ws = hip.ops.DeviceBuffer(256)
    for m, n in ((0, 256), (16, 0), (0, 0)):
        check(lib().gaje_hip_q4_0_gemm_mfma_noalloc(W.ptr, X.ptr, None, 0, Y.ptr, m, n, k, None))
        check(lib().gaje_hip_q4_0_gemm_mfma(W.ptr, X.ptr, None, 0, Y.ptr, m, n, k, ws.ptr, ws.nbytes, None))
