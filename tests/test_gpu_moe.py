"""GPU parity of the MoE SwiGLU FFN layer (gaje_hip_moe_ffn, and over prepared
experts gaje_hip_moe_ffn_prepared) against the oracle.

The reference has no MoE: the layer is a composition of its primitives
(oracle.moe_ffn).  The routing (dot_product router logits, softmax, top-2,
renormalised weights) is computed in the reference's float order on the
device, so the chosen experts and their weights must equal the oracle's bit
for bit; the expert products run on the MFMA units and are held to the
prefill tolerance, floored max relative error <= 2e-3 (conftest.floored_rel_err).
"""
import numpy as np
import pytest

from conftest import floored_rel_err

pytestmark = pytest.mark.gpu

TOL = 2e-3


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


def _experts(hip, E, h, ffn, seed):
    gu = [hip.synth.q4_0_tensor(seed, f"moe.gu.{e}", 2 * ffn, h) for e in range(E)]
    dn = [hip.synth.q4_0_tensor(seed, f"moe.dn.{e}", h, ffn) for e in range(E)]
    return gu, dn


def _run_prepared(hip, x, router, gu, dn, ffn):
    T, h = x.shape
    E = len(gu)
    ops = hip.ops
    xd = ops.DeviceBuffer.from_array(np.ascontiguousarray(x, np.float32))
    rd = ops.DeviceBuffer.from_array(np.ascontiguousarray(router, np.float32))
    gud = [ops.q4_0_upload(b, 2 * ffn, h) for b in gu]
    dnd = [ops.q4_0_upload(b, h, ffn) for b in dn]
    prep = ops.DeviceBuffer(ops.moe_prepared_bytes(h, ffn, E))
    ops.moe_prepare(gud, dnd, h, ffn, prep)
    y = ops.DeviceBuffer(T * h * 4)
    ti = ops.DeviceBuffer(T * 2 * 4)
    tw = ops.DeviceBuffer(T * 2 * 4)
    ws = ops.DeviceBuffer(ops.moe_ffn_prepared_workspace(T, h, ffn, E))
    out = []
    for _ in range(2):  # twice over the same buffers: the second call sees the first's leftovers
        ops.moe_ffn_prepared(xd, T, h, rd, E, prep, ffn, y, ws, top_idx=ti, top_w=tw)
        ops.synchronize()
        out.append((y.read(np.float32, T * h).reshape(T, h), ti.read(np.int32, 2 * T).reshape(T, 2),
                    tw.read(np.float32, 2 * T).reshape(T, 2)))
    assert all(np.array_equal(a.view(np.uint32), b.view(np.uint32)) for a, b in zip(out[0], out[1]))
    return out[1]


def _run(hip, x, router, gu, dn, ffn):
    T, h = x.shape
    E = len(gu)
    ops = hip.ops
    xd = ops.DeviceBuffer.from_array(np.ascontiguousarray(x, np.float32))
    rd = ops.DeviceBuffer.from_array(np.ascontiguousarray(router, np.float32))
    gud = [ops.q4_0_upload(b, 2 * ffn, h) for b in gu]
    dnd = [ops.q4_0_upload(b, h, ffn) for b in dn]
    y = ops.DeviceBuffer(T * h * 4)
    ti = ops.DeviceBuffer(T * 2 * 4)
    tw = ops.DeviceBuffer(T * 2 * 4)
    ws = ops.DeviceBuffer(ops.moe_ffn_workspace(T, h, ffn, E))
    ops.moe_ffn(xd, T, h, rd, gud, dnd, ffn, y, ws, top_idx=ti, top_w=tw)
    ops.synchronize()
    return (y.read(np.float32, T * h).reshape(T, h), ti.read(np.int32, 2 * T).reshape(T, 2),
            tw.read(np.float32, 2 * T).reshape(T, 2))


@pytest.mark.parametrize("T,h,ffn,E,skew", [(256, 1536, 4096, 8, 0.0), (37, 256, 512, 4, 0.0), (1, 64, 96, 2, 0.0),
                                            (100, 256, 256, 5, 3.0), (1500, 128, 128, 16, 0.0),
                                            (2100, 64, 96, 3, 4.0)])
def test_moe_ffn(hip, O, T, h, ffn, E, skew):
    x = hip.synth.normal(51, f"moe.x.{T}.{h}", T * h).reshape(T, h)
    router = hip.synth.normal(52, f"moe.r.{E}.{h}", E * h, 0.0, 0.02).reshape(E, h)
    if skew:  # a skewed load: one expert's router row dominates
        router[1] += np.float32(skew * 0.02) * x.mean(axis=0)
    gu, dn = _experts(hip, E, h, ffn, 53)
    y, idx, w = _run(hip, x, router, gu, dn, ffn)
    ry, ridx, rw = O.moe_ffn(x, router, gu, dn, ffn)
    counts = np.bincount(ridx.reshape(-1), minlength=E)
    err = floored_rel_err(y, ry)
    print(f"moe T={T} h={h} ffn={ffn} E={E}: expert loads {counts.tolist()}, floored err {err:.3e}")
    assert np.array_equal(idx, ridx)
    assert np.array_equal(w.view(np.uint32), rw.view(np.uint32))
    assert err <= TOL


@pytest.mark.parametrize("T,h,ffn,E,skew", [(256, 1536, 4096, 8, 0.0), (37, 256, 512, 4, 0.0), (1, 64, 96, 2, 0.0),
                                            (100, 256, 256, 5, 3.0), (1500, 128, 128, 16, 0.0),
                                            (2100, 64, 96, 3, 4.0), (300, 160, 224, 6, 6.0)])
def test_moe_ffn_prepared(hip, O, T, h, ffn, E, skew):
    """The grouped block-scaled products over prepared experts: routing bit-exact,
    the layer within the same tolerance; skewed loads put several row tiles in
    one expert and leave others nearly empty."""
    x = hip.synth.normal(51, f"moe.x.{T}.{h}", T * h).reshape(T, h)
    router = hip.synth.normal(52, f"moe.r.{E}.{h}", E * h, 0.0, 0.02).reshape(E, h)
    if skew:
        router[1] += np.float32(skew * 0.02) * x.mean(axis=0)
    gu, dn = _experts(hip, E, h, ffn, 53)
    y, idx, w = _run_prepared(hip, x, router, gu, dn, ffn)
    ry, ridx, rw = O.moe_ffn(x, router, gu, dn, ffn)
    counts = np.bincount(ridx.reshape(-1), minlength=E)
    err = floored_rel_err(y, ry)
    print(f"moe prepared T={T} h={h} ffn={ffn} E={E}: expert loads {counts.tolist()}, floored err {err:.3e}")
    assert np.array_equal(idx, ridx)
    assert np.array_equal(w.view(np.uint32), rw.view(np.uint32))
    assert err <= TOL


def test_moe_ffn_prepared_arguments(hip):
    from gaje_hip._lib import GajeError
    assert hip.ops.moe_prepared_bytes(48, 64, 4) == -1
    assert hip.ops.moe_prepared_bytes(64, 64, 1) == -1
    assert hip.ops.moe_ffn_prepared_workspace(4, 64, 64, 17) == -1
    gu, dn = _experts(hip, 2, 64, 64, 54)
    gud = [hip.ops.q4_0_upload(b, 128, 64) for b in gu]
    dnd = [hip.ops.q4_0_upload(b, 64, 64) for b in dn]
    small = hip.ops.DeviceBuffer(hip.ops.moe_prepared_bytes(64, 64, 2) - 256)
    with pytest.raises(GajeError):
        hip.ops.moe_prepare(gud, dnd, 64, 64, small)
    prep = hip.ops.DeviceBuffer(hip.ops.moe_prepared_bytes(64, 64, 2))
    hip.ops.moe_prepare(gud, dnd, 64, 64, prep)
    x = hip.ops.DeviceBuffer(4 * 64 * 4)
    r = hip.ops.DeviceBuffer(2 * 64 * 4)
    y = hip.ops.DeviceBuffer(4 * 64 * 4)
    ws = hip.ops.DeviceBuffer(hip.ops.moe_ffn_prepared_workspace(4, 64, 64, 2) - 256)
    with pytest.raises(GajeError):
        hip.ops.moe_ffn_prepared(x, 4, 64, r, 2, prep, 64, y, ws)


def test_moe_ffn_arguments(hip):
    from gaje_hip._lib import GajeError
    assert hip.ops.moe_ffn_workspace(4, 48, 64, 4) == -1  # h not a multiple of 32
    assert hip.ops.moe_ffn_workspace(4, 64, 64, 1) == -1  # one expert
    assert hip.ops.moe_ffn_workspace(4, 64, 64, 17) == -1
    x = hip.ops.DeviceBuffer(4 * 64 * 4)
    r = hip.ops.DeviceBuffer(2 * 64 * 4)
    y = hip.ops.DeviceBuffer(4 * 64 * 4)
    gu, dn = _experts(hip, 2, 64, 64, 54)
    gud = [hip.ops.q4_0_upload(b, 128, 64) for b in gu]
    dnd = [hip.ops.q4_0_upload(b, 64, 64) for b in dn]
    small = hip.ops.DeviceBuffer(hip.ops.moe_ffn_workspace(4, 64, 64, 2) - 256)
    with pytest.raises(GajeError):
        hip.ops.moe_ffn(x, 4, 64, r, gud, dnd, 64, y, small)
