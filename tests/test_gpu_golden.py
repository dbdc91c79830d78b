"""The HIP path against the committed golden fixtures, bit for bit (the
fixtures are the oracle's outputs on small seeded inputs; see
tests/golden/make_golden.py)."""
import os
import sys

import numpy as np
import pytest

from conftest import REPO

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(REPO, "tests", "golden", "golden.npz")


@pytest.fixture(scope="module")
def g():
    return dict(np.load(GOLDEN, allow_pickle=False))


@pytest.fixture(scope="module")
def hip():
    import gaje_hip
    if gaje_hip.ops.device_count() < 1:
        pytest.fail("no HIP device visible")
    return gaje_hip


def same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def dev(hip, a):
    return hip.ops.DeviceBuffer.from_array(a)


@pytest.mark.parametrize("tag", ["q4a", "q4b"])
def test_q4_0_gemv_golden(hip, g, tag):
    b, x, bias, ref = g[f"{tag}.blocks"], g[f"{tag}.x"], g[f"{tag}.bias"], g[f"{tag}.y"]
    n, k = ref.size, x.size
    y = hip.ops.DeviceBuffer(n * 4)
    hip.ops.q4_0_gemv(hip.ops.q4_0_upload(b, n, k), dev(hip, x), y, n, k, bias=dev(hip, bias), bias_len=bias.size)
    assert same(y.read(np.float32), ref)


def test_f32_lut_dequant_golden(hip, g):
    y = hip.ops.DeviceBuffer(33 * 4)
    hip.ops.f32_gemv(dev(hip, g["f32.w"]), dev(hip, g["f32.x"]), y, 33, 100)
    assert same(y.read(np.float32), g["f32.y"])
    y = hip.ops.DeviceBuffer(20 * 4)
    hip.ops.lut4_gemv(dev(hip, g["lut.codes"]), dev(hip, g["lut.tables"]), g["lut.tables"].size,
                      dev(hip, g["lut.x"]), y, 20, 64)
    assert same(y.read(np.float32), g["lut.y"])
    nb = g["q4a.blocks"].size // 20
    out = hip.ops.DeviceBuffer(nb * 128)
    hip.ops.q4_0_dequant(dev(hip, g["q4a.blocks"]), out, nb)
    assert same(out.read(np.float32), g["dequant.y"])


def test_elementwise_golden(hip, g):
    y = hip.ops.DeviceBuffer(896 * 4)
    hip.ops.rmsnorm(dev(hip, g["norm.x"]), dev(hip, g["norm.w"]), 1e-6, y, 896)
    assert same(y.read(np.float32), g["norm.y"])
    y = hip.ops.DeviceBuffer(256 * 4)
    hip.ops.swiglu(dev(hip, g["swiglu.g"]), dev(hip, g["swiglu.u"]), y, 256)
    assert same(y.read(np.float32), g["swiglu.y"])
    y = hip.ops.DeviceBuffer(512 * 4)
    hip.ops.expf(dev(hip, g["expf.x"]), y, 512)
    assert same(y.read(np.float32), g["expf.y"])


@pytest.mark.parametrize("cap_pad", [0, 3])  # streaming kernel (cap % 4 == 0) and the generic one
def test_attention_golden(hip, g, cap_pad):
    ctx, nh, nkv, hd = (int(v) for v in g["att.shape"])
    cap = (ctx + 3) // 4 * 4 + cap_pad
    kh = np.zeros((nkv, hd, cap), np.float32)  # K and V: [head][dim][pos]
    vh = np.zeros((nkv, hd, cap), np.float32)
    kh[:, :, :ctx] = g["att.k"].reshape(ctx, nkv, hd).transpose(1, 2, 0)
    vh[:, :, :ctx] = g["att.v"].reshape(ctx, nkv, hd).transpose(1, 2, 0)
    out = hip.ops.DeviceBuffer(nh * hd * 4)
    hip.ops.attention(dev(hip, g["att.q"]), dev(hip, kh), dev(hip, vh), ctx, cap, nh, nkv, hd, out)
    assert same(out.read(np.float32), g["att.y"])


def test_model_logits_golden(hip, g, tmp_path):
    sys.path.insert(0, os.path.join(REPO, "tests", "golden"))
    import make_golden
    path = make_golden.model_file(str(tmp_path))
    m = hip.load_genomic_auto(path, device=0)
    m.set_k_wta_ratio(0.0)
    for i, t in enumerate(g["model.tokens"]):
        assert same(m.forward(int(t), i == 0), g["model.logits"][i]), i
    m.close()
