"""The oracle (and the host reader) against the reference's own known answers
and against what mathematics fixes, on the CPU.

Pins, by oracle function:
  FlatHeaderV2 / readers   header KATs of src/io/header/tests.rs:7-48
  q4_0 dequant             Q4_0 round trip of src/io/header/tests.rs:51-88;
                           closed form (two roundings) over every code and
                           f16 scale/min pairs incl. subnormals, -0, inf
  Q4_0 linear              2x32 GEMV KAT of src/nn/linear/tests.rs:7-100
  dot_q4_0 / dot_f32 /     fp64 dot within Higham's bound gamma_n * sum|w x|;
  dot_4bit                 the dequantised-row form for Q4_0
  rms_norm                 fp64 closed form
  swiglu_balanced          torch silu(g) * u in fp64 (|g| < 64), closed form beyond
  kwta                     brute-force sort (k-th largest threshold, strict '<')
  rope                     torch fp64 rotation of HF's rotate_half (split) and the
                           interleaved pair rotation, same angle table
  attention                torch fp64 softmax attention with the GQA head map
A plausible slip (a swapped nibble, a wrong sign, a transposed operand) moves
each of these far outside its bound.
"""
import struct

import numpy as np
import pytest
import torch

from oracle import oracle as O
from oracle import flat as OF

U = 2.0 ** -24  # unit roundoff of f32


def gamma(n):
    return n * U / (1 - n * U)


# ------------------------------------------------------------ header KATs --

def _hdr(version, **fields):
    b = bytearray(4096)
    b[0:4] = b"GAJE"
    b[4:8] = struct.pack("<I", version)
    for off, val in fields.values():
        b[off:off + 4] = struct.pack("<I", val)
    return bytes(b)


def test_header_v1_backward_compatibility():
    """header/tests.rs:7-23"""
    import gaje_hip
    b = _hdr(0x000907, flags=(8, 1), num_tensors=(12, 12))
    for parse in (OF.FlatHeader.from_bytes, gaje_hip.flat.header_from_bytes):
        h = parse(b)
        get = (lambda k: h[k]) if isinstance(h, dict) else (lambda k: getattr(h, k))
        qt = get("quantization_type") if isinstance(h, dict) else h.quantization_type()
        eg = get("effective_group_size") if isinstance(h, dict) else h.effective_group_size()
        assert qt == "LegacyCentroids" and eg == 16
        assert get("num_tensors") == 12 and get("version") == 0x000907


def test_header_v2_q4_0():
    """header/tests.rs:25-38"""
    import gaje_hip
    b = _hdr(0x000908, group=(48, 32), quant=(52, 1))
    h = OF.FlatHeader.from_bytes(b)
    assert h.quantization_type() == "Q4_0" and h.effective_group_size() == 32 and h.version == 0x000908
    c = gaje_hip.flat.header_from_bytes(b)
    assert c["quantization_type"] == "Q4_0" and c["effective_group_size"] == 32 and c["version"] == 0x000908


def test_invalid_magic_and_short_header():
    """header/tests.rs:40-48 (InvalidMagic), and TooShort below 4096 bytes."""
    import gaje_hip
    bad = bytearray(4096)
    bad[0:4] = b"XGAJ"
    with pytest.raises(OF.InvalidMagic):
        OF.FlatHeader.from_bytes(bytes(bad))
    with pytest.raises(gaje_hip.GajeIOError) as e:
        gaje_hip.flat.header_from_bytes(bytes(bad))
    assert e.value.code == gaje_hip._lib.ERR_INVALID_MAGIC
    with pytest.raises(OF.TooShort):
        OF.FlatHeader.from_bytes(b"GAJE" + bytes(100))
    with pytest.raises(gaje_hip.GajeIOError) as e:
        gaje_hip.flat.header_from_bytes(b"GAJE" + bytes(100))
    assert e.value.code == gaje_hip._lib.ERR_TOO_SHORT


# ------------------------------------------------------------- Q4_0 KATs --

def _round_half_away(x):
    """f32::round (half away from zero)."""
    return np.sign(x) * np.floor(np.abs(x) + np.float32(0.5))


def _make_block(row, mn, mx):
    """The quantiser of header/tests.rs:51-70 and linear/tests.rs:14-47 (f32 arithmetic)."""
    row = np.asarray(row, np.float32)
    mn, mx = np.float32(mn), np.float32(mx)
    scale = np.float32((mx - mn) / np.float32(15.0))
    inv = np.float32(np.float32(1.0) / scale) if scale > 0 else np.float32(0.0)
    q = np.clip(_round_half_away(((row - mn) * inv).astype(np.float32)), 0, 15).astype(np.uint8)
    qs = q[0::2] | (q[1::2] << 4)
    blk = np.zeros(20, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(scale).tobytes(), np.uint8)  # half::f16::from_f32 (RNE)
    blk[2:4] = np.frombuffer(np.float16(mn).tobytes(), np.uint8)
    blk[4:] = qs
    return blk


def test_q4_0_block_roundtrip():
    """header/tests.rs:51-88: weights i*0.1 come back within 0.11."""
    w = (np.arange(32, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    blk = _make_block(w, 0.0, 3.1)
    d = O.q4_0_dequant(blk)
    assert np.all(np.abs(w - d) <= 0.11)


def test_q4_0_linear_forward_kat():
    """linear/tests.rs:7-100: 2x32 Q4_0 GEMV on ones vs the dequantised row sums (1e-4)."""
    r0 = (np.arange(32, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    r1 = (np.arange(32, dtype=np.float32) * np.float32(-0.1)).astype(np.float32)
    blocks = np.concatenate([_make_block(r0, 0.0, 3.1), _make_block(r1, -3.1, 0.0)])
    L = O.GenomicLinear(blocks, b"", None, 2, 32, None, 4)
    assert L.kind == O.KIND_Q4_0  # bit_depth 4 + empty centroids selects GenomicQ4_0
    out = L.forward_core(np.ones(32, np.float32))
    for r in range(2):
        d = O.q4_0_dequant(blocks[20 * r:20 * (r + 1)])
        expected = np.float32(0.0)
        for v in d:  # Iterator::sum, left to right in f32
            expected = np.float32(expected + v)
        assert abs(out[r] - expected) < 1e-4


F16_EDGES = np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0x7BFF, 0xBC00, 0xFBFF,
                      0x2E66, 0x1400, 0x7C00, 0xFC00, 0x3555, 0xC1A3], np.uint16)


def test_dequant_closed_form_every_code():
    """w = f32(q) * f32(scale) rounded, + f32(min) rounded (blocks.rs:18-30), all codes x f16 edges."""
    rng = np.random.default_rng(5)
    hs = np.concatenate([F16_EDGES, rng.integers(0, 0x7C00, 40, dtype=np.uint16),
                         rng.integers(0x8000, 0xFC00, 20, dtype=np.uint16)])
    blocks, expect = [], []
    codes = np.array([(2 * i) % 16 | (((2 * i + 1) % 16) << 4) for i in range(16)], np.uint8)
    q = np.empty(32, np.float32)
    q[0::2], q[1::2] = codes & 15, codes >> 4
    for s in hs:
        for m in hs[::3]:
            b = np.zeros(20, np.uint8)
            b[0:2] = np.frombuffer(np.uint16(s).tobytes(), np.uint8)
            b[2:4] = np.frombuffer(np.uint16(m).tobytes(), np.uint8)
            b[4:] = codes
            blocks.append(b)
            sf = np.uint16(s).view(np.float16).astype(np.float32)
            mf = np.uint16(m).view(np.float16).astype(np.float32)
            with np.errstate(invalid="ignore", over="ignore"):
                expect.append(((q * sf).astype(np.float32) + mf).astype(np.float32))
    got = O.q4_0_dequant(np.concatenate(blocks))
    ref = np.concatenate(expect)
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all()


# -------------------------------------------------------------- dot bounds --

def _q4_rows(seed, n, k):
    import gaje_hip
    return gaje_hip.synth.q4_0_tensor(seed, f"kat.{n}.{k}", n, k).reshape(n, k // 32, 20)


def _exact_q4_row(blocks):
    """fma(q, scale, min) in exact fp64 (the GEMV's dequantisation before its one rounding)."""
    sc = blocks[:, 0:2].copy().view(np.float16).astype(np.float64).reshape(-1, 1)
    mn = blocks[:, 2:4].copy().view(np.float16).astype(np.float64).reshape(-1, 1)
    qs = blocks[:, 4:]
    q = np.empty((blocks.shape[0], 32))
    q[:, 0::2], q[:, 1::2] = qs & 15, qs >> 4
    return (q * sc + mn).reshape(-1)


@pytest.mark.parametrize("k", [32, 896, 4864])
def test_dot_q4_0_within_higham_bound(k):
    blocks = _q4_rows(21, 6, k)
    x = np.random.default_rng(k).standard_normal(k).astype(np.float32)
    for r in range(blocks.shape[0]):
        got = O.dot_q4_0(blocks[r], x)
        d = _exact_q4_row(blocks[r])
        ref = float(np.dot(d, x.astype(np.float64)))
        bound = gamma(k // 8 + 4) * float(np.abs(d * x).sum()) + 1e-6  # + the 1e-6 flush
        assert abs(got - ref) <= bound, (r, got, ref, bound)
        # the scalar fallback is the same sum in another order: same bound
        assert abs(O.dot_q4_0(blocks[r], x, scalar=True) - ref) <= gamma(k + 4) * float(np.abs(d * x).sum()) + 1e-6


def test_dot_q4_0_nibble_order_matters():
    """Swapping the low/high nibble (a plausible slip) leaves the bound by far."""
    blocks = _q4_rows(22, 1, 896)
    x = np.random.default_rng(1).standard_normal(896).astype(np.float32)
    d = _exact_q4_row(blocks[0])
    swapped = blocks[0].copy()
    swapped[:, 4:] = ((swapped[:, 4:] & 15) << 4) | (swapped[:, 4:] >> 4)
    ref = float(np.dot(d, x.astype(np.float64)))
    bound = gamma(116) * float(np.abs(d * x).sum())
    assert abs(O.dot_q4_0(swapped, x) - ref) > 100 * bound


@pytest.mark.parametrize("k", [8, 12, 100, 896, 1536])
def test_dot_f32_within_higham_bound(k):
    rng = np.random.default_rng(k + 7)
    a = rng.standard_normal(k).astype(np.float32)
    b = rng.standard_normal(k).astype(np.float32)
    ref = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
    bound = gamma(k // 8 + k % 8 + 4) * float(np.abs(a.astype(np.float64) * b).sum())
    assert abs(O.dot_f32(a, b) - ref) <= bound


def test_dot_4bit_within_bound_and_high_nibble_first():
    """genomic_dot_product_4bit: even element = high nibble (genomic.rs:148-204)."""
    rng = np.random.default_rng(3)
    codes = rng.integers(0, 256, 28 * 16, dtype=np.uint8)
    table = np.sort(rng.standard_normal(16)).astype(np.float32)
    x = rng.standard_normal(896).astype(np.float32)
    idx = np.empty(896, np.int64)
    idx[0::2], idx[1::2] = codes >> 4, codes & 15
    w = table[idx].astype(np.float64)
    ref = float(np.dot(w, x))
    bound = gamma(896 // 4 + 4) * float(np.abs(w * x).sum()) + 1e-6
    assert abs(O.dot_4bit(codes, x, table) - ref) <= bound


# ------------------------------------------------- norm / activation / kwta --

@pytest.mark.parametrize("n", [8, 13, 576, 896, 4864])
def test_rms_norm_closed_form(n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    eps = 1e-6
    xd = x.astype(np.float64)
    ref = xd / np.sqrt(np.mean(xd * xd) + eps) * w
    got = O.rms_norm(x, w, eps)
    assert np.max(np.abs(got - ref) / np.abs(ref).max()) < (n // 8 + 16) * U


def test_swiglu_matches_torch_silu():
    rng = np.random.default_rng(9)
    g = (rng.standard_normal(4096) * 8).astype(np.float32)
    u = rng.standard_normal(4096).astype(np.float32)
    got = O.swiglu_balanced(g, u)
    ref = (torch.nn.functional.silu(torch.from_numpy(g).double()) * torch.from_numpy(u).double()).numpy()
    assert np.max(np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)) < 8 * U
    # the clamp of activation.rs:40-49 beyond |g| = 64: sigmoid(+-64), not silu(g)
    g2 = np.array([-100.0, -64.5, 70.0, 1e4], np.float32)
    u2 = np.ones(4, np.float32)
    got2 = O.swiglu_balanced(g2, u2)
    sig = np.where(g2 >= 0, 1 / (1 + np.exp(-64.0)), np.exp(-64.0) / (1 + np.exp(-64.0)))
    assert np.allclose(got2, g2 * sig, rtol=1e-6)


@pytest.mark.parametrize("n,ratio", [(151936 // 16, 0.5), (1000, 0.1), (37, 0.9)])
def test_kwta_brute_force(n, ratio):
    rng = np.random.default_rng(n)
    s = rng.standard_normal(n).astype(np.float32)
    s[::7] = s[3]  # ties at the threshold stay
    k = max(int(np.float32(n) * np.float32(ratio)), 1)
    thr = np.sort(s)[::-1][k - 1]
    ref = np.where(s < thr, np.float32(-1e9), s)
    got = O.kwta(s, k)
    assert np.array_equal(got, ref)


# ------------------------------------------------------------- RoPE, attention --

def _angles(head_dim, base, pos):
    """The host table the reference builds (attention.rs:66-68): f32 powf / sinf / cosf."""
    i = np.arange(head_dim // 2, dtype=np.float32)
    freq = (np.float32(1.0) / np.power(np.float32(base), (np.float32(2.0) * i) / np.float32(head_dim))).astype(np.float32)
    return (np.float32(pos) * freq).astype(np.float32)


@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("pos", [0, 1, 17, 300])
def test_rope_is_the_rotation(split, pos):
    heads, hd, base = 3, 64, 1e6
    v = np.random.default_rng(pos).standard_normal(heads * hd).astype(np.float32)
    got = O.rope(v, heads, hd, base, pos, split)
    th = torch.from_numpy(_angles(hd, base, pos).astype(np.float64))
    cos, sin = torch.cos(th), torch.sin(th)
    x = torch.from_numpy(v.astype(np.float64)).view(heads, hd)
    if split:  # HF rotate_half: (x1, x2) -> (x1 cos - x2 sin, x2 cos + x1 sin)
        x1, x2 = x[:, : hd // 2], x[:, hd // 2:]
        ref = torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=1)
    else:  # interleaved pairs (2i, 2i+1)
        x1, x2 = x[:, 0::2], x[:, 1::2]
        ref = torch.stack([x1 * cos - x2 * sin, x1 * sin + x2 * cos], dim=2).reshape(heads, hd)
    ref = ref.reshape(-1).numpy()
    assert np.max(np.abs(got - ref)) < 8 * U * np.abs(v).max()
    # a rotation keeps each pair's length
    g = got.astype(np.float64).reshape(heads, hd)
    pair = (lambda a: a[:, : hd // 2] ** 2 + a[:, hd // 2:] ** 2) if split else (lambda a: a[:, 0::2] ** 2 + a[:, 1::2] ** 2)
    assert np.allclose(pair(g), pair(v.astype(np.float64).reshape(heads, hd)), rtol=1e-5)


@pytest.mark.parametrize("ctx,n_head,n_kv,hd", [(1, 4, 2, 64), (9, 14, 2, 64), (300, 9, 3, 64), (77, 12, 2, 128)])
def test_attention_matches_torch_softmax(ctx, n_head, n_kv, hd):
    rng = np.random.default_rng(ctx + hd)
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    k = rng.standard_normal(ctx * n_kv * hd).astype(np.float32)
    v = rng.standard_normal(ctx * n_kv * hd).astype(np.float32)
    got = O.attention(q, k, v, ctx, n_head, n_kv, hd)
    Q = torch.from_numpy(q.astype(np.float64)).view(n_head, 1, hd)
    K = torch.from_numpy(k.astype(np.float64)).view(ctx, n_kv, hd).permute(1, 0, 2)
    V = torch.from_numpy(v.astype(np.float64)).view(ctx, n_kv, hd).permute(1, 0, 2)
    rep = n_head // n_kv  # query head h reads kv head h // rep
    K, V = K.repeat_interleave(rep, 0), V.repeat_interleave(rep, 0)
    ref = torch.softmax(Q @ K.transpose(1, 2) / np.sqrt(hd), dim=-1) @ V
    ref = ref.reshape(-1).numpy()
    assert np.max(np.abs(got - ref)) < 64 * U * max(1.0, np.abs(v).max())
    if ctx == 1:  # one position: the output is v itself (weight exp(0) / (1 + 1e-12))
        assert np.array_equal(got, np.repeat(v.reshape(n_kv, hd), rep, 0).reshape(-1))
