"""The native .gaje.flat writer and its quantisers (csrc/quantize.cpp, csrc/writer.cpp).

What pins them:
  quantize_q4_0_native  src/io/header/tests.rs:51-88 (weights i * 0.1 come back
                        within 0.11 after dequantize_weight), and hand-worked
                        blocks for the rules the KAT leaves open: a flat block
                        (scale <= 1e-7: every code 0), f32::round's halves away
                        from zero (2.5 -> 3, where numpy's round gives 2), and the
                        f16 storage of scale and min (numpy's float16 cast, RNE)
  quantize_q8_0_native  src/io/header/tests.rs:121-165 through the oracle's
                        restatement (pinned there), byte for byte
  genomize_4bit_core    linear centroids min + j * step on a block whose step is
                        exactly 1; nearest centroid with ties to the lower index;
                        high nibble first; anchors by absolute threshold, by
                        density and off (the buffer is always written with the
                        pointers {0, count}); the LUT layer it produces, loaded by
                        the oracle, against a float64 composition
  export_gaje_flat      the header fields, the JSON directory and the 64-byte
                        sub-blob alignment of scripts/export_gaje_flat.py:184-483,
                        read back by both readers, with tensors equal to their
                        quantisation byte for byte
"""
import json
import struct

import numpy as np
import pytest

import gaje_hip
from gaje_hip import writer as W
from oracle import oracle as O
from oracle.flat import FlatFile

F16 = np.float16


def _blocks(b):
    return np.frombuffer(b, np.uint8).reshape(-1, 20)


def test_q4_0_roundtrip_kat():
    w = (np.arange(32, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    d = O.q4_0_dequant(np.frombuffer(W.quantize_q4_0_native(w), np.uint8))
    assert np.all(np.abs(d - w) <= 0.11)


def test_q4_0_rules():
    # scale (15 - 0) / 15 = 1, inv = 1: codes round(w) with halves away from zero
    w = np.zeros(32, np.float32)
    w[1] = 15.0
    w[2], w[3], w[4], w[5] = 2.5, 0.5, 14.5, 7.49999
    blk = _blocks(W.quantize_q4_0_native(w))[0]
    codes = np.empty(32, np.uint8)
    codes[0::2], codes[1::2] = blk[4:] & 0xF, blk[4:] >> 4
    assert list(codes[:6]) == [0, 15, 3, 1, 15, 7]
    assert blk[0:2].view(F16)[0] == F16(1.0) and blk[2:4].view(F16)[0] == F16(0.0)
    # a flat block: scale 0 <= 1e-7, every code 0, min stored as f16
    flat = np.full(32, 0.3, np.float32)
    blk = _blocks(W.quantize_q4_0_native(flat))[0]
    assert not blk[4:].any() and blk[0:2].view(F16)[0] == F16(0.0)
    assert blk[2:4].view(F16)[0] == F16(np.float32(0.3))
    # scale and min as f16 rounded to nearest even, codes from the f32 scale
    rng = np.random.default_rng(3)
    w = rng.standard_normal(32 * 64).astype(np.float32)
    b = _blocks(W.quantize_q4_0_native(w))
    for j in range(64):
        blk32 = w[32 * j:32 * j + 32]
        mn, mx = blk32.min(), blk32.max()
        scale = np.float32((mx - mn) / np.float32(15.0))
        assert b[j, 0:2].view(F16)[0] == F16(scale) and b[j, 2:4].view(F16)[0] == F16(mn)
    # dequantised error within half a step of the f16-rounded grid, plus its rounding
    d = O.q4_0_dequant(b.reshape(-1)).reshape(64, 32)
    for j in range(64):
        s = float(b[j, 0:2].view(F16)[0])
        m = float(b[j, 2:4].view(F16)[0])
        blk32 = w[32 * j:32 * j + 32].astype(np.float64)
        assert np.all(np.abs(d[j] - blk32) <= 0.5 * s + abs(m - blk32.min()) + 15 * abs(
            s - (blk32.max() - blk32.min()) / 15) + 1e-6)


def test_q4_0_length_error():
    with pytest.raises(gaje_hip.GajeError, match="divisible by 32"):
        W.quantize_q4_0_native(np.zeros(33, np.float32))


def test_q8_0_matches_oracle():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal(32 * 100) * 0.05).astype(np.float32)
    w[:32] = 0.0
    w[32:64] = 1e-9
    assert W.quantize_q8_0_native(w) == O.q8_0_quantize(w).tobytes()


def test_genomize_centroids_ties_and_nibbles():
    blk = np.zeros(32, np.float32)
    blk[0], blk[1] = 15.0, 0.0  # min 0, max 15: step 1, centroids 0..15
    blk[2], blk[3] = 2.5, 2.5000002
    blk[4], blk[5] = 7.0, 14.9
    codes, cent, anc = W.genomize_4bit_core(blk, 32, -1.0)
    assert cent == [float(j) for j in range(16)]
    c = np.frombuffer(codes, np.uint8)
    hi, lo = c >> 4, c & 0xF  # element 2k is the high nibble
    assert (hi[0], lo[0]) == (15, 0)
    assert (hi[1], lo[1]) == (2, 3)  # 2.5 ties between 2 and 3: the lower index
    assert (hi[2], lo[2]) == (7, 15)
    # anchors off: the buffer still holds "GAJE", count 0 and the pointers {0, 0}
    assert anc == b"GAJE" + struct.pack("<I", 0) + struct.pack("<QQ", 0, 0)


def test_genomize_anchor_thresholds():
    rng = np.random.default_rng(5)
    w = rng.standard_normal(96).astype(np.float32)
    for thr, want in ((1.5, np.nonzero(np.abs(w) >= 1.5)[0]), (0.0, np.arange(96))):
        _, _, anc = W.genomize_4bit_core(w, 32, thr)
        cnt = struct.unpack_from("<I", anc, 4)[0]
        idx = np.frombuffer(anc, "<u4", cnt, 8)
        val = np.frombuffer(anc, "<u2", cnt, 8 + 4 * cnt).view(F16)
        ptr = np.frombuffer(anc, "<u8", 2, 8 + 6 * cnt)
        assert list(idx) == list(want) and list(ptr) == [0, cnt]
        assert np.array_equal(val, w[want].astype(F16))
    # density 0.25: the threshold is the 24th largest |w| (index int(96 * 0.25)),
    # and every |w| at or above it is an anchor
    _, _, anc = W.genomize_4bit_core(w, 32, 0.25)
    cnt = struct.unpack_from("<I", anc, 4)[0]
    thr = np.sort(np.abs(w))[::-1][24]
    assert list(np.frombuffer(anc, "<u4", cnt, 8)) == list(np.nonzero(np.abs(w) >= thr)[0])
    assert cnt == 25


def test_genomize_layer_in_the_oracle():
    """A LUT layer built by genomize_4bit_core (per-(row, block) tables, its anchor
    buffer, whose two pointers send every anchor to its row by flat index) against a
    float64 composition of the centroid lookup and the anchors."""
    rng = np.random.default_rng(6)
    n, k = 6, 64
    w = rng.standard_normal((n, k)).astype(np.float32)
    x = rng.standard_normal(k).astype(np.float32)
    codes, cent, anc = W.genomize_4bit_core(w, 32, 1.8)
    L = O.GenomicLinear(np.frombuffer(codes, np.uint8), anc, np.array(cent, np.float32), n, k, None, 4)
    c = np.frombuffer(codes, np.uint8).reshape(n, k // 2)
    q = np.empty((n, k), np.int64)
    q[:, 0::2], q[:, 1::2] = c >> 4, c & 0xF
    t = np.array(cent, np.float64).reshape(n, k // 32, 16)
    D = np.array([[t[r, j // 32, q[r, j]] for j in range(k)] for r in range(n)])
    ref = D @ x.astype(np.float64)
    big = np.abs(w) >= 1.8
    ref += (np.where(big, w.astype(F16).astype(np.float64), 0.0) * x.astype(np.float64)).sum(axis=1)
    bound = 1e-6 * (k + 8) * (np.abs(D) @ np.abs(x)) + 1e-5
    assert np.all(np.abs(L.forward_core(x) - ref) <= bound)


def _tiny_tensors(rng, h=64, heads=4, kv=2, blocks=2, ffn=96, vocab=120):
    hd = h // heads
    T = {"token_embd.weight": 0.02 * rng.standard_normal((vocab, h)),
         "output_norm.weight": 1 + 0.1 * rng.standard_normal(h),
         "lm_head.weight": 0.02 * rng.standard_normal((vocab, h))}
    for i in range(blocks):
        p = f"blk.{i}."
        T[p + "attn_norm.weight"] = 1 + 0.1 * rng.standard_normal(h)
        T[p + "ffn_norm.weight"] = 1 + 0.1 * rng.standard_normal(h)
        T[p + "attn_q.weight"] = 0.1 * rng.standard_normal((heads * hd, h))
        T[p + "attn_k.weight"] = 0.1 * rng.standard_normal((kv * hd, h))
        T[p + "attn_v.weight"] = 0.1 * rng.standard_normal((kv * hd, h))
        for t, n in (("q", heads * hd), ("k", kv * hd), ("v", kv * hd)):
            T[p + f"attn_{t}.bias"] = 0.02 * rng.standard_normal(n)
        T[p + "attn_output.weight"] = 0.1 * rng.standard_normal((h, heads * hd))
        T[p + "ffn_gate.weight"] = 0.1 * rng.standard_normal((ffn, h))
        T[p + "ffn_up.weight"] = 0.1 * rng.standard_normal((ffn, h))
        T[p + "ffn_down.weight"] = 0.1 * rng.standard_normal((h, ffn))
    return {k: v.astype(np.float32) for k, v in T.items()}


@pytest.mark.parametrize("body,quant_embed", [("q4_0", False), ("q4_0", True), ("lut4", False)])
def test_export_layout(tmp_models, body, quant_embed):
    T = _tiny_tensors(np.random.default_rng(7))
    p = str(tmp_models / f"export_{body}_{int(quant_embed)}.flat")
    W.export_gaje_flat(p, T, n_embd=64, n_head=4, n_head_kv=2, n_blocks=2, vocab_size=120, eps=1e-6,
                       rope_base=1e6, arch_family=3, quant_embed=quant_embed, body=body, anchor_threshold=0.3)
    ff = FlatFile(p)
    h = ff.header
    assert h.version == 0x000908 and h.group_size == 32 and h.arch_family == 3 and h.flags == 3
    assert h.weights_offset % 4096 == 0 and h.weights_offset >= 4096 + h.meta_len + h.dir_len
    meta = json.loads(ff.metadata_json)
    assert meta["n_embd"] == 64 and meta["config"]["rope_base"] == 1e6 and meta["eps"] == 1e-6
    names = list(ff.tensors)
    assert names[:3] == ["token_embd", "output_norm", "lm_head"]
    assert names[3:9] == ["blk.0.attn_norm", "blk.0.ffn_norm", "blk.0.attn_qkv", "blk.0.attn_output",
                          "blk.0.ffn_gate_up", "blk.0.ffn_down"]
    for e in ff.tensors.values():
        for k in ("dna_off", "c_off", "anc_off", "bias_off"):
            assert e[k] % 64 == 0
    qkv = ff.tensors["blk.0.attn_qkv"]
    w_qkv = np.concatenate([T["blk.0.attn_q.weight"], T["blk.0.attn_k.weight"], T["blk.0.attn_v.weight"]])
    b_qkv = np.concatenate([T[f"blk.0.attn_{t}.bias"] for t in "qkv"])
    assert qkv["out_features"] == 128 and qkv["in_features"] == 64
    assert np.array_equal(ff.get_f32_slice(qkv["bias_off"], qkv["bias_len"]), b_qkv)
    dna = bytes(ff.get_slice(qkv["dna_off"], qkv["dna_len"]))
    if body == "q4_0":
        assert qkv["bit_depth"] == 4 and qkv["c_len"] == 0 and qkv["anc_len"] == 0
        assert dna == W.quantize_q4_0_native(w_qkv)
    else:
        codes, cent, anc = W.genomize_4bit_core(w_qkv, 32, 0.3)
        assert dna == codes and qkv["c_len"] == len(cent) * 4
        assert bytes(ff.get_slice(qkv["anc_off"], qkv["anc_len"])) == anc
    emb = ff.tensors["token_embd"]
    if quant_embed:
        assert emb["bit_depth"] == 8
        assert bytes(ff.get_slice(emb["dna_off"], emb["dna_len"])) == W.quantize_q8_0_native(T["token_embd.weight"])
    else:
        assert emb["bit_depth"] == 32
        assert np.array_equal(ff.get_f32_slice(emb["dna_off"], emb["dna_len"]), T["token_embd.weight"].reshape(-1))
    n = ff.tensors["blk.1.ffn_norm"]
    assert n["in_features"] == 1 and n["c_off"] == 0 and n["anc_off"] == 0
    # the C++ reader agrees, and the oracle runs the model
    info = gaje_hip.flat.inspect(p)
    assert info["n_embd"] == 64 and info["n_blocks"] == 2 and info["n_tensors"] == len(names)
    r = O.load_genomic(p)
    r.set_k_wta_ratio(0.0)
    logits = r.forward_core(5, True)
    assert logits.shape == (120,) and np.all(np.isfinite(logits))
