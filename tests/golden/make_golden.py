#!/usr/bin/env python3
"""Writes tests/golden/golden.npz: small seeded inputs and the oracle's outputs.

The oracle (oracle/gaje_oracle.c, the line-faithful AVX2 restatement of the
reference kernels) computes every expected output here; the inputs come from
the synthetic writer's documented PRNG.  The CPU suite checks that the oracle
still reproduces these files bit for bit and the GPU suite checks the HIP
path against them.  Regenerate with:  python tests/golden/make_golden.py
"""
import hashlib
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
for p in (REPO, os.path.join(REPO, "gaje-semantic-compression_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

from gaje_hip import synth  # noqa: E402  (host-only writer and PRNG)
from oracle import oracle as O  # noqa: E402

MODEL = dict(n_embd=128, n_head=4, n_head_kv=2, n_blocks=2, ffn=256, vocab_size=300, eps=1e-6,
             rope_base=1e4, arch_family=1, qkv_bias=1, tied_embeddings=0, seed=77)
MODEL_TOKENS = np.array([3, 141, 59, 26, 0], np.uint32)


def model_file(d: str) -> str:
    path = os.path.join(d, "golden_model.flat")
    synth.write_flat(path, **MODEL)
    return path


def build() -> dict:
    g = {}
    # Q4_0 matvecs (a partial packed group at K=160, the Qwen2 hidden size)
    for tag, n, k in (("q4a", 37, 160), ("q4b", 48, 896)):
        b = synth.q4_0_tensor(101, f"golden.{tag}", n, k)
        x = synth.normal(102, f"golden.{tag}.x", k)
        bias = synth.normal(103, f"golden.{tag}.b", n // 2, 0.0, 0.02)
        g[f"{tag}.blocks"], g[f"{tag}.x"], g[f"{tag}.bias"] = b, x, bias
        g[f"{tag}.y"] = O.GenomicLinear(b, b"", None, n, k, bias, 4).forward_core(x)
    # f32 matvec with a scalar tail (K % 8 == 4)
    w = synth.normal(104, "golden.f32.w", 33 * 100)
    x = synth.normal(105, "golden.f32.x", 100)
    g["f32.w"], g["f32.x"] = w, x
    g["f32.y"] = O.GenomicLinear(w.view(np.uint8), b"", None, 33, 100, None, 32).forward_core(x)
    # LUT 4-bit, one table per row and block
    codes, lut = synth.lut4_tensor(106, "golden.lut", 20, 64)
    x = synth.normal(107, "golden.lut.x", 64)
    g["lut.codes"], g["lut.tables"], g["lut.x"] = codes, lut, x
    g["lut.y"] = O.GenomicLinear(codes, b"", lut, 20, 64, None, 4).forward_core(x)
    # Q4_0 dequant
    g["dequant.y"] = O.q4_0_dequant(g["q4a.blocks"])
    # rms_norm, swiglu, expf
    x = synth.normal(108, "golden.norm.x", 896)
    wn = synth.normal(109, "golden.norm.w", 896, 1.0, 0.1)
    g["norm.x"], g["norm.w"], g["norm.y"] = x, wn, O.rms_norm(x, wn, 1e-6)
    gt = synth.normal(110, "golden.swiglu.g", 256, 0.0, 8.0)
    up = synth.normal(111, "golden.swiglu.u", 256)
    g["swiglu.g"], g["swiglu.u"], g["swiglu.y"] = gt, up, O.swiglu_balanced(gt, up)
    ex = synth.normal(112, "golden.expf.x", 512, 0.0, 30.0)
    g["expf.x"], g["expf.y"] = ex, O.expf(ex)
    # GQA attention, 37 positions, 4 query heads over 2 kv heads, head_dim 64
    ctx, nh, nkv, hd = 37, 4, 2, 64
    q = synth.normal(113, "golden.att.q", nh * hd)
    k = synth.normal(114, "golden.att.k", ctx * nkv * hd)
    v = synth.normal(115, "golden.att.v", ctx * nkv * hd)
    g["att.q"], g["att.k"], g["att.v"] = q, k, v
    g["att.shape"] = np.array([ctx, nh, nkv, hd], np.int64)
    g["att.y"] = O.attention(q, k, v, ctx, nh, nkv, hd)
    # a tiny model's logits for a few tokens (K-WTA off), from a regenerated file
    with tempfile.TemporaryDirectory() as d:
        path = model_file(d)
        g["model.sha256"] = np.frombuffer(hashlib.sha256(open(path, "rb").read()).digest(), np.uint8)
        r = O.load_genomic(path)
        r.set_k_wta_ratio(0.0)
        g["model.tokens"] = MODEL_TOKENS
        g["model.logits"] = np.stack([r.forward_core(int(t), i == 0) for i, t in enumerate(MODEL_TOKENS)])
    return g


if __name__ == "__main__":
    g = build()
    out = os.path.join(HERE, "golden.npz")
    np.savez_compressed(out, **g)
    print(f"wrote {out} ({os.path.getsize(out)} bytes, {len(g)} arrays)")
