"""A float64 composition of the reference forward, for the tests only.

forward_fp64 runs the reference's block wiring (RustGenomicBlock::forward_core,
src/nn/block/forward.rs:10-157; GenomicLLM::forward_core,
src/nn/llm/forward.rs:7-64) over a whole prompt at once, in float64, with the
file's weights dequantised exactly (Q4_0: q * scale + min, LUT: the table
value, F32: the stored float).  Its only roundings are float64's, so its
distance from the float32 oracle measures the oracle's own float32 noise.

It restates the semantics, not the rounding sequence:
  rms_norm            x / sqrt(mean(x^2) + eps) * w          (norm.rs:17-131)
  linear rows         W x, |t| < 1e-6 flushed to 0, + bias   (linear/forward.rs:11-117,
                                                              genomic.rs:331-335)
  RoPE                split pairs (i, i + hd/2) or interleaved (2i, 2i+1),
                      theta = pos / base^(2i/hd)             (attention.rs:56-84)
  attention           softmax(q.k / sqrt(hd)) with the +1e-12 of the sum,
                      kv head h / (n_head / n_head_kv)      (attention.rs:87-127)
  swiglu_balanced     g * sigmoid(clamp(g, -64, 64)) * u     (activation.rs:35-51)
  use_genomic_norm    ffn_out * h_scale / rms when rms > h_scale, h_scale 1
                                                             (block/forward.rs:115-123,
                                                              flat_reader.rs:220)
It is pinned against HF transformers' Qwen2 model in float64
(tests/test_oracle_model.py).
"""
from __future__ import annotations

import numpy as np


def tensor_weights(ff, name: str):
    """Exact float64 weights [out][in] and bias of a flat tensor."""
    e = ff.tensors[name]
    n, k = e["out_features"], e["in_features"]
    dna = np.asarray(ff.get_slice(e["dna_off"], e["dna_len"]))
    bias = ff.get_f32_slice(e["bias_off"], e["bias_len"]).astype(np.float64)
    if e["bit_depth"] == 32:
        w = np.frombuffer(dna.tobytes(), np.float32)[: n * k].reshape(n, k).astype(np.float64)
        return w, bias
    nb = k // 32
    if e["c_len"] == 0:  # Q4_0 blocks: q * scale + min exactly (f16 scale / min)
        b = dna[: n * nb * 20].reshape(n * nb, 20)
        sc = b[:, 0:2].copy().view(np.float16).astype(np.float64)
        mn = b[:, 2:4].copy().view(np.float16).astype(np.float64)
        q = np.empty((n * nb, 32))
        q[:, 0::2], q[:, 1::2] = b[:, 4:] & 15, b[:, 4:] >> 4
        return (q * sc + mn).reshape(n, k), bias
    # LUT 4-bit: high nibble = even element; tables expanded as init.rs:109-124
    t = ff.get_f32_slice(e["c_off"], e["c_len"]).astype(np.float64)
    if t.size == 16:
        t = np.tile(t, n * nb)
    elif t.size == nb * 16:
        t = np.tile(t, n)
    t = t[: n * nb * 16].reshape(n * nb, 16)
    c = dna[: n * nb * 16].reshape(n * nb, 16)
    idx = np.empty((n * nb, 32), np.int64)
    idx[:, 0::2], idx[:, 1::2] = c >> 4, c & 15
    return np.take_along_axis(t, idx, axis=1).reshape(n, k), bias


def _linear(ff, name, x):
    """Rows of a [tokens][in] batch: W x with the 1e-6 flush, then the bias
    (a bias shorter than the rows leaves the later rows without one)."""
    w, b = tensor_weights(ff, name)
    y = x @ w.T
    y[np.abs(y) < 1e-6] = 0.0
    nb = min(b.size, y.shape[1])
    y[:, :nb] += b[:nb]
    return y


def _rms(x, w, eps):
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w


def _rope(v, heads, hd, base, pos, interleaved, f32_angles):
    """v: [tokens][heads * hd]; pos: [tokens].  With f32_angles the angle is
    the reference's float32 value, theta = f32(pos) * (1 / powf(base, f32(2i) / f32(hd)))
    rounded as attention.rs:66-67 rounds it (powf taken as the correctly
    rounded power); only sin and cos are then exact."""
    if f32_angles:
        i = np.arange(hd // 2)
        e = (np.float32(2.0) * i.astype(np.float32)) / np.float32(hd)
        pw = (np.float64(np.float32(base)) ** e.astype(np.float64)).astype(np.float32)
        freq = (np.float32(1.0) / pw).astype(np.float32)
        th = (pos[:, None].astype(np.float32) * freq[None, :]).astype(np.float32).astype(np.float64)
    else:
        i = np.arange(hd // 2, dtype=np.float64)
        freq = 1.0 / base ** (2.0 * i / hd)
        th = pos[:, None].astype(np.float64) * freq[None, :]
    c, s = np.cos(th)[:, None, :], np.sin(th)[:, None, :]
    v = v.reshape(v.shape[0], heads, hd).copy()
    if interleaved:
        a, b = v[:, :, 0::2].copy(), v[:, :, 1::2].copy()
        v[:, :, 0::2], v[:, :, 1::2] = a * c - b * s, a * s + b * c
    else:
        a, b = v[:, :, : hd // 2].copy(), v[:, :, hd // 2:].copy()
        v[:, :, : hd // 2], v[:, :, hd // 2:] = a * c - b * s, a * s + b * c
    return v.reshape(v.shape[0], heads * hd)


def _swiglu(g, u):
    gs = np.clip(g, -64.0, 64.0)
    return g * (1.0 / (1.0 + np.exp(-gs))) * u


def forward_fp64(ff, cfg, ids, logits_for="last", h_scale=1.0, stats=None, f32_angles=False):
    """Float64 logits of a prompt fed from an empty cache: the last token's
    ([vocab]) or every token's ([tokens][vocab]) with logits_for="all".
    stats, when given, counts in "gnorm_fired" the (token, block) pairs whose
    use_genomic_norm scaling applies (a test of that branch must make it fire).
    f32_angles keeps the reference's float32 RoPE angles (see _rope)."""
    E, H, KV, L = cfg.n_embd, cfg.n_head, cfg.n_head_kv, cfg.n_blocks
    hd = E // H
    base = float(cfg.config["rope_base"])
    interleaved = cfg.config["rope_style"] != "split"
    gnorm = bool(cfg.config["use_genomic_norm"])
    eps = float(np.float32(cfg.eps))
    ids = np.asarray(ids, np.int64)
    T = ids.size
    pos = np.arange(T)
    f32 = lambda name: ff.get_f32_slice(ff.tensors[name]["dna_off"], ff.tensors[name]["dna_len"]).astype(np.float64)
    emb, _ = tensor_weights(ff, "token_embd")
    x = emb[ids].copy()
    del emb
    mask = np.triu(np.full((T, T), -np.inf), 1)
    for i in range(L):
        p = f"blk.{i}."
        xn = _rms(x, f32(p + "attn_norm"), eps)
        if p + "attn_qkv" in ff.tensors:
            qkv = _linear(ff, p + "attn_qkv", xn)
            q, k, v = qkv[:, : H * hd], qkv[:, H * hd:(H + KV) * hd], qkv[:, (H + KV) * hd:(H + 2 * KV) * hd]
        else:
            q, k, v = (_linear(ff, p + t, xn) for t in ("attn_q", "attn_k", "attn_v"))
        q = _rope(q, H, hd, base, pos, interleaved, f32_angles).reshape(T, H, hd)
        k = _rope(k, KV, hd, base, pos, interleaved, f32_angles).reshape(T, KV, hd)
        v = v.reshape(T, KV, hd)
        att = np.empty((T, H, hd))
        for h in range(H):
            kh = h // (H // KV)
            s = q[:, h, :] @ k[:, kh, :].T / np.sqrt(hd) + mask
            e = np.exp(s - s.max(axis=1, keepdims=True))
            w = e / (e.sum(axis=1, keepdims=True) + 1e-12)
            att[:, h, :] = w @ v[:, kh, :]
        x = x + _linear(ff, p + "attn_output", att.reshape(T, H * hd))
        xf = _rms(x, f32(p + "ffn_norm"), eps)
        if p + "ffn_gate_up" in ff.tensors:
            gu = _linear(ff, p + "ffn_gate_up", xf)
            n = gu.shape[1] // 2
            g, u = gu[:, :n], gu[:, n:2 * n]
        else:
            g, u = (_linear(ff, p + t, xf) for t in ("ffn_gate", "ffn_up"))
        f = _swiglu(g, u)
        if gnorm:
            rms = np.sqrt(np.mean(f * f, axis=1, keepdims=True) + eps)
            if stats is not None:
                stats["gnorm_fired"] = stats.get("gnorm_fired", 0) + int((rms > h_scale).sum())
            f = np.where(rms > h_scale, f * (h_scale / rms), f)
        x = x + _linear(ff, p + "ffn_down", f)
    hn = _rms(x if logits_for == "all" else x[-1:], f32("output_norm"), eps)
    logits = _linear(ff, "lm_head", hn)
    return logits if logits_for == "all" else logits[0]
