"""Native `.gaje.flat` writer over f32 weights (csrc/writer.cpp, csrc/quantize.cpp).

Mirrors the reference's export path: `export_gaje_flat` follows
scripts/export_gaje_flat.py:184-483 (tensor order, fused QKV and gate/up rows,
metadata JSON, 4096-byte header), and the quantisers are the ones its
GenomicLayer calls (python/gaje/nn/stabilized.py:242-323):
`quantize_q4_0_native` and `quantize_q8_0_native`
(src/compute/quantize/python.rs:151-300) and `genomize_4bit_core`
(src/compute/quantize/genomize.rs:286-382).  Weights are taken in the
reference's split (HuggingFace) row order; the GGUF Q/K un-permutation the
exporter applies to Llama-family GGUF files is the caller's.
"""
from __future__ import annotations

import ctypes
import json
import os

import numpy as np

from ._lib import FlatWriterHeader, check, lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def quantize_q4_0_native(weights) -> bytes:
    w = _f32(weights).reshape(-1)
    out = np.empty(w.size // 32 * 20, np.uint8)
    check(lib().gaje_quantize_q4_0(w.ctypes.data, w.size, out.ctypes.data))
    return out.tobytes()


def quantize_q8_0_native(weights) -> bytes:
    w = _f32(weights).reshape(-1)
    out = np.empty(w.size // 32 * 34, np.uint8)
    check(lib().gaje_quantize_q8_0(w.ctypes.data, w.size, out.ctypes.data))
    return out.tobytes()


def genomize_4bit_core(weights, block_size: int = 32, anchor_threshold: float = -1.0):
    """(codes bytes, centroids list, anchor buffer bytes), as genomize_4bit_core returns them."""
    w = _f32(weights).reshape(-1)
    nb = w.size // block_size
    codes = np.empty(max(nb * (block_size // 2), 1), np.uint8)
    cent = np.empty(max(nb * 16, 1), np.float32)
    n_anc = ctypes.c_int64(0)
    check(lib().gaje_genomize_4bit(w.ctypes.data, w.size, block_size, float(anchor_threshold), codes.ctypes.data,
                                   cent.ctypes.data, None, ctypes.byref(n_anc)))
    anc = np.empty(n_anc.value, np.uint8)
    check(lib().gaje_genomize_4bit(w.ctypes.data, w.size, block_size, float(anchor_threshold), None, None,
                                   anc.ctypes.data, ctypes.byref(n_anc)))
    return codes[:nb * (block_size // 2)].tobytes(), [float(c) for c in cent[:nb * 16]], anc.tobytes()


class FlatWriter:
    """Tensors in file order, then write()."""

    def __init__(self):
        h = ctypes.c_void_p()
        check(lib().gaje_flat_writer_create(ctypes.byref(h)))
        self._h = h.value

    def close(self):
        if self._h:
            lib().gaje_flat_writer_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def add_norm(self, name: str, w):
        w = _f32(w).reshape(-1)
        check(lib().gaje_flat_writer_add_norm(self._h, name.encode(), w.ctypes.data, w.size))

    def add(self, name: str, w, fmt: str = "q4_0", bias=None, anchor_threshold: float = -1.0):
        """fmt: 'f32' (bit_depth 32), 'q4_0', 'q8_0' or 'lut4' (genomize_4bit_core)."""
        w = _f32(w)
        out_f, in_f = w.shape
        b = _f32(bias).reshape(-1) if bias is not None else None
        bp, bn = (b.ctypes.data, b.size) if b is not None and b.size else (None, 0)
        L = lib()
        if fmt == "f32":
            check(L.gaje_flat_writer_add_f32(self._h, name.encode(), w.ctypes.data, out_f, in_f, bp, bn))
        elif fmt == "q4_0":
            check(L.gaje_flat_writer_add_q4_0(self._h, name.encode(), w.ctypes.data, out_f, in_f, bp, bn))
        elif fmt == "q8_0":
            check(L.gaje_flat_writer_add_q8_0(self._h, name.encode(), w.ctypes.data, out_f, in_f, bp, bn))
        elif fmt == "lut4":
            check(L.gaje_flat_writer_add_lut4(self._h, name.encode(), w.ctypes.data, out_f, in_f,
                                              float(anchor_threshold), bp, bn))
        else:
            raise ValueError(f"unknown tensor format {fmt!r}")

    def write(self, path: str, metadata: dict, arch_family: int, n_embd: int, n_head: int, n_head_kv: int,
              n_blocks: int, qk_permute: bool = False, flags: int = 0x3, quant_format: int = 1):
        h = FlatWriterHeader(flags=flags, group_size=32, quant_format=quant_format, arch_family=arch_family,
                             n_embd=n_embd, n_head=n_head, n_head_kv=n_head_kv, n_blocks=n_blocks,
                             qk_permute=int(bool(qk_permute)))
        check(lib().gaje_flat_writer_write(self._h, os.fsencode(path), json.dumps(metadata).encode(),
                                           ctypes.byref(h)))


def export_gaje_flat(path: str, tensors, n_embd: int, n_head: int, n_head_kv: int, n_blocks: int,
                     vocab_size: int, eps: float, rope_base: float, arch_family: int = 3,
                     name: str = "qwen2", quant_embed: bool = False, body: str = "q4_0",
                     anchor_threshold: float = -1.0, tokenizer_id: str = "", tokenizer: str = "") -> str:
    """export_gaje_flat over f32 tensors keyed by their GGUF names (token_embd.weight,
    output_norm.weight, lm_head.weight (else the tied token_embd), blk.{i}.attn_norm.weight,
    blk.{i}.ffn_norm.weight, blk.{i}.attn_{q,k,v}.weight (+ .bias), blk.{i}.attn_output.weight,
    blk.{i}.ffn_{gate,up,down}.weight), each [out][in].

    body="q4_0" (the default) is the reference exporter's output: Q4_0 blocks and
    quant_format 1 (scripts/export_gaje_flat.py).  body="lut4" is an extension
    with no counterpart in that exporter: it writes quant_format 0 and runs
    genomize_4bit_core over each whole tensor, where the reference's GenomicLayer
    splits tensors over 100 MB into 10000-row chunks with their own thresholds
    and anchor buffers; files it writes for such tensors are not what the
    reference would write."""
    T = {k: _f32(v) for k, v in tensors.items()}
    emb = "q8_0" if quant_embed else "f32"
    w = FlatWriter()
    w.add("token_embd", T["token_embd.weight"], emb)
    w.add_norm("output_norm", T["output_norm.weight"])
    w.add("lm_head", T.get("lm_head.weight", T["token_embd.weight"]), emb)
    for i in range(n_blocks):
        p = f"blk.{i}."
        for nm in ("attn_norm", "ffn_norm"):
            if p + nm + ".weight" in T:
                w.add_norm(p + nm, T[p + nm + ".weight"])
        qkv = np.concatenate([T[p + "attn_q.weight"], T[p + "attn_k.weight"], T[p + "attn_v.weight"]], axis=0)
        bias = None
        if all(p + f"attn_{t}.bias" in T for t in "qkv"):
            bias = np.concatenate([T[p + f"attn_{t}.bias"] for t in "qkv"])
        w.add(p + "attn_qkv", qkv, body, bias=bias, anchor_threshold=anchor_threshold)
        w.add(p + "attn_output", T[p + "attn_output.weight"], body, bias=T.get(p + "attn_output.bias"),
              anchor_threshold=anchor_threshold)
        gu = np.concatenate([T[p + "ffn_gate.weight"], T[p + "ffn_up.weight"]], axis=0)
        w.add(p + "ffn_gate_up", gu, body, anchor_threshold=anchor_threshold)
        w.add(p + "ffn_down", T[p + "ffn_down.weight"], body, anchor_threshold=anchor_threshold)
    metadata = {"config": {"name": name, "version": "0.9.8", "tokenizer_id": tokenizer_id, "rope_base": rope_base,
                           "ffn_act": "swiglu" if arch_family != 5 else "geglu", "use_genomic_norm": False},
                "n_embd": n_embd, "n_head": n_head, "n_head_kv": n_head_kv, "n_blocks": n_blocks,
                "vocab_size": vocab_size, "eps": eps, "tokenizer": tokenizer}
    w.write(path, metadata, arch_family, n_embd, n_head, n_head_kv, n_blocks,
            quant_format=1 if body == "q4_0" else 0)
    w.close()
    return path
