"""Random-init `.gaje.flat` models for the benchmark shapes.

No checkpoints exist in this environment, so the benchmark configurations are
materialised by the C++ writer (csrc/synth.cpp) with a counter-based PRNG; the
recipe is documented there.  Presets:

  smollm2-135m   hidden 576, 30 layers, 9/3 heads, ffn 1536, vocab 49152,
                 eps 1e-5, RoPE theta 1e4 (arch family 1), tied f32 embeddings
  qwen2-0.5b     hidden 896, 24 layers, 14/2 heads, ffn 4864, vocab 151936,
                 eps 1e-6, theta 1e6 (family 3), QKV bias
  qwen2.5-1.5b   hidden 1536, 28 layers, 12/2 heads, ffn 8960, vocab 151936,
                 eps 1e-6, theta 1e6 (family 4), QKV bias
Norm weights are 1 + 0.1 N(0,1); f32 embeddings / lm_head and biases N(0, 0.02);
the 4-bit body follows the 16-quantile x per-block-scale recipe.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from ._lib import SynthConfig, check, lib

Q4_0 = 1
LUT4 = 2
BIT2 = 4  # Genomic2Bit (bit_depth 2)

PRESETS = {
    "smollm2-135m": dict(n_embd=576, n_head=9, n_head_kv=3, n_blocks=30, ffn=1536, vocab_size=49152,
                         eps=1e-5, rope_base=1e4, arch_family=1, qkv_bias=0, tied_embeddings=1),
    "qwen2-0.5b": dict(n_embd=896, n_head=14, n_head_kv=2, n_blocks=24, ffn=4864, vocab_size=151936,
                       eps=1e-6, rope_base=1e6, arch_family=3, qkv_bias=1, tied_embeddings=0),
    "qwen2.5-1.5b": dict(n_embd=1536, n_head=12, n_head_kv=2, n_blocks=28, ffn=8960,
                         vocab_size=151936, eps=1e-6, rope_base=1e6, arch_family=4, qkv_bias=1,
                         tied_embeddings=0),
}


def make_config(body_format: int = Q4_0, fused: bool = True, seed: int = 0, **shape) -> SynthConfig:
    c = SynthConfig()
    for k, v in shape.items():
        setattr(c, k, v)
    c.body_format = int(body_format)
    c.fused = int(bool(fused))
    c.seed = int(seed)
    return c


def write_flat(path: str, preset: str | None = None, body_format: int = Q4_0, fused: bool = True,
               seed: int = 0, **shape) -> str:
    """Write a synthetic model; `preset` names a shape in PRESETS, keywords override it."""
    args = dict(PRESETS[preset]) if preset else {}
    args.update(shape)
    cfg = make_config(body_format=body_format, fused=fused, seed=seed, **args)
    check(lib().gaje_synth_write_flat(os.fsencode(path), ctypes.byref(cfg)))
    return path


def q4_0_tensor(seed: int, name: str, n: int, k: int) -> np.ndarray:
    """[n][k/32] Q4_0 blocks (20 bytes each) of the C0 recipe, as a flat byte array."""
    out = np.empty(n * (k // 32) * 20, dtype=np.uint8)
    check(lib().gaje_synth_q4_0(seed, name.encode(), n, k, out.ctypes.data))
    return out


def lut4_tensor(seed: int, name: str, n: int, k: int):
    """([n][k/32][16] code bytes, [n][k/32][16] f32 tables) of the C0-LUT recipe."""
    codes = np.empty(n * (k // 32) * 16, dtype=np.uint8)
    lut = np.empty(n * (k // 32) * 16, dtype=np.float32)
    check(lib().gaje_synth_lut4(seed, name.encode(), n, k, codes.ctypes.data, lut.ctypes.data))
    return codes, lut


def bit2_tensor(seed: int, name: str, n: int, k: int):
    """([n][k/32][8] code bytes, [n][k/32][4] f32 centroids) of the 2-bit recipe."""
    codes = np.empty(n * (k // 32) * 8, dtype=np.uint8)
    cent = np.empty(n * (k // 32) * 4, dtype=np.float32)
    check(lib().gaje_synth_2bit(seed, name.encode(), n, k, codes.ctypes.data, cent.ctypes.data))
    return codes, cent


def normal(seed: int, name: str, count: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(count, dtype=np.float32)
    check(lib().gaje_synth_normal(seed, name.encode(), count, mean, std, out.ctypes.data))
    return out
