"""CPU oracle for the GAJE quantised decode path.

TEST INFRASTRUCTURE ONLY.  tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg are the only users; the product never imports this module.

The arithmetic lives in gaje_oracle.c (line-faithful AVX2 restatement of the
reference kernels); this module restates the orchestration around it:

  GenomicLinear::new dispatch, LUT expansion, anchors  src/nn/linear/init.rs:12-160
  GenomicLinear::forward_core / get_row_core           src/nn/linear/forward.rs:119-285
  GenomicAttention::forward_attention_core             src/nn/attention.rs:45-128
  RustGenomicBlock::forward_core                       src/nn/block/forward.rs:10-157
  GenomicLLM::forward_core / forward_with_hidden_core  src/nn/llm/forward.rs:7-113
  GenomicLLM::clear_cache_core / generate_native_core  src/nn/llm/forward.rs:174-330
  GajeFlatFileReader::get_linear / load_genomic        src/io/flat_reader.rs:92-236
  set_k_wta_ratio                                       src/nn/llm/python.rs:53-59

What pins each part (tests/test_oracle_*.py):
  Q4_0 dequant              reference KATs (header/tests.rs:51-88, linear/tests.rs:7-100),
                            closed form over all 16 codes x f16 pairs
  Q4_0 / LUT / f32 dots     fp64 dot with a Higham bound; the scalar factored form;
                            the dequantised-row dot; linear/tests.rs:7-100 KAT
  Q8_0 dequant / dot        closed form (q * scale exact) over all 256 codes x f16 edge
                            scales; header/tests.rs:121-165 round-trip KAT through the
                            restated writer; fp64 dot with a Higham bound; scalar form
  rms_norm                  closed form in fp64; torch CPU RMSNorm
  RoPE                      HF-style rotate_half on the CPU (split) and the
                            interleaved definition of tests/unit/test_rope_logic.py
  attention                 torch CPU scaled_dot_product_attention with GQA repeat;
                            brute force at ctx 1
  swiglu_balanced           torch CPU silu(g)*u (g >= -64), closed form below
  K-WTA                     brute-force sort
  header / reader           header/tests.rs:7-48 KATs, exporter layout
  whole forward             torch CPU fp32 composition from the dequantised weights
  sampling branch            its distribution (chi-square against softmax(l / T)), the
                            near-greedy limit and the penalty before the draw
  use_genomic_norm           a float64 composition (tests/fp64_model.py) where it fires
Parity unpinned: the exact bits of glibc expf/powf/sinf/cosf as the Rust build
would see them (no Rust toolchain here); the sampled tokens themselves
(thread_rng upstream, so nothing fixes its draws; the device's splitmix draws
are restated by SplitMixDraws).
"""
from __future__ import annotations

import ctypes
import os
import struct

import numpy as np

from .flat import FlatFile, ModelConfig

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

Q4_0_BLOCK_BYTES = 20
BLOCK_SIZE = 32  # hard-coded by load_genomic (flat_reader.rs:141)

KIND_F32, KIND_Q4_0, KIND_LUT4, KIND_Q8_0, KIND_2BIT = 0, 1, 2, 3, 4
Q8_0_BLOCK_BYTES = 34

_fp = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)


class _OrcLinear(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int), ("out_features", ctypes.c_int64),
                ("in_features", ctypes.c_int64), ("db", ctypes.c_void_p),
                ("db_len", ctypes.c_int64), ("centroids", ctypes.c_void_p),
                ("centroids_len", ctypes.c_int64), ("bias", ctypes.c_void_p),
                ("bias_len", ctypes.c_int64), ("anchor_indices", ctypes.c_void_p),
                ("anchor_values", ctypes.c_void_p), ("anchor_row_ptrs", ctypes.c_void_p),
                ("n_anchors", ctypes.c_int64)]


def lib():
    """Load oracle/liboracle.so (built by oracle/Makefile)."""
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"oracle library missing: {path} (run `make -C oracle`)")
        L = ctypes.CDLL(path)
        L.orc_init.restype = ctypes.c_int
        if L.orc_init() != 0:
            raise RuntimeError("oracle needs an AVX2+FMA+F16C host (the reference's x86 path)")
        L.orc_set_threads.argtypes = [ctypes.c_int]
        L.orc_get_threads.restype = ctypes.c_int
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_expf_batch.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
        L.orc_q4_0_dequant_weight.argtypes = [ctypes.c_void_p, ctypes.c_int]
        L.orc_q4_0_dequant_weight.restype = ctypes.c_float
        L.orc_q4_0_dequant.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        for fn in ("orc_dot_q4_0_avx2", "orc_dot_q4_0_scalar", "orc_dot_q8_0_avx2", "orc_dot_q8_0_scalar"):
            getattr(L, fn).argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
            getattr(L, fn).restype = ctypes.c_float
        L.orc_q8_0_dequant_weight.argtypes = [ctypes.c_void_p, ctypes.c_int]
        L.orc_q8_0_dequant_weight.restype = ctypes.c_float
        L.orc_q8_0_dequant.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        L.orc_q8_0_quantize.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        L.orc_dot_4bit.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                   ctypes.c_size_t, ctypes.c_size_t]
        L.orc_dot_4bit.restype = ctypes.c_float
        for fn in ("orc_dot_2bit", "orc_dot_2bit_scalar"):
            getattr(L, fn).argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                       ctypes.c_size_t, ctypes.c_size_t, ctypes.c_void_p]
            getattr(L, fn).restype = ctypes.c_float
        L.orc_dequant_2bit.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p]
        L.orc_dot_f32.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]
        L.orc_dot_f32.restype = ctypes.c_float
        L.orc_rms_norm.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float,
                                   ctypes.c_size_t, ctypes.c_void_p]
        L.orc_swiglu_balanced.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                          ctypes.c_size_t]
        L.orc_kwta.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t]
        L.orc_rope.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_float,
                               ctypes.c_size_t, ctypes.c_int]
        L.orc_attention.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                    ctypes.c_size_t, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_void_p]
        L.orc_linear_forward.argtypes = [ctypes.POINTER(_OrcLinear), ctypes.c_void_p,
                                         ctypes.c_int64, ctypes.c_void_p]
        L.orc_linear_row.argtypes = [ctypes.POINTER(_OrcLinear), ctypes.c_int64,
                                     ctypes.c_void_p, ctypes.c_int64]
        L.orc_linear_row.restype = ctypes.c_float
        L.orc_linear_get_row.argtypes = [ctypes.POINTER(_OrcLinear), ctypes.c_int64,
                                         ctypes.c_void_p]
        _LIB = L
    return _LIB


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def get_threads() -> int:
    return lib().orc_get_threads()


def _ptr(a: np.ndarray):
    return a.ctypes.data if a is not None and a.size else None


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------- kernels ---

def f16_to_f32(h: int) -> float:
    return lib().orc_f16_to_f32(h)


def f32_to_f16(f: float) -> int:
    return lib().orc_f32_to_f16(f)


def expf(x: np.ndarray) -> np.ndarray:
    """f32::exp as the reference calls it: the host C library's expf."""
    x = _f32(x)
    y = np.empty_like(x)
    lib().orc_expf_batch(_ptr(x), _ptr(y), x.size)
    return y


def attention(q, k_cache, v_cache, seq_len, n_head, n_head_kv, head_dim):
    """forward_attention_core's attention over an appended cache (attention.rs:87-127);
    caches are [seq_len][n_head_kv * head_dim]."""
    q, k, v = _f32(q), _f32(k_cache), _f32(v_cache)
    out = np.empty(n_head * head_dim, dtype=np.float32)
    lib().orc_attention(_ptr(q), _ptr(k), _ptr(v), seq_len, n_head, n_head_kv, head_dim, _ptr(out))
    return out


def q4_0_dequant(blocks: np.ndarray) -> np.ndarray:
    """Q4_0Block::dequantize_weight over whole blocks (blocks.rs:18-30)."""
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    nb = b.size // Q4_0_BLOCK_BYTES
    out = np.empty(nb * 32, dtype=np.float32)
    lib().orc_q4_0_dequant(_ptr(b), nb, _ptr(out))
    return out


def dot_q4_0(blocks: np.ndarray, x: np.ndarray, scalar: bool = False) -> float:
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    x = _f32(x)
    fn = lib().orc_dot_q4_0_scalar if scalar else lib().orc_dot_q4_0_avx2
    return fn(_ptr(b), _ptr(x), b.size // Q4_0_BLOCK_BYTES)


def q8_0_dequant(blocks: np.ndarray) -> np.ndarray:
    """Q8_0Block::dequantize_weight over whole blocks (blocks.rs:43-49)."""
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    nb = b.size // Q8_0_BLOCK_BYTES
    out = np.empty(nb * 32, dtype=np.float32)
    lib().orc_q8_0_dequant(_ptr(b), nb, _ptr(out))
    return out


def dot_q8_0(blocks: np.ndarray, x: np.ndarray, scalar: bool = False) -> float:
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    x = _f32(x)
    fn = lib().orc_dot_q8_0_scalar if scalar else lib().orc_dot_q8_0_avx2
    return fn(_ptr(b), _ptr(x), b.size // Q8_0_BLOCK_BYTES)


def q8_0_quantize(w: np.ndarray) -> np.ndarray:
    """quantize_q8_0_native's blocks (compute/quantize/python.rs:235-300) as bytes."""
    w = _f32(w).reshape(-1)
    if w.size % 32:
        raise ValueError("Weights length must be divisible by 32")
    out = np.zeros(w.size // 32 * Q8_0_BLOCK_BYTES, dtype=np.uint8)
    lib().orc_q8_0_quantize(_ptr(w), w.size // 32, _ptr(out))
    return out


def dot_4bit(codes: np.ndarray, x: np.ndarray, centroids: np.ndarray) -> float:
    """genomic_dot_product_4bit over one row: centroids are per block ([n_blocks][16]);
    a single 16-entry table is shared by every block, as init.rs:109-124 expands it."""
    c = np.ascontiguousarray(codes, dtype=np.uint8).reshape(-1)
    nb = c.size // 16
    t = _f32(centroids)
    if t.size == 16:
        t = np.ascontiguousarray(np.tile(t, nb))
    if t.size < nb * 16:
        raise ValueError("dot_4bit needs 16 centroids per block")
    return lib().orc_dot_4bit(_ptr(c), _ptr(_f32(x)), _ptr(t), 16, nb)


def dot_2bit(codes: np.ndarray, x: np.ndarray, centroids: np.ndarray, modulation=None,
             scalar: bool = False, stride: int = 8) -> float:
    """genomic_dot_product over one row (genomic.rs:17-144): `stride` code bytes per
    block, centroids read 4 per block from the row's base ([n_blocks][4]; a single
    4-entry table is tiled first, as init.rs:125-139 expands it)."""
    c = np.ascontiguousarray(codes, dtype=np.uint8).reshape(-1)
    nb = c.size // stride
    t = _f32(centroids)
    if t.size == 4:
        t = np.ascontiguousarray(np.tile(t, nb))
    if t.size < nb * 4:
        raise ValueError("dot_2bit needs 4 centroids per block")
    m = _f32(modulation) if modulation is not None else None
    fn = lib().orc_dot_2bit_scalar if scalar else lib().orc_dot_2bit
    return fn(_ptr(c), _ptr(_f32(x)), _ptr(t), stride, nb, _ptr(m) if m is not None else None)


def quantize_embedding(vector, thresholds=None) -> bytes:
    """quantize_embedding (compute/quantize/python.rs:38-71): 2-bit codes, MSB first,
    00 below t0, 01 below t1, 11 below t2, 10 otherwise."""
    t = [-0.43, 0.0, 0.43] if thresholds is None else list(thresholds)
    v = np.asarray(vector, dtype=np.float32)
    out = bytearray()
    for i in range(0, v.size, 4):
        byte = 0
        for j in range(4):
            if i + j < v.size:
                val = v[i + j]
                bits = 0b00 if val < t[0] else 0b01 if val < t[1] else 0b11 if val < t[2] else 0b10
                byte = ((byte << 2) | bits) & 0xFF
        out.append(byte)
    return bytes(out)


def dequantize_embedding(packed, dims: int, centroids=None) -> np.ndarray:
    """dequantize_embedding_core (compute/quantize/dequantize.rs:6-42), including its
    per-dimension table form (4 centroids per dimension when len == dims * 4)."""
    c = np.asarray([-0.68, -0.17, 0.17, 0.68] if centroids is None else centroids, dtype=np.float32)
    multi = c.size == dims * 4
    rec = []
    for byte in bytes(packed):
        for j in range(4):
            if len(rec) >= dims:
                break
            bits = (byte >> ((3 - j) * 2)) & 3
            slot = {0: 0, 1: 1, 3: 2, 2: 3}[bits]
            rec.append(c[len(rec) * 4 + slot] if multi else c[slot])
    return np.asarray(rec, dtype=np.float32)


def dot_f32(a: np.ndarray, b: np.ndarray) -> float:
    a, b = _f32(a), _f32(b)
    return lib().orc_dot_f32(_ptr(a), _ptr(b), a.size)


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x, w = _f32(x), _f32(w)
    out = np.empty_like(x)
    lib().orc_rms_norm(_ptr(x), _ptr(w), ctypes.c_float(eps), x.size, _ptr(out))
    return out


def swiglu_balanced(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    g, u = _f32(gate), _f32(up)
    out = np.empty_like(g)
    lib().orc_swiglu_balanced(_ptr(g), _ptr(u), _ptr(out), g.size)
    return out


def kwta(scores: np.ndarray, k: int) -> np.ndarray:
    s = _f32(scores).copy()
    lib().orc_kwta(_ptr(s), s.size, int(k))
    return s


def rope(vec: np.ndarray, heads: int, head_dim: int, rope_base: float, pos: int,
         is_split: bool) -> np.ndarray:
    v = _f32(vec).copy()
    lib().orc_rope(_ptr(v), heads, head_dim, ctypes.c_float(rope_base), pos, int(is_split))
    return v


# ----------------------------------------------------------------- modules ---

class GenomicLinear:
    """GenomicLinear restricted to the flat-file formats (F32, Q4_0, Q8_0, LUT-4bit, 2-bit)."""

    def __init__(self, database, anchors_u8, centroids, out_features, in_features, bias,
                 bit_depth):
        self.out_features, self.in_features = int(out_features), int(in_features)
        self.db = np.ascontiguousarray(np.frombuffer(bytes(database), dtype=np.uint8)) \
            if not isinstance(database, np.ndarray) else np.ascontiguousarray(database, np.uint8)
        centroids = _f32(centroids) if centroids is not None else np.zeros(0, np.float32)
        self.bias = _f32(bias) if bias is not None else np.zeros(0, np.float32)
        # variant dispatch (init.rs:29-54)
        if bit_depth == 4:
            self.kind = KIND_Q4_0 if centroids.size == 0 else KIND_LUT4
        elif bit_depth == 32:
            self.kind = KIND_F32
        elif bit_depth == 8:
            self.kind = KIND_Q8_0
        else:
            self.kind = KIND_2BIT  # every other bit_depth is Genomic2Bit (init.rs:53)
        # centroid expansion (init.rs:109-139)
        n_blocks = self.in_features // BLOCK_SIZE
        if bit_depth == 4 and centroids.size == 16:
            centroids = np.tile(centroids, self.out_features * n_blocks)
        elif bit_depth == 4 and n_blocks and centroids.size == n_blocks * 16:
            centroids = np.tile(centroids, self.out_features)
        elif self.kind == KIND_2BIT and centroids.size == 4:
            centroids = np.tile(centroids, self.out_features * n_blocks)
        elif self.kind == KIND_2BIT and n_blocks and centroids.size == n_blocks * 4:
            centroids = np.tile(centroids, self.out_features)
        if self.kind == KIND_2BIT and 0 < centroids.size < max(4, n_blocks * 4):
            # the reference's row dot would read past such a table (forward.rs:40-45
            # hands the dot the table's start for rows without their own centroids)
            raise ValueError(f"2-bit centroid table of {centroids.size} floats")
        self.centroids = np.ascontiguousarray(centroids)
        self._parse_anchors(bytes(anchors_u8) if anchors_u8 is not None else b"")
        self._c = _OrcLinear(self.kind, self.out_features, self.in_features, _ptr(self.db),
                             self.db.size, _ptr(self.centroids), self.centroids.size,
                             _ptr(self.bias), self.bias.size, _ptr(self.a_idx),
                             _ptr(self.a_val), _ptr(self.a_ptr), self.a_idx.size)

    def _parse_anchors(self, buf: bytes):
        """Sparse f16 anchors in the "GAJE" buffer layout (init.rs:61-107)."""
        n_out, n_in = self.out_features, self.in_features
        if len(buf) >= 4 and buf[:4] == b"GAJE":
            count = struct.unpack_from("<I", buf, 4)[0]
            idx_s, val_s = 8, 8 + count * 4
            ptr_s = val_s + count * 2
            self.a_idx = np.frombuffer(buf, dtype="<u4", count=count, offset=idx_s).copy()
            self.a_val = np.frombuffer(buf, dtype="<u2", count=count, offset=val_s).copy()
            ptrs = np.zeros(n_out + 1, dtype=np.int64)
            if len(buf) >= ptr_s + (n_out + 1) * 8:
                ptrs[:] = np.frombuffer(buf, dtype="<u8", count=n_out + 1, offset=ptr_s)
            else:
                cur = 0
                for a, flat in enumerate(self.a_idx):
                    r = int(flat) // n_in
                    while cur < r:
                        ptrs[cur + 1] = a
                        cur += 1
                while cur < n_out:
                    ptrs[cur + 1] = len(self.a_idx)
                    cur += 1
            self.a_ptr = ptrs
        else:
            self.a_idx = np.zeros(0, np.uint32)
            self.a_val = np.zeros(0, np.uint16)
            self.a_ptr = np.zeros(n_out + 1, np.int64)

    def forward_core(self, x: np.ndarray) -> np.ndarray:
        x = _f32(x)
        out = np.empty(self.out_features, dtype=np.float32)
        lib().orc_linear_forward(ctypes.byref(self._c), _ptr(x), x.size, _ptr(out))
        return out

    def row(self, i: int, x: np.ndarray) -> float:
        x = _f32(x)
        return lib().orc_linear_row(ctypes.byref(self._c), i, _ptr(x), x.size)

    def get_row_core(self, idx: int) -> np.ndarray:
        out = np.empty(self.in_features, dtype=np.float32)
        lib().orc_linear_get_row(ctypes.byref(self._c), int(idx), _ptr(out))
        return out


class GenomicAttention:
    """GenomicAttention with its f32 KV cache (attention.rs:10-40,130-136)."""

    def __init__(self, n_head, n_head_kv, head_dim, rmsnorm_weight, eps, rope_base, rope_style):
        self.n_head, self.n_head_kv, self.head_dim = n_head, n_head_kv, head_dim
        self.rmsnorm_weight = _f32(rmsnorm_weight)
        self.eps = np.float32(eps)
        self.rope_base = np.float32(rope_base)
        self.rope_style = rope_style
        kv = n_head_kv * head_dim
        self._k = np.zeros((16, kv), np.float32)
        self._v = np.zeros((16, kv), np.float32)
        self.len = 0

    def k_cache_len(self) -> int:
        return self.len

    def clear_cache_core(self):
        self.len = 0

    def forward_attention_core(self, q, k, v, pos):
        is_split = self.rope_style == "split"
        q_rope = rope(q, self.n_head, self.head_dim, self.rope_base, pos, is_split)
        k_rope = rope(k, self.n_head_kv, self.head_dim, self.rope_base, pos, is_split)
        if self.len == self._k.shape[0]:
            self._k = np.concatenate([self._k, np.zeros_like(self._k)])
            self._v = np.concatenate([self._v, np.zeros_like(self._v)])
        self._k[self.len] = k_rope
        self._v[self.len] = v
        self.len += 1
        out = np.empty(self.n_head * self.head_dim, dtype=np.float32)
        lib().orc_attention(_ptr(q_rope), _ptr(self._k), _ptr(self._v), self.len, self.n_head,
                            self.n_head_kv, self.head_dim, _ptr(out))
        return out


class RustGenomicBlock:
    """RustGenomicBlock for flat loads: fused or split qkv / gate_up, no topology."""

    def __init__(self, idx, attn, w_o, w_down, ffn_norm, eps, use_genomic_norm,
                 fused_qkv=None, fused_gate_up=None, qkv_split=None, gate_up_split=None,
                 h_scale=1.0):
        self.idx, self.attn, self.w_o, self.w_down = idx, attn, w_o, w_down
        self.ffn_norm = _f32(ffn_norm)
        self.eps = np.float32(eps)
        self.use_genomic_norm = use_genomic_norm
        self.fused_qkv, self.fused_gate_up = fused_qkv, fused_gate_up
        self.qkv_split, self.gate_up_split = qkv_split, gate_up_split
        self.h_scale = np.float32(h_scale)
        self.k_wta_ratio = 0.0  # block/init.rs:42

    def forward_core(self, x: np.ndarray, pos: int) -> np.ndarray:
        if np.isnan(x).any():
            raise ValueError("Input x is NaN")
        a = self.attn
        if a.rmsnorm_weight.size:
            x_norm = rms_norm(x, a.rmsnorm_weight, a.eps)
            if np.isnan(x_norm).any():
                raise ValueError("NaN after attn rms_norm")
        else:
            x_norm = x.copy()
        q_dim, kv_dim = a.n_head * a.head_dim, a.n_head_kv * a.head_dim
        if self.fused_qkv is not None:
            qkv = self.fused_qkv.forward_core(x_norm)
            q, k, v = qkv[:q_dim], qkv[q_dim:q_dim + kv_dim], qkv[q_dim + kv_dim:q_dim + 2 * kv_dim]
        else:
            q, k, v = (l.forward_core(x_norm) for l in self.qkv_split)
        attn_out = a.forward_attention_core(q, k, v, pos)
        proj = self.w_o.forward_core(attn_out)
        x_post = (x + proj).astype(np.float32)
        x_ffn_n = rms_norm(x_post, self.ffn_norm, self.eps)
        if self.fused_gate_up is not None:
            gu = self.fused_gate_up.forward_core(x_ffn_n)
            ffn = gu.size // 2
            gate, up = gu[:ffn], gu[ffn:2 * ffn]
        else:
            gate, up = (l.forward_core(x_ffn_n) for l in self.gate_up_split)
        if np.isnan(up).any():
            raise ValueError("NaN in up")
        ffn_out = swiglu_balanced(gate, up)
        if np.isnan(ffn_out).any():
            raise ValueError("NaN in ffn_out")
        if self.use_genomic_norm:
            # block/forward.rs:115-123.  Upstream sums with a rayon reduction
            # whose order is not fixed; here (and on the device) a sequential
            # float32 sum of the rounded squares, in element order.
            sq = (ffn_out * ffn_out).astype(np.float32)
            ss = np.cumsum(sq, dtype=np.float32)[-1] if sq.size else np.float32(0.0)
            rms = np.float32(np.sqrt(np.float32(np.float32(ss / np.float32(ffn_out.size)) + self.eps)))
            if rms > self.h_scale:
                ffn_out = (ffn_out * np.float32(self.h_scale / rms)).astype(np.float32)
        proj_ffn = self.w_down.forward_core(ffn_out)
        if np.isnan(proj_ffn).any():
            raise ValueError("NaN in projected_ffn")
        final = (x_post + proj_ffn).astype(np.float32)
        if np.isnan(final).any():
            raise ValueError("NaN after projected_ffn addition")
        if 0.0 < self.k_wta_ratio < 1.0:
            k = max(int(np.float32(final.size) * np.float32(self.k_wta_ratio)), 1)
            final = kwta(final, k)
        return final

    def clear_cache_core(self):
        self.attn.clear_cache_core()


class GenomicLLM:
    """GenomicLLM as returned by load_genomic (k_wta_ratio 0.5, no topology)."""

    def __init__(self, embeddings, blocks, output_norm, lm_head, eps):
        self.embeddings, self.blocks = embeddings, blocks
        self.output_norm = _f32(output_norm)
        self.lm_head = lm_head
        self.eps = np.float32(eps)
        self.k_wta_ratio = 0.5  # flat_reader.rs:234

    @property
    def vocab_size(self):
        return self.embeddings.out_features

    def set_k_wta_ratio(self, ratio: float):
        self.k_wta_ratio = float(np.float32(ratio))
        for b in self.blocks:
            b.k_wta_ratio = self.k_wta_ratio

    def clear_cache_core(self):
        for b in self.blocks:
            b.clear_cache_core()

    def _hidden(self, token_id: int, clear_cache: bool) -> np.ndarray:
        if clear_cache:
            self.clear_cache_core()
        pos = self.blocks[0].attn.k_cache_len() if self.blocks else 0
        h = self.embeddings.get_row_core(token_id)
        for b in self.blocks:
            h = b.forward_core(h, pos)
        return rms_norm(h, self.output_norm, self.eps)

    def forward_core(self, token_id: int, clear_cache: bool = False) -> np.ndarray:
        h_norm = self._hidden(token_id, clear_cache)
        if self.lm_head.out_features == 0:
            raise ValueError("LM Head out_features is 0!")
        logits = self.lm_head.forward_core(h_norm)
        if 0.0 < self.k_wta_ratio < 1.0:
            k = max(int(np.float32(logits.size) * np.float32(self.k_wta_ratio)), 1)
            logits = kwta(logits, k)
        return logits

    def forward_with_hidden_core(self, token_id: int, clear_cache: bool = False):
        h_norm = self._hidden(token_id, clear_cache)
        return self.lm_head.forward_core(h_norm), h_norm

    def generate_native_core(self, prompt_tokens, max_new_tokens, temperature,
                             repetition_penalty, eos_token_ids, rng=None):
        if len(prompt_tokens) == 0:
            raise ValueError("Prompt tokens cannot be empty")
        self.clear_cache_core()
        last = None
        for t in prompt_tokens:
            last = self.forward_core(int(t), False)
        generated = []
        for _ in range(max_new_tokens):
            if last is None or last.size == 0:
                break
            logits = last.copy()
            if repetition_penalty > 1.0:
                seen = set(generated) - set(eos_token_ids)
                for t in seen:
                    if t < logits.size:
                        if logits[t] < 0.0:
                            logits[t] = np.float32(logits[t] * np.float32(repetition_penalty))
                        else:
                            logits[t] = np.float32(logits[t] / np.float32(repetition_penalty))
            if np.float32(temperature) <= np.float32(1e-5):
                nxt = argmax_first(logits)
            else:
                nxt = sample_next(logits, temperature, rng)
            generated.append(int(nxt))
            if nxt in eos_token_ids:
                break
            rep = False
            for w in range(2, 49):
                if len(generated) >= w * 3:
                    a = generated[-w:]
                    if a == generated[-2 * w:-w] and a == generated[-3 * w:-2 * w]:
                        rep = True
                        break
            if rep:
                break
            last = self.forward_core(int(nxt), False)
        return generated


def moe_route(x: np.ndarray, router: np.ndarray):
    """Top-2 routing of the MoE layer (no reference function; the composition the
    device layer defines): logits by dot_product (dot.rs:23-94), softmax with
    expf(l - max) and a serial sum in expert order, p_e = e_e / sum, the two
    largest p (ties to the lower id), weights p / (p_a + p_b).  Parity of the
    routing semantics themselves is unpinned (nothing in the reference fixes
    them); the arithmetic is float32 throughout."""
    x = _f32(x)
    router = _f32(router)
    T, E = x.shape[0], router.shape[0]
    idx = np.zeros((T, 2), np.int32)
    w = np.zeros((T, 2), np.float32)
    for t in range(T):
        l = np.array([dot_f32(x[t], router[e]) for e in range(E)], np.float32)
        mx = l[0]
        for e in range(1, E):
            mx = l[e] if l[e] > mx else mx
        ex = expf((l - mx).astype(np.float32))
        s = np.float32(0.0)
        for e in range(E):
            s = np.float32(s + ex[e])
        p = (ex / s).astype(np.float32)
        a = 0
        for e in range(1, E):
            if p[e] > p[a]:
                a = e
        b = 1 if a == 0 else 0
        for e in range(E):
            if e != a and p[e] > p[b]:
                b = e
        den = np.float32(p[a] + p[b])
        idx[t] = (a, b)
        w[t] = (np.float32(p[a] / den), np.float32(p[b] / den))
    return idx, w


def moe_ffn(x: np.ndarray, router: np.ndarray, gate_up, down, ffn: int):
    """The MoE layer through the oracle's GenomicLinear rows: expert e is
    down_e(swiglu_balanced(gate_e(x), up_e(x))) with Q4_0 blocks gate_up[e]
    ([2 ffn][h]) and down[e] ([h][ffn]); y = (w_a f_a) + (w_b f_b)."""
    x = _f32(x)
    T, h = x.shape
    idx, w = moe_route(x, router)
    gu = [GenomicLinear(b, b"", None, 2 * ffn, h, None, 4) for b in gate_up]
    dn = [GenomicLinear(b, b"", None, h, ffn, None, 4) for b in down]
    y = np.zeros((T, h), np.float32)
    for t in range(T):
        f = []
        for k in range(2):
            e = int(idx[t, k])
            g = gu[e].forward_core(x[t])
            f.append(dn[e].forward_core(swiglu_balanced(g[:ffn], g[ffn:])))
        y[t] = (w[t, 0] * f[0]).astype(np.float32) + (w[t, 1] * f[1]).astype(np.float32)
    return y, idx, w


def sample_next(logits: np.ndarray, temperature: float, rng) -> int:
    """The multinomial branch of generate_native_core (forward.rs:272-297):
    max by strict '>', p_i = exp((l_i - max) / T), a sequential float32 sum,
    r = u * sum with one uniform draw u, then the first i whose running sum
    reaches r (0 if none)."""
    if rng is None:
        raise ValueError("sampling needs an rng (upstream uses thread_rng)")
    logits = _f32(logits)
    fin = logits[~np.isnan(logits)]
    m = fin.max() if fin.size else np.float32(-np.inf)
    p = expf(((logits - m) / np.float32(temperature)).astype(np.float32))
    c = np.cumsum(p, dtype=np.float32)
    r = np.float32(np.float32(_draw(rng)) * c[-1])
    hit = np.nonzero(r <= c)[0]
    return int(hit[0]) if hit.size else 0


class SplitMixDraws:
    """The uniform draws of the device library's sampler: a splitmix64 stream,
    state += 0x9E3779B97F4A7C15, u = (mix(state) >> 40) * 2^-24, a float32 in
    [0, 1) with 24 random bits (the form of rand's gen::<f32>() that
    forward.rs:287 draws from thread_rng).  Seeded like gaje_hip_generate."""

    def __init__(self, seed: int):
        self.state = int(seed) & 0xFFFFFFFFFFFFFFFF

    @staticmethod
    def mix(z: int) -> int:
        M = 0xFFFFFFFFFFFFFFFF
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
        return z ^ (z >> 31)

    def __call__(self) -> np.float32:
        self.state = (self.state + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
        return np.float32((self.mix(self.state) >> 40) * 2.0 ** -24)


def _draw(rng) -> np.float32:
    """One uniform float32 in [0, 1): rng is a callable (SplitMixDraws) or a
    numpy Generator (24 random bits, as rand's gen::<f32>())."""
    if callable(rng):
        return np.float32(rng())
    return np.float32(int(rng.integers(0, 1 << 24)) * 2.0 ** -24)


def argmax_first(logits: np.ndarray) -> int:
    """Greedy argmax with the reference's strict '>' (llm/forward.rs:262-271)."""
    v = np.where(np.isnan(logits), -np.inf, np.asarray(logits, dtype=np.float32))
    if v.size == 0:
        return 0
    i = int(np.argmax(v))  # first occurrence of the maximum
    return 0 if v[i] == -np.inf else i


def get_linear(ff: FlatFile, name: str) -> GenomicLinear:
    """GajeFlatFileReader::get_linear (flat_reader.rs:92-122)."""
    if name not in ff.tensors:
        raise FileNotFoundError(f"Flat tensor entry '{name}' not found")
    e = ff.tensors[name]
    dna = ff.get_slice(e["dna_off"], e["dna_len"])
    cent = ff.get_f32_slice(e["c_off"], e["c_len"])
    anc = ff.get_slice(e["anc_off"], e["anc_len"])
    bias = ff.get_f32_slice(e["bias_off"], e["bias_len"])
    return GenomicLinear(np.asarray(dna), bytes(anc), cent, e["out_features"],
                         e["in_features"], bias, e["bit_depth"])


def load_genomic(path: str) -> GenomicLLM:
    """GajeFlatFileReader::open + load_genomic (flat_reader.rs:33-69,124-236)."""
    ff = FlatFile(path)
    cfg: ModelConfig = ff.model_config()
    head_dim = cfg.n_embd // cfg.n_head
    embd = get_linear(ff, "token_embd")
    on = ff.tensors["output_norm"]
    output_norm = ff.get_f32_slice(on["dna_off"], on["dna_len"])
    lm_head = get_linear(ff, "lm_head")
    blocks = []
    for i in range(cfg.n_blocks):
        p = f"blk.{i}."
        an = ff.tensors[p + "attn_norm"]
        fn = ff.tensors[p + "ffn_norm"]
        attn_norm = ff.get_f32_slice(an["dna_off"], an["dna_len"])
        ffn_norm = ff.get_f32_slice(fn["dna_off"], fn["dna_len"])
        fused_qkv = qkv_split = fused_gu = gu_split = None
        if p + "attn_qkv" in ff.tensors:
            fused_qkv = get_linear(ff, p + "attn_qkv")
        else:
            qkv_split = [get_linear(ff, p + n) for n in ("attn_q", "attn_k", "attn_v")]
        w_o = get_linear(ff, p + "attn_output")
        if p + "ffn_gate_up" in ff.tensors:
            fused_gu = get_linear(ff, p + "ffn_gate_up")
        else:
            gu_split = [get_linear(ff, p + n) for n in ("ffn_gate", "ffn_up")]
        w_down = get_linear(ff, p + "ffn_down")
        attn = GenomicAttention(cfg.n_head, cfg.n_head_kv, head_dim, attn_norm, cfg.eps,
                                cfg.config["rope_base"], cfg.config["rope_style"])
        blocks.append(RustGenomicBlock(i, attn, w_o, w_down, ffn_norm, cfg.eps,
                                       bool(cfg.config["use_genomic_norm"]), fused_qkv, fused_gu,
                                       qkv_split, gu_split))
    llm = GenomicLLM(embd, blocks, output_norm, lm_head, cfg.eps)
    llm.flat = ff
    llm.config = cfg
    return llm
