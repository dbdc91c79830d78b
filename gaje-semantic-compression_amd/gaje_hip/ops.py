"""Operator-level API over device buffers (mirrors the reference kernel entry
points of src/compute/kernels/mod.rs:19-28 one level up: whole matvecs instead
of single rows)."""
from __future__ import annotations

import ctypes

import numpy as np

from ._lib import check, lib


class DeviceBuffer:
    """A device allocation made through the C ABI (freed on close / GC)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(lib().gaje_hip_malloc(ctypes.byref(p), self.nbytes))
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.write(a)
        return b

    def write(self, a: np.ndarray, offset: int = 0) -> None:
        """Copy a host array into the buffer at byte `offset`."""
        a = np.ascontiguousarray(a)
        if offset < 0 or offset + a.nbytes > self.nbytes:
            raise ValueError("array beyond the device buffer")
        check(lib().gaje_hip_memcpy_h2d(self.ptr + offset, a.ctypes.data, a.nbytes))

    def read(self, dtype, count: int | None = None) -> np.ndarray:
        dtype = np.dtype(dtype)
        n = self.nbytes // dtype.itemsize if count is None else int(count)
        out = np.empty(n, dtype=dtype)
        check(lib().gaje_hip_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes))
        return out

    def close(self):
        if getattr(self, "ptr", None):
            lib().gaje_hip_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _p(b):
    return None if b is None else b.ptr


def memcpy_d2d(dst: DeviceBuffer, src: DeviceBuffer, nbytes: int) -> None:
    if nbytes > min(dst.nbytes, src.nbytes):
        raise ValueError("copy larger than a buffer")
    check(lib().gaje_hip_memcpy_d2d(dst.ptr, src.ptr, int(nbytes)))


def synchronize() -> None:
    check(lib().gaje_hip_device_synchronize())


def device_count() -> int:
    n = ctypes.c_int()
    check(lib().gaje_hip_device_count(ctypes.byref(n)))
    return n.value


def device_name(device: int = 0) -> str:
    buf = ctypes.create_string_buffer(256)
    check(lib().gaje_hip_device_name(device, buf, 256))
    return buf.value.decode()


def q4_0_packed_bytes(n: int, k: int) -> int:
    v = lib().gaje_hip_q4_0_packed_bytes(int(n), int(k))
    if v < 0:
        raise ValueError(f"Q4_0 needs k to be a positive multiple of 32 (got {k})")
    return v


def q4_0_pack(blocks: DeviceBuffer, packed: DeviceBuffer, n: int, k: int, stream=None) -> None:
    """Q4_0Block rows (file layout) -> the matvec's packed layout, on the device."""
    check(lib().gaje_hip_q4_0_pack(blocks.ptr, packed.ptr, n, k, stream))


def q4_0_upload(blocks: np.ndarray, n: int, k: int) -> DeviceBuffer:
    """Uploads n rows of Q4_0Blocks and returns them packed for q4_0_gemv."""
    raw = DeviceBuffer.from_array(np.ascontiguousarray(blocks, dtype=np.uint8))
    packed = DeviceBuffer(max(q4_0_packed_bytes(n, k), 1))
    q4_0_pack(raw, packed, n, k)
    synchronize()
    raw.close()
    return packed


def q4_0_gemv(packed: DeviceBuffer, x: DeviceBuffer, y: DeviceBuffer, n: int, k: int,
              bias: DeviceBuffer | None = None, bias_len: int = 0, stream=None) -> None:
    check(lib().gaje_hip_q4_0_gemv(packed.ptr, x.ptr, _p(bias), bias_len, y.ptr, n, k, stream))


def q4_0_gemv_tol(packed: DeviceBuffer, x: DeviceBuffer, y: DeviceBuffer, n: int, k: int,
                  bias: DeviceBuffer | None = None, bias_len: int = 0, stream=None) -> None:
    """q4_0_gemv in tolerance mode: within 1e-4 of each row's sum of |w x|
    (regrouped by block on the long streams), not bit for bit."""
    check(lib().gaje_hip_q4_0_gemv_tol(packed.ptr, x.ptr, _p(bias), bias_len, y.ptr, n, k, stream))


def q4_0_gemv_blocks(blocks: DeviceBuffer, x: DeviceBuffer, y: DeviceBuffer, n: int, k: int,
                     bias: DeviceBuffer | None = None, bias_len: int = 0, stream=None) -> None:
    """The Q4_0 matvec on the file's own Q4_0Block rows (no packing)."""
    check(lib().gaje_hip_q4_0_gemv_blocks(blocks.ptr, x.ptr, _p(bias), bias_len, y.ptr, n, k, stream))


def q4_0_gemm(packed: DeviceBuffer, X: DeviceBuffer, Y: DeviceBuffer, m: int, n: int, k: int,
              bias: DeviceBuffer | None = None, bias_len: int = 0, stream=None) -> None:
    check(lib().gaje_hip_q4_0_gemm(packed.ptr, X.ptr, _p(bias), bias_len, Y.ptr, m, n, k, stream))


def q4_0_gemm_mfma_workspace(m: int, n: int, k: int) -> int:
    return int(lib().gaje_hip_q4_0_gemm_mfma_workspace(m, n, k))


def q4_0_gemm_mfma(packed: DeviceBuffer, X: DeviceBuffer, Y: DeviceBuffer, m: int, n: int, k: int,
                   workspace: DeviceBuffer, bias: DeviceBuffer | None = None, bias_len: int = 0,
                   stream=None) -> None:
    """Y = X W^T (+ bias) on the MFMA units: the reference dot product to fp32
    accuracy (f16 hi/lo operand pairs), not bit-exact; see gaje_hip.h."""
    check(lib().gaje_hip_q4_0_gemm_mfma(packed.ptr, X.ptr, _p(bias), bias_len, Y.ptr, m, n, k,
                                        workspace.ptr, workspace.nbytes, stream))


def moe_ffn_workspace(T: int, h: int, ffn: int, n_expert: int) -> int:
    return int(lib().gaje_hip_moe_ffn_workspace(T, h, ffn, n_expert))


def moe_ffn(x: DeviceBuffer, T: int, h: int, router: DeviceBuffer, gate_up, down, ffn: int,
            y: DeviceBuffer, workspace: DeviceBuffer, top_idx: DeviceBuffer | None = None,
            top_w: DeviceBuffer | None = None, stream=None) -> None:
    """Top-2 MoE SwiGLU FFN over packed Q4_0 experts (gaje_hip_moe_ffn)."""
    E = len(gate_up)
    gu = (ctypes.c_void_p * E)(*[b.ptr for b in gate_up])
    dn = (ctypes.c_void_p * E)(*[b.ptr for b in down])
    check(lib().gaje_hip_moe_ffn(x.ptr, T, h, router.ptr, E, gu, dn, ffn, y.ptr, _p(top_idx), _p(top_w),
                                 workspace.ptr, workspace.nbytes, stream))


def moe_prepared_bytes(h: int, ffn: int, n_expert: int) -> int:
    return int(lib().gaje_hip_moe_prepared_bytes(h, ffn, n_expert))


def moe_prepare(gate_up, down, h: int, ffn: int, prepared: DeviceBuffer, stream=None) -> None:
    """The block-scaled weight operands of every expert (gaje_hip_moe_prepare)."""
    E = len(gate_up)
    gu = (ctypes.c_void_p * E)(*[b.ptr for b in gate_up])
    dn = (ctypes.c_void_p * E)(*[b.ptr for b in down])
    check(lib().gaje_hip_moe_prepare(gu, dn, h, ffn, E, prepared.ptr, prepared.nbytes, stream))


def moe_ffn_prepared_workspace(T: int, h: int, ffn: int, n_expert: int) -> int:
    return int(lib().gaje_hip_moe_ffn_prepared_workspace(T, h, ffn, n_expert))


def moe_ffn_prepared(x: DeviceBuffer, T: int, h: int, router: DeviceBuffer, n_expert: int, prepared: DeviceBuffer,
                     ffn: int, y: DeviceBuffer, workspace: DeviceBuffer, top_idx: DeviceBuffer | None = None,
                     top_w: DeviceBuffer | None = None, stream=None) -> None:
    """Top-2 MoE SwiGLU FFN over prepared experts (gaje_hip_moe_ffn_prepared)."""
    check(lib().gaje_hip_moe_ffn_prepared(x.ptr, T, h, router.ptr, n_expert, prepared.ptr, ffn, y.ptr,
                                          _p(top_idx), _p(top_w), workspace.ptr, workspace.nbytes, stream))


def q8_0_packed_bytes(n: int, k: int) -> int:
    return int(lib().gaje_hip_q8_0_packed_bytes(n, k))


def q8_0_upload(blocks: np.ndarray, n: int, k: int) -> DeviceBuffer:
    """Q8_0Block rows (34 bytes per block) -> packed device rows."""
    raw = DeviceBuffer.from_array(np.ascontiguousarray(blocks, np.uint8))
    packed = DeviceBuffer(max(q8_0_packed_bytes(n, k), 1))
    check(lib().gaje_hip_q8_0_pack(raw.ptr, packed.ptr, n, k, None))
    synchronize()
    raw.close()
    return packed


def q8_0_gemv(packed: DeviceBuffer, x: DeviceBuffer, y: DeviceBuffer, n: int, k: int,
              bias: DeviceBuffer | None = None, bias_len: int = 0, stream=None) -> None:
    check(lib().gaje_hip_q8_0_gemv(packed.ptr, x.ptr, _p(bias), bias_len, y.ptr, n, k, stream))


def q8_0_dequant(blocks: DeviceBuffer, out: DeviceBuffer, nblocks: int, stream=None) -> None:
    check(lib().gaje_hip_q8_0_dequant(blocks.ptr, out.ptr, nblocks, stream))


def lut4_gemv(codes: DeviceBuffer, lut: DeviceBuffer, lut_len: int, x: DeviceBuffer,
              y: DeviceBuffer, n: int, k: int, bias: DeviceBuffer | None = None,
              bias_len: int = 0, stream=None) -> None:
    check(lib().gaje_hip_lut4_gemv(codes.ptr, lut.ptr, lut_len, x.ptr, _p(bias), bias_len, y.ptr,
                                   n, k, stream))


def bit2_gemv(codes: DeviceBuffer, centroids: DeviceBuffer | None, c_len: int, x: DeviceBuffer,
              y: DeviceBuffer, n: int, k: int, modulation=None, bias: DeviceBuffer | None = None,
              bias_len: int = 0, stream=None) -> None:
    """GenomicLinear::forward_core on Genomic2Bit rows (gaje_hip_2bit_gemv)."""
    mod = None
    if modulation is not None:
        mod = np.ascontiguousarray(modulation, dtype=np.float32).reshape(4)
    check(lib().gaje_hip_2bit_gemv(codes.ptr, _p(centroids), c_len, mod.ctypes.data if mod is not None else None,
                                   x.ptr, _p(bias), bias_len, y.ptr, n, k, stream))


def f32_gemv(w: DeviceBuffer, x: DeviceBuffer, y: DeviceBuffer, n: int, k: int,
             bias: DeviceBuffer | None = None, bias_len: int = 0, stream=None) -> None:
    check(lib().gaje_hip_f32_gemv(w.ptr, x.ptr, _p(bias), bias_len, y.ptr, n, k, stream))


def q4_0_dequant(blocks: DeviceBuffer, out: DeviceBuffer, nblocks: int, stream=None) -> None:
    check(lib().gaje_hip_q4_0_dequant(blocks.ptr, out.ptr, nblocks, stream))


def rmsnorm(x: DeviceBuffer, w: DeviceBuffer, eps: float, y: DeviceBuffer, n: int, stream=None):
    check(lib().gaje_hip_rmsnorm(x.ptr, w.ptr, float(eps), y.ptr, n, stream))


def swiglu(gate: DeviceBuffer, up: DeviceBuffer, out: DeviceBuffer, n: int, stream=None):
    check(lib().gaje_hip_swiglu(gate.ptr, up.ptr, out.ptr, n, stream))


def expf(x: DeviceBuffer, y: DeviceBuffer, n: int, stream=None):
    check(lib().gaje_hip_expf(x.ptr, y.ptr, n, stream))


def attention(q: DeviceBuffer, k_cache: DeviceBuffer, v_cache: DeviceBuffer, seq_len: int,
              capacity: int, n_head: int, n_head_kv: int, head_dim: int, out: DeviceBuffer,
              stream=None):
    """k_cache and v_cache are both [n_head_kv][head_dim][capacity]."""
    check(lib().gaje_hip_attention(q.ptr, k_cache.ptr, v_cache.ptr, seq_len, capacity, n_head,
                                   n_head_kv, head_dim, out.ptr, stream))


def kwta(scores: DeviceBuffer, n: int, k: int, stream=None):
    check(lib().gaje_hip_kwta(scores.ptr, n, k, stream))


def kwta_at(scores: DeviceBuffer, first: int, n: int, k: int, stream=None):
    """kwta over the n floats that start at float `first` of the buffer."""
    if first < 0 or (first + n) * 4 > scores.nbytes:
        raise ValueError("kwta range beyond the buffer")
    check(lib().gaje_hip_kwta(scores.ptr + 4 * first, n, k, stream))


def argmax(x: DeviceBuffer, n: int, idx: DeviceBuffer, stream=None):
    check(lib().gaje_hip_argmax(x.ptr, n, idx.ptr, stream))


def bench_gemv(fmt: int, w: DeviceBuffer, copy_stride: int, copies: int, x: DeviceBuffer,
               y: DeviceBuffer, n: int, k: int, iters: int, lut: DeviceBuffer | None = None,
               lut_stride: int = 0) -> float:
    """Average ms per launch of the matvec over `copies` weight copies (graph replays)."""
    ms = ctypes.c_float()
    check(lib().gaje_hip_bench_gemv(int(fmt), w.ptr, int(copy_stride), _p(lut), int(lut_stride),
                                    int(copies), x.ptr, y.ptr, int(n), int(k), int(iters),
                                    ctypes.byref(ms)))
    return ms.value


def bench_floor(buf: DeviceBuffer | None, nbytes: int, grid: int, block: int, iters: int) -> float:
    """Average ms per launch of an empty kernel (nbytes == 0) or of a plain read of
    nbytes of buf, with the given grid (graph replays, as bench_gemv)."""
    ms = ctypes.c_float()
    check(lib().gaje_hip_bench_floor(_p(buf), int(nbytes), int(grid), int(block), int(iters),
                                     ctypes.byref(ms)))
    return ms.value


class Stream:
    def __init__(self):
        s = ctypes.c_void_p()
        check(lib().gaje_hip_stream_create(ctypes.byref(s)))
        self.handle = s.value

    def synchronize(self):
        check(lib().gaje_hip_stream_synchronize(self.handle))

    def close(self):
        if self.handle:
            lib().gaje_hip_stream_destroy(self.handle)
            self.handle = None


class Event:
    def __init__(self):
        e = ctypes.c_void_p()
        check(lib().gaje_hip_event_create(ctypes.byref(e)))
        self.handle = e.value

    def record(self, stream=None):
        check(lib().gaje_hip_event_record(self.handle, stream))

    def synchronize(self):
        check(lib().gaje_hip_event_synchronize(self.handle))

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(lib().gaje_hip_event_elapsed_ms(self.handle, end.handle, ctypes.byref(ms)))
        return ms.value

    def close(self):
        if self.handle:
            lib().gaje_hip_event_destroy(self.handle)
            self.handle = None
