"""ctypes binding of lib/libgaje_hip.so (the C ABI declared in include/gaje_hip.h).

There is no CPU fallback: if the shared library is missing the import of any
entry point raises, so a caller never silently runs something else.
"""
from __future__ import annotations

import ctypes
import os

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_PKG_DIR), "lib", "libgaje_hip.so")

GAJE_OK = 0
ERR_INVALID_ARG = -1
ERR_IO = -2
ERR_TOO_SHORT = -3
ERR_INVALID_MAGIC = -4
ERR_INVALID_DATA = -5
ERR_NOT_FOUND = -6
ERR_NAN = -7
ERR_MODEL = -8
ERR_UNSUPPORTED = -9
ERR_HIP = -10
ERR_NO_DEVICE = -11

c_i64 = ctypes.c_int64
c_vp = ctypes.c_void_p


class GajeError(Exception):
    """A non-zero status from the C ABI, with gaje_hip_last_error()'s text."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class GajeValueError(GajeError, ValueError):
    """Err(String) of the reference forward path (PyValueError upstream)."""


class GajeIOError(GajeError, OSError):
    """std::io::Error / HeaderError of the reference reader."""


class FlatWriterHeader(ctypes.Structure):
    _fields_ = [("flags", ctypes.c_uint32), ("group_size", ctypes.c_uint32), ("quant_format", ctypes.c_uint32),
                ("arch_family", ctypes.c_uint32), ("n_embd", ctypes.c_uint32), ("n_head", ctypes.c_uint32),
                ("n_head_kv", ctypes.c_uint32), ("n_blocks", ctypes.c_uint32), ("qk_permute", ctypes.c_uint32)]


class ModelInfo(ctypes.Structure):
    _fields_ = [("n_embd", c_i64), ("n_head", c_i64), ("n_head_kv", c_i64), ("n_blocks", c_i64),
                ("head_dim", c_i64), ("ffn", c_i64), ("vocab_size", c_i64), ("eps", ctypes.c_float),
                ("rope_base", ctypes.c_float), ("rope_split", ctypes.c_int32),
                ("arch_family", ctypes.c_int32), ("body_format", ctypes.c_int32),
                ("use_genomic_norm", ctypes.c_int32), ("max_ctx", c_i64), ("weight_bytes", c_i64),
                ("n_logits", c_i64)]


class FlatHeader(ctypes.Structure):
    _fields_ = [("version", ctypes.c_uint32), ("flags", ctypes.c_uint32), ("num_tensors", ctypes.c_uint32),
                ("group_size", ctypes.c_uint32), ("quant_format", ctypes.c_uint32),
                ("arch_family", ctypes.c_uint32), ("arch_n_embd", ctypes.c_uint32),
                ("arch_n_head", ctypes.c_uint32), ("arch_n_head_kv", ctypes.c_uint32),
                ("arch_n_blocks", ctypes.c_uint32), ("arch_qk_permute", ctypes.c_uint32),
                ("quant_type", ctypes.c_int32), ("effective_group_size", ctypes.c_uint32),
                ("pad_", ctypes.c_uint32), ("meta_len", ctypes.c_uint64), ("dir_len", ctypes.c_uint64),
                ("weights_offset", ctypes.c_uint64), ("weights_len", ctypes.c_uint64)]


class FlatInfo(ctypes.Structure):
    _fields_ = [("header", FlatHeader), ("n_embd", c_i64), ("n_head", c_i64), ("n_head_kv", c_i64),
                ("n_blocks", c_i64), ("vocab_size", c_i64), ("eps", ctypes.c_float),
                ("rope_base", ctypes.c_float), ("rope_split", ctypes.c_int32),
                ("use_genomic_norm", ctypes.c_int32), ("has_descriptor", ctypes.c_int32),
                ("n_tensors", ctypes.c_int32)]


class FlatTensor(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in ("bit_depth", "out_features", "in_features", "dna_off",
                                               "dna_len", "c_off", "c_len", "anc_off", "anc_len",
                                               "bias_off", "bias_len")]


class SynthConfig(ctypes.Structure):
    _fields_ = [("n_embd", c_i64), ("n_head", c_i64), ("n_head_kv", c_i64), ("n_blocks", c_i64),
                ("ffn", c_i64), ("vocab_size", c_i64), ("eps", ctypes.c_float),
                ("rope_base", ctypes.c_float), ("arch_family", ctypes.c_int32),
                ("qkv_bias", ctypes.c_int32), ("tied_embeddings", ctypes.c_int32),
                ("body_format", ctypes.c_int32), ("fused", ctypes.c_int32),
                ("rope_interleaved", ctypes.c_int32), ("use_genomic_norm", ctypes.c_int32),
                ("quant_embed", ctypes.c_int32), ("g2_tables", ctypes.c_int32),
                ("anchors", ctypes.c_int32), ("seed", ctypes.c_uint64)]


# (name, restype, argtypes): every symbol include/gaje_hip.h declares.
SIGNATURES = [
    ("gaje_hip_last_error", ctypes.c_char_p, []),
    ("gaje_hip_device_count", ctypes.c_int, [ctypes.POINTER(ctypes.c_int)]),
    ("gaje_hip_set_device", ctypes.c_int, [ctypes.c_int]),
    ("gaje_hip_device_name", ctypes.c_int, [ctypes.c_int, ctypes.c_char_p, ctypes.c_size_t]),
    ("gaje_hip_malloc", ctypes.c_int, [ctypes.POINTER(c_vp), ctypes.c_size_t]),
    ("gaje_hip_free", ctypes.c_int, [c_vp]),
    ("gaje_hip_memcpy_h2d", ctypes.c_int, [c_vp, c_vp, ctypes.c_size_t]),
    ("gaje_hip_memcpy_d2h", ctypes.c_int, [c_vp, c_vp, ctypes.c_size_t]),
    ("gaje_hip_memcpy_d2d", ctypes.c_int, [c_vp, c_vp, ctypes.c_size_t]),
    ("gaje_hip_memset", ctypes.c_int, [c_vp, ctypes.c_int, ctypes.c_size_t]),
    ("gaje_hip_device_synchronize", ctypes.c_int, []),
    ("gaje_hip_stream_create", ctypes.c_int, [ctypes.POINTER(c_vp)]),
    ("gaje_hip_stream_destroy", ctypes.c_int, [c_vp]),
    ("gaje_hip_stream_synchronize", ctypes.c_int, [c_vp]),
    ("gaje_hip_event_create", ctypes.c_int, [ctypes.POINTER(c_vp)]),
    ("gaje_hip_event_destroy", ctypes.c_int, [c_vp]),
    ("gaje_hip_event_record", ctypes.c_int, [c_vp, c_vp]),
    ("gaje_hip_event_synchronize", ctypes.c_int, [c_vp]),
    ("gaje_hip_event_elapsed_ms", ctypes.c_int, [c_vp, c_vp, ctypes.POINTER(ctypes.c_float)]),
    ("gaje_hip_q4_0_packed_bytes", c_i64, [c_i64, c_i64]),
    ("gaje_hip_q4_0_pack", ctypes.c_int, [c_vp, c_vp, c_i64, c_i64, c_vp]),
    ("gaje_hip_q4_0_gemv", ctypes.c_int, [c_vp, c_vp, c_vp, c_i64, c_vp, c_i64, c_i64, c_vp]),
    ("gaje_hip_q4_0_gemv_blocks", ctypes.c_int, [c_vp, c_vp, c_vp, c_i64, c_vp, c_i64, c_i64, c_vp]),
    ("gaje_hip_q4_0_gemv_tol", ctypes.c_int, [c_vp, c_vp, c_vp, c_i64, c_vp, c_i64, c_i64, c_vp]),
    ("gaje_hip_q4_0_gemm", ctypes.c_int, [c_vp, c_vp, c_vp, c_i64, c_vp, c_i64, c_i64, c_i64, c_vp]),
    ("gaje_hip_q4_0_gemm_mfma_workspace", c_i64, [c_i64, c_i64, c_i64]),
    ("gaje_hip_q4_0_gemm_mfma", ctypes.c_int, [c_vp, c_vp, c_vp, c_i64, c_vp, c_i64, c_i64, c_i64, c_vp,
                                               c_i64, c_vp]),
    ("gaje_hip_q4_0_gemm_mfma_noalloc", ctypes.c_int, [c_vp, c_vp, c_vp, c_i64, c_vp, c_i64, c_i64, c_i64, c_vp]),
    ("gaje_hip_moe_ffn_workspace", c_i64, [c_i64, c_i64, c_i64, c_i64]),
    ("gaje_hip_moe_ffn", ctypes.c_int, [c_vp, c_i64, c_i64, c_vp, c_i64, c_vp, c_vp, c_i64, c_vp, c_vp, c_vp,
                                        c_vp, c_i64, c_vp]),
    ("gaje_hip_moe_prepared_bytes", c_i64, [c_i64, c_i64, c_i64]),
    ("gaje_hip_moe_prepare", ctypes.c_int, [c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp]),
    ("gaje_hip_moe_ffn_prepared_workspace", c_i64, [c_i64, c_i64, c_i64, c_i64]),
    ("gaje_hip_moe_ffn_prepared", ctypes.c_int, [c_vp, c_i64, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_vp, c_vp,
                                                 c_vp, c_i64, c_vp]),
    ("gaje_hip_q8_0_packed_bytes", c_i64, [c_i64, c_i64]),
    ("gaje_hip_q8_0_pack", ctypes.c_int, [c_vp, c_vp, c_i64, c_i64, c_vp]),
    ("gaje_hip_q8_0_gemv", ctypes.c_int, [c_vp, c_vp, c_vp, c_i64, c_vp, c_i64, c_i64, c_vp]),
    ("gaje_hip_q8_0_dequant", ctypes.c_int, [c_vp, c_vp, c_i64, c_vp]),
    ("gaje_hip_lut4_gemv", ctypes.c_int, [c_vp, c_vp, c_i64, c_vp, c_vp, c_i64, c_vp, c_i64, c_i64, c_vp]),
    ("gaje_hip_2bit_gemv", ctypes.c_int, [c_vp, c_vp, c_i64, c_vp, c_vp, c_vp, c_i64, c_vp, c_i64, c_i64, c_vp]),
    ("gaje_hip_f32_gemv", ctypes.c_int, [c_vp, c_vp, c_vp, c_i64, c_vp, c_i64, c_i64, c_vp]),
    ("gaje_hip_q4_0_dequant", ctypes.c_int, [c_vp, c_vp, c_i64, c_vp]),
    ("gaje_hip_rmsnorm", ctypes.c_int, [c_vp, c_vp, ctypes.c_float, c_vp, c_i64, c_vp]),
    ("gaje_hip_swiglu", ctypes.c_int, [c_vp, c_vp, c_vp, c_i64, c_vp]),
    ("gaje_hip_expf", ctypes.c_int, [c_vp, c_vp, c_i64, c_vp]),
    ("gaje_hip_attention", ctypes.c_int, [c_vp, c_vp, c_vp, c_i64, c_i64, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int, c_vp, c_vp]),
    ("gaje_hip_kwta", ctypes.c_int, [c_vp, c_i64, c_i64, c_vp]),
    ("gaje_hip_argmax", ctypes.c_int, [c_vp, c_i64, c_vp, c_vp]),
    ("gaje_hip_open", ctypes.c_int, [ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(c_vp)]),
    ("gaje_hip_close", None, [c_vp]),
    ("gaje_hip_model_info_get", ctypes.c_int, [c_vp, ctypes.POINTER(ModelInfo)]),
    ("gaje_hip_forward", ctypes.c_int, [c_vp, ctypes.c_uint32, ctypes.c_int, c_vp]),
    ("gaje_hip_forward_hidden", ctypes.c_int, [c_vp, ctypes.c_uint32, ctypes.c_int, c_vp, c_vp]),
    ("gaje_hip_clear_cache", ctypes.c_int, [c_vp]),
    ("gaje_hip_cache_len", ctypes.c_int, [c_vp, ctypes.POINTER(c_i64)]),
    ("gaje_hip_set_kwta", ctypes.c_int, [c_vp, ctypes.c_float]),
    ("gaje_hip_get_kwta", ctypes.c_int, [c_vp, ctypes.POINTER(ctypes.c_float)]),
    ("gaje_hip_reserve", ctypes.c_int, [c_vp, c_i64]),
    ("gaje_hip_prefill", ctypes.c_int, [c_vp, c_vp, c_i64, c_vp]),
    ("gaje_hip_prefill_mfma", ctypes.c_int, [c_vp, c_vp, c_i64, c_vp]),
    ("gaje_hip_batch_open", ctypes.c_int, [c_vp, c_i64, c_i64, ctypes.POINTER(c_vp)]),
    ("gaje_hip_batch_close", None, [c_vp]),
    ("gaje_hip_batch_reset", ctypes.c_int, [c_vp, c_i64]),
    ("gaje_hip_batch_cache_len", ctypes.c_int, [c_vp, c_i64, ctypes.POINTER(c_i64)]),
    ("gaje_hip_batch_feed", ctypes.c_int, [c_vp, c_vp, c_i64, c_vp, c_vp]),
    ("gaje_hip_batch_decode_greedy", ctypes.c_int, [c_vp, c_vp, c_i64, c_vp, c_vp]),
    ("gaje_hip_greedy_next", ctypes.c_int, [c_vp, ctypes.c_uint32, ctypes.POINTER(ctypes.c_uint32)]),
    ("gaje_hip_decode_greedy", ctypes.c_int, [c_vp, ctypes.c_uint32, c_i64, c_vp]),
    ("gaje_hip_generate", ctypes.c_int, [c_vp, c_vp, c_i64, c_i64, ctypes.c_float, ctypes.c_float,
                                         c_vp, c_i64, ctypes.c_uint64, c_vp, ctypes.POINTER(c_i64)]),
    ("gaje_hip_last_timing", ctypes.c_int, [c_vp, ctypes.POINTER(ctypes.c_float),
                                            ctypes.POINTER(ctypes.c_float)]),
    ("gaje_hip_truncate_cache", ctypes.c_int, [c_vp, c_i64]),
    ("gaje_hip_time_stage", ctypes.c_int, [c_vp, ctypes.c_int, c_i64, ctypes.c_int,
                                           ctypes.POINTER(ctypes.c_float), ctypes.POINTER(c_i64)]),
    ("gaje_hip_bench_gemv", ctypes.c_int, [ctypes.c_int, c_vp, ctypes.c_size_t, c_vp, ctypes.c_size_t,
                                           ctypes.c_int, c_vp, c_vp, c_i64, c_i64, ctypes.c_int,
                                           ctypes.POINTER(ctypes.c_float)]),
    ("gaje_hip_bench_floor", ctypes.c_int, [c_vp, c_i64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                            ctypes.POINTER(ctypes.c_float)]),
    ("gaje_flat_header_from_bytes", ctypes.c_int, [c_vp, ctypes.c_size_t, ctypes.POINTER(FlatHeader)]),
    ("gaje_flat_inspect", ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(FlatInfo)]),
    ("gaje_flat_tensor_entry", ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(FlatTensor)]),
    ("gaje_flat_writer_create", ctypes.c_int, [ctypes.POINTER(c_vp)]),
    ("gaje_flat_writer_free", None, [c_vp]),
    ("gaje_flat_writer_add_norm", ctypes.c_int, [c_vp, ctypes.c_char_p, c_vp, c_i64]),
    ("gaje_flat_writer_add_f32", ctypes.c_int, [c_vp, ctypes.c_char_p, c_vp, c_i64, c_i64, c_vp, c_i64]),
    ("gaje_flat_writer_add_q4_0", ctypes.c_int, [c_vp, ctypes.c_char_p, c_vp, c_i64, c_i64, c_vp, c_i64]),
    ("gaje_flat_writer_add_q8_0", ctypes.c_int, [c_vp, ctypes.c_char_p, c_vp, c_i64, c_i64, c_vp, c_i64]),
    ("gaje_flat_writer_add_lut4", ctypes.c_int, [c_vp, ctypes.c_char_p, c_vp, c_i64, c_i64, ctypes.c_float, c_vp,
                                                 c_i64]),
    ("gaje_flat_writer_write", ctypes.c_int, [c_vp, ctypes.c_char_p, ctypes.c_char_p,
                                              ctypes.POINTER(FlatWriterHeader)]),
    ("gaje_quantize_q4_0", ctypes.c_int, [c_vp, c_i64, c_vp]),
    ("gaje_quantize_q8_0", ctypes.c_int, [c_vp, c_i64, c_vp]),
    ("gaje_genomize_4bit", ctypes.c_int, [c_vp, c_i64, c_i64, ctypes.c_float, c_vp, c_vp, c_vp,
                                          ctypes.POINTER(c_i64)]),
    ("gaje_synth_write_flat", ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(SynthConfig)]),
    ("gaje_synth_q4_0", ctypes.c_int, [ctypes.c_uint64, ctypes.c_char_p, c_i64, c_i64, c_vp]),
    ("gaje_synth_lut4", ctypes.c_int, [ctypes.c_uint64, ctypes.c_char_p, c_i64, c_i64, c_vp, c_vp]),
    ("gaje_synth_2bit", ctypes.c_int, [ctypes.c_uint64, ctypes.c_char_p, c_i64, c_i64, c_vp, c_vp]),
    ("gaje_synth_normal", ctypes.c_int, [ctypes.c_uint64, ctypes.c_char_p, c_i64, ctypes.c_float,
                                         ctypes.c_float, c_vp]),
]

_LIB = None


def lib() -> ctypes.CDLL:
    """The loaded HIP library (raises if it has not been built)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"HIP library missing: {LIB_PATH}; build it with "
                               f"`make -C gaje-semantic-compression_amd` (or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def last_error() -> str:
    msg = lib().gaje_hip_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(rc: int) -> None:
    """Raise the Python exception matching a C-ABI status."""
    if rc == GAJE_OK:
        return
    msg = last_error()
    if rc in (ERR_NAN, ERR_MODEL):
        raise GajeValueError(rc, msg)
    if rc == ERR_NOT_FOUND:
        e = GajeIOError(rc, msg)
        e.errno = 2
        raise e
    if rc in (ERR_IO, ERR_TOO_SHORT, ERR_INVALID_MAGIC, ERR_INVALID_DATA):
        raise GajeIOError(rc, msg)
    raise GajeError(rc, msg)
