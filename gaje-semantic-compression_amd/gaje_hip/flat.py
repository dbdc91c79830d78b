"""The .gaje.flat reader of the C ABI (host-only; no GPU needed).

Mirrors the reference reader's inspection surface: FlatHeaderV2::from_bytes
with quantization_type / effective_group_size (src/io/header/flat.rs:46-79),
GajeFlatFileReader::open and load_genomic's config resolution
(src/io/flat_reader.rs:33-69,124-139), and the FlatTensorEntry directory
(flat_reader.rs:9-22).
"""
from __future__ import annotations

import ctypes
import os

from ._lib import FlatHeader, FlatInfo, FlatTensor, check, lib

QUANT_TYPES = {0: "LegacyCentroids", 1: "Q4_0", 2: "Q8_0", 3: "Unknown"}


def _as_dict(st) -> dict:
    out = {}
    for name, _ in st._fields_:
        if name == "pad_":
            continue
        v = getattr(st, name)
        out[name] = _as_dict(v) if isinstance(v, ctypes.Structure) else v
    return out


def header_from_bytes(b: bytes) -> dict:
    """The header fields; raises GajeIOError (TooShort / InvalidMagic) as the reference does."""
    h = FlatHeader()
    buf = ctypes.create_string_buffer(bytes(b), len(b)) if len(b) else None
    check(lib().gaje_flat_header_from_bytes(buf, len(b), ctypes.byref(h)))
    d = _as_dict(h)
    d["quantization_type"] = QUANT_TYPES.get(h.quant_type, "Unknown")
    return d


def inspect(path: str) -> dict:
    """Header and resolved model config of a .gaje.flat file."""
    info = FlatInfo()
    check(lib().gaje_flat_inspect(os.fsencode(path), ctypes.byref(info)))
    d = _as_dict(info)
    d["header"]["quantization_type"] = QUANT_TYPES.get(info.header.quant_type, "Unknown")
    return d


def tensor_entry(path: str, name: str) -> dict:
    e = FlatTensor()
    check(lib().gaje_flat_tensor_entry(os.fsencode(path), name.encode(), ctypes.byref(e)))
    return _as_dict(e)
