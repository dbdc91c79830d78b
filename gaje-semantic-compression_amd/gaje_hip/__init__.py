"""MI355X (gfx950) implementation of the GAJE quantised decode path.

The compute runs in lib/libgaje_hip.so (hand-written HIP kernels behind the C
ABI of include/gaje_hip.h); this package is its Python binding, shaped like the
reference's PyO3 surface (`load_genomic_auto`, `RustGenomicLLM.forward`, ...).
"""
from ._lib import (GajeError, GajeIOError, GajeValueError, LIB_PATH, SIGNATURES, last_error,
                   lib)
from .model import BATCH_INACTIVE, GenomicBatch, GenomicLLM, load_genomic_auto
from . import flat, gguf, ops, synth, writer

RustGenomicLLM = GenomicLLM

__all__ = ["BATCH_INACTIVE", "GajeError", "GajeIOError", "GajeValueError", "GenomicBatch", "GenomicLLM", "RustGenomicLLM",
           "LIB_PATH", "SIGNATURES", "flat", "gguf", "last_error", "lib", "load_genomic_auto", "ops", "synth", "writer"]
