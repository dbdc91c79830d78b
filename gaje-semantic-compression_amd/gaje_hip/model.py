"""Model-level mirror of the reference's Python surface.

`load_genomic_auto(path)` and the returned `GenomicLLM` follow the PyO3 API of
the reference (src/io/ffi.rs:66-71, src/nn/llm/python.rs:33-119): same method
names, argument meaning and error behaviour (ValueError with the reference's
messages for the forward-path Err(String)s, OSError for reader failures).
"""
from __future__ import annotations

import ctypes

import numpy as np

from ._lib import ModelInfo, check, lib


class GenomicLLM:
    """RustGenomicLLM backed by a device-resident model on one MI355X."""

    def __init__(self, path: str, device: int = 0):
        h = ctypes.c_void_p()
        check(lib().gaje_hip_open(str(path).encode(), int(device), ctypes.byref(h)))
        self._h = h
        info = ModelInfo()
        check(lib().gaje_hip_model_info_get(self._h, ctypes.byref(info)))
        self.info = {f: getattr(info, f) for f, _ in ModelInfo._fields_}
        self.n_logits = int(self.info["n_logits"])

    # -- lifetime ------------------------------------------------------------
    def close(self):
        if getattr(self, "_h", None):
            lib().gaje_hip_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- reference getters / setters (python.rs:33-59) ------------------------
    @property
    def vocab_size(self) -> int:
        return self.info["vocab_size"]

    @property
    def n_embd(self) -> int:
        return self.info["n_embd"]

    @property
    def k_wta_ratio(self) -> float:
        r = ctypes.c_float()
        check(lib().gaje_hip_get_kwta(self._h, ctypes.byref(r)))
        return r.value

    def set_k_wta_ratio(self, ratio: float) -> None:
        check(lib().gaje_hip_set_kwta(self._h, float(ratio)))

    # -- forward path (python.rs:68-100) -------------------------------------
    def forward(self, token_id: int, clear_cache: bool = False) -> np.ndarray:
        out = np.empty(self.n_logits, dtype=np.float32)
        check(lib().gaje_hip_forward(self._h, int(token_id) & 0xFFFFFFFF, int(bool(clear_cache)),
                                     out.ctypes.data))
        return out

    def forward_with_hidden(self, token_id: int, clear_cache: bool = False):
        logits = np.empty(self.n_logits, dtype=np.float32)
        hidden = np.empty(self.n_embd, dtype=np.float32)
        check(lib().gaje_hip_forward_hidden(self._h, int(token_id) & 0xFFFFFFFF,
                                            int(bool(clear_cache)), logits.ctypes.data,
                                            hidden.ctypes.data))
        return logits, hidden

    def clear_cache_py(self) -> None:
        check(lib().gaje_hip_clear_cache(self._h))

    def generate_native_py(self, prompt_tokens, max_new_tokens: int = 30, temperature: float = 0.7,
                           repetition_penalty: float = 1.0, eos_token_ids=(2, 151643, 151645),
                           seed: int = 0):
        prompt = np.ascontiguousarray(prompt_tokens, dtype=np.uint32)
        eos = np.ascontiguousarray(list(eos_token_ids), dtype=np.uint32)
        out = np.empty(max(int(max_new_tokens), 1), dtype=np.uint32)
        n = ctypes.c_int64()
        check(lib().gaje_hip_generate(self._h, prompt.ctypes.data if prompt.size else None, prompt.size,
                                      int(max_new_tokens), float(temperature),
                                      float(repetition_penalty),
                                      eos.ctypes.data if eos.size else None, eos.size,
                                      int(seed) & 0xFFFFFFFFFFFFFFFF, out.ctypes.data,
                                      ctypes.byref(n)))
        return [int(t) for t in out[: n.value]]

    # -- device fast paths ---------------------------------------------------
    def cache_len(self) -> int:
        n = ctypes.c_int64()
        check(lib().gaje_hip_cache_len(self._h, ctypes.byref(n)))
        return n.value

    def reserve(self, positions: int) -> None:
        check(lib().gaje_hip_reserve(self._h, int(positions)))

    def prefill(self, ids, want_logits: bool = False):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        out = np.empty(self.n_logits, dtype=np.float32) if want_logits else None
        check(lib().gaje_hip_prefill(self._h, ids.ctypes.data if ids.size else None, ids.size,
                                     out.ctypes.data if out is not None else None))
        return out

    def prefill_mfma(self, ids, want_logits: bool = False):
        """prefill() with the prompt processed as MFMA matrix products: fp32
        accuracy, not the reference's bits (gaje_hip_prefill_mfma)."""
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        out = np.empty(self.n_logits, dtype=np.float32) if want_logits else None
        check(lib().gaje_hip_prefill_mfma(self._h, ids.ctypes.data if ids.size else None, ids.size,
                                          out.ctypes.data if out is not None else None))
        return out

    def greedy_next(self, token: int) -> int:
        nxt = ctypes.c_uint32()
        check(lib().gaje_hip_greedy_next(self._h, int(token), ctypes.byref(nxt)))
        return nxt.value

    def decode_greedy(self, first_token: int, n: int) -> np.ndarray:
        out = np.empty(max(int(n), 1), dtype=np.uint32)
        check(lib().gaje_hip_decode_greedy(self._h, int(first_token), int(n), out.ctypes.data))
        return out[: int(n)]

    def truncate_cache(self, length: int) -> None:
        check(lib().gaje_hip_truncate_cache(self._h, int(length)))

    STAGES = {"qkv": 1, "attention": 2, "o": 3, "gate_up": 4, "down": 5, "lm_head": 6, "token": 7}

    def time_stage(self, stage: str, layer: int = 0, iters: int = 50):
        """(average ms per launch, algorithmic bytes per launch) of one stage's kernel."""
        ms, nbytes = ctypes.c_float(), ctypes.c_int64()
        check(lib().gaje_hip_time_stage(self._h, self.STAGES[stage], int(layer), int(iters),
                                        ctypes.byref(ms), ctypes.byref(nbytes)))
        return ms.value, nbytes.value

    def last_timing(self):
        b, hd = ctypes.c_float(), ctypes.c_float()
        check(lib().gaje_hip_last_timing(self._h, ctypes.byref(b), ctypes.byref(hd)))
        return b.value, hd.value


def load_genomic_auto(path: str, device: int = 0) -> GenomicLLM:
    """load_genomic_auto for .gaje.flat files (src/io/flat_reader.rs:240-252)."""
    return GenomicLLM(path, device)


BATCH_INACTIVE = 0xFFFFFFFF


class GenomicBatch:
    """n_seq independent sequences over one GenomicLLM's weights, stepped
    together (gaje_hip_batch_*): each sequence's logits are bit-identical to its
    own GenomicLLM.forward_core."""

    def __init__(self, model: GenomicLLM, n_seq: int, capacity: int):
        h = ctypes.c_void_p()
        check(lib().gaje_hip_batch_open(model._h, int(n_seq), int(capacity), ctypes.byref(h)))
        self._h = h
        self.model = model
        self.n_seq = int(n_seq)

    def close(self):
        if getattr(self, "_h", None):
            lib().gaje_hip_batch_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self, seq: int = -1) -> None:
        check(lib().gaje_hip_batch_reset(self._h, int(seq)))

    def cache_len(self, seq: int) -> int:
        n = ctypes.c_int64()
        check(lib().gaje_hip_batch_cache_len(self._h, int(seq), ctypes.byref(n)))
        return n.value

    def feed(self, ids, want_logits: bool = False, status: bool = False):
        """ids: [n_seq][n] token ids (BATCH_INACTIVE skips a sequence's step).
        Returns the last step's logits [n_seq][n_logits] (or None), and the
        per-sequence status when asked."""
        ids = np.ascontiguousarray(ids, dtype=np.uint32).reshape(self.n_seq, -1)
        out = np.empty((self.n_seq, self.model.n_logits), np.float32) if want_logits else None
        st = np.zeros(self.n_seq, np.int32)
        rc = lib().gaje_hip_batch_feed(self._h, ids.ctypes.data, ids.shape[1],
                                       out.ctypes.data if out is not None else None, st.ctypes.data)
        if status:
            return out, st, rc
        check(rc)
        return out

    def decode_greedy(self, first, n: int, status: bool = False):
        first = np.ascontiguousarray(first, dtype=np.uint32).reshape(self.n_seq)
        out = np.zeros((self.n_seq, int(n)), np.uint32)
        st = np.zeros(self.n_seq, np.int32)
        rc = lib().gaje_hip_batch_decode_greedy(self._h, first.ctypes.data, int(n), out.ctypes.data,
                                                st.ctypes.data)
        if status:
            return out, st, rc
        check(rc)
        return out
