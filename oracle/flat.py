"""numpy restatement of the `.gaje.flat` v2 reader.

TEST INFRASTRUCTURE ONLY (parity oracle).  It is independent of the product
reader (C++, in the package's csrc/) so the two can check each other.

Restates:
  - FlatHeaderV2 layout / from_bytes / quantization_type / effective_group_size
    / architecture_descriptor   (src/io/header/flat.rs:14-148, types.rs:7-29)
  - ArchConfig / ModelConfig serde defaults             (src/io/config.rs:17-145)
  - FlatTensorEntry and GajeFlatFileReader::open / get_slice / get_f32_slice
                                                         (src/io/flat_reader.rs:9-90)
  - the descriptor-over-JSON precedence of load_genomic  (src/io/flat_reader.rs:124-142)
"""
from __future__ import annotations

import json
import struct
from dataclasses import dataclass, field

import numpy as np

HEADER_SIZE = 4096
# "<4sIIIQQQQIIIIIIII": the field order of FlatHeaderV2 (flat.rs:14-41), which
# is also the pack format of the exporter (scripts/export_gaje_flat.py:450-471).
HEADER_FMT = "<4sIIIQQQQIIIIIIII"


class HeaderError(Exception):
    """HeaderError::{TooShort, InvalidMagic} (src/io/header/types.rs:15-27)."""


class TooShort(HeaderError):
    def __init__(self):
        super().__init__("Header buffer is less than 4096 bytes")


class InvalidMagic(HeaderError):
    def __init__(self):
        super().__init__("Invalid magic bytes (expected 'GAJE')")


# family code -> (rope_base, rope_style, ffn_act)  (flat.rs:100-136)
_FAMILY = {
    1: ("Llama", 10000.0, "split", "swiglu"),
    2: ("SmolLM", 100000.0, "split", "swiglu"),
    3: ("Qwen2", 1000000.0, "split", "swiglu"),
    4: ("Qwen2_5", 1000000.0, "split", "swiglu"),
    5: ("Gemma", 10000.0, "split", "geglu"),
}


@dataclass
class FlatHeader:
    magic: bytes
    version: int
    flags: int
    num_tensors: int
    meta_len: int
    dir_len: int
    weights_offset: int
    weights_len: int
    group_size: int
    quant_format: int
    arch_family: int
    arch_n_embd: int
    arch_n_head: int
    arch_n_head_kv: int
    arch_n_blocks: int
    arch_qk_permute: int

    @classmethod
    def from_bytes(cls, b: bytes) -> "FlatHeader":
        if len(b) < HEADER_SIZE:
            raise TooShort()
        h = cls(*struct.unpack_from(HEADER_FMT, b, 0))
        if h.magic != b"GAJE":
            raise InvalidMagic()
        return h

    def quantization_type(self) -> str:
        return {0: "LegacyCentroids", 1: "Q4_0", 2: "Q8_0"}.get(self.quant_format, "Unknown")

    def effective_group_size(self) -> int:
        return 16 if self.group_size == 0 else self.group_size

    def architecture_descriptor(self):
        if self.arch_family == 0:
            return None
        fam, base, style, act = _FAMILY.get(self.arch_family, ("Unknown", 10000.0, "split", "silu"))
        head_dim = self.arch_n_embd // self.arch_n_head if self.arch_n_head > 0 else 0
        return dict(family=fam, n_embd=self.arch_n_embd, n_head=self.arch_n_head,
                    n_head_kv=self.arch_n_head_kv, n_blocks=self.arch_n_blocks,
                    head_dim=head_dim, rope_base=np.float32(base), rope_style=style,
                    ffn_act=act, qk_permute=self.arch_qk_permute != 0)


_ARCH_DEFAULTS = dict(name="GAJE-Model", version="1.0.0-alpha", tokenizer_id="gpt2",
                      rope_base=10000.0, ffn_act="swiglu", use_genomic_norm=False,
                      rope_style="split", anchor_threshold=0.1, ffn_anchor_threshold=0.1,
                      rna_threshold=0.5, unpermute_weights=False,
                      apply_smollm_rope_patch=False, tie_word_embeddings=False)


@dataclass
class ModelConfig:
    """ModelConfig + ArchConfig (src/io/config.rs:17-48,137-145)."""
    n_embd: int
    n_head: int
    n_head_kv: int
    n_blocks: int
    vocab_size: int | None
    eps: np.float32
    config: dict = field(default_factory=dict)

    @classmethod
    def from_json(cls, text: str) -> "ModelConfig":
        d = json.loads(text)
        for req in ("config", "n_embd", "n_head", "n_head_kv", "n_blocks", "eps"):
            if req not in d:
                raise ValueError(f"missing field `{req}`")
        cfg = dict(_ARCH_DEFAULTS)
        cfg.update({k: v for k, v in d["config"].items() if k in _ARCH_DEFAULTS})
        cfg["rope_base"] = np.float32(cfg["rope_base"])
        return cls(int(d["n_embd"]), int(d["n_head"]), int(d["n_head_kv"]), int(d["n_blocks"]),
                   d.get("vocab_size"), np.float32(d["eps"]), cfg)


ENTRY_FIELDS = ("name", "bit_depth", "out_features", "in_features", "dna_off", "dna_len",
                "c_off", "c_len", "anc_off", "anc_len", "bias_off", "bias_len")


class FlatFile:
    """GajeFlatFileReader (src/io/flat_reader.rs:24-90)."""

    def __init__(self, path: str):
        self.mm = np.memmap(path, dtype=np.uint8, mode="r")
        self.header = FlatHeader.from_bytes(bytes(self.mm[:HEADER_SIZE]))
        h = self.header
        ms, me = HEADER_SIZE, HEADER_SIZE + h.meta_len
        self.metadata_json = bytes(self.mm[ms:me]).decode("utf-8")
        entries = json.loads(bytes(self.mm[me:me + h.dir_len]))
        self.tensors = {}
        for e in entries:
            self.tensors[e["name"]] = {k: e[k] for k in ENTRY_FIELDS}
        self.weights_offset = h.weights_offset

    def get_slice(self, off: int, length: int) -> np.ndarray:
        if length == 0:
            return np.zeros(0, dtype=np.uint8)
        s = self.weights_offset + off
        return self.mm[s:s + length]

    def get_f32_slice(self, off: int, length: int) -> np.ndarray:
        if length == 0:
            return np.zeros(0, dtype=np.float32)
        b = self.get_slice(off, length)
        return np.frombuffer(bytes(b[: (len(b) // 4) * 4]), dtype=np.float32)

    def model_config(self) -> ModelConfig:
        """load_genomic's config resolution (flat_reader.rs:125-142)."""
        cfg = ModelConfig.from_json(self.metadata_json)
        desc = self.header.architecture_descriptor()
        if desc is not None:
            cfg.n_embd = desc["n_embd"]
            cfg.n_head = desc["n_head"]
            cfg.n_head_kv = desc["n_head_kv"]
            cfg.n_blocks = desc["n_blocks"]
            cfg.config["rope_base"] = desc["rope_base"]
            cfg.config["rope_style"] = desc["rope_style"]
            cfg.config["ffn_act"] = desc["ffn_act"]
            cfg.config["unpermute_weights"] = desc["qk_permute"]
        return cfg
