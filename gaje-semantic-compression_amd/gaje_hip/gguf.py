"""GGUF importer: a GGUF checkpoint (F32 / F16 / Q8_0 tensors) to `.gaje.flat`.

The container is read as published (GGUF v2/v3): the magic "GGUF", a u32
version, u64 tensor and metadata counts, the metadata key/value pairs (13 value
types, arrays included), the tensor infos (name, dims innermost first, type,
offset), and the tensor data from the first multiple of `general.alignment`
(default 32) after the infos.  The reference reads the same fields and tensor
types (src/io/gguf/reader.rs:29-125, tensor sizes :239-250), turns F16 into f32
and Q8_0 blocks (f16 scale d, 32 int8) into f32(q) * d
(src/compute/quantize/dequantize.rs:47-72), and un-permutes the Llama-family
Q/K rows from GGUF's interleaved RoPE order to the split order
(src/io/gguf_loader/tensors.rs:91-92,133-155; the exporter's
unpermute_to_split, python/gaje/utils/quantization.py:51-61).

`import_gguf` reads the architecture the way scripts/export_gaje_flat.py:57-124
does (family from `general.architecture` and the file name; Q/K un-permuted
for the Llama / SmolLM families) and hands the f32 tensors, keyed by their
GGUF names, to the native writer (`writer.export_gaje_flat`).  `write_gguf` is
the inverse container writer, for round trips.
"""
from __future__ import annotations

import mmap
import os
import struct

import numpy as np

# value types (GGUF spec; src/io/gguf/types.rs:7-21)
U8, I8, U16, I16, U32, I32, F32V, BOOL, STRING, ARRAY, U64, I64, F64V = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32V: "<f", BOOL: "<?",
           U64: "<Q", I64: "<q", F64V: "<d"}
# tensor types read here (ggml type ids)
GGML_F32, GGML_F16, GGML_Q8_0 = 0, 1, 8
Q8_0_BYTES = 34


class GGUFError(ValueError):
    pass


class _Cursor:
    """Reads fields from a buffer whose slices are copies (an mmap), so no view
    of the file outlives the parse."""

    def __init__(self, buf):
        self.buf, self.pos = buf, 0

    def take(self, n: int):
        if self.pos + n > len(self.buf):
            raise GGUFError("GGUF file truncated")
        v = self.buf[self.pos:self.pos + n]
        self.pos += n
        return v

    def scalar(self, fmt: str):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        return bytes(self.take(self.scalar("<Q"))).decode("utf-8")

    def value(self, vtype: int):
        if vtype in _SCALAR:
            return self.scalar(_SCALAR[vtype])
        if vtype == STRING:
            return self.string()
        if vtype == ARRAY:
            etype, count = self.scalar("<I"), self.scalar("<Q")
            return [self.value(etype) for _ in range(count)]
        raise GGUFError(f"unknown GGUF value type {vtype}")


def tensor_nbytes(dims, ttype: int) -> int:
    n = int(np.prod(dims, dtype=np.int64)) if len(dims) else 1
    if ttype == GGML_F32:
        return 4 * n
    if ttype == GGML_F16:
        return 2 * n
    if ttype == GGML_Q8_0:
        return (n + 31) // 32 * Q8_0_BYTES
    raise GGUFError(f"unsupported tensor type {ttype}")


class GGUFFile:
    """A parsed GGUF file: `metadata`, `tensors` (name -> (dims, type,
    offset)), and the tensor data as f32 through `f32`."""

    def __init__(self, path: str):
        self._f = open(path, "rb")
        self._mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        try:
            self._parse()
        except BaseException:
            self.close()
            raise

    def _parse(self):
        c = _Cursor(self._mm)
        if bytes(c.take(4)) != b"GGUF":
            raise GGUFError("Not a GGUF file")
        self.version = c.scalar("<I")
        if self.version not in (2, 3):
            raise GGUFError(f"Unsupported GGUF version: {self.version}")
        n_tensors, n_kv = c.scalar("<Q"), c.scalar("<Q")
        self.metadata = {}
        for _ in range(n_kv):
            key = c.string()
            self.metadata[key] = c.value(c.scalar("<I"))
        self.tensors = {}
        for _ in range(n_tensors):
            name = c.string()
            dims = tuple(c.scalar("<Q") for _ in range(c.scalar("<I")))
            ttype = c.scalar("<I")
            if ttype not in (GGML_F32, GGML_F16, GGML_Q8_0):
                raise GGUFError(f"Unsupported tensor type: {ttype}")
            self.tensors[name] = (dims, ttype, c.scalar("<Q"))
        align = self.metadata.get("general.alignment", 32)
        if not isinstance(align, int) or align <= 0:
            raise GGUFError("bad general.alignment")
        self.data_offset = (c.pos + align - 1) // align * align
        for name, (dims, ttype, off) in self.tensors.items():
            if self.data_offset + off + tensor_nbytes(dims, ttype) > len(self._mm):
                raise GGUFError(f"Tensor {name} offset out of bounds")

    def close(self):
        if self._mm is not None:
            self._mm.close()
            self._f.close()
            self._mm = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _view(self, name: str) -> np.ndarray:
        dims, ttype, off = self.tensors[name]
        return np.frombuffer(self._mm, np.uint8, tensor_nbytes(dims, ttype), self.data_offset + off)

    def raw(self, name: str) -> np.ndarray:
        """The tensor's stored bytes (a copy)."""
        return self._view(name).copy()

    def f32(self, name: str) -> np.ndarray:
        """The tensor as f32, [out][in] for 2-D tensors (GGUF dims are innermost
        first: dims = (in, out)), flat otherwise."""
        if name not in self.tensors:
            raise KeyError(f"Tensor not found: {name}")
        dims, ttype, _ = self.tensors[name]
        b = self._view(name)
        if ttype == GGML_F32:
            v = b.view(np.float32).copy()
        elif ttype == GGML_F16:
            v = b.view(np.float16).astype(np.float32)
        else:  # Q8_0: f32(q) * f32(d), rounded once (dequantize.rs:61-67)
            blk = b.reshape(-1, Q8_0_BYTES)
            d = blk[:, :2].copy().view(np.float16).astype(np.float32)
            q = blk[:, 2:].view(np.int8).astype(np.float32)
            v = (q * d).reshape(-1)[: int(np.prod(dims))]
        return v.reshape(dims[1], dims[0]) if len(dims) == 2 else v


def unpermute_qk(w: np.ndarray, n_head: int, head_dim: int) -> np.ndarray:
    """GGUF's interleaved Q/K rows to the split RoPE order: row h hd + a hd/2 + i
    of the result is row h hd + 2 i + a of w (tensors.rs:137-155)."""
    out_f, in_f = w.shape
    if head_dim % 2 or out_f % head_dim:
        raise GGUFError("un-permute needs rows in whole heads of even head_dim")
    return w.reshape(out_f // head_dim, head_dim // 2, 2, in_f).transpose(0, 2, 1, 3).reshape(out_f, in_f)


def permute_qk(w: np.ndarray, n_head: int, head_dim: int) -> np.ndarray:
    """The inverse: split rows to GGUF's interleaved order (what a Llama
    checkpoint converter does to Q and K)."""
    out_f, in_f = w.shape
    return w.reshape(out_f // head_dim, 2, head_dim // 2, in_f).transpose(0, 2, 1, 3).reshape(out_f, in_f)


def infer_family(arch: str, file_name: str):
    """(arch_family, qk_permute) as scripts/export_gaje_flat.py:99-124 maps them."""
    n, a = file_name.lower(), arch.lower()
    for key, fam, perm in (("qwen2.5", 4, False), ("qwen2", 3, False), ("smollm2", 2, True), ("smollm", 2, True),
                           ("gemma", 5, False), ("llama", 1, True)):
        if key in n or key in a:
            return fam, perm
    return 6, False


def model_config(g: GGUFFile) -> dict:
    """Shapes and hyper-parameters from the metadata (src/io/gguf_loader/metadata.rs:34-75)."""
    md = g.metadata
    arch = md.get("general.architecture", "llama")

    def get(key, default=None):
        for k in (f"{arch}.{key}", f"llama.{key}"):
            if k in md:
                return md[k]
        if default is None:
            raise GGUFError(f"{key} not found")
        return default

    n_embd, n_head = int(get("embedding_length")), int(get("attention.head_count"))
    return dict(arch=arch, n_embd=n_embd, n_head=n_head, n_head_kv=int(get("attention.head_count_kv", n_head)),
                n_blocks=int(get("block_count")), eps=float(md.get(f"{arch}.attention.layer_norm_rms_epsilon", 1e-6)),
                rope_base=float(get("rope.freq_base", 10000.0)), name=str(md.get("general.name", "GGUF-Model")))


def import_gguf(gguf_path: str, flat_path: str, quant_embed: bool = False, body: str = "q4_0",
                qk_permute: bool | None = None, arch_family: int | None = None) -> str:
    """Convert a GGUF checkpoint into a `.gaje.flat` file through the native
    writer.  Q/K rows are un-permuted for the Llama / SmolLM families unless
    `qk_permute` says otherwise."""
    from .writer import export_gaje_flat
    with GGUFFile(gguf_path) as g:
        cfg = model_config(g)
        fam, perm = infer_family(cfg["arch"], os.path.basename(gguf_path))
        fam = fam if arch_family is None else arch_family
        perm = perm if qk_permute is None else qk_permute
        hd = cfg["n_embd"] // cfg["n_head"]
        T = {}
        for name in g.tensors:
            w = g.f32(name)
            if perm and (name.endswith("attn_q.weight") or name.endswith("attn_k.weight")):
                heads = cfg["n_head"] if name.endswith("attn_q.weight") else cfg["n_head_kv"]
                w = unpermute_qk(w, heads, hd)
            T["lm_head.weight" if name == "output.weight" else name] = w
        vocab = T["token_embd.weight"].shape[0]
    return export_gaje_flat(flat_path, T, cfg["n_embd"], cfg["n_head"], cfg["n_head_kv"], cfg["n_blocks"], vocab,
                            cfg["eps"], cfg["rope_base"], arch_family=fam, name=cfg["name"], quant_embed=quant_embed,
                            body=body)


# ---- writer (round trips) ---------------------------------------------------------------------------

def _pack_value(vtype: int, v) -> bytes:
    if vtype in _SCALAR:
        return struct.pack(_SCALAR[vtype], v)
    if vtype == STRING:
        b = v.encode("utf-8")
        return struct.pack("<Q", len(b)) + b
    raise GGUFError(f"cannot pack value type {vtype}")


def _value_type(v):
    if isinstance(v, bool):
        return BOOL
    if isinstance(v, int):
        return U32 if 0 <= v < 2 ** 32 else I64
    if isinstance(v, float):
        return F32V
    if isinstance(v, str):
        return STRING
    raise GGUFError(f"no GGUF type for {type(v)}")


def quantize_q8_0_gguf(w: np.ndarray) -> bytes:
    """ggml's Q8_0 blocks: d = max|x| / 127 (stored f16), q = round(x / d)."""
    x = np.asarray(w, np.float32).reshape(-1, 32)
    amax = np.abs(x).max(axis=1)
    d = (amax / 127.0).astype(np.float32)
    inv = np.where(d > 0, 1.0 / np.where(d > 0, d, 1.0), 0.0).astype(np.float32)
    q = np.clip(np.rint(x * inv[:, None]), -127, 127).astype(np.int8)
    out = np.empty((x.shape[0], Q8_0_BYTES), np.uint8)
    out[:, :2] = d.astype(np.float16)[:, None].view(np.uint8)
    out[:, 2:] = q.view(np.uint8)
    return out.tobytes()


def write_gguf(path: str, metadata: dict, tensors: dict, types: dict | None = None, alignment: int = 32,
               version: int = 3, value_types: dict | None = None) -> str:
    """Write a GGUF file: metadata (key -> value; value_types may force a
    type, lists are arrays of their first element's type) and tensors (name ->
    f32 array, 2-D as [out][in]) stored as F32, or as types[name] (GGML_F16 /
    GGML_Q8_0)."""
    types, value_types = types or {}, value_types or {}
    kv = b""
    md = dict(metadata)
    if alignment != 32:
        md["general.alignment"] = alignment
    for k, v in md.items():
        kv += _pack_value(STRING, k)
        if isinstance(v, list):
            et = value_types.get(k, _value_type(v[0]) if v else U32)
            kv += struct.pack("<IIQ", ARRAY, et, len(v)) + b"".join(_pack_value(et, e) for e in v)
        else:
            vt = value_types.get(k, _value_type(v))
            kv += struct.pack("<I", vt) + _pack_value(vt, v)
    infos, blobs, off = b"", [], 0
    for name, w in tensors.items():
        w = np.asarray(w, np.float32)
        t = types.get(name, GGML_F32)
        dims = (w.shape[1], w.shape[0]) if w.ndim == 2 else (w.size,)
        data = (w.astype(np.float16).tobytes() if t == GGML_F16 else quantize_q8_0_gguf(w) if t == GGML_Q8_0
                else w.tobytes())
        infos += _pack_value(STRING, name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        infos += struct.pack("<IQ", t, off)
        blobs.append((off, data))
        off = (off + len(data) + alignment - 1) // alignment * alignment
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(md)) + kv + infos
    start = (len(head) + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(head + bytes(start - len(head)))
        for o, data in blobs:
            f.seek(start + o)
            f.write(data)
        f.truncate(start + off)
    return path
