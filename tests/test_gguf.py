"""The GGUF importer (gaje_hip.gguf): container parsing, the Q/K un-permutation
and the conversion to .gaje.flat.

Pinned without the reference's own loader (Rust, unbuildable here) or the
`gguf` Python package (absent): the un-permutation against its closed form on a
matrix whose rows carry their own index (src/io/gguf_loader/tensors.rs:137-155)
and as the inverse of the converter's permutation; the container through round
trips of files written by gaje_hip.gguf.write_gguf (every value type, F32 / F16
/ Q8_0 tensors, alignments 32 and 64, GGUF v2 and v3), Q8_0 values against the
reference's f32(q) * f32(d) (src/compute/quantize/dequantize.rs:61-67); and the
import as the writer's own export of the same f32 tensors, byte for byte.
"""
import os

import numpy as np
import pytest

from oracle import oracle as O
from oracle.flat import FlatFile


@pytest.fixture(scope="module")
def G():
    import gaje_hip
    return gaje_hip.gguf


def test_unpermute_closed_form(G):
    # rows labelled by their index: row h hd + a hd/2 + i of the result is row h hd + 2 i + a
    n_head, hd, k = 3, 8, 5
    w = np.repeat(np.arange(n_head * hd, dtype=np.float32)[:, None], k, axis=1)
    u = G.unpermute_qk(w, n_head, hd)
    expect = [h * hd + 2 * i + a for h in range(n_head) for a in range(2) for i in range(hd // 2)]
    assert list(u[:, 0].astype(int)) == expect
    # the Rust loop (tensors.rs:141-152): new_j = 2 j (j < hd/2) else 2 (j - hd/2) + 1
    rust = [h * hd + (2 * j if j < hd // 2 else 2 * (j - hd // 2) + 1) for h in range(n_head) for j in range(hd)]
    assert list(u[:, 0].astype(int)) == rust
    # the converter's permutation and the un-permutation are inverses
    x = np.random.default_rng(0).normal(size=(n_head * hd, k)).astype(np.float32)
    assert np.array_equal(G.unpermute_qk(G.permute_qk(x, n_head, hd), n_head, hd), x)
    assert not np.array_equal(G.permute_qk(x, n_head, hd), x)


@pytest.mark.parametrize("version,alignment", [(3, 32), (2, 64)])
def test_container_round_trip(G, tmp_path, version, alignment):
    rng = np.random.default_rng(1)
    md = {"general.architecture": "qwen2", "general.name": "tiny", "qwen2.block_count": 2,
          "qwen2.rope.freq_base": 1e6, "u8": 7, "i8": -3, "u16": 65000, "i16": -2000, "i32": -7, "u64": 2 ** 40,
          "i64": -(2 ** 40), "f64": 0.1, "flag": True, "tokens": ["a", "bc", ""], "scores": [0.5, -1.0]}
    vt = {"u8": G.U8, "i8": G.I8, "u16": G.U16, "i16": G.I16, "i32": G.I32, "u64": G.U64, "i64": G.I64,
          "f64": G.F64V, "scores": G.F32V}
    T = {"a": rng.normal(size=(3, 64)).astype(np.float32), "b": rng.normal(size=(64,)).astype(np.float32),
         "c": rng.normal(size=(5, 32)).astype(np.float32), "d": rng.normal(size=(2, 96)).astype(np.float32)}
    p = G.write_gguf(str(tmp_path / "t.gguf"), md, T, types={"c": G.GGML_F16, "d": G.GGML_Q8_0},
                     alignment=alignment, version=version, value_types=vt)
    with G.GGUFFile(p) as g:
        assert g.version == version and g.data_offset % alignment == 0
        for k, v in md.items():
            got = g.metadata[k]
            assert (abs(got - v) < 1e-6 if isinstance(v, float) else got == v), k
        assert g.metadata["scores"] == [0.5, -1.0]
        assert g.tensors["a"][0] == (64, 3) and g.tensors["b"][0] == (64,)
        assert np.array_equal(g.f32("a"), T["a"]) and np.array_equal(g.f32("b"), T["b"])
        assert np.array_equal(g.f32("c"), T["c"].astype(np.float16).astype(np.float32))
        # Q8_0: f32(q) * f32(d) per block of 32 (dequantize.rs:61-67)
        raw = g.raw("d").reshape(-1, 34)
        d = raw[:, :2].copy().view(np.float16).astype(np.float32)
        q = raw[:, 2:].view(np.int8).astype(np.float32)
        assert np.array_equal(g.f32("d").reshape(-1, 32), (q * d).astype(np.float32))
        assert np.max(np.abs(g.f32("d") - T["d"])) < np.max(np.abs(T["d"])) / 100


def test_bad_files(G, tmp_path):
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUX" + bytes(64))
    with pytest.raises(G.GGUFError, match="Not a GGUF"):
        G.GGUFFile(str(bad))
    bad.write_bytes(b"GGUF" + (4).to_bytes(4, "little") + bytes(16))
    with pytest.raises(G.GGUFError, match="version"):
        G.GGUFFile(str(bad))
    p = G.write_gguf(str(tmp_path / "q4.gguf"), {"x": 1}, {"w": np.zeros((2, 32), np.float32)})
    data = bytearray(open(p, "rb").read())
    i = data.index(b"w") + 1 + 4 + 16  # name, n_dims, two dims: the type field
    data[i:i + 4] = (2).to_bytes(4, "little")  # ggml Q4_0: not read here (nor by the reference)
    open(p, "wb").write(bytes(data))
    with pytest.raises(G.GGUFError, match="Unsupported tensor type"):
        G.GGUFFile(p)
    short = tmp_path / "short.gguf"
    short.write_bytes(open(G.write_gguf(str(tmp_path / "s.gguf"), {}, {"w": np.ones(64, np.float32)}), "rb").read()[:-40])
    with pytest.raises(G.GGUFError, match="out of bounds"):
        G.GGUFFile(str(short))


def _tiny_tensors(rng, E=64, H=4, KV=2, L=2, F=96, V=50, bias=True):
    hd = E // H
    T = {"token_embd.weight": rng.normal(0, 0.02, (V, E)), "output_norm.weight": 1 + 0.1 * rng.normal(size=E),
         "output.weight": rng.normal(0, 0.02, (V, E))}
    for i in range(L):
        p = f"blk.{i}."
        T[p + "attn_norm.weight"] = 1 + 0.1 * rng.normal(size=E)
        T[p + "ffn_norm.weight"] = 1 + 0.1 * rng.normal(size=E)
        T[p + "attn_q.weight"] = rng.normal(0, 0.05, (H * hd, E))
        T[p + "attn_k.weight"] = rng.normal(0, 0.05, (KV * hd, E))
        T[p + "attn_v.weight"] = rng.normal(0, 0.05, (KV * hd, E))
        if bias:
            for t, n in (("q", H), ("k", KV), ("v", KV)):
                T[p + f"attn_{t}.bias"] = rng.normal(0, 0.02, n * hd)
        T[p + "attn_output.weight"] = rng.normal(0, 0.05, (E, H * hd))
        T[p + "ffn_gate.weight"] = rng.normal(0, 0.05, (F, E))
        T[p + "ffn_up.weight"] = rng.normal(0, 0.05, (F, E))
        T[p + "ffn_down.weight"] = rng.normal(0, 0.05, (E, F))
    return {k: np.asarray(v, np.float32) for k, v in T.items()}


def _md(arch, E=64, H=4, KV=2, L=2, eps=1e-6, base=1e6):
    return {"general.architecture": arch, "general.name": f"tiny-{arch}", f"{arch}.embedding_length": E,
            f"{arch}.attention.head_count": H, f"{arch}.attention.head_count_kv": KV, f"{arch}.block_count": L,
            f"{arch}.attention.layer_norm_rms_epsilon": eps, f"{arch}.rope.freq_base": base}


@pytest.mark.parametrize("arch,ext_types", [("qwen2", {}), ("llama", {}), ("qwen2", "f16")])
def test_import_equals_direct_export(G, tmp_path, arch, ext_types):
    """import_gguf = read + (Llama: un-permute Q/K) + the writer's export of the
    same f32 tensors: the two .gaje.flat files are identical byte for byte."""
    import gaje_hip
    rng = np.random.default_rng(5)
    T = _tiny_tensors(rng, bias=arch == "qwen2")
    hd = 64 // 4
    stored = dict(T)
    if arch == "llama":  # the checkpoint converter's interleaved Q/K rows
        for i in range(2):
            stored[f"blk.{i}.attn_q.weight"] = G.permute_qk(T[f"blk.{i}.attn_q.weight"], 4, hd)
            stored[f"blk.{i}.attn_k.weight"] = G.permute_qk(T[f"blk.{i}.attn_k.weight"], 2, hd)
    types = {}
    if ext_types == "f16":
        types = {k: G.GGML_F16 for k in T if k.endswith(".weight") and T[k].ndim == 2}
        T = {k: (v.astype(np.float16).astype(np.float32) if k in types else v) for k, v in T.items()}
    src = G.write_gguf(str(tmp_path / f"{arch}.gguf"), _md(arch), stored, types=types)
    got = G.import_gguf(src, str(tmp_path / "imported.flat"))
    fam, _ = G.infer_family(arch, "x")
    direct = dict(T)
    direct["lm_head.weight"] = direct.pop("output.weight")
    eps = float(np.float32(1e-6))  # the metadata stores eps as an f32 (metadata.rs:60-62)
    ref = gaje_hip.writer.export_gaje_flat(str(tmp_path / "direct.flat"), direct, 64, 4, 2, 2, 50, eps, 1e6,
                                           arch_family=fam, name=f"tiny-{arch}")
    assert open(got, "rb").read() == open(ref, "rb").read()
    # and the file loads: the oracle's forward runs on it
    r = O.load_genomic(got)
    r.set_k_wta_ratio(0.0)
    assert np.isfinite(r.forward_core(3, True)).all()
    ff = FlatFile(got)
    assert ff.model_config().n_blocks == 2 and ff.header.arch_family == fam


def test_import_q8_0_tensors_and_family(G, tmp_path):
    """Q8_0 tensors dequantised as the reference does; the family and the
    un-permutation follow the architecture and the file name."""
    import gaje_hip
    rng = np.random.default_rng(6)
    T = _tiny_tensors(rng, bias=False)
    types = {k: G.GGML_Q8_0 for k in T if T[k].ndim == 2}
    path = G.write_gguf(str(tmp_path / "SmolLM2-tiny.gguf"), _md("llama"), T, types=types)
    with G.GGUFFile(path) as g:
        deq = {k: g.f32(k) for k in T}
    assert G.infer_family("llama", "SmolLM2-tiny.gguf") == (2, True)
    got = G.import_gguf(path, str(tmp_path / "q8.flat"), qk_permute=False)
    direct = dict(deq)
    direct["lm_head.weight"] = direct.pop("output.weight")
    ref = gaje_hip.writer.export_gaje_flat(str(tmp_path / "q8_direct.flat"), direct, 64, 4, 2, 2, 50,
                                           float(np.float32(1e-6)), 1e6, arch_family=2, name="tiny-llama")
    assert open(got, "rb").read() == open(ref, "rb").read()
