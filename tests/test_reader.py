"""The C++ .gaje.flat reader (the model loader's, through its host-only C
ABI) against the oracle's numpy reader on synthetic files, and its errors on
damaged files (GajeFlatFileReader::open, src/io/flat_reader.rs:33-69)."""
import os

import numpy as np
import pytest

from oracle import flat as OF

ENTRY = ("bit_depth", "out_features", "in_features", "dna_off", "dna_len", "c_off", "c_len",
         "anc_off", "anc_len", "bias_off", "bias_len")


def _write(tmp_path, name, **kw):
    import gaje_hip
    path = str(tmp_path / name)
    args = dict(n_embd=128, n_head=4, n_head_kv=2, n_blocks=2, ffn=256, vocab_size=500, eps=1e-5,
                rope_base=1e4, arch_family=1, qkv_bias=1, tied_embeddings=0, seed=9)
    args.update(kw)
    gaje_hip.synth.write_flat(path, **args)
    return path


@pytest.mark.parametrize("kw", [dict(), dict(fused=False), dict(body_format=2), dict(arch_family=3),
                                dict(arch_family=0, rope_interleaved=1, use_genomic_norm=1),
                                dict(tied_embeddings=1, qkv_bias=0)])
def test_cpp_reader_matches_numpy_reader(tmp_path, kw):
    import gaje_hip
    path = _write(tmp_path, "m.flat", **kw)
    ff = OF.FlatFile(path)
    cfg = ff.model_config()
    info = gaje_hip.flat.inspect(path)
    h = ff.header
    for f in ("version", "flags", "num_tensors", "group_size", "quant_format", "arch_family", "meta_len",
              "dir_len", "weights_offset", "weights_len"):
        assert info["header"][f] == getattr(h, f), f
    assert info["header"]["quantization_type"] == h.quantization_type()
    assert (info["n_embd"], info["n_head"], info["n_head_kv"], info["n_blocks"]) == \
        (cfg.n_embd, cfg.n_head, cfg.n_head_kv, cfg.n_blocks)
    assert np.float32(info["eps"]) == cfg.eps
    assert np.float32(info["rope_base"]) == np.float32(cfg.config["rope_base"])
    assert info["rope_split"] == (cfg.config["rope_style"] == "split")
    assert info["use_genomic_norm"] == bool(cfg.config["use_genomic_norm"])
    assert info["has_descriptor"] == (h.arch_family != 0)
    assert info["n_tensors"] == len(ff.tensors)
    for name, e in ff.tensors.items():
        got = gaje_hip.flat.tensor_entry(path, name)
        assert all(got[k] == e[k] for k in ENTRY), name
    if kw.get("arch_family") == 3:  # the descriptor's family rope base wins over the JSON (flat.rs:100-136)
        assert info["rope_base"] == 1e6


def test_reader_errors(tmp_path):
    import gaje_hip
    from gaje_hip import _lib
    path = _write(tmp_path, "ok.flat")
    data = open(path, "rb").read()

    def damaged(name, b):
        p = str(tmp_path / name)
        with open(p, "wb") as f:
            f.write(b)
        return p

    cases = {
        "missing.flat": (None, _lib.ERR_IO),
        "magic.flat": (b"XGAJ" + data[4:], _lib.ERR_INVALID_MAGIC),
        "short.flat": (data[:1000], _lib.ERR_TOO_SHORT),
        # serde: a required field (eps) absent from the metadata JSON
        "noeps.flat": (data.replace(b'"eps"', b'"epz"', 1), _lib.ERR_INVALID_DATA),
        # metadata that is not UTF-8
        "utf8.flat": (data[:4096] + b"\xff" + data[4097:], _lib.ERR_INVALID_DATA),
    }
    for name, (content, code) in cases.items():
        p = str(tmp_path / name) if content is None else damaged(name, content)
        with pytest.raises(gaje_hip.GajeError) as e:
            gaje_hip.flat.inspect(p)
        assert e.value.code == code, (name, e.value.code, str(e.value))
    with pytest.raises(gaje_hip.GajeIOError) as e:
        gaje_hip.flat.tensor_entry(path, "blk.9.attn_qkv")
    assert e.value.code == _lib.ERR_NOT_FOUND and "not found" in str(e.value)
    assert os.path.getsize(path) > 4096
