"""The C ABI: every entry point include/gaje_hip.h declares is exported by the
built library and bound by the Python mirror with the header's struct layouts.

CPU only: symbols are resolved, and the host-only entry points are called, but
nothing touches a device.
"""
import ctypes
import os
import re
import subprocess

import pytest

from conftest import REPO

HEADER = os.path.join(REPO, "include", "gaje_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^[A-Za-z_][\w \*]*?\b(gaje_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_header_declares_the_boundary():
    names = declared_functions()
    # the operator, model, reader and writer groups are all present
    for must in ("gaje_hip_q4_0_gemv", "gaje_hip_q4_0_pack", "gaje_hip_f32_gemv", "gaje_hip_attention",
                 "gaje_hip_rmsnorm", "gaje_hip_open", "gaje_hip_forward", "gaje_hip_decode_greedy",
                 "gaje_flat_inspect", "gaje_synth_write_flat", "gaje_hip_last_error"):
        assert must in names
    assert len(names) >= 50


def test_library_exports_every_declared_symbol():
    import gaje_hip
    assert os.path.exists(gaje_hip.LIB_PATH), "build the library first (__graft_entry__.build())"
    raw = ctypes.CDLL(gaje_hip.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(raw, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_python_mirror_binds_exactly_the_header():
    import gaje_hip
    bound = sorted(n for n, _, _ in gaje_hip.SIGNATURES)
    assert bound == declared_functions()
    gaje_hip.lib()  # every signature resolves and gets its argtypes


def test_status_codes_match_header():
    from gaje_hip import _lib
    text = open(HEADER).read()
    codes = dict(re.findall(r"\b(GAJE_(?:OK|ERR_\w+))\s*=\s*(-?\d+)", text))
    assert int(codes["GAJE_OK"]) == _lib.GAJE_OK
    for name, val in codes.items():
        if name == "GAJE_OK":
            continue
        assert getattr(_lib, name[len("GAJE_"):]) == int(val), name


STRUCTS = {"gaje_hip_model_info": "ModelInfo", "gaje_synth_config": "SynthConfig",
           "gaje_flat_header": "FlatHeader", "gaje_flat_info": "FlatInfo", "gaje_flat_tensor": "FlatTensor"}


def test_struct_layouts_match_a_c_compiler(tmp_path):
    """sizeof and every field offset as gcc lays the header's structs out."""
    from gaje_hip import _lib
    src = ['#include <stdio.h>', '#include <stddef.h>', '#include "gaje_hip.h"', "int main(void) {"]
    for cname, pyname in STRUCTS.items():
        st = getattr(_lib, pyname)
        src.append(f'printf("{pyname} size %zu\\n", sizeof({cname}));')
        for f, _ in st._fields_:
            src.append(f'printf("{pyname} {f} %zu\\n", offsetof({cname}, {f}));')
    src.append("return 0; }")
    c = tmp_path / "layout.c"
    c.write_text("\n".join(src))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(REPO, "include"), str(c), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    for line in filter(None, out):
        pyname, field, val = line.split()
        st = getattr(_lib, pyname)
        got = ctypes.sizeof(st) if field == "size" else getattr(st, field).offset
        assert got == int(val), f"{pyname}.{field}: ctypes {got} vs C {val}"


def test_host_entry_points_run_without_a_device(tmp_path):
    import numpy as np
    import gaje_hip
    assert gaje_hip.ops.q4_0_packed_bytes(4864, 896) == 4864 * 7 * 80 + 2048
    with pytest.raises(ValueError):
        gaje_hip.ops.q4_0_packed_bytes(3, 100)
    b = gaje_hip.synth.q4_0_tensor(1, "abi", 2, 64)
    assert b.shape == (2 * 2 * 20,) and b.dtype == np.uint8
    path = str(tmp_path / "m.flat")
    gaje_hip.synth.write_flat(path, n_embd=64, n_head=2, n_head_kv=1, n_blocks=1, ffn=128, vocab_size=50,
                              eps=1e-6, rope_base=1e4, arch_family=1, qkv_bias=1, tied_embeddings=0, seed=3)
    info = gaje_hip.flat.inspect(path)
    assert info["n_embd"] == 64 and info["n_blocks"] == 1 and info["header"]["quantization_type"] == "Q4_0"
