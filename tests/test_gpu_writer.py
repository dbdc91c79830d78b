"""Files written by the native writer from f32 weights (export_gaje_flat's layout and
quantisers) run on the device bit for bit like the oracle."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def same_bits(a, b) -> bool:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("body,quant_embed,anchors", [("q4_0", False, -1.0), ("q4_0", True, -1.0),
                                                       ("lut4", False, 0.2)])
def test_exported_model_stream(tmp_models, body, quant_embed, anchors):
    import gaje_hip
    from gaje_hip import writer as W
    from oracle import oracle as O
    from test_writer import _tiny_tensors
    if gaje_hip.ops.device_count() < 1:
        pytest.fail("no HIP device visible")
    T = _tiny_tensors(np.random.default_rng(17), h=128, heads=4, kv=2, blocks=2, ffn=256, vocab=500)
    p = str(tmp_models / f"gpu_export_{body}_{int(quant_embed)}.flat")
    W.export_gaje_flat(p, T, n_embd=128, n_head=4, n_head_kv=2, n_blocks=2, vocab_size=500, eps=1e-6,
                       rope_base=1e6, arch_family=3, quant_embed=quant_embed, body=body, anchor_threshold=anchors)
    g = gaje_hip.load_genomic_auto(p)
    r = O.load_genomic(p)
    g.set_k_wta_ratio(0.0)
    r.set_k_wta_ratio(0.0)
    toks = [int(t) for t in np.random.default_rng(18).integers(0, 500, 8)]
    for i, t in enumerate(toks):
        assert same_bits(g.forward(t, i == 0), r.forward_core(t, i == 0)), f"token {i}"
    g.close()


@pytest.mark.parametrize("arch", ["llama", "qwen2"])
def test_imported_gguf_stream(tmp_models, arch):
    """A GGUF checkpoint (Llama-family Q/K rows interleaved as converters store
    them) imported to .gaje.flat runs on the device bit for bit like the oracle."""
    import gaje_hip
    from gaje_hip import gguf as G
    from oracle import oracle as O
    from test_gguf import _md, _tiny_tensors
    if gaje_hip.ops.device_count() < 1:
        pytest.fail("no HIP device visible")
    T = _tiny_tensors(np.random.default_rng(19), E=128, H=4, KV=2, L=2, F=256, V=500, bias=arch == "qwen2")
    if arch == "llama":
        for i in range(2):
            T[f"blk.{i}.attn_q.weight"] = G.permute_qk(T[f"blk.{i}.attn_q.weight"], 4, 32)
            T[f"blk.{i}.attn_k.weight"] = G.permute_qk(T[f"blk.{i}.attn_k.weight"], 2, 32)
    src = G.write_gguf(str(tmp_models / f"imp_{arch}.gguf"), _md(arch, E=128), T,
                       types={k: G.GGML_F16 for k in T if k.startswith("blk.") and T[k].ndim == 2})
    p = G.import_gguf(src, str(tmp_models / f"imp_{arch}.flat"))
    g = gaje_hip.load_genomic_auto(p)
    r = O.load_genomic(p)
    g.set_k_wta_ratio(0.0)
    r.set_k_wta_ratio(0.0)
    for i, t in enumerate([int(v) for v in np.random.default_rng(20).integers(0, 500, 6)]):
        assert same_bits(g.forward(t, i == 0), r.forward_core(t, i == 0)), f"token {i}"
    g.close()
