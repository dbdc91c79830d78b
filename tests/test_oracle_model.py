"""The oracle's whole forward against an independent composition: HF
transformers' Qwen2ForCausalLM built from a local config (no download), in
float64, with its weights set to the file's tensors dequantised exactly.

This pins what the per-kernel tests cannot: the block wiring of
RustGenomicBlock::forward_core (residuals, the fused QKV / gate_up split,
RoPE on q and k only, GQA head mapping, SwiGLU, the final norm and lm_head).
Tolerance: logits within a floored relative error of 1e-3.  The oracle
computes in fp32 and HF here in fp64, and fp32 rounding alone already reaches
~1.2e-4 on this measure; a wiring slip is off by O(1) (checked below).  K-WTA is off, as in the
benchmark; the genomic norm and the 2-bit paths are not part of HF's model.
"""
import numpy as np
import pytest

from conftest import GNORM_MODEL, floored_rel_err, write_genomic_norm_model

torch = pytest.importorskip("torch")
transformers = pytest.importorskip("transformers")

from oracle import oracle as O  # noqa: E402
from oracle.flat import FlatFile  # noqa: E402
from fp64_model import forward_fp64, tensor_weights  # noqa: E402


def hf_model(ff: FlatFile, cfg, vocab, ffn, rope_base):
    from transformers import Qwen2Config, Qwen2ForCausalLM
    E, H, KV, L = cfg.n_embd, cfg.n_head, cfg.n_head_kv, cfg.n_blocks
    hd = E // H
    hc = Qwen2Config(vocab_size=vocab, hidden_size=E, intermediate_size=ffn, num_hidden_layers=L,
                     num_attention_heads=H, num_key_value_heads=KV, rms_norm_eps=float(cfg.eps),
                     rope_theta=float(rope_base), max_position_embeddings=256, tie_word_embeddings=False,
                     attn_implementation="eager")
    m = Qwen2ForCausalLM(hc).double().eval()
    sd = {}
    f32 = lambda name: ff.get_f32_slice(ff.tensors[name]["dna_off"], ff.tensors[name]["dna_len"]).astype(np.float64)
    sd["model.embed_tokens.weight"] = tensor_weights(ff, "token_embd")[0]
    sd["model.norm.weight"] = f32("output_norm")
    sd["lm_head.weight"] = tensor_weights(ff, "lm_head")[0]
    for i in range(L):
        p, q = f"blk.{i}.", f"model.layers.{i}."
        sd[q + "input_layernorm.weight"] = f32(p + "attn_norm")
        sd[q + "post_attention_layernorm.weight"] = f32(p + "ffn_norm")
        if p + "attn_qkv" in ff.tensors:
            w, b = tensor_weights(ff, p + "attn_qkv")
            b = np.concatenate([b, np.zeros(w.shape[0] - b.size)])
            parts = np.split(np.arange(w.shape[0]), [H * hd, H * hd + KV * hd])
            for nm, rows in zip(("q_proj", "k_proj", "v_proj"), parts):
                sd[q + f"self_attn.{nm}.weight"] = w[rows]
                sd[q + f"self_attn.{nm}.bias"] = b[rows]
        else:
            for nm, t in zip(("q_proj", "k_proj", "v_proj"), ("attn_q", "attn_k", "attn_v")):
                w, b = tensor_weights(ff, p + t)
                sd[q + f"self_attn.{nm}.weight"] = w
                sd[q + f"self_attn.{nm}.bias"] = np.concatenate([b, np.zeros(w.shape[0] - b.size)])
        sd[q + "self_attn.o_proj.weight"] = tensor_weights(ff, p + "attn_output")[0]
        if p + "ffn_gate_up" in ff.tensors:
            w, _ = tensor_weights(ff, p + "ffn_gate_up")
            sd[q + "mlp.gate_proj.weight"], sd[q + "mlp.up_proj.weight"] = w[:ffn], w[ffn:2 * ffn]
        else:
            sd[q + "mlp.gate_proj.weight"] = tensor_weights(ff, p + "ffn_gate")[0]
            sd[q + "mlp.up_proj.weight"] = tensor_weights(ff, p + "ffn_up")[0]
        sd[q + "mlp.down_proj.weight"] = tensor_weights(ff, p + "ffn_down")[0]
    m.load_state_dict({k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in sd.items()}, strict=True)
    return m


@pytest.mark.parametrize("body_format,fused", [(1, 1), (2, 1), (1, 0)])
def test_oracle_forward_matches_hf_qwen2(tmp_path, body_format, fused):
    import gaje_hip
    vocab, ffn, base = 300, 192, 10000.0
    path = str(tmp_path / "m.flat")
    gaje_hip.synth.write_flat(path, n_embd=128, n_head=4, n_head_kv=2, n_blocks=2, ffn=ffn, vocab_size=vocab,
                              eps=1e-6, rope_base=base, arch_family=1, qkv_bias=1, tied_embeddings=0,
                              body_format=body_format, fused=bool(fused), seed=31)
    r = O.load_genomic(path)
    r.set_k_wta_ratio(0.0)
    m = hf_model(r.flat, r.config, vocab, ffn, base)
    ids = [5, 299, 17, 0, 123, 42]
    with torch.no_grad():
        ref = m(torch.tensor([ids])).logits[0].numpy()
    for i, t in enumerate(ids):
        got = r.forward_core(t, i == 0)
        err = floored_rel_err(got, ref[i])
        assert err < 1e-3, (i, err)
    # a wiring slip is not small: the logits of the wrong position are far off
    assert floored_rel_err(r.forward_core(ids[0], True), ref[1]) > 1e-2


def test_fp64_composition_matches_hf(tmp_path):
    """tests/fp64_model.forward_fp64 (the float64 reference for deep-model noise
    floors) is the same function as HF's Qwen2 in float64.  HF keeps its
    RMSNorm statistics and rotary tables in float32 even in a float64 model,
    which leaves ~1e-7 of the largest logit; a wiring slip is O(1)."""
    import gaje_hip
    vocab, ffn, base = 300, 192, 10000.0
    path = str(tmp_path / "m.flat")
    gaje_hip.synth.write_flat(path, n_embd=128, n_head=4, n_head_kv=2, n_blocks=2, ffn=ffn, vocab_size=vocab,
                              eps=1e-6, rope_base=base, arch_family=1, qkv_bias=1, tied_embeddings=0, seed=31)
    ff = FlatFile(path)
    m = hf_model(ff, ff.model_config(), vocab, ffn, base)
    ids = [5, 299, 17, 0, 123, 42, 7, 7]
    with torch.no_grad():
        ref = m(torch.tensor([ids])).logits[0].numpy()
    got = forward_fp64(ff, ff.model_config(), ids, logits_for="all")
    assert np.max(np.abs(got - ref)) < 1e-6 * np.max(np.abs(ref))
    assert np.allclose(forward_fp64(ff, ff.model_config(), ids), got[-1], rtol=0, atol=1e-12)


def test_genomic_norm_branch_fp64(tmp_path):
    """use_genomic_norm (block/forward.rs:115-123, h_scale 1 from flat_reader.rs:220):
    where the SwiGLU output's rms exceeds 1 it is scaled to rms 1.  The oracle
    against the float64 composition, on a model where the branch fires in
    every block; without the scaling the logits are far off."""
    path = write_genomic_norm_model(str(tmp_path))
    r = O.load_genomic(path)
    r.set_k_wta_ratio(0.0)
    assert r.blocks[0].use_genomic_norm
    ids = [5, 299, 17, 0, 123, 42]
    stats = {}
    ref = forward_fp64(r.flat, r.config, ids, logits_for="all", stats=stats)
    assert stats["gnorm_fired"] >= len(ids) * GNORM_MODEL["n_blocks"] // 2
    for i, t in enumerate(ids):
        err = floored_rel_err(r.forward_core(t, i == 0), ref[i])
        assert err < 1e-3, (i, err)
    import copy
    cfg = copy.deepcopy(r.config)
    cfg.config["use_genomic_norm"] = False
    off = forward_fp64(r.flat, cfg, ids, logits_for="all")
    assert floored_rel_err(off[-1], ref[-1]) > 1e-2
