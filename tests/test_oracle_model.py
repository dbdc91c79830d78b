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

from conftest import floored_rel_err

torch = pytest.importorskip("torch")
transformers = pytest.importorskip("transformers")

from oracle import oracle as O  # noqa: E402
from oracle.flat import FlatFile  # noqa: E402


def tensor_weights(ff: FlatFile, name: str):
    """Exact float64 weights [out][in] and bias of a flat tensor."""
    e = ff.tensors[name]
    n, k = e["out_features"], e["in_features"]
    dna = np.asarray(ff.get_slice(e["dna_off"], e["dna_len"]))
    bias = ff.get_f32_slice(e["bias_off"], e["bias_len"]).astype(np.float64)
    if e["bit_depth"] == 32:
        w = np.frombuffer(dna.tobytes(), np.float32)[: n * k].reshape(n, k).astype(np.float64)
        return w, bias
    nb = k // 32
    if e["c_len"] == 0:  # Q4_0 blocks: q * scale + min exactly (f16 scale / min)
        b = dna[: n * nb * 20].reshape(n * nb, 20)
        sc = b[:, 0:2].copy().view(np.float16).astype(np.float64)
        mn = b[:, 2:4].copy().view(np.float16).astype(np.float64)
        q = np.empty((n * nb, 32))
        q[:, 0::2], q[:, 1::2] = b[:, 4:] & 15, b[:, 4:] >> 4
        return (q * sc + mn).reshape(n, k), bias
    # LUT 4-bit: high nibble = even element; tables expanded as init.rs:109-124
    t = ff.get_f32_slice(e["c_off"], e["c_len"]).astype(np.float64)
    if t.size == 16:
        t = np.tile(t, n * nb)
    elif t.size == nb * 16:
        t = np.tile(t, n)
    t = t[: n * nb * 16].reshape(n * nb, 16)
    c = dna[: n * nb * 16].reshape(n * nb, 16)
    idx = np.empty((n * nb, 32), np.int64)
    idx[:, 0::2], idx[:, 1::2] = c >> 4, c & 15
    return np.take_along_axis(t, idx, axis=1).reshape(n, k), bias


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
