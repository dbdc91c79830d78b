"""GPU parity of the whole decode path against the CPU oracle.

The device path reproduces the reference's rounding sequence end to end
(matvec accumulation orders, RMSNorm, RoPE table, glibc expf, the serial softmax
sums), so logits must match the oracle bit for bit and greedy decoding must
produce the same tokens.  That is stricter than the task's bars (floored max
relative error <= 1e-4 on logits, argmax agreement where the top-2 margin exceeds
the tolerance); the floored error is printed for information.
"""
import os
import struct

import numpy as np
import pytest

from conftest import floored_rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-4

TINY = dict(n_embd=128, n_head=4, n_head_kv=2, n_blocks=2, ffn=256, vocab_size=1000, eps=1e-6,
            rope_base=1e4, arch_family=1, qkv_bias=1, tied_embeddings=0)


@pytest.fixture(scope="module")
def hip():
    import gaje_hip
    if gaje_hip.ops.device_count() < 1:
        pytest.fail("no HIP device visible")
    return gaje_hip


@pytest.fixture(scope="module")
def O():
    from oracle import oracle
    return oracle


def _write(hip, path, **kw):
    if not os.path.exists(path):
        hip.synth.write_flat(str(path), **kw)
    return str(path)


@pytest.fixture(scope="module")
def tiny(hip, tmp_models):
    return _write(hip, tmp_models / "tiny_q4.flat", seed=3, **TINY)


def _margin_ok(logits, tol=TOL):
    """True if the top-2 margin of the reference logits exceeds tol * |top1|."""
    v = np.sort(np.where(np.isnan(logits), -np.inf, logits))[::-1]
    return (v[0] - v[1]) > tol * abs(v[0])


def same_bits(a, b) -> bool:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _tokens(n, vocab, seed):
    return [int(t) for t in np.random.default_rng(seed).integers(0, vocab, n)]


def _compare_stream(hip, O, path, tokens, kwta=0.0, hidden=False):
    g = hip.load_genomic_auto(path)
    r = O.load_genomic(path)
    g.set_k_wta_ratio(kwta)
    r.set_k_wta_ratio(kwta)
    worst = 0.0
    for i, t in enumerate(tokens):
        if hidden:
            gl, gh = g.forward_with_hidden(t, i == 0)
            rl, rh = r.forward_with_hidden_core(t, i == 0)
            assert same_bits(gh, rh), f"h_norm differs at token {i}"
        else:
            gl = g.forward(t, i == 0)
            rl = r.forward_core(t, i == 0)
        worst = max(worst, floored_rel_err(gl, rl))
        assert same_bits(gl, rl), f"logits differ at token {i} (floored rel err {worst:.2e})"
    assert g.cache_len() == len(tokens) == r.blocks[0].attn.k_cache_len()
    g.close()
    return worst


def test_tiny_logits_stream(hip, O, tiny):
    err = _compare_stream(hip, O, tiny, _tokens(24, TINY["vocab_size"], 1))
    print(f"tiny logits worst err {err:.3e}")
    assert err <= TOL


def test_tiny_forward_with_hidden(hip, O, tiny):
    err = _compare_stream(hip, O, tiny, _tokens(6, TINY["vocab_size"], 2), hidden=True)
    assert err <= TOL


def test_tiny_kwta_logits(hip, O, tiny):
    """K-WTA on (the flat-load default 0.5, flat_reader.rs:234)."""
    g = hip.load_genomic_auto(tiny)
    r = O.load_genomic(tiny)
    assert abs(g.k_wta_ratio - 0.5) < 1e-7 and r.k_wta_ratio == 0.5
    for i, t in enumerate(_tokens(5, TINY["vocab_size"], 3)):
        gl = g.forward(t, i == 0)
        rl = r.forward_core(t, i == 0)
        assert (rl == np.float32(-1e9)).sum() == TINY["vocab_size"] // 2
        assert same_bits(gl, rl)
    g.close()


def test_tiny_block_kwta(hip, O, tiny):
    """set_k_wta_ratio also filters every block output (python.rs:55-57)."""
    g = hip.load_genomic_auto(tiny)
    r = O.load_genomic(tiny)
    g.set_k_wta_ratio(0.75)
    r.set_k_wta_ratio(0.75)
    for i, t in enumerate([7, 11, 13]):
        gl = g.forward(t, i == 0)
        rl = r.forward_core(t, i == 0)
        assert same_bits(gl, rl)
    g.close()


def test_tiny_block_kwta_ratio_change(hip, O, tiny):
    """Changing the ratio on one handle changes the blocks' k (block/forward.rs:144-148)
    in the captured token step: 0.75, decode, 0.25, decode, then off."""
    g = hip.load_genomic_auto(tiny)
    r = O.load_genomic(tiny)
    toks = _tokens(9, TINY["vocab_size"], 12)
    for j, ratio in enumerate((0.75, 0.25, 0.0, 0.75)):
        g.set_k_wta_ratio(ratio)
        r.set_k_wta_ratio(ratio)
        for i, t in enumerate(toks[j * 2:j * 2 + 3]):
            gl = g.forward(t, j == 0 and i == 0)
            rl = r.forward_core(t, j == 0 and i == 0)
            assert same_bits(gl, rl), f"ratio {ratio}: logits differ at token {i}"
        # the greedy loop replays the same graph
        out = g.decode_greedy(toks[j], 2)
        feed = int(toks[j])
        for tok in out:
            assert int(tok) == O.argmax_first(r.forward_core(feed, False))
            feed = int(tok)
    g.close()


def _check_greedy(gen, O, path, first, n, prompt=None):
    r = O.load_genomic(path)
    r.set_k_wta_ratio(0.0)
    if prompt is not None:
        for i, t in enumerate(prompt):
            r.forward_core(t, i == 0)
    tok = first
    for i in range(n):
        logits = r.forward_core(tok, prompt is None and i == 0)
        ref = O.argmax_first(logits)
        assert gen[i] == ref, f"greedy token differs at step {i} (margin ok: {_margin_ok(logits)})"
        tok = ref
    return n


def test_tiny_decode_greedy(hip, O, tiny):
    g = hip.load_genomic_auto(tiny)
    g.set_k_wta_ratio(0.0)
    g.clear_cache_py()
    out = g.decode_greedy(17, 40)
    assert g.cache_len() == 40
    matched = _check_greedy(out, O, tiny, 17, 40)
    print(f"greedy steps matched: {matched}/40")
    g.close()


def test_tiny_prefill_truncate_decode(hip, O, tiny):
    prompt = _tokens(20, TINY["vocab_size"], 4)
    g = hip.load_genomic_auto(tiny)
    g.set_k_wta_ratio(0.0)
    g.clear_cache_py()
    g.prefill(prompt)
    assert g.cache_len() == 20
    a = g.decode_greedy(prompt[-1], 12)
    g.truncate_cache(20)
    b = g.decode_greedy(prompt[-1], 12)
    assert np.array_equal(a, b), "replay from the same prompt state must be identical"
    _check_greedy(a, O, tiny, prompt[-1], 12, prompt=prompt)
    nxt = g.greedy_next(int(b[-1]))
    assert g.cache_len() == 33
    assert 0 <= nxt < TINY["vocab_size"]
    g.close()


def test_tiny_generate_greedy_matches_oracle(hip, O, tiny):
    """generate_native_core: penalty, greedy argmax, EOS and the loop detector."""
    prompt = _tokens(8, TINY["vocab_size"], 5)
    penalty = 1.3
    g = hip.load_genomic_auto(tiny)
    r = O.load_genomic(tiny)
    got = g.generate_native_py(prompt, max_new_tokens=40, temperature=0.0,
                               repetition_penalty=penalty, eos_token_ids=[2])
    ref = r.generate_native_core(prompt, 40, 0.0, penalty, [2])
    print(f"generate: {len(got)} vs {len(ref)} tokens")
    assert got == ref
    g.close()


def _oracle_generate(O, path, prompt, max_new, penalty, eos, kwta):
    r = O.load_genomic(path)
    r.set_k_wta_ratio(kwta)
    out = r.generate_native_core(prompt, max_new, 0.0, penalty, eos)
    return out, r.blocks[0].attn.k_cache_len()


@pytest.mark.parametrize("penalty,kwta,max_new", [(1.3, 0.0, 40), (1.15, 0.5, 70), (1.0, 0.0, 70),
                                                  (1.0, 0.5, 33), (2.5, 0.25, 100)])
def test_tiny_generate_device_loop(hip, O, tiny, penalty, kwta, max_new):
    """The greedy loop on the device (penalty over the K-WTA-filtered logits, EOS, the
    loop detector, chunks of 32 steps): the oracle's tokens and cache length."""
    prompt = _tokens(9, TINY["vocab_size"], 13)
    g = hip.load_genomic_auto(tiny)
    g.set_k_wta_ratio(kwta)
    ref, ref_len = _oracle_generate(O, tiny, prompt, max_new, penalty, [2], kwta)
    got = g.generate_native_py(prompt, max_new_tokens=max_new, temperature=0.0, repetition_penalty=penalty,
                               eos_token_ids=[2])
    print(f"generate penalty {penalty} kwta {kwta}: {len(got)} tokens, ref {len(ref)}")
    assert got == ref
    assert g.cache_len() == ref_len
    g.close()


def test_tiny_generate_eos_and_host_path(hip, O, tiny):
    """An EOS id the stream reaches ends the loop there (the EOS is returned, not fed);
    more EOS ids than the device list holds take the host loop, with the same tokens."""
    prompt = _tokens(7, TINY["vocab_size"], 14)
    g = hip.load_genomic_auto(tiny)
    g.set_k_wta_ratio(0.0)
    free = g.generate_native_py(prompt, max_new_tokens=20, temperature=0.0, repetition_penalty=1.4,
                                eos_token_ids=[])
    eos = free[4]
    cut = free[:free.index(eos) + 1]
    ref, ref_len = _oracle_generate(O, tiny, prompt, 20, 1.4, [eos], 0.0)
    assert ref == cut
    got = g.generate_native_py(prompt, max_new_tokens=20, temperature=0.0, repetition_penalty=1.4,
                               eos_token_ids=[eos])
    assert got == ref and g.cache_len() == ref_len == len(prompt) + len(ref) - 1
    many = [eos] + list(range(TINY["vocab_size"] - 80, TINY["vocab_size"]))
    ref2, _ = _oracle_generate(O, tiny, prompt, 20, 1.4, many, 0.0)
    assert g.generate_native_py(prompt, max_new_tokens=20, temperature=0.0, repetition_penalty=1.4,
                                eos_token_ids=many) == ref2
    g.close()


@pytest.mark.parametrize("temperature,penalty,kwta,seed", [(0.7, 1.0, 0.0, 0), (0.7, 1.3, 0.0, 11),
                                                            (1.5, 1.1, 0.5, 42), (0.05, 1.0, 0.0, 5)])
def test_tiny_generate_sampling_matches_oracle(hip, O, tiny, temperature, penalty, kwta, seed):
    """The multinomial branch (forward.rs:272-297) with the device library's
    seeded splitmix draws: the oracle, handed the same draw stream, samples the
    same tokens, since the logits are the same bits and the exponentials, the
    sequential sum and the running-sum search are the reference's."""
    prompt = _tokens(6, TINY["vocab_size"], 21)
    g = hip.load_genomic_auto(tiny)
    g.set_k_wta_ratio(kwta)
    r = O.load_genomic(tiny)
    r.set_k_wta_ratio(kwta)
    got = g.generate_native_py(prompt, max_new_tokens=40, temperature=temperature,
                               repetition_penalty=penalty, eos_token_ids=[2], seed=seed)
    ref = r.generate_native_core(prompt, 40, temperature, penalty, [2], rng=O.SplitMixDraws(seed))
    print(f"sampling T={temperature} penalty={penalty} kwta={kwta}: {len(got)} tokens, {len(set(got))} distinct")
    assert got == ref
    assert g.cache_len() == r.blocks[0].attn.k_cache_len()
    g.close()


def test_tiny_generate_empty_prompt_error(hip, tiny):
    g = hip.load_genomic_auto(tiny)
    with pytest.raises(ValueError, match="Prompt tokens cannot be empty"):
        g.generate_native_py([], max_new_tokens=3)
    g.close()


def test_split_tensors_and_lut_body(hip, O, tmp_models):
    p1 = _write(hip, tmp_models / "tiny_split.flat", seed=5, fused=False, **TINY)
    assert _compare_stream(hip, O, p1, _tokens(10, TINY["vocab_size"], 6)) <= TOL
    p2 = _write(hip, tmp_models / "tiny_lut.flat", seed=6, body_format=hip.synth.LUT4, **TINY)
    assert _compare_stream(hip, O, p2, _tokens(10, TINY["vocab_size"], 7)) <= TOL


def test_json_config_interleaved_rope_genomic_norm(hip, O, tmp_models):
    """arch_family 0: shapes, rope_base and rope_style come from the metadata
    JSON; interleaved RoPE pairs (2i, 2i+1); use_genomic_norm scales ffn_out."""
    kw = dict(TINY)
    kw.update(arch_family=0, rope_base=5e5, rope_interleaved=1, use_genomic_norm=1)
    p = _write(hip, tmp_models / "tiny_json.flat", seed=8, **kw)
    r = O.load_genomic(p)
    assert r.config.config["rope_style"] == "interleaved" and r.blocks[0].use_genomic_norm
    assert _compare_stream(hip, O, p, _tokens(8, TINY["vocab_size"], 8)) <= TOL


def test_genomic_norm_branch_fires(hip, O, tmp_models):
    """use_genomic_norm where its scaling fires (rms > h_scale in most blocks):
    bit for bit with the oracle, whose branch a float64 composition pins
    (tests/test_oracle_model.py)."""
    from conftest import write_genomic_norm_model
    p = write_genomic_norm_model(str(tmp_models))
    assert _compare_stream(hip, O, p, _tokens(10, 300, 31)) == 0.0


def test_nan_embedding_row_raises(hip, O, tmp_models, tiny):
    from oracle.flat import FlatFile
    p = str(tmp_models / "tiny_nan.flat")
    data = bytearray(open(tiny, "rb").read())
    ff = FlatFile(tiny)
    e = ff.tensors["token_embd"]
    off = ff.weights_offset + e["dna_off"] + 42 * TINY["n_embd"] * 4
    data[off:off + 4] = struct.pack("<f", float("nan"))
    open(p, "wb").write(bytes(data))
    g = hip.load_genomic_auto(p)
    r = O.load_genomic(p)
    with pytest.raises(ValueError, match="Input x is NaN"):
        r.forward_core(42, True)
    with pytest.raises(ValueError, match="Input x is NaN"):
        g.forward(42, True)
    # a clean token afterwards works (the halted state is cleared per call)
    g.set_k_wta_ratio(0.0)
    r.set_k_wta_ratio(0.0)
    assert same_bits(g.forward(5, True), r.forward_core(5, True))
    g.close()


def test_kv_growth_preserves_cache(hip, O, tiny):
    tokens = _tokens(12, TINY["vocab_size"], 9)
    g = hip.load_genomic_auto(tiny)
    r = O.load_genomic(tiny)
    g.set_k_wta_ratio(0.0)
    r.set_k_wta_ratio(0.0)
    for i, t in enumerate(tokens):
        if i == 6:
            g.reserve(5000)  # reallocates and copies the cache mid-sequence
        assert same_bits(g.forward(t, i == 0), r.forward_core(t, i == 0))
    g.close()


def test_bad_files(hip, tmp_models, tiny):
    bad = tmp_models / "bad_magic.flat"
    bad.write_bytes(b"XGAJ" + bytes(5000))
    with pytest.raises(OSError, match="Invalid magic"):
        hip.load_genomic_auto(str(bad))
    short = tmp_models / "short.flat"
    short.write_bytes(b"GAJE" + bytes(100))
    with pytest.raises(OSError, match="less than 4096"):
        hip.load_genomic_auto(str(short))
    with pytest.raises(OSError):
        hip.load_genomic_auto(str(tmp_models / "missing.flat"))


@pytest.mark.parametrize("preset,ntok", [("smollm2-135m", 4), ("qwen2-0.5b", 3)])
def test_benchmark_shapes(hip, O, tmp_models, preset, ntok):
    p = _write(hip, tmp_models / f"{preset}.flat", preset=preset, seed=0)
    vocab = hip.synth.PRESETS[preset]["vocab_size"]
    err = _compare_stream(hip, O, p, _tokens(ntok, vocab, 10))
    print(f"{preset}: worst logits err {err:.3e}")
    assert err <= TOL
