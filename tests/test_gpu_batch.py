"""GPU parity of the batched decode (gaje_hip_batch_*) against the CPU oracle.

A batch of n sequences is n independent GenomicLLM instances stepping
together (the reference has no batched path; its oracle is n sequential
forward_core runs).  The batched matvecs run every sequence's accumulation
chains in the batch-1 order, so each sequence's logits must equal the oracle's
bit for bit and greedy decoding must give the same tokens.
"""
import os
import struct

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TINY = dict(n_embd=128, n_head=4, n_head_kv=2, n_blocks=2, ffn=256, vocab_size=1000, eps=1e-6,
            rope_base=1e4, arch_family=1, qkv_bias=1, tied_embeddings=0)
HD64 = dict(n_embd=256, n_head=4, n_head_kv=2, n_blocks=2, ffn=512, vocab_size=1000, eps=1e-6,
            rope_base=1e4, arch_family=1, qkv_bias=1, tied_embeddings=0)
# gate/up rows >= 16384: the two-rows-per-lane batched matvec
WIDE = dict(n_embd=128, n_head=4, n_head_kv=2, n_blocks=1, ffn=8192, vocab_size=1000, eps=1e-6,
            rope_base=1e4, arch_family=1, qkv_bias=1, tied_embeddings=0)
# the same rows with K = 1024: the two-rows-per-lane matvec over two activation chunks
WIDE_K = dict(n_embd=1024, n_head=8, n_head_kv=2, n_blocks=1, ffn=8192, vocab_size=1000, eps=1e-6,
              rope_base=1e4, arch_family=1, qkv_bias=1, tied_embeddings=0)
HD128 = dict(n_embd=256, n_head=2, n_head_kv=1, n_blocks=1, ffn=256, vocab_size=512, eps=1e-6,
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


def same_bits(a, b) -> bool:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _prompts(n_seq, lengths, vocab, seed):
    rng = np.random.default_rng(seed)
    return [[int(t) for t in rng.integers(0, vocab, lengths[s % len(lengths)])] for s in range(n_seq)]


def _padded(prompts, inactive):
    """Left-aligned [n_seq][max_len] ids; shorter prompts end in inactive steps."""
    n = max(len(p) for p in prompts)
    ids = np.full((len(prompts), n), inactive, np.uint32)
    for s, p in enumerate(prompts):
        ids[s, :len(p)] = p
    return ids


def _oracle_run(O, path, prompt, n_gen):
    r = O.load_genomic(path)
    r.set_k_wta_ratio(0.0)
    r.clear_cache_core()
    last = None
    for t in prompt:
        last = r.forward_core(int(t))
    toks = []
    tok = O.argmax_first(last)
    for _ in range(n_gen):
        toks.append(tok)
        tok = O.argmax_first(r.forward_core(tok))
    return last, toks


@pytest.mark.parametrize("cfg,name,n_seq,lengths", [(TINY, "tiny", 3, [5, 9, 7]), (HD64, "hd64", 5, [12, 4, 8]),
                                                    (HD64, "hd64", 16, [6]), (TINY, "tiny", 1, [10]),
                                                    (WIDE, "wide", 16, [5, 3]), (WIDE, "wide", 8, [4]),
                                                    (WIDE_K, "widek", 16, [4, 2]), (WIDE_K, "widek", 11, [3])])
def test_batch_matches_independent_runs(hip, O, tmp_models, cfg, name, n_seq, lengths):
    p = _write(hip, tmp_models / f"batch_{name}.flat", seed=21, **cfg)
    prompts = _prompts(n_seq, lengths, cfg["vocab_size"], 22 + n_seq)
    g = hip.load_genomic_auto(p)
    g.set_k_wta_ratio(0.0)
    b = hip.GenomicBatch(g, n_seq, 64)
    ids = _padded(prompts, hip.BATCH_INACTIVE)
    # the sequences whose prompt ends on the last step report their logits there
    logits = b.feed(ids, want_logits=True)
    for s, pr in enumerate(prompts):
        assert b.cache_len(s) == len(pr)
    n_gen = 8
    firsts = []
    refs = []
    for s, pr in enumerate(prompts):
        last, toks = _oracle_run(O, p, pr, n_gen)
        refs.append(toks)
        firsts.append(toks[0])
        if len(pr) == ids.shape[1]:
            assert same_bits(logits[s], last), f"sequence {s}: last prompt logits differ"
    out = b.decode_greedy(firsts, n_gen)
    for s in range(n_seq):
        # out[s][i] is the argmax after feeding refs[s][i]: the oracle's token i+1
        assert list(out[s][:n_gen - 1]) == refs[s][1:], f"sequence {s}"
        assert b.cache_len(s) == len(prompts[s]) + n_gen
    b.close()
    g.close()


@pytest.mark.parametrize("lengths", [[300, 140, 7], [1, 129, 257, 64]])
def test_batch_long_context_hd128(hip, O, tmp_models, lengths):
    """128-wide heads at contexts of several key rounds and V blocks, ragged across the batch."""
    p = _write(hip, tmp_models / "batch_hd128.flat", seed=23, **HD128)
    prompts = _prompts(len(lengths), lengths, HD128["vocab_size"], 24)
    g = hip.load_genomic_auto(p)
    g.set_k_wta_ratio(0.0)
    b = hip.GenomicBatch(g, len(lengths), 320)
    b.feed(_padded(prompts, hip.BATCH_INACTIVE))
    n_gen = 6
    firsts, refs = [], []
    for pr in prompts:
        _, toks = _oracle_run(O, p, pr, n_gen)
        firsts.append(toks[0])
        refs.append(toks)
    out = b.decode_greedy(firsts, n_gen)
    for s in range(len(prompts)):
        assert list(out[s][:n_gen - 1]) == refs[s][1:], f"sequence {s}"
    b.close()
    g.close()


@pytest.mark.parametrize("n_seq", [4, 11, 16])
def test_batch_benchmark_shape(hip, O, tmp_models, n_seq):
    """The Qwen2.5-1.5B block shapes (hd 128, GQA 6:1, ffn 8960, QKV bias), two blocks; at 16 and
    11 sequences the 17920-row gate_up runs the two-rows-per-lane matvec over three chunks."""
    p = _write(hip, tmp_models / "batch_c3_2blk.flat", preset="qwen2.5-1.5b", seed=0, n_blocks=2,
               vocab_size=4096)
    prompts = _prompts(n_seq, [12], 4096, 31)
    g = hip.load_genomic_auto(p)
    g.set_k_wta_ratio(0.0)
    b = hip.GenomicBatch(g, n_seq, 128)
    logits = b.feed(_padded(prompts, hip.BATCH_INACTIVE), want_logits=True)
    firsts = []
    refs = []
    for s, pr in enumerate(prompts):
        last, toks = _oracle_run(O, p, pr, 4)
        assert same_bits(logits[s], last), f"sequence {s}"
        firsts.append(toks[0])
        refs.append(toks)
    out = b.decode_greedy(firsts, 4)
    for s in range(n_seq):
        assert list(out[s][:3]) == refs[s][1:], f"sequence {s}"
    b.close()
    g.close()


def test_batch_reset_and_capacity(hip, O, tmp_models):
    from gaje_hip._lib import GajeError
    p = _write(hip, tmp_models / "batch_tiny.flat", seed=21, **TINY)
    g = hip.load_genomic_auto(p)
    g.set_k_wta_ratio(0.0)
    b = hip.GenomicBatch(g, 2, 16)  # capacity rounds up to 64
    prompts = _prompts(2, [5], TINY["vocab_size"], 41)
    b.feed(np.array(prompts, np.uint32))
    b.reset(1)
    assert b.cache_len(0) == 5 and b.cache_len(1) == 0
    logits = b.feed(np.array([[3], [prompts[1][0]]], np.uint32), want_logits=True)
    r = O.load_genomic(p)
    r.set_k_wta_ratio(0.0)
    assert same_bits(logits[1], r.forward_core(prompts[1][0], True))
    with pytest.raises(GajeError):
        b.decode_greedy([1, 2], 100)  # past the capacity
    b.close()
    g.close()


def test_batch_nan_guard_halts_one_sequence(hip, O, tmp_models):
    from oracle.flat import FlatFile
    base = _write(hip, tmp_models / "batch_tiny.flat", seed=21, **TINY)
    p = str(tmp_models / "batch_nan.flat")
    data = bytearray(open(base, "rb").read())
    ff = FlatFile(base)
    e = ff.tensors["token_embd"]
    off = ff.weights_offset + e["dna_off"] + 42 * TINY["n_embd"] * 4
    data[off:off + 4] = struct.pack("<f", float("nan"))
    open(p, "wb").write(bytes(data))
    g = hip.load_genomic_auto(p)
    g.set_k_wta_ratio(0.0)
    b = hip.GenomicBatch(g, 2, 64)
    logits, status, rc = b.feed(np.array([[5, 6], [7, 42]], np.uint32), want_logits=True, status=True)
    assert rc != 0 and status[0] == 0 and status[1] == 1  # stage 0 ("Input x is NaN") + 1
    assert b.cache_len(0) == 2 and b.cache_len(1) == 1
    r = O.load_genomic(p)
    r.set_k_wta_ratio(0.0)
    r.forward_core(5, True)
    assert same_bits(logits[0], r.forward_core(6))
    b.close()
    lut = _write(hip, tmp_models / "batch_lut.flat", seed=6, body_format=hip.synth.LUT4, **TINY)
    g2 = hip.load_genomic_auto(lut)
    with pytest.raises(Exception):
        hip.GenomicBatch(g2, 2, 64)
    g2.close()
    g.close()
