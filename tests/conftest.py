"""Shared test setup.

Tests marked `gpu` need an MI355X and the built lib/libgaje_hip.so; everything
else runs on the CPU (oracle against the reference's known answers, the reader,
host logic, and the C-ABI symbol table).
"""
import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "gaje-semantic-compression_amd")
for p in (REPO, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


def floored_rel_err(got, ref) -> float:
    """max_i |got_i - ref_i| / max(|ref_i|, tau) with tau = 1e-3 * max|ref|.

    A plain elementwise relative error is ill-posed for these outputs: the
    reference flushes |t| < 1e-6 to 0 and summation-order noise dominates near
    zero, so the denominator is floored at a thousandth of the largest output.
    """
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if ref.size == 0:
        return 0.0
    tau = 1e-3 * float(np.max(np.abs(ref)))
    den = np.maximum(np.abs(ref), tau)
    den[den == 0] = 1.0
    return float(np.max(np.abs(got - ref) / den))


@pytest.fixture(scope="session")
def tmp_models(tmp_path_factory):
    """Directory for synthetic .gaje.flat files written during the session."""
    return tmp_path_factory.mktemp("models")


def scale_ffn_norms(path: str, out: str, factor: float) -> str:
    """A copy of a flat file whose ffn_norm weights are multiplied by factor."""
    from oracle.flat import FlatFile
    ff = FlatFile(path)
    data = bytearray(open(path, "rb").read())
    for name, e in ff.tensors.items():
        if name.endswith(".ffn_norm"):
            off = ff.weights_offset + e["dna_off"]
            w = np.frombuffer(bytes(data[off:off + e["dna_len"]]), np.float32) * np.float32(factor)
            data[off:off + e["dna_len"]] = w.astype(np.float32).tobytes()
    open(out, "wb").write(bytes(data))
    return out


# a model whose metadata sets use_genomic_norm, with interleaved RoPE from the JSON
GNORM_MODEL = dict(n_embd=128, n_head=4, n_head_kv=2, n_blocks=3, ffn=192, vocab_size=300, eps=1e-6,
                   rope_base=5e5, arch_family=0, rope_interleaved=1, use_genomic_norm=1, qkv_bias=1,
                   tied_embeddings=0)


def write_genomic_norm_model(directory: str, seed: int = 8) -> str:
    """GNORM_MODEL with its ffn_norm weights scaled 12x, so that the SwiGLU
    output's rms exceeds h_scale = 1 and use_genomic_norm's scaling fires
    (with the synthetic recipe's unit norms it never would)."""
    import gaje_hip
    raw = os.path.join(directory, f"gnorm_raw_{seed}.flat")
    gaje_hip.synth.write_flat(raw, seed=seed, **GNORM_MODEL)
    return scale_ffn_norms(raw, os.path.join(directory, f"gnorm_{seed}.flat"), 12.0)
