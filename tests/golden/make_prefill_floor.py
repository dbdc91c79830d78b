"""Writes prefill_floor_qwen2.5-1.5b_512.npz: the float64 noise floor of the
28-layer, 512-token Qwen2.5-1.5B-shape prompt that the MFMA prefill test runs.

The reference feeds a prompt through forward_core one token at a time
(src/nn/llm/forward.rs:229-232); the oracle restates that in float32, bit for
bit.  tests/fp64_model.forward_fp64 computes the same function in float64 with
the file's weights dequantised exactly and the reference's float32 RoPE angles
(theta = f32(pos) * f32 freq, attention.rs:66-67: part of the function the
reference defines, and identical in every float32 path here).  The floored
relative error between
the two at the last token's logits is the oracle's own float32 noise at this
depth: a float32 computation in any other summation order cannot be expected
to land closer to the oracle than that.

With exact angles instead the distance is 1.9e-2: the angles' float32
rounding at positions up to 511 dominates it, and it is not summation noise.

Stored: the float64 logits (rounded to float32, 6e-8 relative, far below the
floor), the floor, and the oracle's top-2 logits and argmax.

Run from the repository root:  python tests/golden/make_prefill_floor.py
(the HIP library's host code writes the synthetic model; ~2 minutes on 8 CPUs).
"""
import os
import sys
import tempfile
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [REPO, os.path.join(REPO, "gaje-semantic-compression_amd"), os.path.dirname(HERE)]

import gaje_hip  # noqa: E402
from conftest import floored_rel_err  # noqa: E402
from fp64_model import forward_fp64  # noqa: E402
from oracle import oracle as O  # noqa: E402

PRESET, SEED, PROMPT_SEED, PROMPT_LEN = "qwen2.5-1.5b", 0, 10, 512
OUT = os.path.join(HERE, "prefill_floor_qwen2.5-1.5b_512.npz")


def main():
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "m.flat")
        gaje_hip.synth.write_flat(path, preset=PRESET, seed=SEED)
        r = O.load_genomic(path)
        r.set_k_wta_ratio(0.0)
        prompt = np.random.default_rng(PROMPT_SEED).integers(0, r.vocab_size, PROMPT_LEN).astype(np.uint32)
        t = time.time()
        for i, tok in enumerate(prompt):
            last = r.forward_core(int(tok), i == 0)
        print(f"oracle: {time.time() - t:.1f} s", flush=True)
        t = time.time()
        ref64 = forward_fp64(r.flat, r.config, prompt, f32_angles=True)
        print(f"float64 composition: {time.time() - t:.1f} s", flush=True)
    floor = floored_rel_err(last, ref64)
    top = np.sort(last)[::-1][:2]
    print(f"floor {floor:.3e}; oracle argmax {O.argmax_first(last)}, float64 argmax {int(np.argmax(ref64))}; "
          f"top-2 margin {(top[0] - top[1]) / abs(top[0]):.3e}")
    np.savez_compressed(OUT, logits_fp64=ref64.astype(np.float32), floor=np.float64(floor),
                        oracle_top2=top.astype(np.float32), oracle_argmax=np.int64(O.argmax_first(last)),
                        prompt=prompt, preset=np.array(PRESET), seed=np.int64(SEED))
    print("wrote", OUT)


if __name__ == "__main__":
    main()
