#!/usr/bin/env python3
"""Decode benchmark of the MI355X GAJE path on one GPU.

Workload (the metric's configuration): a random-init Qwen2-0.5B-shaped model
(hidden 896, 24 layers, 14/2 heads, ffn 4864, vocab 151936, Q4_0 body, f32
token_embd / lm_head, QKV bias), batch-1 greedy decode.  One step = the
fixed-length argmax -> forward loop of benchmarks/performance/gaje_flat_benchmark.py:94-96
for 256 tokens from the state after a 512-token prompt (KV cache 512 -> 768),
K-WTA off as in benchmarks/performance/bench_decode.py:158-159.  The prompt is
prefilled once before timing; every step rewinds the cache to the prompt.

Also reported on the same run:
  - per-stage device time of the exact kernels of the decode step (HIP events
    on the model stream) and the roofline of the dominant one;
  - the single Q4_0 matvec at K=896, N=4864 (the C0 shape), cycling 128 weight
    copies (348 MB, beyond the 256 MB last-level cache) and hot in cache;
  - the CPU oracle (AVX2 restatement of the reference kernels) on the host cores.

Secondary workloads (same JSON line, under "workloads"):
  - Qwen2.5-1.5B-shaped (hidden 1536, 28 layers, 12/2 heads, ffn 8960,
    vocab 151936) 512-token prompt prefill on the MFMA units, and batch-16
    greedy decode (each sequence fed a 1024-token random context, then 128
    steps, bit-exact per sequence);
  - a Q4_0 MoE SwiGLU FFN layer: hidden 1536, 8 experts of ffn 4096, top-2,
    256 tokens.

Prints ONE JSON line on stdout; progress goes to stderr.
"""
import argparse
import json
import os
import sys
import tempfile
import time

REPO = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(REPO, "gaje-semantic-compression_amd")
for _p in (REPO, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E, published
METRIC = "Q4_0 GEMV HBM GB/s (% of peak); decode tok/s, Qwen2-0.5B shape, batch 1"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def model_path(preset: str, seed: int, d: str, quant_embed: int = 0, body_format: int = 1) -> str:
    from gaje_hip import synth
    tag = ("_q8embed" if quant_embed else "") + ("_2bit" if body_format == synth.BIT2 else "")
    path = os.path.join(d, f"gaje_{preset}_s{seed}{tag}.flat")
    if not os.path.exists(path):
        t = time.perf_counter()
        synth.write_flat(path + ".tmp", preset=preset, seed=seed, quant_embed=quant_embed, body_format=body_format)
        os.replace(path + ".tmp", path)
        log(f"[bench] wrote {path} ({os.path.getsize(path) / 1e9:.2f} GB) in {time.perf_counter() - t:.1f}s")
    return path


def q4_gemv_c0(iters: int = 1024, hot: bool = True, stream: bool = True):
    """The C0 matvec: Q4_0 K=896 N=4864, cold (128 copies) and hot (1 copy); the
    launch floors of its grid; and one launch over all 128 copies as a single
    622,592-row matrix (348 MB), the kernel's streaming rate."""
    from gaje_hip import ops, synth
    n, k = 4864, 896
    blocks = synth.q4_0_tensor(0, "c0.gemv", n, k)
    wbytes = n * ((k + 127) // 128) * 80  # the same 2,723,840 bytes, GEMV order
    packed = ops.q4_0_upload(blocks, n, k).read(np.uint8)[:wbytes]
    stride = (wbytes + 255) // 256 * 256
    copies = 128
    w = ops.DeviceBuffer(stride * copies + 4096)  # + the tail the prefetch ring may read past the last row
    host = np.zeros(stride * copies + 4096, dtype=np.uint8)
    for c in range(copies):
        host[c * stride:c * stride + wbytes] = packed
    w.write(host)
    del host
    x = ops.DeviceBuffer.from_array(synth.normal(0, "c0.x", k))
    y = ops.DeviceBuffer(n * copies * 4)
    algo = blocks.nbytes + k * 4 + n * 4  # weights + x + y
    cold_ms = ops.bench_gemv(1, w, stride, copies, x, y, n, k, iters)
    hot_ms = ops.bench_gemv(1, w, stride, 1, x, y, n, k, iters) if hot else None
    # floors of a launch with the C0 grid (n rows x 8 chain lanes, 256 threads)
    grid = (n * 8 + 255) // 256
    empty_ms = ops.bench_floor(None, 0, grid, 256, iters)
    read_ms = ops.bench_floor(w, packed.nbytes, 256, 256, iters)
    out = dict(shape="N=4864 K=896 (Q4_0Block 20 B / 32 weights, packed on device)", algorithmic_bytes=algo,
               launches=iters, cold_us=cold_ms * 1e3, cold_GBps=algo / (cold_ms * 1e-3) / 1e9,
               cold_frac=algo / (cold_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS,
               copies=copies, empty_kernel_us=empty_ms * 1e3, plain_read_us=read_ms * 1e3,
               note="cold = 128 distinct copies cycled (348 MB > 256 MB LLC), graph-replayed back-to-back "
                    "launches, per-launch time including the launch boundary; hot = one copy; "
                    f"empty_kernel_us = an empty kernel of the same grid ({grid} x 256); plain_read_us = a "
                    "read-only kernel over the same 2,723,840 weight bytes (256 x 256 threads)")
    if hot_ms is not None:
        out.update(hot_us=hot_ms * 1e3, hot_GBps=algo / (hot_ms * 1e-3) / 1e9)
    if stream and stride == packed.nbytes:
        ns = n * copies  # the copies are contiguous: one matrix of 622,592 rows
        s_ms = ops.bench_gemv(1, w, 0, 1, x, y, ns, k, 64)
        s_algo = ns * (k // 32) * 20 + k * 4 + ns * 4
        sr_ms = ops.bench_floor(w, ns * (k // 32) * 20, 4096, 256, 64)
        out.update(stream_rows=ns, stream_bytes=s_algo, stream_us=s_ms * 1e3,
                   stream_GBps=s_algo / (s_ms * 1e-3) / 1e9,
                   stream_frac=s_algo / (s_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS,
                   stream_plain_read_GBps=ns * (k // 32) * 20 / (sr_ms * 1e-3) / 1e9)
    w.close()
    return out


TRAFFIC_FILE = os.path.join(REPO, "profiles", "q4_0_gemv_c0_traffic.json")


def read_traffic():
    """HBM bytes per C0 launch from the committed rocprofv3 counter runs (FETCH_SIZE +
    WRITE_SIZE, scaled by a plain copy's reading), or None if they were not collected."""
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)["traffic_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def cpu_baseline(path: str, prompt, seconds: float, threads: int):
    """The oracle's decode on the host cores: greedy chain from the prompt's first token."""
    from oracle import oracle as O
    O.set_threads(threads)
    r = O.load_genomic(path)
    r.set_k_wta_ratio(0.0)
    tok = int(prompt[0])
    r.forward_core(tok, True)  # first token also pages the weights in (untimed)
    n, t0 = 0, time.perf_counter()
    while True:
        logits = r.forward_core(tok, False)
        tok = O.argmax_first(logits)
        n += 1
        el = time.perf_counter() - t0
        if (el >= seconds and n >= 4) or n >= 512:
            break
    return dict(value=n / el, unit="tok/s", cores=O.get_threads(), kind="port",
                sample=f"{n} greedy decode tokens (ctx 2..{n + 1}) of the same model on the host, "
                       f"{O.get_threads()} threads; AVX2 restatement of the reference kernels")


def c3_workloads(d: str, seed: int, prefill_tokens: int = 512, batch: int = 16, ctx: int = 1024, gen: int = 128):
    """Qwen2.5-1.5B-shaped MFMA prefill and batch-16 decode."""
    import gaje_hip
    from gaje_hip import ops
    path = model_path("qwen2.5-1.5b", seed, d)
    g = gaje_hip.load_genomic_auto(path)
    g.set_k_wta_ratio(0.0)
    rng = np.random.default_rng(seed + 1)
    ids = rng.integers(0, g.vocab_size, prefill_tokens).astype(np.uint32)
    g.reserve(prefill_tokens + 1)
    times = []
    for _ in range(4):
        g.clear_cache_py()
        ops.synchronize()
        t = time.perf_counter()
        g.prefill_mfma(ids)
        ops.synchronize()
        times.append(time.perf_counter() - t)
    pf = min(times[1:])
    body_flop = 2.0 * prefill_tokens * sum(
        n * k for n, k in ((2048, 1536), (1536, 1536), (17920, 1536), (1536, 8960))) * g.info["n_blocks"]
    prefill = dict(tokens=prefill_tokens, ms=round(pf * 1e3, 3), tok_s=round(prefill_tokens / pf, 1),
                   body_TFLOPs=round(body_flop / pf / 1e12, 2), body_flop=body_flop,
                   precision="f16 hi/lo operand pairs, fp32 accumulation (fp32-level accuracy)")
    log(f"[bench] C3 prefill {prefill_tokens}: {pf * 1e3:.2f} ms = {prefill_tokens / pf:.0f} tok/s, "
        f"body {body_flop / pf / 1e12:.1f} TFLOP/s")
    b = gaje_hip.GenomicBatch(g, batch, ctx + 2 * gen + 1)
    ctx_ids = rng.integers(0, g.vocab_size, (batch, ctx)).astype(np.uint32)
    t = time.perf_counter()
    logits = b.feed(ctx_ids, want_logits=True)
    ops.synchronize()
    feed_s = time.perf_counter() - t
    first = logits.argmax(axis=1).astype(np.uint32)
    b.decode_greedy(first, 8)  # warm-up steps
    ops.synchronize()
    t = time.perf_counter()
    out = b.decode_greedy(first, gen)
    ops.synchronize()
    el = time.perf_counter() - t
    decode = dict(batch=batch, context=ctx, steps=gen, ms_per_step=round(el / gen * 1e3, 3),
                  tok_s=round(batch * gen / el, 1), feed_s=round(feed_s, 2),
                  note="each sequence bit-exact with its own forward_core; contexts fed through batched steps")
    log(f"[bench] C3 batch-{batch} decode: {el / gen * 1e3:.2f} ms/step = {batch * gen / el:.0f} tok/s "
        f"(context {ctx}+, fed in {feed_s:.1f}s)")
    b.close()
    g.close()
    return prefill, decode, [int(v) for v in out[0, :4]]


def variant_decode_workload(d: str, seed: int, preset: str, prompt_len: int, gen: int, steps: int,
                            quant_embed: int = 0, body_format: int = 1):
    """Batch-1 greedy decode of the same shape in another format: Q8_0 token_embd / lm_head
    (quant_embed=1, the --quant-embed export: the lm_head reads 34 B per 32 weights instead
    of 128) or a 2-bit body (body_format=4, Genomic2Bit with per-block centroids)."""
    import gaje_hip
    from gaje_hip import ops
    path = model_path(preset, seed, d, quant_embed=quant_embed, body_format=body_format)
    g = gaje_hip.load_genomic_auto(path)
    g.set_k_wta_ratio(0.0)
    prompt = np.random.default_rng(seed).integers(0, g.vocab_size, prompt_len).astype(np.uint32)
    g.reserve(prompt_len + gen + 1)
    g.clear_cache_py()
    g.prefill(prompt)

    def step():
        g.truncate_cache(prompt_len)
        return g.decode_greedy(int(prompt[-1]), gen)

    step()
    ops.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    ops.synchronize()
    el = time.perf_counter() - t0
    g.truncate_cache(prompt_len + gen - 1)
    stages = {}
    for st in (("lm_head",) if quant_embed else ("qkv", "o", "gate_up", "down")):
        ms, nbytes = g.time_stage(st, iters=200)
        gbps = nbytes / (ms * 1e-3) / 1e9
        stages[st] = dict(us=round(ms * 1e3, 3), bytes=int(nbytes), GBps=round(gbps, 1),
                          frac=round(gbps / HBM_PEAK_GBPS, 4))
    g.close()
    out = dict(tok_s=round(gen * steps / el, 2), ms_per_token=round(el / (gen * steps) * 1e3, 4),
               prompt=prompt_len, gen=gen, steps=steps, stages=stages)
    what = "Q8_0 embed/lm_head" if quant_embed else "2-bit body"
    log(f"[bench] {what} decode: {out['tok_s']:.1f} tok/s; " +
        ", ".join(f"{k} {v['us']:.2f} us" for k, v in stages.items()))
    return out


def moe_workload(seed: int, T: int = 256, h: int = 1536, ffn: int = 4096, E: int = 8, iters: int = 50):
    from gaje_hip import ops, synth
    x = synth.normal(seed + 51, "moe.x", T * h).reshape(T, h)
    router = synth.normal(seed + 52, "moe.r", E * h, 0.0, 0.02).reshape(E, h)
    gu = [ops.q4_0_upload(synth.q4_0_tensor(seed + 53, f"moe.gu.{e}", 2 * ffn, h), 2 * ffn, h) for e in range(E)]
    dn = [ops.q4_0_upload(synth.q4_0_tensor(seed + 53, f"moe.dn.{e}", h, ffn), h, ffn) for e in range(E)]
    xd, rd = ops.DeviceBuffer.from_array(x), ops.DeviceBuffer.from_array(router)
    y = ops.DeviceBuffer(T * h * 4)
    ws = ops.DeviceBuffer(ops.moe_ffn_workspace(T, h, ffn, E))
    for _ in range(3):
        ops.moe_ffn(xd, T, h, rd, gu, dn, ffn, y, ws)
    ops.synchronize()
    e0, e1 = ops.Event(), ops.Event()
    e0.record()
    for _ in range(iters):
        ops.moe_ffn(xd, T, h, rd, gu, dn, ffn, y, ws)
    e1.record()
    e1.synchronize()
    ms = e0.elapsed_ms(e1) / iters
    flop = 2.0 * T * 2 * (2 * ffn * h + h * ffn)
    wbytes = E * (2 * ffn * h + h * ffn) * 20 // 32
    log(f"[bench] C4 MoE layer: {ms * 1e3:.1f} us, {flop / ms / 1e9:.1f} TFLOP/s (expert products)")
    return dict(tokens=T, hidden=h, ffn=ffn, experts=E, top_k=2, us_per_layer=round(ms * 1e3, 2),
                expert_TFLOPs=round(flop / ms / 1e9, 2), expert_flop=flop, expert_weight_bytes=wbytes,
                tokens_per_s=round(T / ms * 1e3, 1))


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--preset", default="qwen2-0.5b")
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--gen", type=int, default=256)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--model-dir", default=None)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-stages", action="store_true")
    ap.add_argument("--no-c3", action="store_true", help="skip the Qwen2.5-1.5B prefill and batched decode")
    ap.add_argument("--c3-ctx", type=int, default=1024, help="context fed to each batched sequence")
    ap.add_argument("--c3-gen", type=int, default=128, help="batched greedy steps timed")
    ap.add_argument("--no-decode", action="store_true",
                    help="skip the Qwen2-0.5B decode, its stages and the C0 matvec (profiling runs of the other workloads)")
    ap.add_argument("--no-moe", action="store_true", help="skip the MoE layer")
    ap.add_argument("--no-q8", action="store_true", help="skip the Q8_0 token_embd/lm_head decode")
    ap.add_argument("--no-2bit", action="store_true", help="skip the 2-bit body decode")
    ap.add_argument("--gemv-only", action="store_true",
                    help="only the C0 Q4_0 matvec (cold) and a 256 MiB device copy, for counter runs")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build runs on exactly one GPU (asked for {max(args.gpus, world)}); "
              "the decode path is not sharded across GPUs", file=sys.stderr)
        sys.exit(2)

    import gaje_hip
    from gaje_hip import ops
    if ops.device_count() < 1:
        print("bench.py: no HIP device", file=sys.stderr)
        sys.exit(1)
    log(f"[bench] device: {ops.device_name(0)}")
    if args.gemv_only:
        # a copy kernel of known size (the counters' scale) and the C0 matvec
        nbytes = 256 << 20
        a, b = ops.DeviceBuffer(nbytes), ops.DeviceBuffer(nbytes)
        ops.memcpy_d2d(b, a, nbytes)
        ops.synchronize()
        gemv = q4_gemv_c0(hot=False)
        log(f"[bench] Q4_0 GEMV C0: cold {gemv['cold_us']:.2f} us = {gemv['cold_GBps']:.0f} GB/s")
        print(json.dumps({"q4_0_gemv": gemv, "copy_bytes": nbytes}), flush=True)
        return

    d = args.model_dir or tempfile.gettempdir()
    tok_s = el = None
    toks = []
    stages, gemv, roofline, path, prompt = {}, None, None, None, None
    if not args.no_decode:
        path = model_path(args.preset, args.seed, d)
        t = time.perf_counter()
        g = gaje_hip.load_genomic_auto(path)
        log(f"[bench] loaded {g.info['weight_bytes'] / 1e9:.2f} GB of weights into HBM in {time.perf_counter() - t:.1f}s")
        g.set_k_wta_ratio(0.0)
        vocab = g.vocab_size
        prompt = np.random.default_rng(args.seed).integers(0, vocab, args.prompt).astype(np.uint32)
        g.reserve(args.prompt + args.gen + 1)
        g.clear_cache_py()
        t = time.perf_counter()
        g.prefill(prompt)
        log(f"[bench] prefilled {args.prompt} tokens token-by-token in {time.perf_counter() - t:.2f}s")

        def step():
            g.truncate_cache(args.prompt)
            return g.decode_greedy(int(prompt[-1]), args.gen)

        for _ in range(args.warmup):
            step()
        ops.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            toks = step()
        ops.synchronize()
        el = time.perf_counter() - t0
        tok_s = args.gen * args.steps / el
        log(f"[bench] decode: {tok_s:.1f} tok/s ({el / args.steps * 1e3:.1f} ms per {args.gen}-token step)")

        stages = {}
        roofline = None
        if not args.no_stages:
            counts = {"qkv": g.info["n_blocks"], "attention": g.info["n_blocks"], "o": g.info["n_blocks"],
                      "gate_up": g.info["n_blocks"], "down": g.info["n_blocks"], "lm_head": 1}
            g.truncate_cache(args.prompt + args.gen - 1)  # time at the last step's context
            for s in ("qkv", "attention", "o", "gate_up", "down", "lm_head", "token"):
                ms, nbytes = g.time_stage(s, layer=0, iters=200 if s != "token" else 50)
                gbps = nbytes / (ms * 1e-3) / 1e9
                stages[s] = dict(us=round(ms * 1e3, 3), bytes=int(nbytes), GBps=round(gbps, 1),
                                 frac=round(gbps / HBM_PEAK_GBPS, 4))
                if s in counts:
                    stages[s]["per_token_us"] = round(ms * 1e3 * counts[s], 2)
                log(f"[bench] stage {s:9s}: {ms * 1e3:8.2f} us  {gbps:8.1f} GB/s")

        gemv = q4_gemv_c0()
        log(f"[bench] Q4_0 GEMV C0: cold {gemv['cold_us']:.2f} us = {gemv['cold_GBps']:.0f} GB/s "
            f"({100 * gemv['cold_frac']:.1f}% of HBM peak); hot {gemv['hot_us']:.2f} us")
        # the metric's kernel: the C0 Q4_0 matvec, cold, timed with HIP events on its own stream
        roofline = dict(kernel="gemv_kernel<Q4_0> (C0: K=896, N=4864, 128 cold weight copies)", bound="hbm",
                        achieved=round(gemv["cold_GBps"], 1), peak=HBM_PEAK_GBPS, unit="GB/s",
                        frac=round(gemv["cold_frac"], 4), traffic=read_traffic(),
                        bytes_per_launch=gemv["algorithmic_bytes"], us_per_launch=round(gemv["cold_us"], 3))

        g.close()
    workloads = {}
    if not args.no_q8 and not args.no_decode:
        workloads[f"{args.preset}_q8_0_embed_decode"] = variant_decode_workload(
            d, args.seed, args.preset, args.prompt, args.gen, args.steps, quant_embed=1)
    if not args.no_2bit and not args.no_decode:
        workloads[f"{args.preset}_2bit_body_decode"] = variant_decode_workload(
            d, args.seed, args.preset, args.prompt, args.gen, args.steps, body_format=4)
    if not args.no_c3:
        prefill, decode, c3_tokens = c3_workloads(d, args.seed, ctx=args.c3_ctx, gen=args.c3_gen)
        workloads["qwen2.5-1.5b_prefill_512"] = prefill
        workloads["qwen2.5-1.5b_batch16_decode"] = decode
    if not args.no_moe:
        workloads["moe_ffn_256x1536_8x4096_top2"] = moe_workload(args.seed)

    cpu = None
    if not args.no_cpu and path is not None:
        threads = min(16, os.cpu_count() or 1)
        cpu = cpu_baseline(path, prompt, args.cpu_seconds, threads)
        log(f"[bench] cpu oracle: {cpu['value']:.2f} tok/s on {cpu['cores']} threads")

    out = {
        "metric": METRIC,
        "value": round(tok_s, 2) if tok_s else None,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(el / args.steps * 1e3, 3) if el else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (random-init weights, uniform random prompt ids)",
        "config": {"workload": f"{args.preset}-shape batch-1 greedy decode: {args.prompt}-token prompt, "
                               f"then {args.gen} tokens (KV cache {args.prompt}->{args.prompt + args.gen}), "
                               "Q4_0 body, f32 embed/lm_head, K-WTA off",
                   "prompt": args.prompt, "gen": args.gen, "batch": 1, "preset": args.preset},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "q4_0_gemv": gemv,
        "stages": stages,
        "workloads": workloads,
        "last_tokens": [int(t) for t in toks[-4:]],
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
