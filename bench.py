#!/usr/bin/env python3
"""Dual-AR decode benchmark: audio frames/s of the Slow+Fast AR loop, batch 1.

Default workload ("full"): S2-Pro-shaped random-init model (36 Slow layers,
d=2560, 32 q / 8 kv heads, head_dim 128, FFN 9728, vocab 155776; 4 Fast
layers, 10 codebooks x 4096), f16 weights N(0, 0.02) seed 1, a 256-token
uniform-random prompt, greedy, KV cache 768.  One step = one frame (one
Slow-AR decode step + the Fast-AR's 9 codebook passes + sampling); the timed
window runs from after prefill to the last frame's codes (HIP events inside
the library).  Prints one JSON line.

--steps K asks for at least K timed frames: the timed region is the smallest
number of whole generations of the workload (512 frames for "full") that
holds K frames, so the workload's frame count and KV length are never
shortened; "steps" in the output is the number of frames actually timed.
--warmup W runs the smallest number of untimed generations holding W frames
(at least one).

Workload "codec": the RVQ codec decode that follows code generation
(decode_waveform, crates/fish_s2_infer/src/codec.rs:1690-1714) on a seeded
synthetic codec: 512 code frames (the "full" workload's output length) ->
4 x 512 latent frames -> 1,048,576 samples at 44.1 kHz.  One step = one
whole decode with codes and samples resident in device memory; `value` is
code frames/s.  The default run also reports this decode under "codec".

Workload "full_b8": the voice-clone batch shape: 8 concurrent requests on
the same f16 model, each a 1500-position prompt (250 text ids, 1000
reference frames with uniform random codes, 250 text ids), MFMA prefill,
then 1024 frames per request decoded together at batch 8, KV cache 2560.
`value` is then the aggregate frames/s of the batch.
"""

import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "fish-s2pro_amd"), ROOT]

HBM_PEAK_GBS = 8000.0

WORKLOADS = {
    # name: (shape, prompt, frames, max_seq, temperature, top_p, top_k, requests, reference frames)
    "full": ("full", 256, 512, 768, 0.0, 1.0, 0, 1, 0),
    "full_q8": ("full_q8", 256, 512, 768, 0.7, 0.9, 0, 1, 0),
    "full_q4": ("full_q4", 256, 1024, 1280, 0.0, 1.0, 0, 1, 0),
    "full_b8": ("full", 1500, 1024, 2560, 0.0, 1.0, 0, 8, 1000),
    "tiny": ("tiny", 32, 16, 64, 0.0, 1.0, 0, 1, 0),
    "tiny_b8": ("tiny", 48, 16, 80, 0.0, 1.0, 0, 8, 32),
}


def log(msg):
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def frame_bytes(spec, shape, avg_t, kv_bytes=4, nseq=1):
    """Algorithmic HBM bytes of one decode step of nseq requests: Slow weights
    once, Fast weights for 9 passes (positions 0 and 1 share one pass), the
    candidate head rows and norms once; per request the embeddings and the KV
    reads/writes at the stored KV dtype (kv_bytes for the Slow-AR cache; the
    Fast-AR cache is f32)."""
    b_w = {1: 2.0, 8: 34 / 32, 2: 18 / 32}[spec["linear_type"]]
    d, L, Lf = spec["dim"], spec["slow_layers"], spec["fast_layers"]
    ncb, C = spec["num_codebooks"], spec["codebook_size"]
    kv = spec["kv_heads"] * spec["head_dim"]
    slow = L * shape.linear_params_per_slow_layer() * b_w
    slow += L * (2 * d + 2 * spec["head_dim"]) * 2 + 2 * d + nseq * (ncb + 1) * d * 2
    slow += (C + 1) * d * 2  # semantic rows + im_end of the tied head
    slow += nseq * (avg_t * L * 2 * kv * kv_bytes + L * 2 * kv * kv_bytes)
    fast_pass = Lf * shape.linear_params_per_fast_layer() * b_w + d * C * b_w + Lf * 2 * d * 2 + 2 * d + nseq * d * 2
    fkv = spec["fast_kv_heads"] * spec["fast_head_dim"]
    fast = (ncb - 1) * fast_pass + nseq * Lf * 2 * fkv * 4 * (ncb * (ncb + 1) // 2 + ncb)
    return slow + fast


def prefill_flops(spec, shape, n_tok, nseq=1):
    """Useful FLOPs of prompt prefill: 2 per weight per token in the Slow-AR
    linears, plus causal attention (QK and PV, 4 hd per query-key pair per
    head)."""
    L = spec["slow_layers"]
    lin = 2.0 * L * shape.linear_params_per_slow_layer() * n_tok
    attn = 2.0 * L * spec["heads"] * spec["head_dim"] * n_tok * (n_tok + 1)
    return nseq * (lin + attn)


def counter_traffic(kernel, workload):
    """HBM bytes per launch of `kernel` from the committed FETCH_SIZE and
    WRITE_SIZE summaries (rocprofv3 --pmc, calibrated against a plain copy),
    or None when no summary exists for this kernel and workload."""
    path = os.path.join(ROOT, "profiles", f"counters_{kernel}_{workload}.txt")
    if not os.path.exists(path):
        return None
    got = {}
    with open(path) as f:
        for line in f:
            m = re.match(r"(FETCH_SIZE|WRITE_SIZE): .* kernel bytes/launch (\d+)", line)
            if m:
                got[m.group(1)] = int(m.group(2))
    if set(got) != {"FETCH_SIZE", "WRITE_SIZE"}:
        return None
    return got["FETCH_SIZE"] + got["WRITE_SIZE"]


def cpu_threads():
    """Threads for the CPU baseline: the box's CPU share as OMP_NUM_THREADS
    states it (the reference's Rayon pool defaults to every CPU the process
    may use), else the CPUs this process may run on."""
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        return int(env)
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(path, shape, threads, prompt_len, frames):
    """The oracle in faithful mode (per-step Slow layer reload + f32 expansion,
    Fast-AR prefix recompute, row-parallel f32 linears) on a bounded sample."""
    from oracle import oracle as O
    from s2hip import synth

    m = O.OracleModel(path, prompt_len + frames + 1, shape.im_end_id,
                      flags=O.FAITHFUL_SLOW_RELOAD | O.FAITHFUL_FAST_RECOMPUTE, threads=threads)
    prompt = synth.synthetic_prompt(shape, prompt_len, seed=shape.seed)
    r = m.generate_codes(prompt, frames, 0.0, 1.0, 0, 1 << 30, 0)
    m.close()
    return r["n_frames"] / r["decode_seconds"], r


CODEC_FRAMES = 512
MFMA_F16_PEAK_TFLOPS = 2500.0
CODEC_CONVS = (["entry"] + [f"b{b}_convT" for b in range(1, 5)] +
               [f"b{b}_r{r}_conv{k}" for b in range(1, 4) for r in range(1, 4) for k in (0, 1)] +
               [f"b4_r{r}_unit" for r in range(1, 4)] +  # 96 channels: k7 + snake + k1 in one launch
               [f"up{s}_{x}" for s in (1, 2) for x in ("convT", "pw1", "pw2")])


def bench_codec(args, full):
    """decode_waveform of CODEC_FRAMES code frames on the GPU (HIP events in
    the library, device-resident codes and samples), the MFMA roofline of the
    convolution with the largest share, and (full) the CPU oracle on a
    bounded sample."""
    from s2hip import Codec, synth

    frames = (args.frames or CODEC_FRAMES) if full else CODEC_FRAMES
    path = synth.ensure_codec_gguf(args.model_dir, threads=min(16, os.cpu_count() or 1))
    timed = max(1, -(-(args.steps or frames) // frames)) if full else 3
    warm = max(1, -(-args.warmup // frames)) if full else 1
    with Codec(path, max_frames=frames, device=0) as c:
        c.time("decode", frames, warm)
        us, conv_flops = c.time("decode", frames, timed)
        per = {}
        for name in CODEC_CONVS:
            per[name] = c.time(name, frames, 5)
    top = max(per, key=lambda n: per[n][0])
    with Codec(path, max_frames=frames, device=0) as c:
        # the dominant launch again, last: a kernel trace's final dispatches
        # of this kernel are these 20
        kus, kfl = c.time(top, frames, 20)
    ach = kfl / kus / 1e6
    fps = frames / (us * 1e-6)
    log(f"codec decode {frames} frames: {us / 1e3:.3f} ms, {fps:.0f} code frames/s; dominant {top} {kus:.1f} us")
    out = {
        "metric": "codec decode_waveform code frames/s (RVQ lookup + post-module + upsample + decoder), one GPU",
        "value": round(fps, 1),
        "unit": "code frames/s",
        "n_gpus": 1,
        "steps": timed * frames,
        "warmup": warm * frames,
        "ms_per_step": round(us / 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 MFMA (f16-rounded conv inputs as the reference; split f16 hi+lo for f32 inputs), f32 accumulate",
        "data": "synthetic codec (seeded random-init, fan-in scaled), fixed pseudo-random codes",
        "config": {"workload": f"codec: decode_waveform of {frames} code frames x 10 codebooks -> {4 * frames} latent "
                               f"frames -> {frames * 2048} samples at 44.1 kHz", "frames": frames,
                   "parallelism": "single GPU"},
        "samples_per_s": round(frames * 2048 / (us * 1e-6)),
        "realtime_factor": round(frames * 2048 / (us * 1e-6) / 44100.0, 1),
        "conv_tflops": round(conv_flops / us / 1e6, 1),
        "roofline": {"bound": "mfma", "kernel": f"conv_gemm {top}", "achieved": round(ach, 1),
                     "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(ach / MFMA_F16_PEAK_TFLOPS, 4),
                     "traffic": counter_traffic(top, "codec"), "flops_per_launch": round(kfl), "avg_us": round(kus, 2)},
        "kernels": {n: round(v[0], 1) for n, v in sorted(per.items(), key=lambda kv: -kv[1][0])[:8]},
    }
    if full and args.cpu_baseline:
        from oracle import oracle as O

        threads = cpu_threads()
        n = max(1, args.cpu_frames)
        rng_codes = [[(f * 7919 + q * 104729 + 17) % (4096 if q == 0 else 1024) for f in range(n)] for q in range(10)]
        t0 = time.time()
        with O.OracleCodec(path, threads) as oc:
            oc.decode_waveform(rng_codes, 10, n)
        dt = time.time() - t0
        out["cpu_baseline"] = {"value": round(n / dt, 4), "unit": "code frames/s", "cores": threads, "kind": "port",
                               "cpu_model": cpu_model(),
                               "sample": f"{n} code frames ({n * 2048} samples), the oracle's decode_waveform in the "
                                         f"reference's summation order, output-frame parallel threads"}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed frames at least (whole generations of the workload's frame count)")
    ap.add_argument("--frames", type=int, default=None, help="frames per generation (default: workload's)")
    ap.add_argument("--prompt", type=int, default=None, help="prompt tokens (default: workload's)")
    ap.add_argument("--warmup", type=int, default=1, help="untimed warm-up frames (whole generations, at least one)")
    ap.add_argument("--workload", default="full", choices=sorted(list(WORKLOADS) + ["codec"]))
    ap.add_argument("--codec", type=int, default=1, help="also time the 512-frame codec decode (default run)")
    ap.add_argument("--model-dir", default=os.environ.get("S2HIP_MODEL_DIR", "/tmp/s2hip_models"))
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--kv", choices=("f32", "f16"), default="f32",
                    help="Slow-AR KV cache dtype (f32 as the reference; f16 halves KV traffic)")
    ap.add_argument("--cpu-baseline", type=int, default=1)
    ap.add_argument("--cpu-frames", type=int, default=2)
    ap.add_argument("--cpu-prompt", type=int, default=None, help="CPU baseline prompt tokens (default: workload's)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for {args.gpus}); the dual-AR loop is a single-GPU "
              "batch-1 path in this build", file=sys.stderr)
        sys.exit(2)

    if args.workload == "codec":
        print(json.dumps(bench_codec(args, full=True)), flush=True)
        return

    from s2hip import Engine, synth

    shape_name, prompt_len, frames, max_seq, temp, top_p, top_k, nseq, ref_frames = WORKLOADS[args.workload]
    if args.frames:
        frames = args.frames
    timed_gens = max(1, -(-(args.steps or frames) // frames))
    warm_gens = max(1, -(-args.warmup // frames))
    if args.prompt:
        prompt_len = args.prompt
        ref_frames = min(ref_frames, prompt_len * 2 // 3)  # keep some text ids around the reference frames
    max_seq = max(max_seq, prompt_len + frames)
    shape = synth.SHAPES[shape_name]
    t0 = time.time()
    os.environ.setdefault("S2SYNTH_PROGRESS", "1")
    path = synth.ensure_gguf(shape, args.model_dir, threads=min(16, os.cpu_count() or 1))
    log(f"model {path} ready in {time.time() - t0:.1f}s")
    t0 = time.time()
    eng = Engine(path, max_seq, shape.im_end_id, use_graph=not args.no_graph, kv_f16=args.kv == "f16")
    spec = eng.spec
    log(f"engine loaded in {time.time() - t0:.1f}s ({spec['weight_bytes'] / 1e9:.2f} GB in HBM)")
    kw = dict(temperature=temp, top_p=top_p, top_k=top_k, min_tokens_before_end=1 << 30)
    if nseq == 1:
        prompt = synth.synthetic_prompt(shape, prompt_len, seed=shape.seed)

        def run():
            return eng.generate_codes(prompt, frames, rng_state=shape.seed, **kw)
    else:
        prompts = [synth.voice_clone_prompt(shape, prompt_len - ref_frames, ref_frames, seed=shape.seed + 100 * b)
                   for b in range(nseq)]

        def run():
            rb = eng.generate_codes_batch(prompts, frames, rng_states=[shape.seed + b for b in range(nseq)], **kw)
            return {"n_frames": rb["total_frames"], "prefill_ms": rb["prefill_ms"], "decode_ms": rb["decode_ms"],
                    "graph_used": rb["graph_used"]}
    for i in range(warm_gens):
        r = run()
        log(f"warmup {i}: {r['n_frames']} frames, prefill {r['prefill_ms']:.1f} ms, decode {r['decode_ms']:.1f} ms")
    n = 0
    dec_ms = prefill_ms = 0.0
    for i in range(timed_gens):
        r = run()
        n += r["n_frames"]
        dec_ms += r["decode_ms"]
        prefill_ms += r["prefill_ms"]
    dec_s = dec_ms / 1e3
    fps = n / dec_s
    log(f"timed: {timed_gens} generation(s), {n} frames ({nseq} requests) in {dec_ms:.1f} ms -> {fps:.1f} frames/s "
        f"(prefill {prefill_ms / timed_gens:.1f} ms per generation)")

    steps = n // nseq  # decode steps timed (frames per request over all timed generations)
    gen_steps = steps // timed_gens
    avg_t = prompt_len + gen_steps / 2.0
    fb = frame_bytes(spec, shape, avg_t, kv_bytes=2 if args.kv == "f16" else 4, nseq=nseq)  # bytes per decode step
    kern = "slow_w13" if nseq == 1 else f"slow_w13_b{nseq}"
    us, kb = eng.time_kernel(kern, reps=5)
    achieved = kb / (us * 1e-6) / 1e9
    log(f"{kern}: {us:.2f} us/launch, {kb / 1e6:.2f} MB -> {achieved:.0f} GB/s")
    other = {}
    names = ["slow_wqkv", "slow_wo", "slow_w2", "slow_head", "slow_attn", "fast_attn", "fast_head",
             "sample_fast", "sample_slow", "sample_fast_topp", "sample_slow_topp", "sample_fast_default",
             "fast_frame", "empty", "hbm_copy"]
    if nseq > 1:
        names = [f"{k}_b{nseq}" for k in ("slow_wqkv", "slow_wo", "slow_w2")] + names
    for k in names:
        ku, kbb = eng.time_kernel(k, reps=5)
        other[k] = {"us": round(ku, 3)}
        if kbb:
            other[k]["GBs"] = round(kbb / (ku * 1e-6) / 1e9, 1)
    eng.close()

    cpu = None
    if args.cpu_baseline:
        threads = cpu_threads()
        cpu_prompt = args.cpu_prompt or min(prompt_len, 256)
        model = cpu_model()
        log(f"cpu baseline: oracle faithful mode, {threads} threads ({model}), prompt {cpu_prompt}, "
            f"{args.cpu_frames} frames")
        t0 = time.time()
        cfps, cr = cpu_baseline(path, shape, threads, cpu_prompt, args.cpu_frames)
        log(f"cpu baseline {cfps:.4f} frames/s ({time.time() - t0:.1f}s wall, prefill {cr['prefill_seconds']:.1f}s)")
        cpu = {"value": round(cfps, 5), "unit": "frames/s", "cores": threads, "kind": "port",
               "cpu_model": model,
               "sample": f"{shape_name} model, {cpu_prompt}-token prompt, {cr['n_frames']} greedy frames "
                         f"after prefill (frames timed; prefill {cr['prefill_seconds']:.1f} s untimed); "
                         f"faithful mode (Slow layers re-read + expanded to f32 every step, Fast-AR prefix "
                         f"recompute), one row-parallel thread pool"}

    out = {
        "metric": "audio frames/sec (Slow+Fast AR) batch-1 f16; % of HBM roofline",
        "value": round(fps, 2),
        "unit": "frames/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec_s * 1e3 / max(1, steps), 4),
        "timed_generations": timed_gens,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {1: "f16", 8: "q8_0", 2: "q4_0"}[spec["linear_type"]] + " weights, f32 accumulate",
        "data": "synthetic (random-init N(0,0.02) weights, uniform random prompt ids)",
        "config": {"workload": f"{args.workload}: {spec['slow_layers']}+{spec['fast_layers']} layers d={spec['dim']}, "
                               f"{nseq} x {prompt_len}-token prompt, {gen_steps} frames per request, KV {max_seq}",
                   "requests": nseq, "prompt_tokens": prompt_len, "reference_frames": ref_frames,
                   "frames": gen_steps, "kv_cache": max_seq, "kv_dtype": args.kv, "sampler":
                       {"temperature": temp, "top_p": top_p, "top_k": top_k}, "parallelism": "single GPU"},
        "codes_per_s": round(fps * spec["num_codebooks"], 1),
        "prefill_ms": round(prefill_ms / timed_gens, 2),
        "prefill_tflops": round(prefill_flops(spec, shape, prompt_len, nseq) / (prefill_ms / timed_gens * 1e-3) / 1e12,
                                2),
        "frame_bytes": round(fb),
        "frame_roofline_frac": round(fb * (steps / dec_s) / (HBM_PEAK_GBS * 1e9), 4),
        "roofline": {"bound": "hbm", "kernel": (f"gemv {kern}" if nseq == 1 else f"batched MFMA product {kern}") +
                     " (fused RMSNorm + w1/w3 + SwiGLU)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": counter_traffic(kern, args.workload),
                     "bytes_per_launch": round(kb), "avg_us": round(us, 3)},
        "kernels": other,
        "cpu_baseline": cpu,
        "graph_used": r["graph_used"],
    }
    if args.codec and args.workload == "full":
        try:
            out["codec"] = bench_codec(args, full=False)
        except Exception as e:  # the decode loop's line must still print
            out["codec"] = {"error": str(e)}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
