"""Benchmark: StrasGPT transformer forward pass on one MI355X.

Workload (one "step" = one full greedy generation, KV cache reset first):
the Mistral-Small-24B-shaped decoder (d 5120, FFN 32768, 40 layers, 32/8
heads of 128, vocab 131072, untied output, RoPE theta 1e8; random-init bf16
N(0, 0.02) weights, norm weights 1.0; 47 GB of weights), a 2048-token
uniform-random prompt, then 128 greedy decode tokens: the largest benchmark
configuration, which fits one MI355X. --config selects another (llama3.2-1b,
qwen3-4b, llama3.1-8b, moe-mxfp4). Weights are read from a seeded synthetic
safetensors directory and are HBM-resident before the timed region.

value = decode tokens/s (decode_count / sum of decode time over the timed
steps); prefill tokens/s is reported beside it (prompt tokens / prefill
time). The roofline object describes the dominant decode kernel (largest
share of event-measured decode time in an eager profiling pass of the
same workload); its duration is timed with one pair of HIP events on the
library's stream around back-to-back launches over every layer's weights
(the per-launch event figure, which also brackets each dispatch gap, is
reported beside it). The cpu_baseline is the reference's own C sources
(oracle/_ref/ref_baseline, built with the reference's flags, -march=x86-64-v3
for -march=native) driven by the reference's greedy loop on a bounded
sample of the same model files on the host cores, with the reference's
timing boundaries (source/strasgpt.c:206-274); where that binary is absent,
and for the MoE model (the reference has no MoE path), the oracle (the C +
OpenMP restatement of the reference forward pass). The
GPU runs the same sample, and cpu_baseline.parity compares the two: greedy
tokens identical, prefill logits within 2e-2 relative / 1e-3 absolute.
Under rocprofv3 (kernel trace or counters) the decode steps are launched
eagerly instead of replayed from the captured graph.
"""
import argparse
import json
import os
import subprocess
import sys
import tempfile
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def model_path(name, seed):
    base = "/dev/shm" if os.access("/dev/shm", os.W_OK) else "/tmp"
    return os.path.join(base, f"strasgpt_bench_{name}_{seed}")


def ensure_model(shp, seed):
    from strasgpt_amd import synth
    d = model_path(shp.name, seed)
    if not os.path.exists(os.path.join(d, "config.json")):
        t0 = time.time()
        synth.write_model(shp, d, seed=seed)
        log(f"wrote {shp.name} ({shp.weight_bytes() / 1e9:.2f} GB) in {time.time() - t0:.1f}s")
    return d


def host_cpu():
    """(threads this process may use, physical cores of the host, CPU model)."""
    avail = len(os.sched_getaffinity(0))
    cores = None
    try:
        out = subprocess.run(["lscpu", "-p=CORE,SOCKET"], capture_output=True, text=True,
                             timeout=30).stdout
        cores = len({ln for ln in out.splitlines() if ln and not ln.startswith("#")})
    except (OSError, subprocess.SubprocessError):
        pass
    model = ""
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return avail, cores, model


RTOL, ATOL = 2e-2, 1e-3  # logits: |gpu - cpu| <= ATOL + RTOL |cpu|


def parity(gpu, cpu_tokens, cpu_logits):
    """The GPU's greedy tokens and prefill logits on the baseline's sample
    against the CPU run's."""
    import numpy as np
    g_tokens, g_logits = gpu
    err = np.abs(g_logits - cpu_logits)
    return {"tokens_match": list(g_tokens) == list(cpu_tokens),
            "tokens_cpu": list(cpu_tokens), "tokens_gpu": list(g_tokens),
            "prefill_logits_max_abs_err": float(err.max()),
            "prefill_logits_within_tol": bool((err <= ATOL + RTOL * np.abs(cpu_logits)).all()),
            "tol": f"{RTOL} rel + {ATOL} abs"}


def under_profiler():
    """Whether rocprofv3 runs this process with kernel tracing or counter
    collection (it sets these variables for its tool library)."""
    return any(os.environ.get(v) == "1" for v in ("ROCPROF_KERNEL_TRACE",
                                                  "ROCPROF_COUNTER_COLLECTION"))


def cpu_baseline(d, shp, prompt, threads, prefill_tokens, decode_tokens, gpu):
    """The reference forward pass on the host cores: a short prefill, then
    `decode_tokens` greedy steps, timed like the reference driver. `gpu` is
    (tokens, prefill logits) of the GPU on the same sample; the CPU run's
    are compared with them."""
    import numpy as np
    from oracle import ref_manifest
    avail, phys, model = host_cpu()
    threads = max(1, min(threads, avail))
    sample_prompt = prompt[:prefill_tokens]
    info = {"cores": threads, "host_physical_cores": phys, "threads_available": avail,
            "cpu_model": model}
    # the reference has no MoE path: MoE models time the oracle (its C +
    # OpenMP restatement with the MoE semantics of this library)
    if os.path.exists(ref_manifest.BASELINE) and not shp.experts:
        with tempfile.TemporaryDirectory(prefix="strasgpt_cpu_") as tmp:
            man = ref_manifest.write(d, sample_prompt, decode_tokens + 1,
                                     os.path.join(tmp, "manifest.txt"))
            env = dict(os.environ, OMP_WAIT_POLICY="ACTIVE")  # as source/strasgpt.c:79
            t0 = time.time()
            r = subprocess.run([ref_manifest.BASELINE, man, os.path.join(tmp, "out.bin"),
                                str(threads)], capture_output=True, text=True, env=env)
            if r.returncode != 0:
                raise RuntimeError(f"reference CPU baseline failed: {r.stderr[-1000:]}")
            fields = [ln for ln in r.stderr.splitlines() if ln.startswith("timing ")][-1].split()
            prefill_s, decode_s, n = float(fields[1]), float(fields[2]), int(fields[3])
            log(f"cpu baseline: reference run in {time.time() - t0:.1f}s ({threads} threads)")
            # out.bin: int32 tokens[n + 1], float32 prefill logits[V], ...
            raw = open(os.path.join(tmp, "out.bin"), "rb").read()
            cpu_tokens = np.frombuffer(raw, np.int32, n + 1).tolist()
            cpu_logits = np.frombuffer(raw, np.float32, shp.vocab, offset=4 * (n + 1))
        return {"value": n / decode_s, "unit": "tok/s", "kind": "reference", **info,
                "prefill_tok_s": len(sample_prompt) / prefill_s,
                "sample": (f"{shp.name}: {len(sample_prompt)}-token prefill then {n} greedy "
                           f"decode steps, the reference's C sources (oracle/_ref/ref_baseline: "
                           f"-O3 -march=x86-64-v3 -ffast-math -fno-finite-math-only -fopenmp), "
                           f"OMP_WAIT_POLICY=ACTIVE, {threads} threads"),
                "parity": parity(gpu, cpu_tokens, cpu_logits)}
    from oracle import oracle as orc
    t0 = time.time()
    om = orc.OracleModel(d, threads=threads)
    log(f"cpu baseline: oracle loaded in {time.time() - t0:.1f}s ({threads} threads)")
    t0 = time.time()
    logits = om.predict(sample_prompt)
    t_prefill = time.time() - t0
    cpu_logits = logits[0].copy()
    amax = lambda row: int(om.lib.oracle_argmax(orc.fptr(row), row.size))  # sample_argmax
    cpu_tokens = [amax(logits[0])]
    t0 = time.time()
    for _ in range(decode_tokens):
        cpu_tokens.append(amax(om.predict([cpu_tokens[-1]])[0]))
    t_decode = time.time() - t0
    om.close()
    return {
        "value": decode_tokens / t_decode, "unit": "tok/s", "kind": "port", **info,
        "prefill_tok_s": len(sample_prompt) / t_prefill,
        "sample": (f"{shp.name}: {len(sample_prompt)}-token prefill then {decode_tokens} "
                   f"greedy decode steps, oracle/oracle.c (OpenMP, {threads} threads)"),
        "parity": parity(gpu, cpu_tokens, cpu_logits),
    }


COPY_PROBE_BYTES = 256 << 20


def traffic_file(config):
    return os.path.join(REPO, "profiles", f"traffic_decode_kernels_{config}.json")


def probe_traffic(t, prompt):
    """Kernels for the HBM traffic counter runs (rocprofv3 --pmc FETCH_SIZE, then
    WRITE_SIZE): copy_probe_kernel of known size, then eager decode steps."""
    import ctypes
    from strasgpt_amd import runtime
    lib = runtime.lib()
    lib.strasgpt_kbench_copy.argtypes = [ctypes.c_size_t, ctypes.c_int,
                                         ctypes.POINTER(ctypes.c_double)]
    us = ctypes.c_double()
    lib.strasgpt_kbench_copy(COPY_PROBE_BYTES, 3, ctypes.byref(us))
    log(f"copy probe: {COPY_PROBE_BYTES} bytes in {us.value:.1f} us")
    t.set_decode_mode(runtime.DECODE_EAGER)
    t.reset()
    t.generate(prompt[:16], 5)
    log("probe decode done")


def probe_mfma():
    """strasgpt_kbench_mfma: the bf16 matrix-core rate with constant and with
    random (toggling) operands, one and two waves per SIMD, for the clock
    counter runs."""
    import ctypes
    from strasgpt_amd import runtime
    lib = runtime.lib()
    lib.strasgpt_kbench_mfma.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                         ctypes.POINTER(ctypes.c_double)]
    tf = ctypes.c_double()
    for rnd in (0, 1):
        for waves in (1, 2):
            if lib.strasgpt_kbench_mfma(rnd, waves, 20000 // waves, 4, ctypes.byref(tf)) != 0:
                raise RuntimeError("strasgpt_kbench_mfma refused its arguments")
            log(f"mfma probe: {'random' if rnd else 'constant'} operands, {waves} wave(s) per SIMD: "
                f"{tf.value:.1f} TFLOP/s ({tf.value / 25:.1f}% of 2.5 PF)")


def traffic_for(kernel, config):
    """HBM bytes per launch of a decode kernel class from the committed counter
    summary of this workload (FETCH_SIZE + WRITE_SIZE, calibrated on
    copy_probe_kernel), or None where no summary exists."""
    try:
        with open(traffic_file(config)) as f:
            table = json.load(f)
        return table["kernels"][kernel]["traffic_bytes"]
    except (OSError, KeyError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--config", default="mistral-small-24b")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--cpu-threads", type=int, default=16,
                    help="upper bound; the baseline uses at most the CPUs this process may run on")
    ap.add_argument("--cpu-prefill-tokens", type=int, default=16)
    ap.add_argument("--cpu-decode-tokens", type=int, default=8)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--precision", type=int, default=0, help="prefill GEMM: 0 bf16x2, 1 bf16")
    ap.add_argument("--kv-cache", choices=["fp32", "bf16"], default="fp32",
                    help="KV-cache storage format (fp32: the reference's)")
    ap.add_argument("--probe-traffic", action="store_true",
                    help="only launch the kernels an HBM-counter run needs (a 256 MiB copy, "
                         "then a 16-token prefill and 4 eager decode steps); prints nothing")
    ap.add_argument("--probe-mfma", action="store_true",
                    help="only run the sustained MFMA rate probe (constant and random operands, "
                         "one and two waves per SIMD) and log its rates; prints nothing")
    ap.add_argument("--probe-prefill", action="store_true",
                    help="only run two prefills of the workload's prompt (for MFMA counter "
                         "runs of the prefill GEMMs); prints nothing")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU; multi-GPU runs are "
                                   "not part of it (run with --gpus 1)"}))
        sys.exit(2)

    from strasgpt_amd import runtime, synth
    if args.probe_mfma:
        probe_mfma()
        return
    shp = synth.shape(args.config)
    d = ensure_model(shp, args.seed)
    prompt = synth.prompt_tokens(shp.vocab, shp.prompt_len, 42)
    steps_per_gen = shp.decode_len + 1

    t0 = time.time()
    t = runtime.Transformer(d)
    load_s = time.time() - t0
    load_bytes = sum(os.path.getsize(os.path.join(d, f)) for f in os.listdir(d) if f.endswith(".safetensors"))
    t.set_prefill_precision(args.precision)
    t.set_kv_cache_format(runtime.KV_BF16 if args.kv_cache == "bf16" else runtime.KV_FP32)
    log(f"loaded into HBM in {load_s:.1f}s ({load_bytes / load_s / 1e9:.1f} GB/s); {runtime.version()}")
    if under_profiler():
        # rocprofv3's kernel tracing and counter collection follow every
        # eager launch; replays of the captured decode graph under its
        # kernel trace ended in a host SIGSEGV inside the HIP runtime
        t.set_decode_mode(runtime.DECODE_EAGER)
        log("under rocprofv3: decode steps launched eagerly (the kernels the graph replays)")

    if args.probe_traffic:
        probe_traffic(t, prompt)
        return
    if args.probe_prefill:
        for i in range(2):  # the first one also warms the clocks up
            t.reset()
            t.predict(prompt)
            log(f"probe prefill {i + 1}/2 done")
        return

    for i in range(args.warmup):
        t.reset()
        t.generate(prompt, steps_per_gen)
        log(f"warmup {i + 1}/{args.warmup} done")

    prefill_s = decode_s = 0.0
    decode_n = 0
    tokens = None
    t_start = time.perf_counter()
    for i in range(args.steps):
        t.reset()
        tokens, tm = t.generate(prompt, steps_per_gen)  # synchronous
        prefill_s += tm.prefill_s
        decode_s += tm.decode_s
        decode_n += tm.decode_count
        log(f"step {i + 1}/{args.steps}: prefill {tm.prefill_s * 1e3:.1f} ms, "
            f"decode {tm.decode_count} tok in {tm.decode_s * 1e3:.1f} ms")
    wall = time.perf_counter() - t_start

    # Eager profiling pass of the same workload: per-kernel event timing.
    t.reset()
    t.profile(True)
    t.generate(prompt, steps_per_gen)
    stats = t.profile_read()
    t.profile(False)

    decode_kernels = ["qkv_gemv", "attention_decode", "o_gemv", "gate_up_gemv", "down_gemv",
                      "logits_gemv", "argmax", "moe_route", "moe_gate_up", "moe_down"]
    dec = {k: stats[k] for k in decode_kernels if k in stats}
    dom = max(dec, key=lambda k: dec[k]["total_ms"])
    # Sustained duration of the dominant kernel: back-to-back launches over
    # every layer's weights between one pair of events on the library's
    # stream (the per-launch event pairs above also bracket each launch's
    # dispatch gap). Classes without this hook keep the per-launch figure.
    rate = t.kernel_rate(dom, reps=4)
    # The CPU baseline's sample on the GPU (greedy tokens and prefill
    # logits), for the comparison with the CPU run.
    gpu_sample = None
    if not args.no_cpu_baseline:
        sample = prompt[:args.cpu_prefill_tokens]
        t.reset()
        sample_logits = t.predict(sample)[0]
        t.reset()
        gpu_sample = (t.generate(sample, args.cpu_decode_tokens + 1)[0], sample_logits)
    t.close()

    prefill_kernels = ["qkv_gemm", "o_gemm", "gate_up_gemm", "down_gemm", "moe_gate_up_prefill",
                       "moe_down_prefill"]
    kernels = {}
    for k, v in stats.items():
        avg_ms = v["total_ms"] / v["launches"]
        e = {"launches": v["launches"], "avg_us": avg_ms * 1e3,
             "bytes_per_launch": v["bytes"] / v["launches"],
             "flop_per_launch": v["flops"] / v["launches"]}
        e["gbs"] = v["bytes"] / (v["total_ms"] * 1e-3) / 1e9 if v["total_ms"] else 0.0
        e["tflops"] = v["flops"] / (v["total_ms"] * 1e-3) / 1e12 if v["total_ms"] else 0.0
        kernels[k] = e
    kd = kernels[dom]
    if rate is not None:
        avg_us, bpl = rate
        gbs, timing = bpl / (avg_us * 1e-6) / 1e9, "back-to-back launches over all layers, one event pair"
    else:
        avg_us, bpl, gbs = kd["avg_us"], kd["bytes_per_launch"], kd["gbs"]
        timing = "one event pair per launch (eager profiling pass)"
    roofline = {"kernel": dom, "bound": "hbm", "achieved": round(gbs, 1),
                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                "traffic": traffic_for(dom, shp.name), "avg_us": round(avg_us, 2),
                "avg_us_per_launch_events": round(kd["avg_us"], 2),
                "bytes_per_launch": bpl, "timing": timing}
    pre = {k: stats[k] for k in prefill_kernels if k in stats}
    roofline_prefill = None
    if pre:
        flops = sum(v["flops"] for v in pre.values())
        ms = sum(v["total_ms"] for v in pre.values())
        tf = flops / (ms * 1e-3) / 1e12
        # bf16x2 issues two bf16 MFMAs per product (activations as hi + lo
        # planes): the matrix cores execute twice the algorithmic FLOP
        issue = 2 if args.precision == 0 else 1
        roofline_prefill = {"kernels": sorted(pre), "bound": "mfma", "achieved": round(tf, 1),
                            "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                            "frac": round(tf / BF16_PEAK_TFLOPS, 4),
                            "precision": "bf16x2" if args.precision == 0 else "bf16",
                            "mfma_issued_tflops": round(issue * tf, 1),
                            "mfma_issued_frac": round(issue * tf / BF16_PEAK_TFLOPS, 4)}
    decode_tok_s = decode_n / decode_s
    prefill_tok_s = args.steps * len(prompt) / prefill_s
    decode_bytes = sum(v["bytes"] for k, v in stats.items() if k in decode_kernels)
    ntok = steps_per_gen - 1
    out = {
        "metric": "decode tok/s @batch1 + prefill tok/s; % of HBM BW / MFMA peak",
        "value": round(decode_tok_s, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 2), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16 weights, fp32 activations",
        "data": "synthetic (seeded random-init weights, uniform-random prompt ids)",
        "config": {"workload": f"{shp.name}-shaped decoder: {shp.prompt_len}-token prefill + "
                               f"{shp.decode_len} greedy decode tokens, batch 1",
                   "global_batch": 1, "seq_len": shp.prompt_len + shp.decode_len,
                   "parallelism": "single GPU", "kv_cache": args.kv_cache},
        "prefill_tok_s": round(prefill_tok_s, 1),
        "decode_ms_per_token": round(decode_s / decode_n * 1e3, 4),
        "decode_effective_gbs": round(decode_bytes / ntok / (decode_s / decode_n) / 1e9, 1),
        "roofline": roofline,
        "roofline_prefill": roofline_prefill,
        # transformer_from_safetensors: headers parsed, tensors read with
        # pread into pinned staging buffers and uploaded while the next one
        # is read (the files were just written, so they come from the page
        # cache)
        "model_load": {"seconds": round(load_s, 2), "file_bytes": load_bytes,
                       "gbs": round(load_bytes / load_s / 1e9, 2)},
        "kernels": {k: {kk: (round(vv, 3) if isinstance(vv, float) else vv)
                        for kk, vv in v.items()} for k, v in kernels.items()},
        "tokens_head": tokens[:8],
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(d, shp, prompt, args.cpu_threads,
                                           args.cpu_prefill_tokens, args.cpu_decode_tokens,
                                           gpu_sample)
        par = out["cpu_baseline"]["parity"]
        log(f"cpu baseline parity: tokens {'identical' if par['tokens_match'] else 'DIFFER'} "
            f"(cpu {par['tokens_cpu']}, gpu {par['tokens_gpu']}); prefill logits max |err| "
            f"{par['prefill_logits_max_abs_err']:.3g}")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
