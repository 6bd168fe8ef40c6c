"""Benchmark of the quantized decode path on one MI355X.

Workload (one "step"): every batch-1 GEMV of a decode token of a Qwen3-4B
shaped HyperVSQ-2 model -- 36 layers x {q, k, v, o, gate, up, down}, 252
launches over 1.05 GB of distinct resident weights (four times the 256 MB
infinity cache, so no step is served from cache) -- each launch reading its
own activation image (int8 token quantized on the device from N(0,1)
fp32, in the layout the kernel stages into LDS).  The
252 launches are captured once in a HIP graph and replayed.

value = algorithmic weight bytes per step / step time (GB/s); roofline is
the per-launch kernel time of the dominant shape (gate/up 9728x2560,
7,198,720 B) from HIP events on the launch stream; cpu_baseline times the
reference's CPU kernels (or the oracle port) on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "quant GEMV effective weight GB/s (% HBM peak); decode tok/s 1.5B-shape Q4_0"
PROFILE_TRAFFIC = os.path.join(ROOT, "profiles", "hvsq2_gemv_gate_9728x2560_traffic.json")


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--layers", type=int, default=36)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--cpu-seconds", type=float, default=4.0,
                   help="CPU work per thread setting in the baseline leg")
    p.add_argument("--q4", action="store_true", help="also sweep the Qwen2-1.5B Q4_0 shapes")
    p.add_argument("--only-gate", action="store_true",
                   help="profiling mode: launch only the gate projection sweep")
    p.add_argument("--decode-only", action="store_true",
                   help="profiling mode: only the Qwen2-1.5B Q4_0 greedy decode")
    p.add_argument("--no-decode", action="store_true", help="skip the decode workload")
    p.add_argument("--decode-new", type=int, default=128, help="greedy tokens of the decode workload")
    p.add_argument("--decode-prompt", type=int, default=32, help="prompt tokens of the decode workload")
    p.add_argument("--copy-probe", action="store_true",
                   help="profiling mode: a plain 64 MiB device copy, the reference point that "
                        "scales the FETCH_SIZE / WRITE_SIZE counters to bytes")
    return p.parse_args()


class Sweep:
    """Resident weights, activations and outputs of one GEMV sweep."""

    def __init__(self, torch, ctx, dtype, shapes, layers, seed):
        import numpy as np

        from qwanto_amd import synth
        self.torch, self.ctx, self.dtype = torch, ctx, dtype
        rng = np.random.default_rng(seed)
        torch.manual_seed(seed)
        self.items = []
        self.weight_bytes = 0
        dev = torch.device("cuda:0")
        for layer in range(layers):
            for proj in synth.PROJECTIONS:
                N, K = shapes[proj]
                w = synth.weights(dtype, rng, N, K)
                h = ctx.upload(w, dtype, N, K)
                ib = ctx.image_bytes(h)
                x = torch.randn(1, K, device=dev, dtype=torch.float32)
                img = torch.zeros(1, ib, device=dev, dtype=torch.uint8)
                sc = torch.zeros(1, device=dev, dtype=torch.float32)
                y = torch.zeros(1, N, device=dev, dtype=torch.float32)
                ctx.quantize_image_device(h, x.data_ptr(), 1, K, img.data_ptr(), ib, sc.data_ptr(),
                                          stream=torch.cuda.current_stream().cuda_stream)
                self.items.append((proj, N, K, h, img, sc, y, ib))
                self.weight_bytes += synth.weight_bytes(dtype, N, K)
        torch.cuda.synchronize()

    def launch(self, item, stream):
        proj, N, K, h, img, sc, y, ib = item
        self.ctx.gemm_image_device(h, img.data_ptr(), ib, y.data_ptr(), 1, N,
                                   scales_ptr=sc.data_ptr(), stream=stream)

    def step(self, stream, only=None):
        for it in self.items:
            if only is None or it[0] == only:
                self.launch(it, stream)


def time_graph(torch, fn, steps, warmup):
    """Capture fn(stream) once, replay warmup + steps times; ms per replay."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn(s.cuda_stream)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn(torch.cuda.current_stream().cuda_stream)
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps, g


def time_launches(torch, sweep, proj, steps, warmup):
    """Mean time per launch of one projection: a graph of its 36 launches
    (distinct weights, 36 x 7.2 MB for gate) replayed `steps` times between
    HIP events on the launch stream.  Includes the graph's per-kernel
    dispatch, so it bounds the profiler's kernel duration from above."""
    n = sum(1 for it in sweep.items if it[0] == proj)
    ms, _ = time_graph(torch, lambda s: sweep.step(s, only=proj), steps, warmup)
    return ms / n


def decode_bench(ctx, new_tokens=128, prompt_len=32, seed=2026):
    """Greedy decode of the Qwen2-1.5B shaped random Q4_0 model (28 layers,
    tied F16 LM head, Q8 KV) on the resident decoder: a 32-token prompt, then
    `new_tokens` greedy steps; tok/s = generated / decode wall time, as
    c/qwanto_decode.c:2121-2122 reports it.  Run twice: the first pass
    captures the step graph."""
    import numpy as np

    from qwanto_amd import abi, synth
    cfg = synth.QWEN2_1P5B_CONFIG
    rng = np.random.default_rng(seed)
    model = synth.decoder_model(rng, cfg, "q4_0")
    prompt = synth.prompt_tokens(rng, cfg["vocab"], prompt_len)
    dec = abi.ResidentDecoder(ctx, model)
    try:
        toks, st = dec.generate(prompt, new_tokens)
        dec.reset()
        toks2, st = dec.generate(prompt, new_tokens)
        assert toks.tolist() == toks2.tolist()
    finally:
        dec.close()
    ms_tok = st.decode_ms / st.generated_tokens
    return {
        "tok_s": round(st.generated_tokens / (st.decode_ms / 1e3), 1),
        "ms_per_token": round(ms_tok, 4),
        "prefill_tok_s": round(st.prompt_tokens / (st.prefill_ms / 1e3), 1),
        "weight_bytes_per_token": int(st.weight_bytes_per_step),
        "weight_gbps": round(st.weight_bytes_per_step / (ms_tok / 1e3) / 1e9, 1),
        "kernels_per_token": int(st.launches_per_step),
        "prompt_tokens": int(st.prompt_tokens), "generated_tokens": int(st.generated_tokens),
        "first_ids": toks[:8].tolist(),
        "workload": "qwen2_1p5b_q4_0 random-init, tied F16 LM head, Q8 KV, greedy, HIP graph per token",
    }


def cpu_baseline(seconds: float):
    """Time the reference's own CPU GEMV (oracle/_ref, built from c/qwanto_kernels.c)
    -- or the oracle port when that build is absent -- over a bounded sample:
    one Qwen3-4B layer's seven HyperVSQ-2 projections from N(0,1) fp32
    activations (quantization included, as qwn_matmul_hypervsq2_f32 does),
    rotating through four distinct layer copies (117 MB, beyond the LLC)."""
    import ctypes

    import numpy as np

    import oracle
    from qwanto_amd import synth
    ref = oracle.load_ref()
    ora = oracle.load()
    kind = "reference" if ref is not None else "port"
    rng = np.random.default_rng(99)
    layers = []
    for _ in range(4):
        layer = []
        for proj in synth.PROJECTIONS:
            N, K = synth.QWEN3_4B_SHAPES[proj]
            layer.append((synth.hvsq2_weights(rng, N, K), synth.activations(rng, 1, K), N))
        layers.append(layer)
    layer_bytes = sum(synth.weight_bytes("hvsq2", N, x.shape[1]) for _, x, N in layers[0])
    gomp = None
    for name in ("libgomp.so.1",):
        try:
            gomp = ctypes.CDLL(name)
        except OSError:
            pass
    ncpu = len(os.sched_getaffinity(0))
    results = {}
    for threads in sorted({8, ncpu}):
        if gomp is not None:
            gomp.omp_set_num_threads(threads)
        done = 0
        t0 = time.perf_counter()
        while True:
            for w, x, N in layers[done % 4]:
                if ref is not None:
                    ref.matmul_hvsq2(w, x, N)
                else:
                    ora.matmul_hvsq2(w, x, N, threads=threads)
            done += 1
            if time.perf_counter() - t0 >= seconds:
                break
        dt = time.perf_counter() - t0
        results[threads] = layer_bytes * done / dt / 1e9
    best_threads = ncpu
    return {
        "value": round(results[best_threads], 3), "unit": "GB/s", "cores": best_threads,
        "kind": kind,
        "kernel": (ref.cpu_kernel_name() if ref is not None else ora.variant_name(ora.best_variant())),
        "sample": f"Qwen3-4B layer, 7 HyperVSQ-2 projections x 4 distinct copies (117 MB), batch 1, "
                  f"fp32 N(0,1) input quantized per call, ~{seconds:.0f}s per thread count",
        "gbps_by_threads": {str(k): round(v, 3) for k, v in results.items()},
    }


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(json.dumps({"error": "qwn_hip runs on one GPU; this benchmark measures one MI355X "
                                   "(the multi-GPU sharding is described in DESIGN.md, not built)",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch

    from qwanto_amd import abi, synth
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs the GPU (no CPU fallback)")
    if args.copy_probe:
        n = 64 << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"profile_mode": "copy", "bytes_read": n, "bytes_written": n}), flush=True)
        return
    lib = abi.load()
    ctx = abi.Context(lib, device=0)
    if args.decode_only:
        print(json.dumps({"profile_mode": "decode",
                          **decode_bench(ctx, args.decode_new, args.decode_prompt)}), flush=True)
        return
    t_setup = time.perf_counter()
    sweep = Sweep(torch, ctx, "hvsq2", synth.QWEN3_4B_SHAPES, args.layers, seed=1)
    setup_s = time.perf_counter() - t_setup
    print(f"# setup: {len(sweep.items)} HyperVSQ-2 tensors, {sweep.weight_bytes / 1e9:.3f} GB "
          f"resident in {setup_s:.1f}s", file=sys.stderr, flush=True)

    if args.only_gate:
        ms, _ = time_graph(torch, lambda s: sweep.step(s, only="gate"), args.steps, args.warmup)
        print(json.dumps({"profile_mode": "gate", "ms_per_replay": ms}), flush=True)
        return

    ms_per_step, _ = time_graph(torch, sweep.step, args.steps, args.warmup)
    value = sweep.weight_bytes / (ms_per_step / 1e3) / 1e9
    print(f"# sweep: {ms_per_step:.4f} ms/step -> {value:.1f} GB/s", file=sys.stderr, flush=True)

    per_shape = {}
    for proj in ("gate", "down", "q", "o", "k"):
        N, K = synth.QWEN3_4B_SHAPES[proj]
        ms = time_launches(torch, sweep, proj, args.steps, args.warmup)
        per_shape[f"{proj} {N}x{K}"] = {
            "kernel_us": round(ms * 1e3, 3),
            "gbps": round(synth.weight_bytes("hvsq2", N, K) / (ms / 1e3) / 1e9, 1)}
    gate = per_shape["gate 9728x2560"]
    gate_bytes = synth.weight_bytes("hvsq2", 9728, 2560)
    traffic = None
    if os.path.exists(PROFILE_TRAFFIC):
        traffic = json.load(open(PROFILE_TRAFFIC)).get("hbm_bytes_per_launch")
    roofline = {"bound": "hbm", "achieved": gate["gbps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gate["gbps"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                "kernel": "gemv_kernel<hvsq2> gate 9728x2560",
                "bytes_per_launch": gate_bytes, "avg_launch_us": gate["kernel_us"]}

    extra = {}
    if args.q4:
        q4 = Sweep(torch, ctx, "q4_0", synth.QWEN2_1P5B_SHAPES, 28, seed=2)
        ms_q4, _ = time_graph(torch, q4.step, args.steps, args.warmup)
        extra["q4_0_sweep_qwen2_1p5b"] = {
            "gbps": round(q4.weight_bytes / (ms_q4 / 1e3) / 1e9, 1), "ms_per_step": round(ms_q4, 4),
            "weight_bytes": q4.weight_bytes}

    if not args.no_decode:
        extra["decode_qwen2_1p5b_q4_0"] = decode_bench(ctx, args.decode_new, args.decode_prompt)
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)
    dev = lib.devices()[0].name.decode()
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "hvsq2_gemv_sweep_qwen3_4b_batch1", "layers": args.layers,
                   "projections": {p: list(synth.QWEN3_4B_SHAPES[p]) for p in synth.PROJECTIONS},
                   "launches_per_step": len(sweep.items), "weight_bytes_per_step": sweep.weight_bytes,
                   "hbm_frac_of_peak": round(value / HBM_PEAK_GBS, 4), "device": dev},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "per_shape_kernel": per_shape,
        **extra,
    }
    print(json.dumps(line), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
