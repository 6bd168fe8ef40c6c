"""Benchmark of the quantized decode path on one MI355X.

Headline workload (one "step"): every batch-1 GEMV of a decode token of a
Qwen3-4B shaped HyperVSQ-2 model (36 layers x {q, k, v, o, gate, up, down},
1.05 GB of distinct resident weights, four times the 256 MB infinity cache,
so no step is served from cache), launched the way the decoder issues them:
per layer q/k/v as one grouped launch (one input), o, gate/up as one grouped
launch, down -- 144 launches, captured once in a HIP graph and replayed.
Each launch reads its own activation image (an int8 token quantized on the
device from N(0,1) fp32) already resident in HBM.

value = algorithmic weight bytes per step / step time (GB/s).  roofline is
the dominant kernel of that step (the gate/up launch, 2 x 9728x2560,
14,397,440 B) from HIP events on the launch stream; cpu_baseline times the
oracle's restatement of the reference's CPU GEMV on this host's cores.

Also reported: the same sweep with one launch per tensor, the Qwen2-1.5B
Q4_0 sweep with its per-launch GB/s, the Q4_0 greedy decode (tok/s, with
the oracle CPU decoder on a bounded sample beside it, and the same decode
through the synchronous host-pointer ABI), the same decode at the Qwen3-4B layer
shapes in HyperVSQ-2, Q8-KV decode attention at the Qwen3-4B shape for 4096
and 32768 cached tokens, the weight upload rate, and the HyperVSQ-2 batch
sweep M = 1..16 (weights read once per launch).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "quant GEMV effective weight GB/s (% HBM peak); decode tok/s 1.5B-shape Q4_0"
PROFILE_TRAFFIC = os.path.join(ROOT, "profiles", "hvsq2_gemv_gate_up_2x9728x2560_traffic.json")


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--layers", type=int, default=36)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    p.add_argument("--cpu-seconds", type=float, default=4.0,
                   help="CPU GEMV work per thread setting in the baseline leg")
    p.add_argument("--no-extras", action="store_true",
                   help="only the headline sweep (no Q4_0 sweep, decode, attention, batch sweep)")
    p.add_argument("--no-decode", action="store_true", help="skip the decode workload")
    p.add_argument("--decode-new", type=int, default=128, help="greedy tokens of the decode workload")
    p.add_argument("--decode-prompt", type=int, default=32, help="prompt tokens of the decode workload")
    p.add_argument("--profile", choices=("gate-up", "fused", "decode", "decode-4b", "drop-in", "attention", "batch",
                                        "upload", "copy", "lm-head", "tree"),
                   help="profiling mode: run only one workload (for rocprofv3)")
    p.add_argument("--batch-m", default="1,2,4,8,16",
                   help="token counts of the batch sweep (comma-separated, each 1..16)")
    return p.parse_args()


def upload_layers(ctx, dtype, shapes, layers, seed) -> list:
    """`layers` layers of resident seeded tensors ({projection: handle})."""
    import numpy as np

    from qwanto_amd import synth
    rng = np.random.default_rng(seed)
    return [{p: ctx.upload(synth.weights(dtype, rng, *shapes[p]), dtype, *shapes[p]) for p in synth.PROJECTIONS}
            for _ in range(layers)]


class Sweep:
    """Resident weights, activation images and outputs of a GEMV sweep over
    `layers` layers of one model shape (`weights`: layers uploaded by the
    caller, who releases them)."""

    def __init__(self, torch, ctx, dtype, shapes, layers, seed, batch=1, weights=None):
        from qwanto_amd import synth
        self.torch, self.ctx, self.dtype, self.batch = torch, ctx, dtype, batch
        torch.manual_seed(seed)
        dev = torch.device("cuda:0")
        self.owned = weights is None
        if weights is None:
            weights = upload_layers(ctx, dtype, shapes, layers, seed)
        self.layers = []
        self.weight_bytes = 0
        self.shapes = shapes
        for handles in weights:
            layer = dict(handles)
            self.weight_bytes += sum(synth.weight_bytes(dtype, *shapes[p]) for p in synth.PROJECTIONS)
            # one image per distinct input: qkv (hidden), o (attention), gu (hidden), down (ffn)
            imgs = {}
            for key, proj in (("qkv", "q"), ("o", "o"), ("gu", "gate"), ("down", "down")):
                h = layer[proj]
                K = shapes[proj][1]
                ib = ctx.image_bytes(h)
                x = torch.randn(batch, K, device=dev, dtype=torch.float32)
                img = torch.zeros(batch, ib, device=dev, dtype=torch.uint8)
                sc = torch.zeros(batch, device=dev, dtype=torch.float32)
                ctx.quantize_image_device(h, x.data_ptr(), batch, K, img.data_ptr(), ib, sc.data_ptr(),
                                          stream=torch.cuda.current_stream().cuda_stream)
                imgs[key] = (img, sc, ib)
            layer["images"] = imgs
            layer["out"] = {p: torch.zeros(batch, shapes[p][0], device=dev, dtype=torch.float32)
                            for p in synth.PROJECTIONS}
            self.layers.append(layer)
        torch.cuda.synchronize()
        self._fused = []
        if batch == 1:
            # decoder-style launches (fused prologues, residual epilogues) over
            # one residual stream x, as qwn_decoder.hip issues them: each
            # launch reads what the one before it wrote
            D, Q, I = shapes["q"][1], shapes["o"][1], shapes["gate"][0]
            self.x = torch.randn(D, device=dev)
            self.attn = torch.randn(Q, device=dev)       # stands for the attention output
            self.gate = torch.zeros(I, device=dev)
            self.up = torch.zeros(I, device=dev)
            self.qkv_out = {p: torch.zeros(shapes[p][0], device=dev) for p in ("q", "k", "v")}
            self.norm = (1.0 + 0.1 * torch.randn(D, device=dev)).contiguous()
            for layer in self.layers:
                specs = (("qkv", ("q", "k", "v"), [self.qkv_out[p].data_ptr() for p in ("q", "k", "v")], "rmsnorm",
                          "store", self.x),
                         ("o", ("o",), [self.x.data_ptr()], "f32", "add", self.attn),
                         ("gu", ("gate", "up"), [self.gate.data_ptr(), self.up.data_ptr()], "rmsnorm", "swiglu",
                          self.x),
                         ("down", ("down",), [self.x.data_ptr()], "f32", "add", self.gate))
                for key, projs, outs, imode, omode, src in specs:
                    req, keep = ctx.gemv_group_request(
                        [layer[p] for p in projs], outs, imode, omode, x_ptr=src.data_ptr(),
                        norm_ptr=self.norm.data_ptr() if imode == "rmsnorm" else None, eps=1e-6)
                    self._fused.append((key, req, keep))
        self._requests = []
        for layer in self.layers:
            for key, projs in (("qkv", ("q", "k", "v")), ("o", ("o",)), ("gu", ("gate", "up")),
                               ("down", ("down",))):
                img, sc, ib = layer["images"][key]
                req, keep = ctx.gemv_group_request(
                    [layer[p] for p in projs], [layer["out"][p].data_ptr() for p in projs], "image",
                    batch=batch, image_ptr=img.data_ptr(), image_stride=ib, scales_ptr=sc.data_ptr())
                self._requests.append((key, req, keep))

    def grouped(self, stream, only=None):
        """Decode-order launches: qkv, o, gate/up, down per layer."""
        for key, req, _ in self._requests:
            if only is None or key == only:
                self.ctx.gemv_group_device(req, stream=stream)

    def fused(self, stream, only=None):
        """Decode-order launches as the resident decoder issues them: each
        builds its own int8 image from the fp32 activations in its prologue
        (RMSNorm for q/k/v and gate/up), o and down add into the residual,
        gate/up writes silu(gate) * up."""
        for key, req, _ in self._fused:
            if only is None or key == only:
                self.ctx.gemv_group_device(req, stream=stream)

    def per_tensor(self, stream, only=None):
        """One launch per tensor."""
        from qwanto_amd import synth
        for layer in self.layers:
            for proj in synth.PROJECTIONS:
                if only is not None and proj != only:
                    continue
                key = {"q": "qkv", "k": "qkv", "v": "qkv", "o": "o", "gate": "gu", "up": "gu",
                       "down": "down"}[proj]
                img, sc, ib = layer["images"][key]
                N = self.shapes[proj][0]
                self.ctx.gemm_image_device(layer[proj], img.data_ptr(), ib, layer["out"][proj].data_ptr(),
                                           self.batch, N, scales_ptr=sc.data_ptr(), stream=stream)

    def bytes_of(self, projs):
        from qwanto_amd import synth
        return sum(synth.weight_bytes(self.dtype, *self.shapes[p]) for p in projs)

    def close(self):
        """Release the resident tensors it uploaded (the ABI holds at most 512)."""
        from qwanto_amd import synth
        if self.owned:
            for layer in self.layers:
                for proj in synth.PROJECTIONS:
                    self.ctx.release(layer[proj])
        self.layers = []
        self._requests = []
        self._fused = []


def time_graph(torch, fn, steps, warmup):
    """Capture fn(stream) once, replay warmup + steps times; ms per replay
    (HIP events on the replay stream)."""
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
    return start.elapsed_time(end) / steps


def decode_model(seed=2026, prompt_len=32, cfg=None, dtype="q4_0", qk_norm=False):
    import numpy as np

    from qwanto_amd import synth
    cfg = cfg or synth.QWEN2_1P5B_CONFIG
    rng = np.random.default_rng(seed)
    model = synth.decoder_model(rng, cfg, dtype, qk_norm=qk_norm)
    prompt = synth.prompt_tokens(rng, cfg["vocab"], prompt_len)
    return model, prompt


DECODE_1P5B = "qwen2_1p5b_q4_0 random-init (seed 2026), tied F16 LM head, Q8 KV, greedy, HIP graph per token"
DECODE_4B = ("qwen3_4b-shaped hvsq2 decoder with per-head q/k norms, random-init (seed 2027), tied F16 LM "
             "head, Q8 KV, greedy, HIP graph per token")


def decode_bench(ctx, model, prompt, new_tokens=128, workload=DECODE_1P5B):
    """Greedy decode of the Qwen2-1.5B shaped random Q4_0 model (28 layers,
    tied F16 LM head, Q8 KV) on the resident decoder: the prompt, then
    `new_tokens` greedy steps; tok/s = generated / decode wall time, as
    c/qwanto_decode.c:2121-2122 reports it.  Run twice: the first pass
    captures the step graph."""
    from qwanto_amd import abi
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
        "workload": workload,
    }


def cpu_decode_baseline(model, prompt, steps=16):
    """The oracle decoder (oracle/qwn_oracle_decoder.c, the C restatement of
    c/qwanto_decode.c's CPU step, bit-identical to it) on the same model: the
    prompt, then `steps` greedy steps, timed; tok/s over the greedy steps
    (c/qwanto_decode.c:2121-2122).  At 8 OpenMP threads (the reference's
    published evidence) and at every CPU this process may use; the reported
    value is the faster.  The oracle splits the tied F16 LM head over the
    threads where the reference runs it on one thread, so this is a faster
    CPU baseline than qwnrun's own."""
    import numpy as np

    import oracle
    allowed = len(os.sched_getaffinity(0))
    by_threads = {}
    for threads in sorted({min(8, allowed), allowed}):
        dec = oracle.load().decoder(model, threads=threads)
        try:
            for t in prompt:
                logits = dec.forward(int(t))
            t0 = time.perf_counter()
            for _ in range(steps):
                logits = dec.forward(int(np.argmax(logits)))
            by_threads[threads] = steps / (time.perf_counter() - t0)
        finally:
            dec.close()
    best = max(by_threads, key=by_threads.get)
    return {"value": round(by_threads[best], 3), "unit": "tok/s", "cores": best, "kind": "port",
            "tok_s_by_threads": {str(k): round(v, 3) for k, v in by_threads.items()},
            "sample": f"oracle CPU decoder (C restatement of the reference step), {len(prompt)} prompt tokens "
                      f"then {steps} greedy steps of the same model, at 8 and {allowed} OpenMP threads",
            **cpu_host_info()}


def host_decode_bench(model, prompt, new_tokens=128):
    """The drop-in path: the host decoder (qwanto_amd/host, the reference
    host step in C) driving every projection, the LM head and the Q8 KV
    cache through the synchronous host-pointer ABI, as an unmodified qwnrun
    does; tok/s = generated / decode wall time."""
    from qwanto_amd.host_decoder import HostDecoder
    dec = HostDecoder(model)
    try:
        # the weights upload on first use, inside the prompt steps (not timed)
        dec.generate(prompt, new_tokens)
        m = dec.metrics()
    finally:
        dec.close()
    calls = m.abi_calls / max(1, m.prompt_tokens + m.generated_tokens)
    return {"tok_s": round(m.generated_tokens / (m.decode_wall_ms / 1e3), 1),
            "ms_per_token": round(m.decode_wall_ms / m.generated_tokens, 3),
            "abi_calls_per_token": round(calls, 1),
            "us_per_abi_call": round(m.decode_wall_ms * 1e3 / max(1, m.generated_tokens) / calls, 2),
            "gpu_matmul_count": int(m.gpu_matmul_count), "cpu_fallback_count": int(m.cpu_fallback_count),
            "backend_reason": m.backend_reason.decode(),
            "workload": "host decoder over the qwn_cuda ABI (synchronous, host pointers), same model and "
                        "prompt, greedy"}


def cpu_host_info() -> dict:
    """CPU model and the GPU-local NUMA node's physical cores on this host."""
    info = {"cpu_model": None, "cpu_family": None, "hypervisor": False, "numa_node": None,
            "node_physical_cores": None}
    try:
        for line in open("/proc/cpuinfo"):
            key, _, val = line.partition(":")
            key, val = key.strip(), val.strip()
            if key == "model name" and info["cpu_model"] is None:
                info["cpu_model"] = val
            elif key == "cpu family" and info["cpu_family"] is None:
                info["cpu_family"] = int(val)
            elif key == "flags" and not info["hypervisor"]:
                info["hypervisor"] = "hypervisor" in val.split()
    except (OSError, ValueError):
        pass
    cpus = gpu_local_cpus()
    if cpus is not None:
        node, cpus = cpus
        info["numa_node"] = node
        info["node_physical_cores"] = len(physical_cores(cpus))
    return info


def gpu_local_cpus():
    """(NUMA node of GPU 0, the CPUs of that node this process may use), or
    None where the node is unknown.  A device that reports no node (-1, as
    under a hypervisor) on a host with a single NUMA node is local to it."""
    try:
        import torch
        p = torch.cuda.get_device_properties(0)
        bus = "%04x:%02x:%02x.0" % (getattr(p, "pci_domain_id", 0), p.pci_bus_id, p.pci_device_id)
        node = int(open(f"/sys/bus/pci/devices/{bus}/numa_node").read())
        if node < 0:
            nodes = [n for n in os.listdir("/sys/devices/system/node") if n.startswith("node") and n[4:].isdigit()]
            if len(nodes) != 1:
                return None
            node = int(nodes[0][4:])
        allowed = os.sched_getaffinity(0)
        cpus = set()
        for part in open(f"/sys/devices/system/node/node{node}/cpulist").read().strip().split(","):
            a, _, b = part.partition("-")
            cpus.update(range(int(a), int(b or a) + 1))
        cpus &= allowed
        return (node, sorted(cpus)) if cpus else None
    except Exception:
        return None


def physical_cores(cpus) -> list:
    """One CPU per physical core among `cpus` (SMT siblings dropped)."""
    seen, out = set(), []
    for c in cpus:
        try:
            key = (open(f"/sys/devices/system/cpu/cpu{c}/topology/physical_package_id").read().strip(),
                   open(f"/sys/devices/system/cpu/cpu{c}/topology/core_id").read().strip())
        except OSError:
            key = ("?", str(c))
        if key not in seen:
            seen.add(key)
            out.append(c)
    return out


def attention_bench(torch, ctx, steps=50):
    """Q8-KV decode attention at the Qwen3-4B shape (32 query heads, 8 KV
    heads, head_dim 128) over 4096 and 32768 cached tokens; K/V N(0,1)
    quantized into the cache on the device, q N(0,1).  Bytes = 2176 per
    cached token (K and V int8 plus the per-group scales), read once.  One
    graph replays a call on each of enough distinct caches to cover 512 MB
    (twice the infinity cache), so every call reads its cache from HBM; the
    figure is per call, gaps between calls included."""
    H, HK, D = 32, 8, 128
    dev = torch.device("cuda:0")
    s = torch.cuda.current_stream()
    out = {}
    for T in (4096, 32768):
        bytes_ = 2176 * T
        n = max(2, -(-(512 << 20) // bytes_))
        k = torch.randn(T, HK * D, device=dev)
        v = torch.randn(T, HK * D, device=dev)
        caches = []
        for _ in range(n):
            cache = ctx.kv_create(T, HK, D)
            ctx.kv_append_device(cache, k.data_ptr(), v.data_ptr(), T, stream=s.cuda_stream)
            caches.append(cache)
        q = torch.randn(H * D, device=dev)
        o = torch.zeros(H * D, device=dev)
        work = torch.zeros(max(ctx.attention_workspace_bytes(caches[0], H, T - 1) // 4, 1), device=dev)

        def fn(st):
            for cache in caches:
                ctx.kv_attention_device(cache, q.data_ptr(), o.data_ptr(), H, T - 1, float(D ** -0.5),
                                        work.data_ptr(), stream=st)
        ms = time_graph(torch, fn, steps, 3) / n
        out[str(T)] = {"us_per_call": round(ms * 1e3, 3), "gbps": round(bytes_ / (ms / 1e3) / 1e9, 1),
                       "kv_bytes": bytes_, "caches": n}
        for cache in caches:
            ctx.kv_destroy(cache)
        del k, v
    return out


def lm_head_bench(torch, ctx, steps=20):
    """The LM head GEMV at the Qwen2-1.5B shape (151936 x 1536) in F16 and in
    BF16 (an untied lm_head.weight), fp32 image input; two copies of each
    (934 MB, beyond the infinity cache) alternate so every launch reads its
    weights from HBM.  GB/s of weight bytes per launch."""
    import numpy as np

    from qwanto_amd import synth
    V, D = 151936, 1536
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(5)
    out = {}
    for dtype in ("f16", "bf16"):
        hs = [ctx.upload(synth.weights(dtype, rng, V, D), dtype, V, D) for _ in range(2)]
        ib = ctx.image_bytes(hs[0])
        x = torch.randn(D, device=dev)
        img = torch.zeros(ib, dtype=torch.uint8, device=dev)
        ctx.prepare_image_device(hs[0], x.data_ptr(), 1, D, img.data_ptr(), ib,
                                 stream=torch.cuda.current_stream().cuda_stream)
        y = torch.zeros(V, device=dev)

        def fn(st):
            for _ in range(4):
                for h in hs:
                    ctx.gemm_image_device(h, img.data_ptr(), ib, y.data_ptr(), 1, V, stream=st)
        ms = time_graph(torch, fn, steps, 3) / 8
        out[dtype] = {"us_per_launch": round(ms * 1e3, 2), "gbps": round(V * D * 2 / (ms / 1e3) / 1e9, 1)}
        for h in hs:
            ctx.release(h)
    out["shape"] = [V, D]
    return out


def tree_verify_bench(ctx, model, prompt, reps=10):
    """Speculative verification on the resident decoder after the prompt: a
    64-node draft tree (qwn_hip_decoder_verify_tree: 3 roots, depth 8, one
    64-node block, the LM head on every node) against a 16-token chain
    verify block (qwn_hip_decoder_verify); ms per call including the
    synchronisation, the per-node greedy ids copied back (not the logits)."""
    import numpy as np

    from qwanto_amd import abi
    rng = np.random.default_rng(9)
    parents, level = [], []
    for k, n in enumerate((3, 5, 7, 9, 9, 10, 10, 11)):
        nxt = []
        for _ in range(n):
            parents.append(-1 if k == 0 else int(level[rng.integers(len(level))]))
            nxt.append(len(parents) - 1)
        level = nxt
    tokens = rng.integers(0, model["cfg"]["vocab"], len(parents)).astype(np.int32)
    dec = abi.ResidentDecoder(ctx, model)
    try:
        dec.prefill(prompt, logits=False)
        dec.verify_tree(tokens, parents, logits=False)  # graph capture
        t0 = time.perf_counter()
        for _ in range(reps):
            dec.verify_tree(tokens, parents, logits=False)
        ms_tree = (time.perf_counter() - t0) / reps * 1e3
        chain = tokens[:16]
        dec.verify(chain, logits=False)
        dec.truncate(len(prompt))
        t0 = time.perf_counter()
        for _ in range(reps):
            dec.verify(chain, logits=False)
            dec.truncate(len(prompt))
        ms_chain = (time.perf_counter() - t0) / reps * 1e3
    finally:
        dec.close()
    return {"tree_nodes": len(parents), "tree_depth": 8, "ms_per_tree": round(ms_tree, 3),
            "nodes_per_s": round(len(parents) / (ms_tree / 1e3), 1),
            "chain16_ms": round(ms_chain, 3), "chain16_tokens_per_s": round(16 / (ms_chain / 1e3), 1)}


class MfmaSweep:
    """Resident HyperVSQ-2 or Q4_0 tensors of `layers` layers with MFMA
    images of M tokens (8..16): int8-MFMA GEMM launches grouped as the
    decoder groups its GEMVs (q/k/v, o, gate/up, down: four per layer; o and
    down accumulate into their outputs, the residual adds)."""

    def __init__(self, torch, ctx, shapes, layers, seed, batch, kind="hvsq2", weights=None):
        from qwanto_amd import synth
        self.ctx, self.batch, self.shapes = ctx, batch, shapes
        torch.manual_seed(seed)
        dev = torch.device("cuda:0")
        s = torch.cuda.current_stream().cuda_stream
        self.items, self.handles = [], []
        self.weight_bytes = 0
        owned = weights is None
        if weights is None:
            weights = upload_layers(ctx, kind, shapes, layers, seed)
        layers = len(weights)
        for layer in weights:
            if owned:
                self.handles += list(layer.values())
            for key, projs in (("qkv", ("q", "k", "v")), ("o", ("o",)), ("gu", ("gate", "up")),
                               ("down", ("down",))):
                h0 = layer[projs[0]]
                K = shapes[projs[0]][1]
                x = torch.randn(batch, K, device=dev)
                q8 = torch.zeros(batch, (K + 255) // 256 * 256, dtype=torch.int8, device=dev)
                sc = torch.zeros(batch, device=dev)
                ctx.quantize_device(x.data_ptr(), batch, K, K, q8.data_ptr(), q8.shape[1], sc.data_ptr(), stream=s)
                img = torch.zeros(ctx.mfma_image_bytes(h0), dtype=torch.uint8, device=dev)
                ctx.mfma_image_device(h0, q8.data_ptr(), batch, q8.shape[1], img.data_ptr(), stream=s)
                outs = [torch.zeros(batch, shapes[p][0], device=dev) for p in projs]
                # o and down add into the residual stream, as the decoder runs them
                self.items.append(([layer[p] for p in projs], img, sc, outs, key in ("o", "down")))
                self.weight_bytes += sum(synth.weight_bytes(kind, *shapes[p]) for p in projs)
        torch.cuda.synchronize()
        self.flops = 2 * batch * sum(shapes[p][0] * shapes[p][1] for p in synth.PROJECTIONS) * layers

    def run(self, stream):
        for hs, img, sc, outs, acc in self.items:
            self.ctx.gemm_mfma_group_device(hs, img.data_ptr(), sc.data_ptr(), [o.data_ptr() for o in outs],
                                            self.batch, stream=stream, accumulate=acc)

    def close(self):
        for h in self.handles:
            self.ctx.release(h)
        self.items, self.handles = [], []


INT8_MFMA_PEAK_TOPS = 5000.0   # MI355X dense int8 MFMA


def upload_bench(ctx, layers=36, seed=3):
    """Weight upload from host memory (as qwnrun's mmap'd .qwn payloads):
    the 252 HyperVSQ-2 tensors of a Qwen3-4B-shaped model (1.05 GB), once
    through qwn_hip_ext_upload_batch (one pipelined call) and once tensor
    by tensor through qwn_cuda_abi_upload_tensor; GB/s of on-disk bytes
    including the repack into the wave-tile layout."""
    import numpy as np

    from qwanto_amd import synth
    rng = np.random.default_rng(seed)
    items = []
    for _ in range(layers):
        for proj in synth.PROJECTIONS:
            N, K = synth.QWEN3_4B_SHAPES[proj]
            items.append((synth.hvsq2_weights(rng, N, K), "hvsq2", N, K))
    total = sum(w.nbytes for w, _, _, _ in items)
    t0 = time.perf_counter()
    hs = ctx.upload_batch(items)
    t_batch = time.perf_counter() - t0
    for h in hs:
        ctx.release(h)
    t0 = time.perf_counter()
    hs = [ctx.upload(*it) for it in items]
    t_single = time.perf_counter() - t0
    for h in hs:
        ctx.release(h)
    return {"bytes": total, "tensors": len(items),
            "batch_gbps": round(total / t_batch / 1e9, 2), "batch_s": round(t_batch, 3),
            "per_tensor_gbps": round(total / t_single / 1e9, 2), "per_tensor_s": round(t_single, 3)}


def batch_sweep(torch, ctx, steps, warmup, ms_list=(1, 2, 4, 8, 16)):
    """GEMM at M = 1, 2, 4, 8, 16 tokens per launch (weights read once per
    launch), rotating through at least 1 GB of distinct layers so every
    launch reads its weights from HBM (beyond the 256 MB infinity cache):
    HyperVSQ-2 on 36 layers of the Qwen3-4B shapes (1.05 GB; 36 layers per
    token in tokens_per_s), and under "q4_0" Q4_0 on 40 layers of the
    Qwen2-1.5B shapes (1.05 GB; 28 layers per token); dot8 grouped launches
    below 2 (HyperVSQ-2) or 3 (Q4_0) tokens, grouped int8-MFMA launches from
    there (MFMA utilisation = useful int8 ops / dense int8 peak).  One set of weights
    per kind serves every M."""
    from qwanto_amd import synth

    def sweep(kind, shapes, layers, model_layers, seed0):
        res = {}
        weights = upload_layers(ctx, kind, shapes, layers, seed0)
        try:
            for M in ms_list:
                # the library's own choice (mfma_batch, weights with the MFMA-order copy)
                mfma = M >= (2 if kind == "hvsq2" else 3)
                if not mfma:
                    sw = Sweep(torch, ctx, kind, shapes, layers, seed=seed0 + M, batch=M, weights=weights)
                    ms = time_graph(torch, sw.grouped, steps, warmup)
                    path = "dot8"
                    flops = 2 * M * sum(shapes[p][0] * shapes[p][1] for p in synth.PROJECTIONS) * layers
                else:
                    sw = MfmaSweep(torch, ctx, shapes, layers, seed=seed0 + M, batch=M, kind=kind,
                                   weights=weights)
                    ms = time_graph(torch, sw.run, steps, warmup)
                    path = "mfma-i8"
                    flops = sw.flops
                tops = flops / (ms / 1e3) / 1e12
                res[str(M)] = {"gbps": round(sw.weight_bytes / (ms / 1e3) / 1e9, 1),
                               "us_per_layer": round(ms * 1e3 / layers, 3),
                               "tokens_per_s": round(M * layers / (ms / 1e3) / model_layers, 1),
                               "path": path, "int8_tops": round(tops, 2),
                               "mfma_util": round(tops / INT8_MFMA_PEAK_TOPS, 5) if mfma else None}
                sw.close()
        finally:
            for layer in weights:
                for h in layer.values():
                    ctx.release(h)
        res["layers"] = layers
        return res

    out = sweep("hvsq2", synth.QWEN3_4B_SHAPES, 36, 36, 50)
    out["q4_0"] = sweep("q4_0", synth.QWEN2_1P5B_SHAPES, 40, 28, 70)
    return out


def cpu_gemv_child(threads: int, seconds: float) -> dict:
    """One thread count of the CPU GEMV baseline (run in a child process so
    its OpenMP pool is pinned to the CPUs it was started on)."""
    import numpy as np

    import oracle
    from qwanto_amd import synth
    ora = oracle.load()
    rng = np.random.default_rng(99)
    layers = []
    for _ in range(4):
        layer = []
        for proj in synth.PROJECTIONS:
            N, K = synth.QWEN3_4B_SHAPES[proj]
            layer.append((synth.hvsq2_weights(rng, N, K), synth.activations(rng, 1, K), N))
        layers.append(layer)
    layer_bytes = sum(synth.weight_bytes("hvsq2", N, x.shape[1]) for _, x, N in layers[0])
    for w, x, N in layers[0]:
        ora.matmul_hvsq2(w, x, N, threads=threads)  # warm-up: thread pool, page faults
    done = 0
    t0 = time.perf_counter()
    while True:
        for w, x, N in layers[done % 4]:
            ora.matmul_hvsq2(w, x, N, threads=threads)
        done += 1
        if time.perf_counter() - t0 >= seconds:
            break
    dt = time.perf_counter() - t0
    return {"gbps": layer_bytes * done / dt / 1e9, "kernel": ora.variant_name(ora.best_variant())}


def cpu_baseline(seconds: float):
    """The reference's production CPU GEMV (qwn_matmul_hypervsq2_f32 with the
    vnni-delayed kernel, c/qwanto_kernels.c:841-918, 998-1176) as restated by
    the oracle, over a bounded sample: one Qwen3-4B layer's seven HyperVSQ-2
    projections from N(0,1) fp32 activations (quantization included),
    rotating through four distinct layer copies (117 MB, beyond the LLC).
    Twice: at 8 OpenMP threads (the reference's published evidence) and on
    every physical core of the GPU-local NUMA node this process may use
    (OMP_PLACES=cores, OMP_PROC_BIND=close), each in a child process pinned
    to those CPUs."""
    import subprocess

    local = gpu_local_cpus()
    allowed = sorted(os.sched_getaffinity(0))
    node_cores = physical_cores(local[1] if local else allowed)
    runs = {}
    for label, cpus in (("8", physical_cores(allowed)[:8] or allowed[:8]), ("node", node_cores)):
        threads = len(cpus)
        env = dict(os.environ, OMP_NUM_THREADS=str(threads), OMP_PLACES="cores", OMP_PROC_BIND="close",
                   GOMP_CPU_AFFINITY=" ".join(map(str, cpus)))
        code = ("import json, os, sys; os.sched_setaffinity(0, %r); sys.path.insert(0, %r); import bench; "
                "print(json.dumps(bench.cpu_gemv_child(%d, %r)))" % (cpus, ROOT, threads, seconds))
        res = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=300)
        if res.returncode != 0:
            raise RuntimeError("CPU baseline child failed: " + res.stderr[-2000:])
        runs[label] = dict(json.loads(res.stdout.strip().splitlines()[-1]), threads=threads)
    best = runs["node"]
    return {
        "value": round(best["gbps"], 3), "unit": "GB/s", "cores": best["threads"], "kind": "port",
        "kernel": best["kernel"],
        "sample": f"Qwen3-4B layer, 7 HyperVSQ-2 projections x 4 distinct copies (117 MB), batch 1, "
                  f"fp32 N(0,1) input quantized per call, ~{seconds:.0f}s per thread count; the oracle's "
                  f"restatement of the reference's vnni-delayed GEMV",
        "gbps_by_threads": {str(r["threads"]): round(r["gbps"], 3) for r in runs.values()},
        "numa_local": local is not None,
        **cpu_host_info(),
    }


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(json.dumps({"error": "qwn_hip runs on one GPU; this benchmark measures one MI355X "
                                   "(sharding across GPUs is a design only, not built)",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch

    from qwanto_amd import abi, synth
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs the GPU (no CPU fallback)")
    if args.profile == "copy":
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
    if args.profile == "decode":
        model, prompt = decode_model(prompt_len=args.decode_prompt)
        print(json.dumps({"profile_mode": "decode", **decode_bench(ctx, model, prompt, args.decode_new)}),
              flush=True)
        return
    if args.profile == "drop-in":
        model, prompt = decode_model(prompt_len=args.decode_prompt)
        print(json.dumps({"profile_mode": "drop-in", **host_decode_bench(model, prompt, args.decode_new)}),
              flush=True)
        return
    if args.profile == "decode-4b":
        model, prompt = decode_model(seed=2027, prompt_len=args.decode_prompt,
                                     cfg=synth.QWEN3_4B_SHAPED_CONFIG, dtype="hvsq2", qk_norm=True)
        print(json.dumps({"profile_mode": "decode-4b",
                          **decode_bench(ctx, model, prompt, args.decode_new, DECODE_4B)}), flush=True)
        return
    if args.profile == "attention":
        print(json.dumps({"profile_mode": "attention", **attention_bench(torch, ctx, args.steps)}), flush=True)
        return
    if args.profile == "upload":
        print(json.dumps({"profile_mode": "upload", **upload_bench(ctx)}), flush=True)
        return
    if args.profile == "lm-head":
        print(json.dumps({"profile_mode": "lm-head", **lm_head_bench(torch, ctx, args.steps)}), flush=True)
        return
    if args.profile == "tree":
        model, prompt = decode_model(prompt_len=args.decode_prompt)
        print(json.dumps({"profile_mode": "tree", **tree_verify_bench(ctx, model, prompt)}), flush=True)
        return
    if args.profile == "batch":
        ms_list = tuple(int(m) for m in args.batch_m.split(","))
        if not ms_list or any(m < 1 or m > 16 for m in ms_list):
            sys.exit("--batch-m: token counts between 1 and 16")
        print(json.dumps({"profile_mode": "batch", **batch_sweep(torch, ctx, args.steps, args.warmup, ms_list)}),
              flush=True)
        return
    t_setup = time.perf_counter()
    sweep = Sweep(torch, ctx, "hvsq2", synth.QWEN3_4B_SHAPES, args.layers, seed=1)
    print(f"# setup: {7 * args.layers} HyperVSQ-2 tensors, {sweep.weight_bytes / 1e9:.3f} GB "
          f"resident in {time.perf_counter() - t_setup:.1f}s", file=sys.stderr, flush=True)
    if args.profile == "gate-up":
        ms = time_graph(torch, lambda st: sweep.grouped(st, only="gu"), args.steps, args.warmup)
        print(json.dumps({"profile_mode": "gate-up", "ms_per_replay": ms}), flush=True)
        return
    if args.profile == "fused":
        ms = time_graph(torch, sweep.fused, args.steps, args.warmup)
        print(json.dumps({"profile_mode": "fused", "ms_per_step": ms,
                          "gbps": sweep.weight_bytes / (ms / 1e3) / 1e9}), flush=True)
        return

    ms_step = time_graph(torch, sweep.grouped, args.steps, args.warmup)
    value = sweep.weight_bytes / (ms_step / 1e3) / 1e9
    print(f"# grouped sweep: {ms_step:.4f} ms/step -> {value:.1f} GB/s", file=sys.stderr, flush=True)
    ms_tensor = time_graph(torch, sweep.per_tensor, args.steps, args.warmup)

    # per-launch kernel times (graph of the 36 launches of one kind / 36)
    per_launch = {}
    for key, projs in (("gu", ("gate", "up")), ("qkv", ("q", "k", "v")), ("down", ("down",)), ("o", ("o",))):
        ms = time_graph(torch, lambda st, k=key: sweep.grouped(st, only=k), args.steps, args.warmup) / args.layers
        b = sweep.bytes_of(projs)
        per_launch[key] = {"us": round(ms * 1e3, 3), "bytes": b, "gbps": round(b / (ms / 1e3) / 1e9, 1)}
    gu = per_launch["gu"]
    traffic = None
    if os.path.exists(PROFILE_TRAFFIC):
        traffic = json.load(open(PROFILE_TRAFFIC)).get("hbm_bytes_per_launch")
    roofline = {"bound": "hbm", "achieved": gu["gbps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gu["gbps"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                "kernel": "gemv_kernel<hvsq2> gate+up grouped launch, 2 x 9728x2560",
                "bytes_per_launch": gu["bytes"], "avg_launch_us": gu["us"]}

    # the same step with the decoder's launches: prologues that normalize and
    # quantize fp32 activations, epilogues that add into the residual stream
    ms_fused = time_graph(torch, sweep.fused, args.steps, args.warmup)
    fused_launch = {}
    for key, projs in (("gu", ("gate", "up")), ("qkv", ("q", "k", "v")), ("down", ("down",)), ("o", ("o",))):
        ms = time_graph(torch, lambda st, k=key: sweep.fused(st, only=k), args.steps, args.warmup) / args.layers
        b = sweep.bytes_of(projs)
        fused_launch[key] = {"us": round(ms * 1e3, 3), "gbps": round(b / (ms / 1e3) / 1e9, 1)}
    extra = {"per_tensor_launches": {"gbps": round(sweep.weight_bytes / (ms_tensor / 1e3) / 1e9, 1),
                                     "ms_per_step": round(ms_tensor, 4), "launches_per_step": 7 * args.layers},
             "per_launch_kernel": per_launch,
             "fused_prologue_sweep": {
                 "gbps": round(sweep.weight_bytes / (ms_fused / 1e3) / 1e9, 1), "ms_per_step": round(ms_fused, 4),
                 "hbm_frac_of_peak": round(sweep.weight_bytes / (ms_fused / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
                 "per_launch_kernel": fused_launch,
                 "workload": "the headline step with the resident decoder's launches: RMSNorm/quantize "
                             "prologues on fp32 activations and residual/SwiGLU epilogues over one residual "
                             "stream (each launch reads what the previous one wrote)"}}
    sweep_bytes = sweep.weight_bytes
    sweep.close()
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)
    if not args.no_extras:
        # 40 distinct Qwen2-1.5B-shaped layers (1.05 GB) in decode order
        q4_layers = 40
        q4 = Sweep(torch, ctx, "q4_0", synth.QWEN2_1P5B_SHAPES, q4_layers, seed=2)
        ms_q4 = time_graph(torch, q4.grouped, args.steps, args.warmup)
        # per-layer GEMV rate of the decode workload's projections (graph of
        # one kind's launches over every layer / layers); a kind's working
        # set is recorded with it: the smaller kinds' weights (q/k/v, o) fit
        # in the 256 MB infinity cache when replayed alone
        q4_launch = {}
        for key, projs in (("qkv", ("q", "k", "v")), ("o", ("o",)), ("gu", ("gate", "up")), ("down", ("down",))):
            ms = time_graph(torch, lambda st, k=key: q4.grouped(st, only=k), args.steps, args.warmup) / q4_layers
            b = q4.bytes_of(projs)
            q4_launch[key] = {"us": round(ms * 1e3, 3), "bytes": b, "gbps": round(b / (ms / 1e3) / 1e9, 1),
                              "working_set_bytes": b * q4_layers}
        extra["q4_0_sweep_qwen2_1p5b"] = {
            "gbps": round(q4.weight_bytes / (ms_q4 / 1e3) / 1e9, 1), "ms_per_step": round(ms_q4, 4),
            "weight_bytes": q4.weight_bytes, "layers": q4_layers, "launches_per_step": 4 * q4_layers,
            "per_layer_launch": q4_launch}
        q4.close()
        if not args.no_decode:
            model, prompt = decode_model(prompt_len=args.decode_prompt)
            dec = decode_bench(ctx, model, prompt, args.decode_new)
            dec["drop_in_abi"] = host_decode_bench(model, prompt, args.decode_new)
            dec["speculative_verify"] = tree_verify_bench(ctx, model, prompt)
            if not args.no_cpu:
                dec["cpu_baseline"] = cpu_decode_baseline(model, prompt)
            extra["decode_qwen2_1p5b_q4_0"] = dec
            del model
            # the HyperVSQ-2 GEMV workload's shapes as a dense decoder
            model, prompt = decode_model(seed=2027, prompt_len=args.decode_prompt,
                                         cfg=synth.QWEN3_4B_SHAPED_CONFIG, dtype="hvsq2", qk_norm=True)
            extra["decode_qwen3_4b_shaped_hvsq2"] = decode_bench(ctx, model, prompt, args.decode_new, DECODE_4B)
            del model
        extra["attention_q8_qwen3_4b"] = attention_bench(torch, ctx, args.steps)
        extra["lm_head_qwen2_1p5b"] = lm_head_bench(torch, ctx)
        extra["upload_hvsq2_qwen3_4b"] = upload_bench(ctx)
        extra["batch_sweep_hvsq2_qwen3_4b"] = batch_sweep(torch, ctx, args.steps, args.warmup)

    dev = lib.devices()[0].name.decode()
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "hvsq2_gemv_qwen3_4b_batch1_decode_order", "layers": args.layers,
                   "projections": {p: list(synth.QWEN3_4B_SHAPES[p]) for p in synth.PROJECTIONS},
                   "launches_per_step": 4 * args.layers,
                   "weight_bytes_per_step": sweep_bytes,
                   "hbm_frac_of_peak": round(value / HBM_PEAK_GBS, 4), "device": dev},
        "roofline": roofline,
        "cpu_baseline": cpu,
        **extra,
    }
    print(json.dumps(line), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
