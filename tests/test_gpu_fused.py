"""Grouped GEMV with fused inputs (qwn_hip_ext_gemv_group_device) through
the C ABI.

The fused prologue quantizes the fp32 input inside every workgroup, so the
int8 activations (and with them the integer sums and the fp32 outputs) must
be exactly those of the ABI GEMV fed with the oracle's quantization of the
same vector (c/qwanto_kernels.c:354-433): outputs are compared bit for bit
with that path, and within 1e-4 with the oracle's GEMV.  RMSNorm and SwiGLU
are pinned bit-exactly on inputs where their fp32 results do not depend on
summation order or on the exp implementation (x = +-2^k with eps = 0:
x/rms = +-1 exactly; gate >= 90: silu(g) = g exactly), and on random inputs
against the oracle's CPU RMSNorm / numpy SwiGLU, where a last-bit
difference may move an int8 value by one (loose bound, stated per test).
"""
import numpy as np
import pytest

from parity import gemv_close
from qwanto_amd import synth

pytestmark = pytest.mark.gpu


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def zeros(n):
    import torch
    return torch.zeros(n, dtype=torch.float32, device="cuda:0")


def stream():
    import torch
    return torch.cuda.current_stream().cuda_stream


def sync():
    import torch
    torch.cuda.synchronize()


def run_group(ctx, hs, rows, mode, out_mode="store", init=None, **kw):
    outs = [zeros(n) if init is None else dev(init[i]) for i, n in enumerate(rows)]
    sc = zeros(1)
    req, keep = ctx.gemv_group_request(hs, [o.data_ptr() for o in outs], mode, out_mode,
                                       scale_out_ptr=sc.data_ptr(), **kw)
    ctx.gemv_group_device(req, stream=stream())
    sync()
    return [o.cpu().numpy() for o in outs], float(sc.cpu().numpy()[0])


def abi_gemv(ctx, h, oracle_lib, y_in, N, K):
    """The ABI GEMV on the oracle's quantization of y_in (host int8 path)."""
    q8, xs, _ = oracle_lib.quantize(y_in[None])
    return ctx.gemm(h, q8, N, K, scales=xs, gemv=True)[0], float(xs[0])


def oracle_gemv(oracle_lib, kind, w, y_in, N, K):
    q8, xs, sums = oracle_lib.quantize(y_in[None])
    if kind == "hvsq2":
        return oracle_lib.gemv_hvsq2(w, q8[0], sums[0], float(xs[0]), K, N)
    return oracle_lib.gemv_q4_0_q8(w, q8[0], float(xs[0]), K, N)


GROUPS = [
    ("hvsq2", [(4096, 2560), (1024, 2560), (1024, 2560)]),   # Qwen3-4B q, k, v
    ("hvsq2", [(9728, 2560), (9728, 2560)]),                 # gate, up
    ("hvsq2", [(2560, 9728)]),                               # down
    ("q4_0", [(1536, 1536), (256, 1536), (256, 1536)]),      # Qwen2-1.5B q, k, v
    ("q4_0", [(1536, 8960)]),                                # down
    ("hvsq2", [(77, 512), (3, 512), (130, 512), (64, 512)]), # four ragged jobs
    ("q4_0", [(5, 96)]),                                     # K not a multiple of 128
    # paired tiles (a one-unit-per-lane layout run two units per lane over
    # two tiles, for grids beyond one workgroup per CU), ragged row counts:
    ("hvsq2", [(40001, 512)]),                               # one lane per row of the pair
    ("q4_0", [(5001, 4096)]),                                # 16 lanes per row
    ("hvsq2", [(12001, 1536)]),                              # second unit slot partly empty
]


@pytest.mark.parametrize("kind,shapes", GROUPS)
def test_group_f32_input_bit_exact(gpu_ctx, oracle_lib, kind, shapes):
    rng = np.random.default_rng(sum(n for n, _ in shapes) + shapes[0][1])
    K = shapes[0][1]
    ws = [synth.weights(kind, rng, N, K) for N, _ in shapes]
    hs = [gpu_ctx.upload(w, kind, N, K) for w, (N, _) in zip(ws, shapes)]
    try:
        x = rng.standard_normal(K).astype(np.float32)
        xd = dev(x)
        ys, scale = run_group(gpu_ctx, hs, [n for n, _ in shapes], "f32", x_ptr=xd.data_ptr())
        _, xs, _ = oracle_lib.quantize(x[None])
        assert np.float32(scale) == xs[0], "activation scale differs from the CPU quantization"
        for i, ((N, _), w, h) in enumerate(zip(shapes, ws, hs)):
            y_abi, _ = abi_gemv(gpu_ctx, h, oracle_lib, x, N, K)
            assert np.array_equal(ys[i], y_abi), f"job {i}: fused input differs from the int8 path"
            ok, worst = gemv_close(ys[i], oracle_gemv(oracle_lib, kind, w, x, N, K))
            assert ok, f"job {i}: worst {worst:.3g} of tolerance"
    finally:
        for h in hs:
            gpu_ctx.release(h)


@pytest.mark.parametrize("kind,N,K", [("hvsq2", 9728, 2560), ("q4_0", 8960, 1536), ("q4_0", 40, 64)])
def test_rmsnorm_input_exact_case(gpu_ctx, oracle_lib, kind, N, K):
    """x = +-2^-3 with eps = 0: mean(x^2) = 2^-6, 1/sqrt = 8, x/rms = +-1 and
    the normalized input is +-w exactly on any summation order."""
    rng = np.random.default_rng(N + K)
    w = synth.weights(kind, rng, N, K)
    h = gpu_ctx.upload(w, kind, N, K)
    try:
        x = (rng.choice([-1.0, 1.0], K) * 0.125).astype(np.float32)
        g = rng.standard_normal(K).astype(np.float32)
        xd, gd = dev(x), dev(g)
        ys, scale = run_group(gpu_ctx, [h], [N], "rmsnorm", x_ptr=xd.data_ptr(), norm_ptr=gd.data_ptr(),
                              eps=0.0)
        expect_in = (np.sign(x) * g).astype(np.float32)
        y_abi, xs = abi_gemv(gpu_ctx, h, oracle_lib, expect_in, N, K)
        assert np.float32(scale) == np.float32(xs)
        assert np.array_equal(ys[0], y_abi)
    finally:
        gpu_ctx.release(h)


@pytest.mark.parametrize("kind,N,K", [("hvsq2", 4096, 2560), ("q4_0", 1536, 1536)])
def test_rmsnorm_input_random(gpu_ctx, oracle_lib, kind, N, K):
    """Random x and norm weights against the oracle's RMSNorm (the CPU's
    eight-lane order, c/qwanto_decode.c:627-652): the scale agrees to 1e-6
    relative; an int8 value may move by one where the normalized input sits
    on a rounding boundary (each such move shifts every output by about
    1e-3 of the outputs' rms), so outputs are held to 2e-2 of their rms at
    most and 5e-3 at the median."""
    rng = np.random.default_rng(7 * N + K)
    w = synth.weights(kind, rng, N, K)
    h = gpu_ctx.upload(w, kind, N, K)
    try:
        x = rng.standard_normal(K).astype(np.float32)
        g = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)
        xd, gd = dev(x), dev(g)
        ys, scale = run_group(gpu_ctx, [h], [N], "rmsnorm", x_ptr=xd.data_ptr(), norm_ptr=gd.data_ptr(),
                              eps=1e-6)
        xn = oracle_lib.rmsnorm(x, g, 1e-6)
        ref = oracle_gemv(oracle_lib, kind, w, xn, N, K)
        _, xs, _ = oracle_lib.quantize(xn[None])
        assert abs(scale - float(xs[0])) <= 1e-6 * float(xs[0])
        rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
        assert float(np.max(np.abs(ys[0] - ref))) <= 2e-2 * rms
        assert float(np.median(np.abs(ys[0] - ref))) <= 5e-3 * rms
    finally:
        gpu_ctx.release(h)


@pytest.mark.parametrize("kind,N,K", [("hvsq2", 2560, 9728), ("q4_0", 1536, 8960)])
def test_swiglu_input(gpu_ctx, oracle_lib, kind, N, K):
    rng = np.random.default_rng(N * 3 + K)
    w = synth.weights(kind, rng, N, K)
    h = gpu_ctx.upload(w, kind, N, K)
    try:
        # exact case: gate >= 90, exp(-gate) vanishes against 1, silu(g) = g
        gate = (90.0 + 10.0 * rng.random(K)).astype(np.float32)
        up = rng.standard_normal(K).astype(np.float32)
        gd, ud = dev(gate), dev(up)
        ys, scale = run_group(gpu_ctx, [h], [N], "swiglu", x_ptr=gd.data_ptr(), x2_ptr=ud.data_ptr())
        y_abi, xs = abi_gemv(gpu_ctx, h, oracle_lib, (gate * up).astype(np.float32), N, K)
        assert np.float32(scale) == np.float32(xs)
        assert np.array_equal(ys[0], y_abi)
        # random case against the numpy SwiGLU (exp may differ in the last bit)
        gate = (2.0 * rng.standard_normal(K)).astype(np.float32)
        gd = dev(gate)
        ys, _ = run_group(gpu_ctx, [h], [N], "swiglu", x_ptr=gd.data_ptr(), x2_ptr=ud.data_ptr())
        hid = ((gate / (np.float32(1.0) + np.exp(-gate))) * up).astype(np.float32)
        ref = oracle_gemv(oracle_lib, kind, w, hid, N, K)
        rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
        assert float(np.max(np.abs(ys[0] - ref))) <= 2e-2 * rms
        assert float(np.median(np.abs(ys[0] - ref))) <= 5e-3 * rms
    finally:
        gpu_ctx.release(h)


@pytest.mark.parametrize("kind,N,K", [("hvsq2", 9728, 2560), ("q4_0", 8960, 1536), ("q4_0", 70, 512),
                                     ("hvsq2", 12001, 1536)])
def test_swiglu_output_pairs_gate_and_up(gpu_ctx, oracle_lib, kind, N, K):
    """Gate and up in one launch, SwiGLU in the epilogue: outputs[0] =
    silu(g) * u of the two GEMV outputs (exp within an ulp of numpy's)."""
    rng = np.random.default_rng(N + 11 * K)
    wg, wu = synth.weights(kind, rng, N, K), synth.weights(kind, rng, N, K)
    hg, hu = gpu_ctx.upload(wg, kind, N, K), gpu_ctx.upload(wu, kind, N, K)
    try:
        x = rng.standard_normal(K).astype(np.float32)
        xd = dev(x)
        ys, _ = run_group(gpu_ctx, [hg, hu], [N, N], "f32", "swiglu", x_ptr=xd.data_ptr())
        g, _ = abi_gemv(gpu_ctx, hg, oracle_lib, x, N, K)
        u, _ = abi_gemv(gpu_ctx, hu, oracle_lib, x, N, K)
        h = ((g / (np.float32(1.0) + np.exp(-g))) * u).astype(np.float32)
        ok, worst = gemv_close(ys[0], h, rtol=1e-5)
        assert ok, f"worst {worst:.3g} of tolerance"
        assert np.all(ys[1] == 0.0), "the up output must not be written"
    finally:
        gpu_ctx.release(hg)
        gpu_ctx.release(hu)


@pytest.mark.parametrize("kind,N,K", [("hvsq2", 2560, 4096), ("q4_0", 1536, 1536), ("q4_0", 5001, 4096)])
def test_residual_add_output(gpu_ctx, oracle_lib, kind, N, K):
    rng = np.random.default_rng(N + 5 * K)
    w = synth.weights(kind, rng, N, K)
    h = gpu_ctx.upload(w, kind, N, K)
    try:
        x = rng.standard_normal(K).astype(np.float32)
        r = rng.standard_normal(N).astype(np.float32)
        xd = dev(x)
        ys, _ = run_group(gpu_ctx, [h], [N], "f32", "add", init=[r], x_ptr=xd.data_ptr())
        y_abi, _ = abi_gemv(gpu_ctx, h, oracle_lib, x, N, K)
        assert np.array_equal(ys[0], (r + y_abi).astype(np.float32))
    finally:
        gpu_ctx.release(h)


@pytest.mark.parametrize("N,K,case", [(151936, 1536, "random"), (5000, 1536, "ties"), (777, 256, "equal")])
def test_f16_lm_head_argmax(gpu_ctx, oracle_lib, N, K, case):
    """The tied-LM-head shape: F16 GEMV with the RMSNorm prologue and the
    per-workgroup argmax; the reduced index is the first maximum of the
    logits the kernel wrote (c/qwanto_decode.c:2048-2065)."""
    import torch
    rng = np.random.default_rng(N + K)
    w = synth.f16_weights(rng, N, K)
    x = rng.standard_normal(K).astype(np.float32)
    if case == "ties":
        y0 = oracle_lib.matmul_f16(w, oracle_lib.rmsnorm(x, np.ones(K, np.float32), 1e-6))[0]
        best = int(np.argmax(y0))
        for r in (3, best // 2, N - 1):
            w[r] = w[best]
    elif case == "equal":
        w[:] = w[0]
    h = gpu_ctx.upload(w, "f16", N, K)
    try:
        xd, gd = dev(x), dev(np.ones(K, np.float32))
        probe, _ = gpu_ctx.gemv_group_request([h], [16], "rmsnorm", "argmax", x_ptr=xd.data_ptr(),
                                              norm_ptr=gd.data_ptr(), partials_ptr=16)
        n = gpu_ctx.gemv_group_partials(probe)
        assert n > 0
        parts = torch.zeros(n, dtype=torch.int64, device="cuda:0")
        idx = torch.full((1,), -1, dtype=torch.int32, device="cuda:0")
        logits = zeros(N)
        req, keep = gpu_ctx.gemv_group_request([h], [logits.data_ptr()], "rmsnorm", "argmax",
                                               x_ptr=xd.data_ptr(), norm_ptr=gd.data_ptr(), eps=1e-6,
                                               partials_ptr=parts.data_ptr())
        gpu_ctx.gemv_group_device(req, stream=stream())
        gpu_ctx.argmax_device(parts.data_ptr(), n, idx.data_ptr(), stream=stream())
        sync()
        y = logits.cpu().numpy()
        assert int(idx.cpu().numpy()[0]) == int(np.argmax(y))
        if case == "equal":
            assert int(idx.cpu().numpy()[0]) == 0
        ref = oracle_lib.matmul_f16(w, oracle_lib.rmsnorm(x, np.ones(K, np.float32), 1e-6))[0]
        ok, worst = gemv_close(y, ref, rtol=2e-4)
        assert ok, f"worst {worst:.3g} of tolerance"
    finally:
        gpu_ctx.release(h)


@pytest.mark.parametrize("kind,N,K", [("q4_0", 40001, 512), ("hvsq2", 40001, 512)])
def test_quantized_head_argmax_paired_tiles(gpu_ctx, oracle_lib, kind, N, K):
    """A quantized LM head (an untied Q4_0 / HyperVSQ-2 head) with the argmax
    epilogue on paired tiles: the logits equal the int8 path's bit for bit
    and the reduced index is their first maximum, with the best row copied
    to earlier rows in both tiles of other pairs."""
    import torch
    rng = np.random.default_rng(N + 3 * K)
    w = synth.weights(kind, rng, N, K).reshape(N, -1)
    x = rng.standard_normal(K).astype(np.float32)
    h = gpu_ctx.upload(w.reshape(-1), kind, N, K)
    try:
        y0, _ = abi_gemv(gpu_ctx, h, oracle_lib, x, N, K)
    finally:
        gpu_ctx.release(h)
    best = int(np.argmax(y0))
    for r in (best // 3, best // 2 + 1, N - 1):   # rows of other tiles and pairs
        w[r] = w[best]
    h = gpu_ctx.upload(w.reshape(-1), kind, N, K)
    try:
        xd = dev(x)
        probe, _ = gpu_ctx.gemv_group_request([h], [16], "f32", "argmax", x_ptr=xd.data_ptr(), partials_ptr=16)
        n = gpu_ctx.gemv_group_partials(probe)
        assert n > 0
        parts = torch.zeros(n, dtype=torch.int64, device="cuda:0")
        idx = torch.full((1,), -1, dtype=torch.int32, device="cuda:0")
        logits = zeros(N)
        req, keep = gpu_ctx.gemv_group_request([h], [logits.data_ptr()], "f32", "argmax", x_ptr=xd.data_ptr(),
                                               partials_ptr=parts.data_ptr())
        gpu_ctx.gemv_group_device(req, stream=stream())
        gpu_ctx.argmax_device(parts.data_ptr(), n, idx.data_ptr(), stream=stream())
        sync()
        y = logits.cpu().numpy()
        y_abi, _ = abi_gemv(gpu_ctx, h, oracle_lib, x, N, K)
        assert np.array_equal(y, y_abi), "argmax-epilogue logits differ from the int8 path"
        assert int(idx.cpu().numpy()[0]) == int(np.argmax(y)) == best // 3
    finally:
        gpu_ctx.release(h)


def test_group_rejects_mismatched_tensors(gpu_ctx):
    from qwanto_amd import abi
    rng = np.random.default_rng(3)
    a = gpu_ctx.upload(synth.hvsq2_weights(rng, 8, 512), "hvsq2", 8, 512)
    b = gpu_ctx.upload(synth.hvsq2_weights(rng, 8, 768), "hvsq2", 8, 768)
    c = gpu_ctx.upload(synth.q4_0_weights(rng, 8, 512), "q4_0", 8, 512)
    try:
        x = dev(np.zeros(768, np.float32))
        o1, o2 = zeros(8), zeros(8)
        for pair in ((a, b), (a, c)):
            req, keep = gpu_ctx.gemv_group_request(list(pair), [o1.data_ptr(), o2.data_ptr()], "f32",
                                                   x_ptr=x.data_ptr())
            with pytest.raises(abi.AbiError):
                gpu_ctx.gemv_group_device(req)
        # fp32 input needs columns that are a multiple of 32
        d = gpu_ctx.upload(synth.hvsq2_weights(rng, 8, 500), "hvsq2", 8, 500)
        req, keep = gpu_ctx.gemv_group_request([d], [o1.data_ptr()], "f32", x_ptr=x.data_ptr())
        with pytest.raises(abi.AbiError):
            gpu_ctx.gemv_group_device(req)
        gpu_ctx.release(d)
    finally:
        for h in (a, b, c):
            gpu_ctx.release(h)
