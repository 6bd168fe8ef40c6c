"""GPU parity of the quantized GEMV/GEMM through the C ABI, against the CPU
oracle on identical seeded inputs.

Bar: integer sums (per HyperVSQ-2 octant, per Q4_0 block) bit-exact via the
library's debug dump, which runs the GEMV's own staging and dot code; fp32
outputs within 1e-4 * max(|y|, rms(y)) per element (tests/parity.py).
"""
import ctypes

import numpy as np
import pytest

from parity import gemv_close
from qwanto_amd import abi, synth

pytestmark = pytest.mark.gpu

QWEN3_SHAPES = sorted(set(synth.QWEN3_4B_SHAPES.values()))
QWEN2_SHAPES = sorted(set(synth.QWEN2_1P5B_SHAPES.values()))


def quantize(oracle_lib, x):
    q8, xs, sums = oracle_lib.quantize(x)
    return q8, xs, sums


def check_hvsq2(ctx, oracle_lib, N, K, seed, M=1):
    rng = np.random.default_rng(seed)
    w = synth.hvsq2_weights(rng, N, K)
    x = synth.activations(rng, M, K)
    q8, xs, sums = quantize(oracle_lib, x)
    h = ctx.upload(w, "hvsq2", N, K)
    try:
        nb = (K + 255) // 256
        got = ctx.debug_int_sums(h, q8[0], N * nb * 8).reshape(N, nb * 8)
        sq, _ = oracle_lib.hvsq2_octant_sums(w, q8[0], K, N)
        assert np.array_equal(got, sq), f"octant sums differ at {np.argwhere(got != sq)[:5]}"
        y = ctx.gemm(h, q8, N, K, scales=xs, gemv=(M == 1))
        for t in range(M):
            ref = oracle_lib.gemv_hvsq2(w, q8[t], sums[t], float(xs[t]), K, N)
            ok, worst = gemv_close(y[t], ref)
            assert ok, f"HyperVSQ-2 N={N} K={K} token {t}: worst {worst:.3g} of tolerance"
    finally:
        ctx.release(h)


def check_q4_0(ctx, oracle_lib, N, K, seed, M=1):
    rng = np.random.default_rng(seed)
    w = synth.q4_0_weights(rng, N, K)
    x = synth.activations(rng, M, K)
    q8, xs, sums = quantize(oracle_lib, x)
    h = ctx.upload(w, "q4_0", N, K)
    try:
        nb = (K + 31) // 32
        got = ctx.debug_int_sums(h, q8[0], N * nb).reshape(N, nb)
        assert np.array_equal(got, oracle_lib.q4_0_block_sums(w, q8[0], K, N))
        y = ctx.gemm(h, q8, N, K, scales=xs, gemv=(M == 1))
        for t in range(M):
            ref = oracle_lib.gemv_q4_0_q8(w, q8[t], float(xs[t]), K, N)
            ok, worst = gemv_close(y[t], ref)
            assert ok, f"Q4_0 N={N} K={K} token {t}: worst {worst:.3g} of tolerance"
    finally:
        ctx.release(h)


def test_abi_known_answer(gpu_ctx, oracle_lib):
    """c/tests/test_qwn_hypervsq2_cuda_abi.cu:84-149, through hypervsq2_gemm."""
    from test_oracle import abi_known_answer_case, abi_known_answer_expected
    w, x, scale, rows, cols = abi_known_answer_case()
    expect = abi_known_answer_expected(w, x, scale, rows, cols)
    before = gpu_ctx.telemetry()
    h = gpu_ctx.upload(w, "hvsq2", rows, cols)
    tm = abi.Telemetry()
    y = gpu_ctx.gemm(h, x, rows, cols, scale=scale, telemetry=tm)
    assert np.max(np.abs(y - expect)) <= 1e-3
    assert tm.gpu_matmul_count > before.gpu_matmul_count and tm.gpu_kernel_launch_count > 0
    assert tm.gpu_upload_count == before.gpu_upload_count + 1
    # the tensor's bytes and its MFMA-order copy, if one was made
    assert tm.gpu_resident_bytes == before.gpu_resident_bytes + w.size + gpu_ctx.tensor_info(h).mfma_copy_bytes
    assert tm.kernel_type.startswith(b"hvsq2-74")
    gpu_ctx.release(h)
    assert gpu_ctx.telemetry().gpu_resident_bytes == before.gpu_resident_bytes


@pytest.mark.parametrize("N,K", QWEN3_SHAPES)
def test_hvsq2_qwen3_4b_shapes(gpu_ctx, oracle_lib, N, K):
    check_hvsq2(gpu_ctx, oracle_lib, N, K, seed=N + K)


@pytest.mark.parametrize("N,K", [(1, 1), (3, 31), (5, 255), (7, 256), (65, 257), (130, 513),
                                 (64, 1000), (1, 4096), (300, 7936)])
def test_hvsq2_edge_shapes(gpu_ctx, oracle_lib, N, K):
    check_hvsq2(gpu_ctx, oracle_lib, N, K, seed=3 * N + K)


@pytest.mark.parametrize("N,K", QWEN2_SHAPES)
def test_q4_0_qwen2_1p5b_shapes(gpu_ctx, oracle_lib, N, K):
    check_q4_0(gpu_ctx, oracle_lib, N, K, seed=N * 7 + K)


def oracle_product(oracle_lib, kind, w, q8, sums, xs, K, N):
    if kind == "hvsq2":
        return oracle_lib.gemv_hvsq2(w, q8, sums, float(xs), K, N)
    return oracle_lib.gemv_q4_0_q8(w, q8, float(xs), K, N)


def run_mfma_group(ctx, oracle_lib, kind, Ns, K, M, seed, accumulate=False):
    """One qwn_hip_ext_mfma_image_device + gemm_mfma_group_device pass over
    tensors of one kind and equal columns; every token of every tensor
    against the oracle (with accumulate: the oracle product added to the
    outputs' prior contents)."""
    import torch
    rng = np.random.default_rng(seed)
    make = synth.hvsq2_weights if kind == "hvsq2" else synth.q4_0_weights
    ws = [make(rng, N, K) for N in Ns]
    x = synth.activations(rng, M, K)
    q8, xs, sums = oracle_lib.quantize(x)
    hs = [ctx.upload(w, kind, N, K) for w, N in zip(ws, Ns)]
    try:
        dev = torch.device("cuda:0")
        q8d = torch.from_numpy(q8).to(dev)
        xsd = torch.from_numpy(xs).to(dev)
        img = torch.zeros(ctx.mfma_image_bytes(hs[0]), dtype=torch.uint8, device=dev)
        if accumulate:
            init = [rng.standard_normal((M, N)).astype(np.float32) for N in Ns]
            ys = [torch.from_numpy(i.copy()).to(dev) for i in init]
        else:
            init = [np.zeros((M, N), np.float32) for N in Ns]
            ys = [torch.full((M, N), float("nan"), dtype=torch.float32, device=dev) for N in Ns]
        s = torch.cuda.current_stream().cuda_stream
        ctx.mfma_image_device(hs[0], q8d.data_ptr(), M, q8.shape[1], img.data_ptr(), stream=s)
        ctx.gemm_mfma_group_device(hs, img.data_ptr(), xsd.data_ptr(), [y.data_ptr() for y in ys], M,
                                   stream=s, accumulate=accumulate)
        torch.cuda.synchronize()
        for w, N, y, i0 in zip(ws, Ns, ys, init):
            yh = y.cpu().numpy()
            for t in range(M):
                ref = oracle_product(oracle_lib, kind, w, q8[t], sums[t], xs[t], K, N)
                ok, worst = gemv_close(yh[t] - i0[t], ref)
                assert ok, f"{kind} tensor {N}x{K} token {t}: worst {worst:.3g}"
    finally:
        for h in hs:
            ctx.release(h)


@pytest.mark.parametrize("Ns,K,M", [((4096, 1024, 1024), 2560, 16), ((9728, 9728), 2560, 16),
                                    ((8200, 77), 777, 9), ((16390, 5), 520, 11), ((300,), 16384, 8),
                                    ((2560,), 9728, 12), ((4096, 1024, 1024), 2560, 3),
                                    ((9728, 9728), 2560, 4), ((2560,), 9728, 5), ((40, 7), 16640, 5)])
def test_hvsq2_mfma_group(gpu_ctx, oracle_lib, Ns, K, M):
    """qwn_hip_ext_gemm_mfma_group_device: one MFMA launch over tensors of
    equal columns sharing one image (q/k/v and gate/up shapes, 32- and
    64-row-group launches with ragged rows, unaligned row counts and partial
    blocks, K beyond one chunk of blocks per wave), every token of every
    tensor against the oracle; 65 units of one row per wave tile, whose odd
    meta tiles are read straight from HBM instead of staged)."""
    run_mfma_group(gpu_ctx, oracle_lib, "hvsq2", Ns, K, M, seed=sum(Ns) + K + M)


@pytest.mark.parametrize("Ns,K,M", [((2560,), 4096, 16), ((77, 1030), 9728, 9), ((2560,), 9728, 16),
                                    ((2560,), 9728, 4), ((1000, 40), 2000, 5), ((65, 130), 700, 12),
                                    ((300,), 16384, 10), ((4100,), 2560, 16), ((33,), 1800, 3)])
def test_hvsq2_mfma_group_accumulate(gpu_ctx, oracle_lib, Ns, K, M):
    """accumulate = 1: outputs += the product (the decoder's residual adds,
    the prior outputs loaded ahead of the products): the o and down shapes
    at 4 and 16 tokens, ragged rows and partial blocks, 3..16 tokens, and K
    beyond what one workgroup stages in LDS."""
    run_mfma_group(gpu_ctx, oracle_lib, "hvsq2", Ns, K, M, seed=sum(Ns) + K + M + 1, accumulate=True)


def mfma_group_outputs(ctx, kind, ws, Ns, K, q8, xs, accumulate, init):
    """Outputs of one grouped MFMA launch over freshly uploaded tensors (so
    the upload-time choice of the MFMA-order copy applies)."""
    import torch
    M = q8.shape[0]
    hs = [ctx.upload(w, kind, N, K) for w, N in zip(ws, Ns)]
    try:
        dev = torch.device("cuda:0")
        q8d = torch.from_numpy(q8).to(dev)
        xsd = torch.from_numpy(xs).to(dev)
        img = torch.zeros(ctx.mfma_image_bytes(hs[0]), dtype=torch.uint8, device=dev)
        ys = [torch.from_numpy(i.copy()).to(dev) for i in init]
        s = torch.cuda.current_stream().cuda_stream
        ctx.mfma_image_device(hs[0], q8d.data_ptr(), M, q8.shape[1], img.data_ptr(), stream=s)
        ctx.gemm_mfma_group_device(hs, img.data_ptr(), xsd.data_ptr(), [y.data_ptr() for y in ys], M,
                                   stream=s, accumulate=accumulate)
        torch.cuda.synchronize()
        return [y.cpu().numpy() for y in ys]
    finally:
        for h in hs:
            ctx.release(h)


@pytest.mark.parametrize("Ns,K,M,accumulate", [((9728, 9728), 2560, 4, False), ((2560,), 9728, 16, True),
                                               ((77, 1030), 700, 9, False), ((40, 7), 16640, 5, True),
                                               ((4096, 1024, 1024), 2560, 3, False), ((33,), 256, 12, True)])
def test_hvsq2_mfma_direct_matches_staged(gpu_ctx, oracle_lib, monkeypatch, Ns, K, M, accumulate):
    """HyperVSQ-2 tensors uploaded with the MFMA-order copy (the GEMM reads
    its operands straight from HBM) and without it (QWN_HIP_MFMA_COPY=0: the
    GEMM stages the wave tiles in LDS, or for long rows reads them from the
    wave-tile layout): both within the oracle's tolerance, and within float
    rounding of each other (the int32 block products are the same, checked
    exactly by the dump tests; the two kernels split K over different wave
    counts, so their float partials are added in a different order)."""
    rng = np.random.default_rng(sum(Ns) + K + M + 11)
    ws = [synth.hvsq2_weights(rng, N, K) for N in Ns]
    q8, xs, sums = oracle_lib.quantize(synth.activations(rng, M, K))
    init = [rng.standard_normal((M, N)).astype(np.float32) if accumulate else np.zeros((M, N), np.float32)
            for N in Ns]
    direct = mfma_group_outputs(gpu_ctx, "hvsq2", ws, Ns, K, q8, xs, accumulate, init)
    monkeypatch.setenv("QWN_HIP_MFMA_COPY", "0")
    staged = mfma_group_outputs(gpu_ctx, "hvsq2", ws, Ns, K, q8, xs, accumulate, init)
    for w, N, yd, ys, i0 in zip(ws, Ns, direct, staged, init):
        # a few float roundings of the partial sums apart, relative to the row
        np.testing.assert_allclose(yd, ys, rtol=0, atol=2e-6 * (1.0 + float(np.max(np.abs(ys)))),
                                   err_msg=f"{N}x{K} M={M}: direct vs staged")
        for t in range(M):
            ref = oracle_product(oracle_lib, "hvsq2", w, q8[t], sums[t], xs[t], K, N)
            ok, worst = gemv_close(yd[t] - i0[t], ref)
            assert ok, f"{N}x{K} token {t}: worst {worst:.3g}"


@pytest.mark.parametrize("Ns,K,M,accumulate", [((8960, 8960), 1536, 16, False), ((1536,), 8960, 16, True),
                                               ((1536,), 1536, 8, True), ((1536, 256, 256), 1536, 16, False),
                                               ((77, 1030), 700, 9, False), ((65, 130), 33, 12, True),
                                               ((300,), 16384, 10, False), ((4100,), 1536, 16, True)])
def test_q4_0_mfma_direct_matches_staged(gpu_ctx, oracle_lib, monkeypatch, Ns, K, M, accumulate):
    """Q4_0 tensors uploaded with the MFMA-order copy (operands straight from
    HBM) and without it (QWN_HIP_MFMA_COPY=0: staged in LDS): both within
    the oracle's tolerance and within float rounding of each other (the
    int32 block products are exact on both paths, checked by the dump tests;
    the paths split K over different waves, and the four-way split of
    residual adds over fewer than 256 row groups adds its partials with
    float atomics, in no fixed order)."""
    rng = np.random.default_rng(sum(Ns) + K + M + 13)
    ws = [synth.q4_0_weights(rng, N, K) for N in Ns]
    q8, xs, sums = oracle_lib.quantize(synth.activations(rng, M, K))
    init = [rng.standard_normal((M, N)).astype(np.float32) if accumulate else np.zeros((M, N), np.float32)
            for N in Ns]
    direct = mfma_group_outputs(gpu_ctx, "q4_0", ws, Ns, K, q8, xs, accumulate, init)
    monkeypatch.setenv("QWN_HIP_MFMA_COPY", "0")
    staged = mfma_group_outputs(gpu_ctx, "q4_0", ws, Ns, K, q8, xs, accumulate, init)
    for w, N, yd, ys, i0 in zip(ws, Ns, direct, staged, init):
        np.testing.assert_allclose(yd, ys, rtol=0, atol=2e-6 * (1.0 + float(np.max(np.abs(ys)))),
                                   err_msg=f"{N}x{K} M={M}: direct vs staged")
        for y in (yd, ys):
            for t in range(M):
                ref = oracle_product(oracle_lib, "q4_0", w, q8[t], sums[t], xs[t], K, N)
                ok, worst = gemv_close(y[t] - i0[t], ref)
                assert ok, f"{N}x{K} token {t}: worst {worst:.3g}"


@pytest.mark.parametrize("kind,K,M", [("hvsq2", 2560, 16), ("hvsq2", 16640, 6), ("q4_0", 1536, 16),
                                      ("q4_0", 100, 11)])
def test_mfma_staged_int32_block_dots(gpu_ctx, oracle_lib, monkeypatch, kind, K, M):
    """The staged (and, for 65-unit HyperVSQ-2 rows, the wave-tile) MFMA
    kernels' int32 block dots, with the MFMA-order copy turned off at
    upload."""
    monkeypatch.setenv("QWN_HIP_MFMA_COPY", "0")
    rng = np.random.default_rng(K + M + 5)
    N = 77
    w = synth.weights(kind, rng, N, K)
    q8, xs, sums = quantize(oracle_lib, synth.activations(rng, M, K))
    h = gpu_ctx.upload(w, kind, N, K)
    try:
        nblk = (K + 255) // 256 if kind == "hvsq2" else (K + 31) // 32
        got = gpu_ctx.debug_mfma_sums(h, q8[:, :K], N, nblk)
        for t in range(M):
            if kind == "hvsq2":
                sq, _ = oracle_lib.hvsq2_octant_sums(w, q8[t], K, N)
                ref = hvsq2_block_products(w, sq, N, K)
            else:
                ref = oracle_lib.q4_0_block_sums(w, q8[t], K, N)
            assert np.array_equal(got[t], ref), f"{kind} token {t}"
    finally:
        gpu_ctx.release(h)


@pytest.mark.parametrize("Ns,K,M", [((1536, 256, 256), 1536, 16), ((8960, 8960), 1536, 16),
                                    ((1536,), 8960, 16), ((8200, 77), 777, 9), ((16390, 5), 520, 11),
                                    ((3,), 31, 8), ((65, 130), 33, 12), ((300,), 16384, 10), ((64,), 224, 13)])
def test_q4_0_mfma_group(gpu_ctx, oracle_lib, Ns, K, M):
    """Q4_0 on the int8 MFMA GEMM (one 16x16x32 MFMA per 32-weight block):
    the Qwen2-1.5B q/k/v, gate/up and down shapes, ragged rows, K not a
    multiple of 32 (the last block partial) or of 128 (the last 4-block unit
    partial), K-splits of 1..8 waves, partial token tiles."""
    run_mfma_group(gpu_ctx, oracle_lib, "q4_0", Ns, K, M, seed=sum(Ns) + K + M + 2)


@pytest.mark.parametrize("Ns,K,M", [((1536,), 8960, 16), ((77, 1030), 1536, 9), ((1536,), 1536, 16),
                                    ((2560,), 9728, 16), ((65, 130), 33, 12), ((3,), 31, 8),
                                    ((1000, 40), 777, 5), ((300,), 16384, 10), ((4100,), 1536, 16)])
def test_q4_0_mfma_group_accumulate(gpu_ctx, oracle_lib, Ns, K, M):
    """accumulate = 1 (the residual adds): launches of fewer than 256 row
    groups take the four-way K split (each split's partial added with float
    atomics), the rest the single-pass kernel; ragged rows, K not a multiple
    of 32 or 128, partial token tiles."""
    run_mfma_group(gpu_ctx, oracle_lib, "q4_0", Ns, K, M, seed=sum(Ns) + K + M + 3, accumulate=True)


@pytest.mark.parametrize("N,K", [(1, 1), (3, 31), (5, 32), (7, 100), (65, 129), (130, 520),
                                 (64, 4064), (2, 16384)])
def test_q4_0_edge_shapes(gpu_ctx, oracle_lib, N, K):
    check_q4_0(gpu_ctx, oracle_lib, N, K, seed=5 * N + K)


@pytest.mark.parametrize("M", [2, 3, 4, 8, 16, 17])
def test_hvsq2_batched(gpu_ctx, oracle_lib, M):
    """Multi-token verify shapes (q 4096x2560) with per-token input_scales."""
    check_hvsq2(gpu_ctx, oracle_lib, 4096, 2560, seed=100 + M, M=M)


@pytest.mark.parametrize("M", [2, 3, 4, 5, 8, 16, 17])
def test_q4_0_batched(gpu_ctx, oracle_lib, M):
    """Through qwn_cuda_abi_gemm: the dot8 GEMV at 2 tokens, the MFMA GEMM
    on the MFMA-order copy from 3, in 16-token tiles (17: a full tile and a
    1-token tile)."""
    check_q4_0(gpu_ctx, oracle_lib, 1536, 8960, seed=200 + M, M=M)


@pytest.mark.parametrize("M", [2, 3])
def test_hvsq2_batched_without_copy(gpu_ctx, oracle_lib, monkeypatch, M):
    """Uploaded without the MFMA-order copy (QWN_HIP_MFMA_COPY=0): the dot8
    GEMV at 2 tokens, the staged MFMA GEMM from 3 (with the copy the MFMA
    GEMM takes 2 tokens already: test_hvsq2_batched)."""
    monkeypatch.setenv("QWN_HIP_MFMA_COPY", "0")
    check_hvsq2(gpu_ctx, oracle_lib, 4096, 2560, seed=110 + M, M=M)


@pytest.mark.parametrize("M", [4, 5, 6])
def test_q4_0_batched_without_copy(gpu_ctx, oracle_lib, monkeypatch, M):
    """Uploaded without the MFMA-order copy (QWN_HIP_MFMA_COPY=0): the dot8
    GEMV up to 5 tokens, the staged MFMA GEMM from 6."""
    monkeypatch.setenv("QWN_HIP_MFMA_COPY", "0")
    check_q4_0(gpu_ctx, oracle_lib, 1536, 8960, seed=210 + M, M=M)


@pytest.mark.parametrize("N,K,M", [(77, 700, 8), (130, 513, 9), (1, 256, 8), (64, 256, 16), (300, 7936, 12),
                                   (2560, 4096, 16), (77, 700, 3), (130, 513, 4), (300, 7936, 7)])
def test_hvsq2_mfma_ragged(gpu_ctx, oracle_lib, N, K, M):
    """HyperVSQ-2 from 3 tokens runs on int8 MFMA tiles (16 rows x 16
    tokens): ragged rows, partial blocks, partial token tiles."""
    check_hvsq2(gpu_ctx, oracle_lib, N, K, seed=N + K + M, M=M)


def test_hvsq2_mfma_fp32_input(gpu_ctx, oracle_lib):
    """INPUT_F32 at 10 tokens: quantized per token on the device, then the
    MFMA path; the whole CPU matmul is the reference."""
    rng = np.random.default_rng(91)
    N, K, M = 1024, 2560, 10
    w = synth.hvsq2_weights(rng, N, K)
    x = synth.activations(rng, M, K)
    h = gpu_ctx.upload(w, "hvsq2", N, K)
    try:
        y = gpu_ctx.gemm(h, x, N, K)
        ref = oracle_lib.matmul_hvsq2(w, x, N)
        for t in range(M):
            ok, worst = gemv_close(y[t], ref[t])
            assert ok, f"token {t}: worst {worst:.3g}"
    finally:
        gpu_ctx.release(h)


def test_hvsq2_mfma_device_entry_points(gpu_ctx, oracle_lib):
    """qwn_hip_ext_mfma_image_device + qwn_hip_ext_gemm_mfma_device on device
    pointers, against the oracle."""
    import torch
    rng = np.random.default_rng(92)
    N, K, M = 2560, 9728, 16
    w = synth.hvsq2_weights(rng, N, K)
    x = synth.activations(rng, M, K)
    q8, xs, sums = oracle_lib.quantize(x)
    h = gpu_ctx.upload(w, "hvsq2", N, K)
    try:
        dev = torch.device("cuda:0")
        q8d = torch.from_numpy(q8).to(dev)
        xsd = torch.from_numpy(xs).to(dev)
        img = torch.zeros(gpu_ctx.mfma_image_bytes(h), dtype=torch.uint8, device=dev)
        y = torch.zeros(M, N, dtype=torch.float32, device=dev)
        s = torch.cuda.current_stream().cuda_stream
        gpu_ctx.mfma_image_device(h, q8d.data_ptr(), M, q8.shape[1], img.data_ptr(), stream=s)
        gpu_ctx.gemm_mfma_device(h, img.data_ptr(), xsd.data_ptr(), y.data_ptr(), M, stream=s)
        torch.cuda.synchronize()
        yh = y.cpu().numpy()
        for t in range(M):
            ref = oracle_lib.gemv_hvsq2(w, q8[t], sums[t], float(xs[t]), K, N)
            ok, worst = gemv_close(yh[t], ref)
            assert ok, f"token {t}: worst {worst:.3g}"
    finally:
        gpu_ctx.release(h)


def test_hvsq2_batched_down_proj(gpu_ctx, oracle_lib):
    check_hvsq2(gpu_ctx, oracle_lib, 2560, 9728, seed=77, M=8)


@pytest.mark.parametrize("N,K,M", [(1000, 1536, 1), (77, 70, 2), (4096, 2560, 1), (33, 4096, 4)])
def test_f16_gemv(gpu_ctx, oracle_lib, N, K, M):
    rng = np.random.default_rng(N + K + M)
    w = synth.f16_weights(rng, N, K)
    x = synth.activations(rng, M, K)
    h = gpu_ctx.upload(w, "f16", N, K)
    y = gpu_ctx.gemm(h, x, N, K)
    ref = oracle_lib.matmul_f16(w, x, threads=0)
    for t in range(M):
        ok, worst = gemv_close(y[t], ref[t])
        assert ok, worst
    gpu_ctx.release(h)


@pytest.mark.parametrize("N,K,M", [(1000, 1536, 1), (77, 70, 2), (4096, 2560, 1), (33, 4096, 4), (300, 8960, 16)])
def test_bf16_gemv(gpu_ctx, oracle_lib, N, K, M):
    """BF16 rows (c/qwanto_kernels.c:287-290, 1508-1527) through the ABI with
    fp32 activations, against the oracle's restatement of qwn_matmul_f32 on
    BF16 (pinned to the reference build); subnormal and negative-zero
    weights included."""
    rng = np.random.default_rng(N * 3 + K + M)
    w = synth.bf16_weights(rng, N, K)
    w[0, :3] = (0x0001, 0x8000, 0x807F)
    x = synth.activations(rng, M, K)
    h = gpu_ctx.upload(w, "bf16", N, K)
    try:
        info = gpu_ctx.tensor_info(h)
        assert info.dtype == abi.TENSOR_BF16 and info.logical_bytes == N * K * 2
        tm = abi.Telemetry()
        y = gpu_ctx.gemm(h, x, N, K, telemetry=tm)
        assert tm.kernel_type.startswith(b"bf16")
        ref = oracle_lib.matmul_bf16(w, x, threads=0)
        for t in range(M):
            ok, worst = gemv_close(y[t], ref[t])
            assert ok, f"token {t}: worst {worst:.3g} of tolerance"
        # the same bits read as F16 give other products: the conversion is the BF16 one
        assert not np.allclose(y, oracle_lib.matmul_f16(w.view(np.float16), x, threads=0), rtol=1e-2)
    finally:
        gpu_ctx.release(h)


def test_request_validation(gpu_ctx, hip_lib):
    rng = np.random.default_rng(1)
    w = synth.hvsq2_weights(rng, 8, 256)
    h = gpu_ctx.upload(w, "hvsq2", 8, 256)
    q8 = np.zeros((2, 256), dtype=np.int8)
    with pytest.raises(abi.AbiError) as e:          # rows mismatch
        gpu_ctx.gemm(h, q8[:1], 9, 256, scale=1.0)
    assert e.value.status == -1
    with pytest.raises(abi.AbiError):               # gemv demands batch == 1
        gpu_ctx.gemm(h, q8, 8, 256, scale=1.0, gemv=True)
    hf = gpu_ctx.upload(synth.f16_weights(rng, 8, 256), "f16", 8, 256)
    with pytest.raises(abi.AbiError):               # int8 input for an F16 tensor
        gpu_ctx.gemm(hf, q8[:1], 8, 256, scale=1.0)
    gpu_ctx.release(hf)
    gpu_ctx.release(h)
    with pytest.raises(abi.AbiError):               # released handle
        gpu_ctx.gemm(h, q8[:1], 8, 256, scale=1.0)
    with pytest.raises(abi.AbiError) as e:          # short payload
        gpu_ctx.upload(w[:100], "hvsq2", 8, 256)
    assert e.value.status == -1
    up = abi.TensorUpload(host_data=w.ctypes.data, data_bytes=w.size, dtype=1, rows=8, cols=256,
                          block_bytes=73)
    out = abi.Handle()
    assert hip_lib.lib.qwn_cuda_abi_upload_tensor(ctypes.byref(gpu_ctx.handle), ctypes.byref(up),
                                                  ctypes.byref(out)) == -5


def test_memory_budget(hip_lib):
    with abi.Context(hip_lib, device=0, budget=1000) as ctx:
        rng = np.random.default_rng(2)
        w = synth.hvsq2_weights(rng, 16, 256)   # 1184 bytes > budget
        with pytest.raises(abi.AbiError) as e:
            ctx.upload(w, "hvsq2", 16, 256)
        assert e.value.status == -4
        ctx.upload(synth.hvsq2_weights(rng, 8, 256), "hvsq2", 8, 256)  # 592 bytes fits


def _free_bytes():
    import torch
    torch.cuda.synchronize()
    return torch.cuda.mem_get_info(0)[0]


def test_mfma_copy_charged_to_budget(hip_lib):
    """The batched GEMM's MFMA-order copy is charged like the tensor's own
    bytes (c/cuda/qwn_hypervsq2_cuda_abi.cu:554-562 caps every device byte a
    tensor holds): tensors plus copies never exceed the budget,
    gpu_resident_bytes reports both and equals the device memory the upload
    took (hipMemGetInfo) up to the device layout's padding and allocation
    rounding, release gives both back, and an upload of one tensor at a time
    under a budget gets no copy (a later tensor would lose room to it)."""
    rng = np.random.default_rng(11)
    shapes = [(9728, 2560, "hvsq2"), (9728, 2560, "hvsq2"), (8960, 1536, "q4_0"), (2560, 9728, "hvsq2")]
    items = [(synth.weights(kind, rng, n, k), kind, n, k) for n, k, kind in shapes]
    logical = [w.nbytes for w, _, _, _ in items]
    granule = 2 << 20  # hipMalloc rounding per allocation, at most
    # no budget: every tensor copied (half the device stays free)
    with abi.Context(hip_lib, device=0) as ctx:
        ctx.upload_batch(items[:1])  # the upload pipeline's staging buffers, allocated once
        base = ctx.telemetry().gpu_resident_bytes
        free0 = _free_bytes()
        hs = ctx.upload_batch(items[1:])
        took = free0 - _free_bytes()
        infos = [ctx.tensor_info(h) for h in hs]
        assert all(i.mfma_copy_bytes > 0 for i in infos)
        reported = ctx.telemetry().gpu_resident_bytes - base
        assert reported == sum(i.logical_bytes + i.mfma_copy_bytes for i in infos)
        device = sum(i.device_bytes + i.mfma_copy_bytes for i in infos)
        assert abs(took - device) <= 2 * len(infos) * granule, (took, device)
        assert abs(device - reported) <= 0.03 * reported, (device, reported)
        ctx.release(hs[0])
        assert ctx.telemetry().gpu_resident_bytes == base + reported - infos[0].logical_bytes - infos[0].mfma_copy_bytes
    # a budget with room for the tensors and some copies: copies only from what
    # the batch's tensors leave, never past the budget
    with abi.Context(hip_lib, device=0) as probe:
        copy_sizes = [probe.tensor_info(h).mfma_copy_bytes for h in probe.upload_batch(items)]
    for extra in (0, copy_sizes[0], copy_sizes[0] + copy_sizes[1] + 4096, sum(copy_sizes)):
        budget = sum(logical) + extra
        with abi.Context(hip_lib, device=0, budget=budget) as ctx:
            hs = ctx.upload_batch(items)
            infos = [ctx.tensor_info(h) for h in hs]
            copies = sum(i.mfma_copy_bytes for i in infos)
            assert ctx.telemetry().gpu_resident_bytes == sum(logical) + copies <= budget
            assert copies <= extra and (extra - copies) < max(copy_sizes)  # none left out that fit
            # a GEMM on a tensor with and without its copy gives the same rows
            x = rng.integers(-127, 128, size=(4, 2560), dtype=np.int8)
            y = ctx.gemm(hs[0], x, 9728, 2560, scales=np.full(4, 0.01, np.float32))
            with abi.Context(hip_lib, device=0) as ref_ctx:
                h = ref_ctx.upload(items[0][0], "hvsq2", 9728, 2560)
                y_ref = ref_ctx.gemm(h, x, 9728, 2560, scales=np.full(4, 0.01, np.float32))
            np.testing.assert_allclose(y, y_ref, rtol=1e-5, atol=1e-5)
    # one tensor at a time under a budget: no copies, every tensor fits
    with abi.Context(hip_lib, device=0, budget=sum(logical) + sum(copy_sizes)) as ctx:
        hs = [ctx.upload(w, kind, n, k) for w, kind, n, k in items]
        assert all(ctx.tensor_info(h).mfma_copy_bytes == 0 for h in hs)
        assert ctx.telemetry().gpu_resident_bytes == sum(logical)


def test_device_enumeration(hip_lib):
    devs = hip_lib.devices()
    assert devs, "no device enumerated"
    d = devs[0]
    assert d.total_vram_bytes > 0 and d.free_vram_bytes > 0
    assert b"gfx" in d.name


@pytest.mark.parametrize("kind,K,M", [("hvsq2", 2560, 1), ("hvsq2", 9728, 3), ("hvsq2", 300, 16),
                                      ("q4_0", 1536, 1), ("q4_0", 8960, 5), ("q4_0", 100, 16)])
def test_device_image_path(gpu_ctx, oracle_lib, kind, K, M):
    """Device pointers end to end: fp32 x -> quantize_image_device (scales,
    int8 tokens, image) -> gemm_image_device for two tensors of the same width
    sharing the one image.  Scales and int8 tokens bit-exact against the
    oracle's quantizer, outputs against the oracle GEMV."""
    import torch
    rng = np.random.default_rng(K * 31 + M)
    x = synth.activations(rng, M, K)
    q8_ref, xs_ref, sums = quantize(oracle_lib, x)
    dev = torch.device("cuda:0")
    rows = (129, 64)
    ws = [synth.weights(kind, rng, n, K) for n in rows]
    hs = [gpu_ctx.upload(w, kind, n, K) for w, n in zip(ws, rows)]
    try:
        ib = gpu_ctx.image_bytes(hs[0])
        assert ib == gpu_ctx.image_bytes(hs[1]) and ib % 16 == 0
        xs_stride = (K + 3) // 4 * 4
        xd = torch.zeros(M, xs_stride, dtype=torch.float32)
        xd[:, :K] = torch.from_numpy(x)
        xd = xd.to(dev)
        q8_stride = q8_ref.shape[1]
        q8 = torch.full((M, q8_stride), 77, dtype=torch.int8, device=dev)
        sc = torch.zeros(M, dtype=torch.float32, device=dev)
        img = torch.zeros(M, ib, dtype=torch.uint8, device=dev)
        s = torch.cuda.current_stream().cuda_stream
        gpu_ctx.quantize_image_device(hs[0], xd.data_ptr(), M, xs_stride, img.data_ptr(), ib,
                                      sc.data_ptr(), q8.data_ptr(), q8_stride, stream=s)
        torch.cuda.synchronize()
        assert np.array_equal(sc.cpu().numpy(), xs_ref)
        assert np.array_equal(q8.cpu().numpy(), q8_ref)
        # an image prepared from the int8 tokens is the same image
        img2 = torch.zeros_like(img)
        gpu_ctx.prepare_image_device(hs[1], q8.data_ptr(), M, q8_stride, img2.data_ptr(), ib,
                                     stream=s)
        torch.cuda.synchronize()
        assert torch.equal(img, img2)
        for h, w, n in zip(hs, ws, rows):
            y = torch.full((M, n + 3), float("nan"), dtype=torch.float32, device=dev)
            gpu_ctx.gemm_image_device(h, img.data_ptr(), ib, y.data_ptr(), M, n + 3,
                                      scales_ptr=sc.data_ptr(), stream=s)
            torch.cuda.synchronize()
            yh = y.cpu().numpy()
            assert np.isnan(yh[:, n:]).all(), "wrote past the row end"
            for t in range(M):
                if kind == "hvsq2":
                    ref = oracle_lib.gemv_hvsq2(w, q8_ref[t], sums[t], float(xs_ref[t]), K, n)
                else:
                    ref = oracle_lib.gemv_q4_0_q8(w, q8_ref[t], float(xs_ref[t]), K, n)
                ok, worst = gemv_close(yh[t, :n], ref)
                assert ok, f"{kind} K={K} rows={n} token {t}: worst {worst:.3g}"
    finally:
        for h in hs:
            gpu_ctx.release(h)


def test_null_stream_ordered_with_context_stream(gpu_ctx, oracle_lib):
    """A device entry point given stream NULL runs on the context's stream,
    which is ordered with the null stream (torch's default stream): an input
    written on the null stream behind several milliseconds of other work is
    read only once it is written (scales bit-exact against the oracle's)."""
    import torch
    assert torch.cuda.current_stream().cuda_stream == 0, "torch's default stream is the null stream"
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(4242)
    K, N = 2560, 64
    h = gpu_ctx.upload(synth.weights("hvsq2", rng, N, K), "hvsq2", N, K)
    x = synth.activations(rng, 1, K)
    _, xs_ref, _ = quantize(oracle_lib, x)
    try:
        src = torch.from_numpy(x).to(dev)
        xd = torch.zeros(1, K, dtype=torch.float32, device=dev)
        ib = gpu_ctx.image_bytes(h)
        img = torch.zeros(1, ib, dtype=torch.uint8, device=dev)
        sc = torch.zeros(1, dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        a = torch.randn(4096, 4096, dtype=torch.float32, device=dev)
        for _ in range(8):
            a = (a @ a) * 1e-3   # fp32 products keep the null stream busy
        xd.copy_(src)            # the input, written behind them
        gpu_ctx.quantize_image_device(h, xd.data_ptr(), 1, K, img.data_ptr(), ib, sc.data_ptr())
        torch.cuda.synchronize()
        assert np.array_equal(sc.cpu().numpy(), xs_ref)
    finally:
        gpu_ctx.release(h)


def test_device_image_f16(gpu_ctx, oracle_lib):
    import torch
    rng = np.random.default_rng(5)
    N, K, M = 300, 1000, 4
    w = synth.f16_weights(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    h = gpu_ctx.upload(w, "f16", N, K)
    try:
        ib = gpu_ctx.image_bytes(h)
        dev = torch.device("cuda:0")
        xd = torch.from_numpy(x).to(dev)
        img = torch.zeros(M, ib, dtype=torch.uint8, device=dev)
        y = torch.zeros(M, N, dtype=torch.float32, device=dev)
        s = torch.cuda.current_stream().cuda_stream
        gpu_ctx.prepare_image_device(h, xd.data_ptr(), M, K, img.data_ptr(), ib, stream=s)
        gpu_ctx.gemm_image_device(h, img.data_ptr(), ib, y.data_ptr(), M, N, stream=s)
        torch.cuda.synchronize()
        ref = oracle_lib.matmul_f16(w, x)
        ok, worst = gemv_close(y.cpu().numpy(), ref)
        assert ok, f"F16 image path: worst {worst:.3g}"
    finally:
        gpu_ctx.release(h)


@pytest.mark.parametrize("kind,N,K,M", [("hvsq2", 1024, 2560, 1), ("hvsq2", 77, 700, 3),
                                        ("q4_0", 1536, 1536, 1), ("q4_0", 40, 8960, 2), ("q4_0", 300, 1000, 16),
                                        ("hvsq2", 300, 1000, 12)])
def test_abi_fp32_input_quantized_on_device(gpu_ctx, oracle_lib, kind, N, K, M):
    """INPUT_F32 with a quantized tensor: the library quantizes per token on
    the device (c/qwanto_kernels.c:354-433) -- the whole CPU matmul
    (qwn_matmul_*_f32) is the reference."""
    rng = np.random.default_rng(N + K + M)
    w = synth.weights(kind, rng, N, K)
    x = synth.activations(rng, M, K)
    h = gpu_ctx.upload(w, kind, N, K)
    try:
        y = gpu_ctx.gemm(h, x, N, K, gemv=(M == 1))
        ref = oracle_lib.matmul_hvsq2(w, x, N) if kind == "hvsq2" else oracle_lib.matmul_q4_0(w, x, N)
        for t in range(M):
            ok, worst = gemv_close(y[t], ref[t])
            assert ok, f"{kind} {N}x{K} token {t}: worst {worst:.3g}"
    finally:
        gpu_ctx.release(h)


def hvsq2_block_products(w, sum_q, N, K):
    """Per 256-weight block: sum over octants of multiplier * sum (code-1)*a,
    the exact integer the MFMA path forms (multipliers: 4 bytes at offset 4
    of each 74-byte block, low nibble = even octant)."""
    nb = (K + 255) // 256
    blocks = w.reshape(N, nb, 74)
    sub = np.stack([(blocks[:, :, 4 + o // 2] >> (4 * (o % 2))) & 15 for o in range(8)], axis=-1)
    return (sub.astype(np.int64) * sum_q.reshape(N, nb, 8).astype(np.int64)).sum(axis=-1)


@pytest.mark.parametrize("kind,N,K,M", [("hvsq2", 300, 2560, 16), ("hvsq2", 77, 4096, 9), ("hvsq2", 40, 700, 12),
                                        ("hvsq2", 300, 2560, 3), ("hvsq2", 77, 9728, 4), ("hvsq2", 40, 16640, 6),
                                        ("q4_0", 200, 1536, 16), ("q4_0", 1536, 8960, 16), ("q4_0", 33, 100, 11)])
def test_mfma_int32_block_dots(gpu_ctx, oracle_lib, kind, N, K, M):
    """The MFMA GEMM's per-block int32 dots, dumped by the same kernel (same
    plan, staging and operand code), bit-exact against the oracle's integer
    sums for every token."""
    rng = np.random.default_rng(N + K + M)
    w = synth.weights(kind, rng, N, K)
    q8, xs, sums = quantize(oracle_lib, synth.activations(rng, M, K))
    h = gpu_ctx.upload(w, kind, N, K)
    try:
        nblk = (K + 255) // 256 if kind == "hvsq2" else (K + 31) // 32
        got = gpu_ctx.debug_mfma_sums(h, q8[:, :K], N, nblk)
        for t in range(M):
            if kind == "hvsq2":
                sq, _ = oracle_lib.hvsq2_octant_sums(w, q8[t], K, N)
                ref = hvsq2_block_products(w, sq, N, K)
            else:
                ref = oracle_lib.q4_0_block_sums(w, q8[t], K, N)
            bad = np.argwhere(got[t] != ref)
            assert bad.size == 0, f"{kind} N={N} K={K} token {t}: block dots differ at {bad[:5]}"
    finally:
        gpu_ctx.release(h)


def test_device_quantize_rounds_halves_to_even(gpu_ctx):
    """Per-token int8 quantization (c/qwanto_kernels.c:354-433, the CPU's
    rintf) on the device: with max|x| = 127 the scale is exactly 1, so every
    value x.5 is a tie and must round to the even integer, as numpy's rint
    does; the kernel rounds by adding 1.5 * 2^23, which this pins for every
    tie in range and both signs."""
    import torch
    halves = np.arange(-126.5, 127.0, 1.0, dtype=np.float32)   # 254 ties
    K = 512
    x = np.zeros((2, K), np.float32)
    x[0, 0], x[1, 0] = 127.0, -127.0
    x[0, 1:1 + halves.size] = halves
    x[1, 1:1 + halves.size] = -halves[::-1]
    x[:, 300:310] = [0.49999997, -0.49999997, 0.5, -0.5, 1.4999999, -1.5000001, 2.5, 3.5, -2.5, -0.0]
    dev = torch.device("cuda:0")
    xd = torch.from_numpy(x).to(dev)
    q8 = torch.full((2, K), 99, dtype=torch.int8, device=dev)
    sc = torch.zeros(2, dtype=torch.float32, device=dev)
    gpu_ctx.quantize_device(xd.data_ptr(), 2, K, K, q8.data_ptr(), K, sc.data_ptr(),
                            stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert sc.cpu().numpy().tolist() == [1.0, 1.0]
    want = np.clip(np.rint(x), -127, 127).astype(np.int8)
    got = q8.cpu().numpy()
    bad = np.nonzero(got != want)
    assert bad[0].size == 0, f"first mismatches at {list(zip(*bad))[:5]}: got {got[bad][:5]}, want {want[bad][:5]}"
