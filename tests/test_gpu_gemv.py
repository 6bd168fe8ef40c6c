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
    assert tm.gpu_resident_bytes == before.gpu_resident_bytes + w.size
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


@pytest.mark.parametrize("N,K", [(1, 1), (3, 31), (5, 32), (7, 100), (65, 129), (130, 520),
                                 (64, 4064), (2, 16384)])
def test_q4_0_edge_shapes(gpu_ctx, oracle_lib, N, K):
    check_q4_0(gpu_ctx, oracle_lib, N, K, seed=5 * N + K)


@pytest.mark.parametrize("M", [2, 3, 4, 8, 16, 17])
def test_hvsq2_batched(gpu_ctx, oracle_lib, M):
    """Multi-token verify shapes (q 4096x2560) with per-token input_scales."""
    check_hvsq2(gpu_ctx, oracle_lib, 4096, 2560, seed=100 + M, M=M)


@pytest.mark.parametrize("M", [2, 5, 16])
def test_q4_0_batched(gpu_ctx, oracle_lib, M):
    check_q4_0(gpu_ctx, oracle_lib, 1536, 8960, seed=200 + M, M=M)


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
    with pytest.raises(abi.AbiError):               # fp32 input for an int8 tensor
        gpu_ctx.gemm(h, q8.astype(np.float32), 8, 256)
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


def test_device_enumeration(hip_lib):
    devs = hip_lib.devices()
    assert devs, "no device enumerated"
    d = devs[0]
    assert d.total_vram_bytes > 0 and d.free_vram_bytes > 0
    assert b"gfx" in d.name
