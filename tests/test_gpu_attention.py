"""GPU parity of the Q8 KV cache (append + split-T attention) through the C
ABI, against the oracle's restatement of qwn_q8_cache_attention_head on the
same inputs.  Bar: 1e-4 absolute on the output (the reference's own
tolerance, c/tests/test_cuda_q8_kv.cu:158)."""
import numpy as np
import pytest

from parity import ATTN_ATOL
from qwanto_amd import abi

pytestmark = pytest.mark.gpu


def run_case(ctx, oracle_lib, T, H, HK, D, pos=None, seed=0, keys=None, values=None):
    rng = np.random.default_rng(seed)
    C = HK * D
    k = rng.standard_normal((T, C), dtype=np.float32) if keys is None else keys
    v = rng.standard_normal((T, C), dtype=np.float32) if values is None else values
    q = rng.standard_normal(H * D, dtype=np.float32)
    pos = T - 1 if pos is None else pos
    scale = np.float32(1.0 / np.sqrt(D))
    h = ctx.kv_create(T, HK, D)
    try:
        for t in range(T):
            ctx.kv_append(h, k[t], v[t], t)
        out = ctx.kv_attention(h, q, H, HK, D, pos, float(scale))
    finally:
        ctx.kv_destroy(h)
    kq, ks = oracle_lib.q8_quantize(k)
    vq, vs = oracle_lib.q8_quantize(v)
    ref = oracle_lib.q8_attention(q, kq, vq, ks, vs, H, HK, D, pos, scale)
    err = float(np.max(np.abs(out - ref)))
    assert err <= ATTN_ATOL, f"T={T} H={H} HK={HK} D={D} pos={pos}: max abs err {err:.3g}"
    return err


def test_known_answer(gpu_ctx, oracle_lib):
    """c/tests/test_cuda_q8_kv.cu:107-164."""
    T, H, HK, D = 2, 4, 2, 4
    i = np.arange(T * HK * D)
    k = ((i - 3) * np.float32(0.17)).astype(np.float32).reshape(T, HK * D)
    v = ((i + 2) * np.float32(-0.11)).astype(np.float32).reshape(T, HK * D)
    q = ((np.arange(H * D) - 5) * np.float32(0.09)).astype(np.float32)
    before = gpu_ctx.telemetry()
    h = gpu_ctx.kv_create(8, HK, D)
    for t in range(T):
        gpu_ctx.kv_append(h, k[t], v[t], t)
    tm = abi.Telemetry()
    out = gpu_ctx.kv_attention(h, q, H, HK, D, T - 1, 0.5, telemetry=tm)
    kq, ks = oracle_lib.q8_quantize(k)
    vq, vs = oracle_lib.q8_quantize(v)
    ref = oracle_lib.q8_attention(q, kq, vq, ks, vs, H, HK, D, T - 1, 0.5)
    assert np.max(np.abs(out - ref)) <= 1e-4
    assert tm.kv_cache_kernel_count - before.kv_cache_kernel_count >= 5
    assert tm.kv_cache_resident_bytes > before.kv_cache_resident_bytes
    gpu_ctx.kv_destroy(h)
    assert gpu_ctx.telemetry().kv_cache_resident_bytes == before.kv_cache_resident_bytes


def test_head_dim_65_and_nonfinite(gpu_ctx, oracle_lib):
    """c/tests/test_kv_cache.c:29-59: groups that span heads, NaN/Inf -> 0."""
    rng = np.random.default_rng(3)
    T, HK, D, H = 20, 2, 65, 4
    k = rng.standard_normal((T, HK * D), dtype=np.float32)
    v = rng.standard_normal((T, HK * D), dtype=np.float32)
    k[5, 0], k[5, 1], v[7, 0], v[7, 1] = np.nan, np.inf, -np.inf, np.nan
    run_case(gpu_ctx, oracle_lib, T, H, HK, D, keys=k, values=v)


@pytest.mark.parametrize("T,H,HK,D,pos", [
    (1, 4, 2, 128, None), (15, 32, 8, 128, None), (17, 32, 8, 128, 9), (300, 12, 2, 128, None),
    (1000, 32, 8, 128, 999), (4096, 32, 8, 128, None), (33, 8, 8, 64, None), (40, 16, 2, 96, 31),
    # MFMA path: 8 query heads per KV head (two row tiles) at D 256, one KV
    # head at D 64 over ten splits, the Qwen3-4B heads over 79 splits
    (70, 16, 2, 256, None), (2500, 8, 1, 64, 2400), (20000, 32, 8, 128, None),
])
def test_shapes(gpu_ctx, oracle_lib, T, H, HK, D, pos):
    run_case(gpu_ctx, oracle_lib, T, H, HK, D, pos=pos, seed=T + H + D)


def test_reset_and_reuse(gpu_ctx, oracle_lib):
    rng = np.random.default_rng(4)
    T, H, HK, D = 10, 8, 2, 128
    h = gpu_ctx.kv_create(T, HK, D)
    for _ in range(2):
        k = rng.standard_normal((T, HK * D), dtype=np.float32)
        v = rng.standard_normal((T, HK * D), dtype=np.float32)
        q = rng.standard_normal(H * D, dtype=np.float32)
        gpu_ctx.kv_reset(h)
        for t in range(T):
            gpu_ctx.kv_append(h, k[t], v[t], t)
        out = gpu_ctx.kv_attention(h, q, H, HK, D, T - 1, 0.125)
        kq, ks = oracle_lib.q8_quantize(k)
        vq, vs = oracle_lib.q8_quantize(v)
        ref = oracle_lib.q8_attention(q, kq, vq, ks, vs, H, HK, D, T - 1, 0.125)
        assert np.max(np.abs(out - ref)) <= ATTN_ATOL
    gpu_ctx.kv_destroy(h)


def test_append_contract(gpu_ctx):
    h = gpu_ctx.kv_create(2, 1, 8)
    z = np.zeros(8, dtype=np.float32)
    with pytest.raises(abi.AbiError):       # token must equal the current count
        gpu_ctx.kv_append(h, z, z, 1)
    gpu_ctx.kv_append(h, z, z, 0)
    gpu_ctx.kv_append(h, z, z, 1)
    with pytest.raises(abi.AbiError):       # full
        gpu_ctx.kv_append(h, z, z, 2)
    with pytest.raises(abi.AbiError):       # position beyond the appended tokens
        gpu_ctx.kv_attention(h, np.zeros(8, np.float32), 1, 1, 8, 2, 1.0)
    with pytest.raises(abi.AbiError):       # wrong channel count
        gpu_ctx.kv_append(h, np.zeros(9, np.float32), np.zeros(9, np.float32), 2)
    gpu_ctx.kv_destroy(h)


def test_device_attention_reused_workspace(gpu_ctx, oracle_lib):
    """qwn_hip_ext_kv_attention_device over many splits, several calls in a
    row on one workspace (varying positions, so the number of splits and the
    partials' layout vary too): each output against the oracle."""
    import torch
    rng = np.random.default_rng(21)
    T, H, HK, D = 9000, 32, 8, 128
    k = rng.standard_normal((T, HK * D), dtype=np.float32)
    v = rng.standard_normal((T, HK * D), dtype=np.float32)
    dev = torch.device("cuda:0")
    h = gpu_ctx.kv_create(T, HK, D)
    try:
        s = torch.cuda.current_stream().cuda_stream
        kd, vd = torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev)
        gpu_ctx.kv_append_device(h, kd.data_ptr(), vd.data_ptr(), T, stream=s)
        work = torch.zeros(gpu_ctx.attention_workspace_bytes(h, H, T - 1) // 4 + 1, device=dev)
        kq, ks = oracle_lib.q8_quantize(k)
        vq, vs = oracle_lib.q8_quantize(v)
        for pos in (T - 1, 4095, 700, T - 1, 2500):
            q = rng.standard_normal(H * D, dtype=np.float32)
            qd = torch.from_numpy(q).to(dev)
            out = torch.full((H * D,), float("nan"), device=dev)
            gpu_ctx.kv_attention_device(h, qd.data_ptr(), out.data_ptr(), H, pos, float(D ** -0.5),
                                        work.data_ptr(), stream=s)
            torch.cuda.synchronize()
            ref = oracle_lib.q8_attention(q, kq, vq, ks, vs, H, HK, D, pos, np.float32(D ** -0.5))
            err = float(np.max(np.abs(out.cpu().numpy() - ref)))
            assert err <= ATTN_ATOL, f"pos {pos}: max abs err {err:.3g}"
    finally:
        gpu_ctx.kv_destroy(h)
