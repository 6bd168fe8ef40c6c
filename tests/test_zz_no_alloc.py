"""qwn_hip_ext_kv_attention_device_noalloc (the attention entry point whose
split partials live in the library's file-scope device array, for callers
that cannot allocate) against qwn_hip_ext_kv_attention_device with a
workspace, through the C ABI: two calls in a row, the second smaller, each
bit-identical to the workspace variant and within 1e-4 of the oracle
(c/tests/test_cuda_q8_kv.cu:158); a request beyond the array is refused, and
so is a call that would run while another stream's call still uses the
array."""
import ctypes

import numpy as np
import pytest

from parity import ATTN_ATOL
from qwanto_amd import abi

pytestmark = pytest.mark.gpu


def noalloc(ctx, cache, q_ptr, out_ptr, H, pos, scale, stream):
    """The C-ABI call itself (argument types bound in qwanto_amd.abi)."""
    return ctx.lib.lib.qwn_hip_ext_kv_attention_device_noalloc(ctx._h, ctypes.byref(cache), q_ptr, out_ptr, H,
                                                               pos, scale, stream)


def test_noalloc_attention_matches_workspace_variant(gpu_ctx, oracle_lib):
    import torch
    dev = torch.device("cuda:0")
    s = torch.cuda.current_stream().cuda_stream
    rng = np.random.default_rng(77)
    T, HK, D = 9000, 8, 128
    k = rng.standard_normal((T, HK * D), dtype=np.float32)
    v = rng.standard_normal((T, HK * D), dtype=np.float32)
    kq, ks = oracle_lib.q8_quantize(k)
    vq, vs = oracle_lib.q8_quantize(v)
    h = gpu_ctx.kv_create(T, HK, D)
    try:
        kd, vd = torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev)  # alive until the append ran
        gpu_ctx.kv_append_device(h, kd.data_ptr(), vd.data_ptr(), T, stream=s)
        torch.cuda.synchronize()
        del kd, vd
        # the second call is smaller: fewer tokens (fewer splits) and fewer query heads
        for H, pos in ((32, T - 1), (8, 700)):
            q = rng.standard_normal(H * D, dtype=np.float32)
            qd = torch.from_numpy(q).to(dev)
            scale = float(D ** -0.5)
            work = torch.zeros(gpu_ctx.attention_workspace_bytes(h, H, pos) // 4 + 1, device=dev)
            ref_out = torch.full((H * D,), float("nan"), device=dev)
            gpu_ctx.kv_attention_device(h, qd.data_ptr(), ref_out.data_ptr(), H, pos, scale, work.data_ptr(),
                                        stream=s)
            out = torch.full((H * D,), float("nan"), device=dev)
            rc = noalloc(gpu_ctx, h, qd.data_ptr(), out.data_ptr(), H, pos, scale, s)
            assert rc == 0, gpu_ctx.lib.last_error()
            torch.cuda.synchronize()
            a, b = out.cpu().numpy(), ref_out.cpu().numpy()
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"H={H} pos={pos}: outputs differ"
            ref = oracle_lib.q8_attention(q, kq, vq, ks, vs, H, HK, D, pos, np.float32(scale))
            assert float(np.max(np.abs(a - ref))) <= ATTN_ATOL
    finally:
        gpu_ctx.kv_destroy(h)


def test_noalloc_attention_refuses_oversize(gpu_ctx):
    """48 query heads on 2 KV heads over 5000 tokens need 7.8 MB of
    partials, more than the 4 MiB array: refused, nothing launched."""
    import torch
    dev = torch.device("cuda:0")
    T, HK, D, H = 5000, 2, 128, 48
    h = gpu_ctx.kv_create(T, HK, D)
    try:
        z = torch.zeros(T, HK * D, device=dev)
        gpu_ctx.kv_append_device(h, z.data_ptr(), z.data_ptr(), T, stream=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert gpu_ctx.attention_workspace_bytes(h, H, T - 1) > 4 << 20
        q = torch.zeros(H * D, device=dev)
        out = torch.zeros(H * D, device=dev)
        rc = noalloc(gpu_ctx, h, q.data_ptr(), out.data_ptr(), H, T - 1, 1.0, None)
        assert rc == -1  # QWN_CUDA_STATUS_INVALID_ARGUMENT
        assert "device array" in gpu_ctx.lib.last_error()
    finally:
        gpu_ctx.kv_destroy(h)


def test_noalloc_attention_refuses_overlap(gpu_ctx):
    """The device array is shared by every call on the GPU, so a call is
    refused (QWN_CUDA_STATUS_UNAVAILABLE) while the previous one, enqueued
    on another stream, has not run: here it waits behind ~20 ms of fp32
    products.  A call on that same stream is ordered behind it and
    accepted; once that stream has finished, a call on the other stream is
    accepted again, and every accepted call's output is the same."""
    import torch
    dev = torch.device("cuda:0")
    T, HK, D, H = 256, 8, 128, 32
    scale = float(D ** -0.5)
    h = gpu_ctx.kv_create(T, HK, D)
    try:
        main = torch.cuda.current_stream()
        kv = torch.randn(T, HK * D, device=dev)
        gpu_ctx.kv_append_device(h, kv.data_ptr(), kv.data_ptr(), T, stream=main.cuda_stream)
        q = torch.randn(H * D, device=dev)
        outs = [torch.full((H * D,), float("nan"), device=dev) for _ in range(3)]
        torch.cuda.synchronize()
        busy = torch.cuda.Stream()
        a = torch.randn(4096, 4096, device=dev)
        with torch.cuda.stream(busy):
            for _ in range(20):
                a = (a @ a) / 64.0
        assert noalloc(gpu_ctx, h, q.data_ptr(), outs[0].data_ptr(), H, T - 1, scale, busy.cuda_stream) == 0
        rc = noalloc(gpu_ctx, h, q.data_ptr(), outs[1].data_ptr(), H, T - 1, scale, main.cuda_stream)
        assert rc == -3, f"overlapping call accepted (rc {rc})"  # QWN_CUDA_STATUS_UNAVAILABLE
        assert "in use" in gpu_ctx.lib.last_error()
        assert noalloc(gpu_ctx, h, q.data_ptr(), outs[1].data_ptr(), H, T - 1, scale, busy.cuda_stream) == 0
        busy.synchronize()
        assert noalloc(gpu_ctx, h, q.data_ptr(), outs[2].data_ptr(), H, T - 1, scale, main.cuda_stream) == 0
        torch.cuda.synchronize()
        ref = outs[0].cpu().numpy()
        assert not np.isnan(ref).any()
        for o in outs[1:]:
            assert np.array_equal(o.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    finally:
        torch.cuda.synchronize()
        gpu_ctx.kv_destroy(h)
