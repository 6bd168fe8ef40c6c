"""The pipelined weight upload (qwn_cuda_abi_upload_tensor and the batch
entry point qwn_hip_ext_upload_batch): whole-row chunks through two pinned
staging slots, repacked per chunk.  Every uploaded tensor is checked by a
GEMV against the oracle on the host bytes it came from, including tensors
of several chunks and a batch of mixed dtypes; a failing batch leaves
nothing resident."""
import numpy as np
import pytest

from parity import gemv_close
from qwanto_amd import abi, synth

pytestmark = pytest.mark.gpu


def check(ctx, oracle_lib, h, dtype, w, N, K, rng):
    x = synth.activations(rng, 1, K)
    if dtype == "f16":
        y = ctx.gemm(h, x, N, K, gemv=True)[0]
        ref = oracle_lib.matmul_f16(w, x)[0]
    else:
        q8, xs, sums = oracle_lib.quantize(x)
        y = ctx.gemm(h, q8, N, K, scale=float(xs[0]), gemv=True)[0]
        if dtype == "hvsq2":
            ref = oracle_lib.gemv_hvsq2(w, q8[0], sums[0], float(xs[0]), K, N)
        else:
            ref = oracle_lib.gemv_q4_0_q8(w, q8[0], float(xs[0]), K, N)
    ok, worst = gemv_close(y, ref)
    assert ok, f"{dtype} {N}x{K} after upload: worst {worst:.3g} of tolerance"


@pytest.mark.parametrize("dtype,N,K", [("q4_0", 8960, 8192), ("hvsq2", 30000, 4096), ("f16", 9000, 2048)])
def test_upload_of_several_chunks(gpu_ctx, oracle_lib, dtype, N, K):
    """Tensors of 41, 35 and 37 MB: two chunks each (32 MB slots), the
    second partial."""
    rng = np.random.default_rng(N + K)
    w = synth.weights(dtype, rng, N, K)
    assert w.nbytes > 32 << 20
    h = gpu_ctx.upload(w, dtype, N, K)
    try:
        check(gpu_ctx, oracle_lib, h, dtype, w, N, K, rng)
    finally:
        gpu_ctx.release(h)


def test_upload_batch_mixed(gpu_ctx, oracle_lib):
    rng = np.random.default_rng(3)
    shapes = [("hvsq2", 4096, 2560), ("q4_0", 1536, 8960), ("f16", 1000, 1536), ("hvsq2", 1024, 2560),
              ("q4_0", 7, 100), ("hvsq2", 3, 513), ("q4_0", 20000, 2048)]
    ws = [synth.weights(d, rng, N, K) for d, N, K in shapes]
    before = gpu_ctx.telemetry()
    hs = gpu_ctx.upload_batch([(w, d, N, K) for w, (d, N, K) in zip(ws, shapes)])
    try:
        after = gpu_ctx.telemetry()
        assert after.gpu_upload_count - before.gpu_upload_count == len(shapes)
        # the tensors' bytes plus the MFMA-order copies made for them
        assert after.gpu_resident_bytes - before.gpu_resident_bytes == sum(
            synth.weight_bytes(d, N, K) for d, N, K in shapes) + sum(
            gpu_ctx.tensor_info(h).mfma_copy_bytes for h in hs)
        for h, w, (d, N, K) in zip(hs, ws, shapes):
            check(gpu_ctx, oracle_lib, h, d, w, N, K, rng)
    finally:
        for h in hs:
            gpu_ctx.release(h)


def test_upload_batch_failure_leaves_nothing(gpu_ctx):
    rng = np.random.default_rng(4)
    good = synth.weights("hvsq2", rng, 256, 512)
    short = good.reshape(-1)[: good.nbytes // 2]   # shorter than its shape
    before = gpu_ctx.telemetry()
    with pytest.raises(abi.AbiError):
        gpu_ctx.upload_batch([(good, "hvsq2", 256, 512), (short, "hvsq2", 256, 512)])
    after = gpu_ctx.telemetry()
    assert after.gpu_resident_bytes == before.gpu_resident_bytes
    assert after.gpu_upload_count == before.gpu_upload_count


def test_plan_auto_budget_on_device(gpu_ctx, hip_lib):
    """QWN_HIP_GPU_BUDGET_AUTO: 90% of the device's free memory -- every
    tensor of a 4B-sized plan lands on the GPU of a 288 GB part."""
    names = [f"model.layers.{i // 7}.mlp.w{i % 7}" for i in range(252)]
    sizes = [7198720] * 252
    items, totals = abi.plan_residency(hip_lib, names, [0] * 252, sizes, abi.GPU_BUDGET_AUTO, 0, ctx=gpu_ctx)
    assert all(p.tier == abi.TIER_GPU for p in items)
    assert totals == (sum(sizes), 0, 0)
