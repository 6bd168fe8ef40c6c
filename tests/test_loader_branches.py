"""The host decoder's ABI loader (qwanto_amd/host/qwn_host_decoder.c, the
reference's qwn_cuda_load, c/qwanto_decode.c:267-462) driven through every
refusal branch on the CPU, with a fake qwn_cuda.so
(tests/fake_abi/fake_qwn_cuda.c) built per branch: each refusal must carry
the reference's cuda_backend_reason string, and an accepted library whose
projections fail must fail closed (no CPU fallback, c/qwanto_decode.c:862-871)."""
import os
import shutil
import subprocess

import numpy as np
import pytest

from qwanto_amd import build, synth
from qwanto_amd.host_decoder import HostDecoder, OpenError

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FAKE_SRC = os.path.join(os.path.dirname(os.path.abspath(__file__)), "fake_abi", "fake_qwn_cuda.c")
TINY = dict(hidden=64, intermediate=128, layers=1, heads=2, kv_heads=1, head_dim=32, vocab=50, max_ctx=8,
            rope_theta=1e4, rms_eps=1e-6)


@pytest.fixture(scope="module")
def host_lib():
    if not os.path.exists(build.HOST_DECODER):
        build.build_host_decoder()
    return build.HOST_DECODER


def fake(tmp_path, *defines) -> str:
    """Build one variant of the fake library; returns its path.  FAKE_COMPUTE
    links the oracle library named by QWN_ORACLE_LIB (the sanitizer run's
    build) or oracle/liboracle.so.  QWN_FAKE_CFLAGS adds compiler flags."""
    out = str(tmp_path / ("fake_" + ("_".join(d.split("=")[0] for d in defines) or "ok") + ".so"))
    link = []
    if "FAKE_COMPUTE" in defines:
        lib = os.environ.get("QWN_ORACLE_LIB") or os.path.join(ROOT, "oracle", "liboracle.so")
        if not os.path.exists(lib):
            subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "liboracle.so"], check=True)
        link = ["-I" + os.path.join(ROOT, "oracle"), lib, "-Wl,-rpath," + os.path.dirname(lib)]
    cmd = [shutil.which("gcc") or "gcc", "-O1", "-shared", "-fPIC", "-std=gnu11", "-Wall",
           *os.environ.get("QWN_FAKE_CFLAGS", "").split(), "-I" + os.path.join(ROOT, "include"),
           *("-D" + d for d in defines), FAKE_SRC, "-o", out, *link]
    subprocess.run(cmd, check=True)
    return out


def tiny_model(dtype="q4_0"):
    return synth.decoder_model(np.random.default_rng(0), TINY, dtype)


@pytest.mark.parametrize("defines,reason", [
    (("FAKE_OMIT_GEMM",), "qwn_cuda_dll_missing_versioned_abi_1"),
    (("FAKE_ABI_VERSION=2",), "abi_capability_or_hypervsq2_layout_rejected"),
    (("FAKE_INFO_SIZE=24",), "abi_capability_or_hypervsq2_layout_rejected"),
    (("FAKE_BLOCK_BYTES=72",), "abi_capability_or_hypervsq2_layout_rejected"),
    (("FAKE_NO_Q8_CAP",), "cuda_q8_kv_capability_unavailable"),
    (("FAKE_OMIT_KV_RESET",), "cuda_q8_kv_capability_unavailable"),
    (("FAKE_CAPS_FAIL",), "cuda_capability_query_failed"),
    (("FAKE_DEVICES=0",), "cuda_device_index_0_not_enumerated"),
    (("FAKE_CONTEXT_FAIL",), "cuda_context_creation_failed_device_0"),
    (("FAKE_NO_Q4_CAP",), "qwn_hip_q4_0_f16_capability_unavailable"),
])
def test_refusal_branches(tmp_path, host_lib, defines, reason):
    path = fake(tmp_path, *defines)
    with pytest.raises(OpenError) as ei:
        HostDecoder(tiny_model(), abi_path=path)
    assert ei.value.reason == reason, str(ei.value)


def test_absent_library(tmp_path, host_lib):
    with pytest.raises(OpenError) as ei:
        HostDecoder(tiny_model(), abi_path=str(tmp_path / "missing" / "qwn_cuda.so"))
    assert ei.value.reason == "qwn_cuda_dll_absent_from_runtime_directory"


def test_device_index_beyond_enumeration(tmp_path, host_lib):
    path = fake(tmp_path, "FAKE_DEVICES=2")
    with pytest.raises(OpenError) as ei:
        HostDecoder(tiny_model(), abi_path=path, device=2)
    assert ei.value.reason == "cuda_device_index_2_not_enumerated"


def test_hvsq2_model_needs_no_q4_capability(tmp_path, host_lib):
    """Only a Q4_0 model needs the Q4_0 capability."""
    dec = HostDecoder(tiny_model("hvsq2"), abi_path=fake(tmp_path, "FAKE_NO_Q4_CAP"))
    assert dec.metrics().backend_reason.decode() == "versioned_abi_1_loaded_device_0"
    dec.close()


@pytest.mark.parametrize("defines", [(), ("FAKE_GEMV_ZERO_COUNT",)])
def test_accepted_library_fails_closed(tmp_path, host_lib, defines):
    """Loaded, but every projection is refused (or returns without a GPU
    matmul counted, c/qwanto_decode.c:833-834): the step fails, nothing runs
    on the CPU instead."""
    dec = HostDecoder(tiny_model(), abi_path=fake(tmp_path, *defines))
    m = dec.metrics()
    assert m.backend_reason.decode() == "versioned_abi_1_loaded_device_0"
    with pytest.raises(RuntimeError, match="GPU projection"):
        dec.forward(3)
    m = dec.metrics()
    assert m.cpu_fallback_count == 0 and m.gpu_matmul_count == 0
    dec.close()


@pytest.mark.parametrize("dtype,extra", [("q4_0", {}), ("hvsq2", {}), ("q4_0", {"qk_norm": True, "biases": "qkvo"}),
                                         ("hvsq2", {"qk_norm": True, "biases": "qkv"}),
                                         # BF16 embedding, untied heads in each dtype
                                         ("q4_0", {"embed_dtype": "bf16"}),
                                         ("q4_0", {"embed_dtype": "bf16", "lm_head": "bf16"}),
                                         ("hvsq2", {"lm_head": "f16"}), ("q4_0", {"lm_head": "q4_0"}),
                                         ("hvsq2", {"embed_dtype": "bf16", "lm_head": "hvsq2"})])
def test_host_decoder_end_to_end_on_cpu(tmp_path, host_lib, dtype, extra):
    """A working CPU library (FAKE_COMPUTE: every projection and Q8 KV call
    computed by the oracle's kernels) under the host decoder: its own step
    arithmetic (RMSNorm, RoPE, q/k norms, biases, per-token quantize, SwiGLU,
    residuals, the request fields it builds) must give the oracle decoder's
    logits bit for bit, step after step, with no device in the loop."""
    import oracle
    cfg = dict(TINY, hidden=128, intermediate=256, layers=2, heads=4, kv_heads=2, vocab=300, max_ctx=24)
    model = synth.decoder_model(np.random.default_rng(5), cfg, dtype, **extra)
    dec = HostDecoder(model, abi_path=fake(tmp_path, "FAKE_COMPUTE"))
    ref = oracle.load().decoder(model)
    try:
        token = 11
        for step in range(20):
            a, b = dec.forward(token), ref.forward(token)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), \
                f"step {step}: max |diff| {np.max(np.abs(a - b)):.3g}"
            token = int(np.argmax(b))
        m = dec.metrics()
        assert m.cpu_fallback_count == 0 and m.gpu_matmul_count == 20 * (7 * cfg["layers"] + 1)
    finally:
        dec.close()
        ref.close()
