"""Compile a probe against a qwn_cuda_abi.h and report every struct's size
and field offsets (used by tests/test_abi.py and the fixture
generator tests/golden/make_abi_layout.py)."""
import json
import os
import subprocess
import tempfile

FIELDS = {
    "QwnCudaAbiHeader": ["struct_size", "abi_version", "reserved"],
    "QwnCudaAbiInfo": ["header", "capability_bits", "max_devices", "max_resident_tensors",
                       "hypervsq2_block_bytes", "hypervsq2_block_elements", "abi_name"],
    "QwnCudaDeviceInfo": ["header", "device_id", "compute_major", "compute_minor",
                          "total_vram_bytes", "free_vram_bytes", "name", "driver"],
    "QwnCudaContextOptions": ["header", "device_id", "flags", "memory_budget_bytes",
                              "context_size"],
    "QwnCudaContextHandle": ["header", "opaque"],
    "QwnCudaTensorHandle": ["header", "opaque"],
    "QwnCudaKvCacheHandle": ["header", "opaque"],
    "QwnCudaKvCacheOptions": ["header", "max_tokens", "kv_heads", "head_dim", "reserved"],
    "QwnCudaKvAppendRequest": ["header", "cache", "host_key", "host_value", "n_channels", "token"],
    "QwnCudaKvAttentionRequest": ["header", "cache", "host_query", "host_output", "query_heads",
                                  "kv_heads", "head_dim", "position", "scale"],
    "QwnCudaTensorUpload": ["header", "host_data", "data_bytes", "dtype", "rows", "cols",
                            "block_bytes"],
    "QwnCudaGemmRequest": ["header", "tensor", "input_q8", "input_scale", "input_scales", "output",
                           "batch", "rows", "cols", "input_stride", "output_stride", "input_mode"],
    "QwnCudaTelemetry": ["header", "gpu_matmul_count", "gpu_kernel_launch_count",
                         "gpu_projection_count", "gpu_upload_count", "gpu_upload_bytes",
                         "gpu_resident_bytes", "cpu_matmul_fallback_count",
                         "unsupported_projection_count", "gpu_kernel_ms", "gpu_transfer_ms",
                         "gpu_sync_ms", "device_id", "reserved_device", "device_name",
                         "kernel_type", "dll_hash", "kv_cache_kernel_count",
                         "kv_cache_upload_bytes", "kv_cache_resident_bytes",
                         "kv_cache_kernel_ms", "kv_cache_transfer_ms", "kv_cache_kernel_type"],
}
CONSTANTS = ["QWN_CUDA_ABI_VERSION", "QWN_CUDA_HYPERVSQ2_BLOCK_BYTES",
             "QWN_CUDA_HYPERVSQ2_BLOCK_ELEMENTS", "QWN_CUDA_MAX_RESIDENT_TENSORS",
             "QWN_CUDA_MAX_RESIDENT_KV_CACHES", "QWN_CUDA_CAP_HYPERVSQ2_GEMV",
             "QWN_CUDA_CAP_HYPERVSQ2_GEMM", "QWN_CUDA_CAP_RESIDENT_WEIGHTS",
             "QWN_CUDA_CAP_TELEMETRY", "QWN_CUDA_CAP_DEVICE_ENUMERATION", "QWN_CUDA_CAP_Q8_KV",
             "QWN_CUDA_STATUS_OK", "QWN_CUDA_STATUS_INVALID_ARGUMENT",
             "QWN_CUDA_STATUS_ABI_MISMATCH", "QWN_CUDA_STATUS_UNAVAILABLE",
             "QWN_CUDA_STATUS_OUT_OF_MEMORY", "QWN_CUDA_STATUS_UNSUPPORTED",
             "QWN_CUDA_STATUS_RUNTIME_ERROR", "QWN_CUDA_TENSOR_HYPERVSQ2_74", "QWN_CUDA_INPUT_Q8"]


def probe_source(header: str) -> str:
    lines = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{header}"',
             "int main(void) {", '  printf("{\\"structs\\": {");']
    for si, (s, fields) in enumerate(FIELDS.items()):
        sep = "," if si else ""
        lines.append(f'  printf("{sep}\\"{s}\\": {{\\"size\\": %zu", sizeof({s}));')
        for f in fields:
            lines.append(f'  printf(", \\"{f}\\": %zu", offsetof({s}, {f}));')
        lines.append('  printf("}");')
    lines.append('  printf("}, \\"constants\\": {");')
    for ci, c in enumerate(CONSTANTS):
        sep = ", " if ci else ""
        lines.append(f'  printf("{sep}\\"{c}\\": %lld", (long long)({c}));')
    lines.append('  printf("}}\\n"); return 0; }')
    return "\n".join(lines)


def probe(header: str) -> dict:
    with tempfile.TemporaryDirectory() as d:
        src = os.path.join(d, "probe.c")
        exe = os.path.join(d, "probe")
        with open(src, "w") as f:
            f.write(probe_source(header))
        subprocess.run(["gcc", "-std=c11", "-o", exe, src], check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    return json.loads(out)
