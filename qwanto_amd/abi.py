"""ctypes binding of the qwn_hip C ABI (include/qwn_cuda_abi.h, qwn_hip_ext.h).

This is the host-side mirror of what qwnrun binds with dlsym
(c/qwanto_decode.c:267-462): the same struct layouts, the same call
sequence (query -> enumerate -> context_create -> upload -> gemv), the same
status codes.  ``Library`` loads the in-tree build and raises if it is
missing; there is no CPU fallback anywhere in this package.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "lib", "libqwn_hip.so")

ABI_VERSION = 1
STATUS = {0: "OK", -1: "INVALID_ARGUMENT", -2: "ABI_MISMATCH", -3: "UNAVAILABLE",
          -4: "OUT_OF_MEMORY", -5: "UNSUPPORTED", -6: "RUNTIME_ERROR"}

CAP_HYPERVSQ2_GEMV = 1 << 0
CAP_HYPERVSQ2_GEMM = 1 << 1
CAP_RESIDENT_WEIGHTS = 1 << 2
CAP_TELEMETRY = 1 << 3
CAP_DEVICE_ENUMERATION = 1 << 4
CAP_Q8_KV = 1 << 5
CAP_Q4_0_GEMV = 1 << 6
CAP_F16_GEMV = 1 << 7
CAP_DEVICE_POINTERS = 1 << 8
CAP_BF16_GEMV = 1 << 9

TENSOR_HYPERVSQ2_74 = 1
TENSOR_Q4_0_18 = 2
TENSOR_F16 = 3
TENSOR_BF16 = 4
INPUT_Q8 = 1
INPUT_F32 = 2

DTYPES = {"hvsq2": (TENSOR_HYPERVSQ2_74, 74), "q4_0": (TENSOR_Q4_0_18, 18), "f16": (TENSOR_F16, 2),
          "bf16": (TENSOR_BF16, 2)}

EXPORTS = (
    "qwn_cuda_abi_query", "qwn_cuda_abi_get_capabilities", "qwn_cuda_abi_enumerate_devices",
    "qwn_cuda_abi_context_create", "qwn_cuda_abi_context_destroy", "qwn_cuda_abi_upload_tensor",
    "qwn_cuda_abi_release_tensor", "qwn_cuda_abi_kv_cache_create", "qwn_cuda_abi_kv_cache_destroy",
    "qwn_cuda_abi_kv_cache_append", "qwn_cuda_abi_kv_cache_attention", "qwn_cuda_abi_kv_cache_reset",
    "qwn_cuda_abi_hypervsq2_gemv", "qwn_cuda_abi_hypervsq2_gemm", "qwn_cuda_abi_synchronize",
    "qwn_cuda_abi_get_telemetry", "qwn_cuda_abi_last_error",
)
EXT_EXPORTS = (
    "qwn_hip_ext_tensor_info", "qwn_hip_ext_activation_image_bytes",
    "qwn_hip_ext_prepare_image_device", "qwn_hip_ext_quantize_image_device",
    "qwn_hip_ext_gemm_image_device", "qwn_hip_ext_quantize_device",
    "qwn_hip_ext_kv_append_device", "qwn_hip_ext_attention_workspace_bytes",
    "qwn_hip_ext_kv_attention_device", "qwn_hip_ext_debug_int_sums",
    "qwn_hip_ext_gemv_group_partials", "qwn_hip_ext_gemv_group_device", "qwn_hip_ext_argmax_device",
    "qwn_hip_ext_mfma_image_bytes", "qwn_hip_ext_mfma_image_device", "qwn_hip_ext_gemm_mfma_device",
    "qwn_hip_ext_gemm_mfma_group_device", "qwn_hip_ext_upload_batch", "qwn_hip_ext_plan_residency",
    "qwn_hip_ext_debug_mfma_int_sums", "qwn_hip_ext_debug_kv_read",
    "qwn_hip_ext_kv_attention_device_noalloc",
)
DECODER_EXPORTS = (
    "qwn_hip_decoder_create", "qwn_hip_decoder_destroy", "qwn_hip_decoder_reset",
    "qwn_hip_decoder_forward", "qwn_hip_decoder_generate", "qwn_hip_decoder_prefill",
    "qwn_hip_decoder_debug_kv_read", "qwn_hip_decoder_verify", "qwn_hip_decoder_truncate",
    "qwn_hip_decoder_verify_tree", "qwn_hip_decoder_commit_path",
)

GEMV_INPUT = {"image": 0, "f32": 1, "rmsnorm": 2, "swiglu": 3}
GEMV_OUTPUT = {"store": 0, "add": 1, "argmax": 2, "swiglu": 3}


class Header(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("abi_version", ctypes.c_uint32),
                ("reserved", ctypes.c_uint32 * 4)]


class _Versioned(ctypes.Structure):
    """Structs whose first member is a Header, initialised on construction."""

    def __init__(self, **kw):
        super().__init__(**kw)
        self.header.struct_size = ctypes.sizeof(self)
        self.header.abi_version = ABI_VERSION


class AbiInfo(_Versioned):
    _fields_ = [("header", Header), ("capability_bits", ctypes.c_uint64),
                ("max_devices", ctypes.c_uint32), ("max_resident_tensors", ctypes.c_uint32),
                ("hypervsq2_block_bytes", ctypes.c_uint32),
                ("hypervsq2_block_elements", ctypes.c_uint32), ("abi_name", ctypes.c_char * 32)]


class DeviceInfo(_Versioned):
    _fields_ = [("header", Header), ("device_id", ctypes.c_int32), ("compute_major", ctypes.c_int32),
                ("compute_minor", ctypes.c_int32), ("total_vram_bytes", ctypes.c_uint64),
                ("free_vram_bytes", ctypes.c_uint64), ("name", ctypes.c_char * 128),
                ("driver", ctypes.c_char * 64)]


class ContextOptions(_Versioned):
    _fields_ = [("header", Header), ("device_id", ctypes.c_int32), ("flags", ctypes.c_uint32),
                ("memory_budget_bytes", ctypes.c_uint64), ("context_size", ctypes.c_uint64)]


class Handle(_Versioned):
    _fields_ = [("header", Header), ("opaque", ctypes.c_void_p)]


ContextHandle = TensorHandle = KvCacheHandle = Handle


class KvCacheOptions(_Versioned):
    _fields_ = [("header", Header), ("max_tokens", ctypes.c_uint32), ("kv_heads", ctypes.c_uint32),
                ("head_dim", ctypes.c_uint32), ("reserved", ctypes.c_uint32)]


class KvAppendRequest(_Versioned):
    _fields_ = [("header", Header), ("cache", Handle), ("host_key", ctypes.c_void_p),
                ("host_value", ctypes.c_void_p), ("n_channels", ctypes.c_uint32),
                ("token", ctypes.c_uint32)]


class KvAttentionRequest(_Versioned):
    _fields_ = [("header", Header), ("cache", Handle), ("host_query", ctypes.c_void_p),
                ("host_output", ctypes.c_void_p), ("query_heads", ctypes.c_uint32),
                ("kv_heads", ctypes.c_uint32), ("head_dim", ctypes.c_uint32),
                ("position", ctypes.c_uint32), ("scale", ctypes.c_float)]


class TensorUpload(_Versioned):
    _fields_ = [("header", Header), ("host_data", ctypes.c_void_p), ("data_bytes", ctypes.c_uint64),
                ("dtype", ctypes.c_uint32), ("rows", ctypes.c_uint32), ("cols", ctypes.c_uint32),
                ("block_bytes", ctypes.c_uint32)]


class GemmRequest(_Versioned):
    _fields_ = [("header", Header), ("tensor", Handle), ("input_q8", ctypes.c_void_p),
                ("input_scale", ctypes.c_float), ("input_scales", ctypes.c_void_p),
                ("output", ctypes.c_void_p), ("batch", ctypes.c_uint32), ("rows", ctypes.c_uint32),
                ("cols", ctypes.c_uint32), ("input_stride", ctypes.c_uint32),
                ("output_stride", ctypes.c_uint32), ("input_mode", ctypes.c_uint32)]


class Telemetry(_Versioned):
    _fields_ = [("header", Header), ("gpu_matmul_count", ctypes.c_uint64),
                ("gpu_kernel_launch_count", ctypes.c_uint64),
                ("gpu_projection_count", ctypes.c_uint64), ("gpu_upload_count", ctypes.c_uint64),
                ("gpu_upload_bytes", ctypes.c_uint64), ("gpu_resident_bytes", ctypes.c_uint64),
                ("cpu_matmul_fallback_count", ctypes.c_uint64),
                ("unsupported_projection_count", ctypes.c_uint64),
                ("gpu_kernel_ms", ctypes.c_double), ("gpu_transfer_ms", ctypes.c_double),
                ("gpu_sync_ms", ctypes.c_double), ("device_id", ctypes.c_int32),
                ("reserved_device", ctypes.c_uint32), ("device_name", ctypes.c_char * 128),
                ("kernel_type", ctypes.c_char * 32), ("dll_hash", ctypes.c_char * 65),
                ("kv_cache_kernel_count", ctypes.c_uint64),
                ("kv_cache_upload_bytes", ctypes.c_uint64),
                ("kv_cache_resident_bytes", ctypes.c_uint64),
                ("kv_cache_kernel_ms", ctypes.c_double), ("kv_cache_transfer_ms", ctypes.c_double),
                ("kv_cache_kernel_type", ctypes.c_char * 32)]


class TensorInfo(_Versioned):
    _fields_ = [("header", Header), ("dtype", ctypes.c_uint32), ("rows", ctypes.c_uint32),
                ("cols", ctypes.c_uint32), ("units_per_row", ctypes.c_uint32),
                ("logical_bytes", ctypes.c_uint64), ("device_bytes", ctypes.c_uint64),
                ("lanes_per_row", ctypes.c_uint32), ("units_per_lane", ctypes.c_uint32),
                ("rows_per_wave", ctypes.c_uint32), ("grid", ctypes.c_uint32),
                ("mfma_copy_bytes", ctypes.c_uint64)]


class GemvGroupRequest(_Versioned):
    _fields_ = [("header", Header), ("count", ctypes.c_uint32), ("input_mode", ctypes.c_uint32),
                ("output_mode", ctypes.c_uint32), ("batch", ctypes.c_uint32),
                ("tensors", ctypes.c_void_p), ("outputs", ctypes.c_void_p),
                ("output_stride", ctypes.c_uint32), ("image_stride", ctypes.c_uint32),
                ("image", ctypes.c_void_p), ("scales", ctypes.c_void_p), ("scale", ctypes.c_float),
                ("eps", ctypes.c_float), ("x", ctypes.c_void_p), ("x2", ctypes.c_void_p),
                ("norm", ctypes.c_void_p), ("scale_out", ctypes.c_void_p),
                ("argmax_partials", ctypes.c_void_p)]


class DecoderDesc(_Versioned):
    _fields_ = [("header", Header)] + \
               [(n, ctypes.c_uint32) for n in ("hidden", "intermediate", "layers", "heads", "kv_heads",
                                               "head_dim", "vocab", "max_ctx")] + \
               [("rope_theta", ctypes.c_float), ("rms_eps", ctypes.c_float),
                ("projections", ctypes.c_void_p), ("embedding", ctypes.c_void_p),
                ("input_norms", ctypes.c_void_p), ("post_norms", ctypes.c_void_p),
                ("final_norm", ctypes.c_void_p), ("q_norms", ctypes.c_void_p), ("k_norms", ctypes.c_void_p),
                ("q_biases", ctypes.c_void_p), ("k_biases", ctypes.c_void_p), ("v_biases", ctypes.c_void_p),
                ("o_biases", ctypes.c_void_p), ("lm_head", ctypes.c_void_p)]


class DecoderStats(_Versioned):
    _fields_ = [("header", Header), ("prompt_tokens", ctypes.c_uint32),
                ("generated_tokens", ctypes.c_uint32), ("position", ctypes.c_uint32),
                ("launches_per_step", ctypes.c_uint32), ("prefill_ms", ctypes.c_double),
                ("decode_ms", ctypes.c_double), ("weight_bytes_per_step", ctypes.c_uint64),
                ("graph", ctypes.c_uint32), ("prefill_block_tokens", ctypes.c_uint32)]


class Placement(ctypes.Structure):
    """QwnHipPlacement (the reference's QwnPlacement layout)."""
    _fields_ = [("name_hash", ctypes.c_uint64), ("byte_offset", ctypes.c_uint64),
                ("byte_size", ctypes.c_uint64), ("tensor_index", ctypes.c_uint32),
                ("tier", ctypes.c_uint8), ("priority", ctypes.c_uint8), ("reserved", ctypes.c_uint16)]


TIER_GPU, TIER_RAM, TIER_FILE = 0, 1, 2
GPU_BUDGET_AUTO = (1 << 64) - 1


def plan_residency(lib: "Library", names, offsets, sizes, gpu_budget: int, ram_budget: int,
                   ctx: "Context | None" = None):
    """qwn_hip_ext_plan_residency: returns ([Placement] in plan order,
    (gpu_bytes, ram_bytes, file_bytes))."""
    n = len(names)
    enc = [str(x).encode() for x in names]
    arr_names = (ctypes.c_char_p * n)(*enc)
    offs = (ctypes.c_uint64 * n)(*[int(v) for v in offsets])
    szs = (ctypes.c_uint64 * n)(*[int(v) for v in sizes])
    items = (Placement * n)()
    totals = (ctypes.c_uint64 * 3)()
    lib.check("plan_residency", lib.lib.qwn_hip_ext_plan_residency(
        ctx._h if ctx is not None else None, arr_names, offs, szs, n, int(gpu_budget),
        int(ram_budget), items, totals))
    return [items[i] for i in range(n)], (totals[0], totals[1], totals[2])


STRUCTS = {
    "QwnCudaAbiHeader": Header, "QwnCudaAbiInfo": AbiInfo, "QwnCudaDeviceInfo": DeviceInfo,
    "QwnCudaContextOptions": ContextOptions, "QwnCudaContextHandle": Handle,
    "QwnCudaTensorHandle": Handle, "QwnCudaKvCacheHandle": Handle,
    "QwnCudaKvCacheOptions": KvCacheOptions, "QwnCudaKvAppendRequest": KvAppendRequest,
    "QwnCudaKvAttentionRequest": KvAttentionRequest, "QwnCudaTensorUpload": TensorUpload,
    "QwnCudaGemmRequest": GemmRequest, "QwnCudaTelemetry": Telemetry,
}


class AbiError(RuntimeError):
    def __init__(self, fn: str, status: int, message: str):
        super().__init__(f"{fn} -> {STATUS.get(status, status)}: {message}")
        self.status = status


def _p(a: np.ndarray | None) -> int | None:
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


class Library:
    """The loaded qwn_hip shared library (no fallback: missing -> error)."""

    def __init__(self, path: str = LIB_PATH):
        if not os.path.exists(path):
            raise FileNotFoundError(
                f"{path} is missing; build it with qwanto_amd.build.build() (the GPU path has no "
                "CPU fallback)")
        self.path = path
        lib = ctypes.CDLL(path)
        self.lib = lib
        P = ctypes.POINTER
        lib.qwn_cuda_abi_query.argtypes = [P(AbiInfo)]
        lib.qwn_cuda_abi_get_capabilities.argtypes = [P(AbiInfo)]
        lib.qwn_cuda_abi_enumerate_devices.argtypes = [P(DeviceInfo), ctypes.c_uint32,
                                                       P(ctypes.c_uint32)]
        lib.qwn_cuda_abi_context_create.argtypes = [P(ContextOptions), P(Handle)]
        lib.qwn_cuda_abi_context_destroy.argtypes = [P(Handle)]
        lib.qwn_cuda_abi_upload_tensor.argtypes = [P(Handle), P(TensorUpload), P(Handle)]
        lib.qwn_cuda_abi_release_tensor.argtypes = [P(Handle), P(Handle)]
        lib.qwn_cuda_abi_kv_cache_create.argtypes = [P(Handle), P(KvCacheOptions), P(Handle)]
        lib.qwn_cuda_abi_kv_cache_destroy.argtypes = [P(Handle), P(Handle)]
        lib.qwn_cuda_abi_kv_cache_append.argtypes = [P(Handle), P(KvAppendRequest), P(Telemetry)]
        lib.qwn_cuda_abi_kv_cache_attention.argtypes = [P(Handle), P(KvAttentionRequest),
                                                        P(Telemetry)]
        lib.qwn_cuda_abi_kv_cache_reset.argtypes = [P(Handle), P(Handle)]
        lib.qwn_cuda_abi_hypervsq2_gemv.argtypes = [P(Handle), P(GemmRequest), P(Telemetry)]
        lib.qwn_cuda_abi_hypervsq2_gemm.argtypes = [P(Handle), P(GemmRequest), P(Telemetry)]
        lib.qwn_cuda_abi_synchronize.argtypes = [P(Handle)]
        lib.qwn_cuda_abi_get_telemetry.argtypes = [P(Handle), P(Telemetry)]
        lib.qwn_cuda_abi_last_error.argtypes = [ctypes.c_char_p, ctypes.c_uint32]
        lib.qwn_hip_ext_tensor_info.argtypes = [P(Handle), P(TensorInfo)]
        V, U32 = ctypes.c_void_p, ctypes.c_uint32
        lib.qwn_hip_ext_activation_image_bytes.argtypes = [P(Handle)]
        lib.qwn_hip_ext_activation_image_bytes.restype = ctypes.c_uint64
        lib.qwn_hip_ext_prepare_image_device.argtypes = [P(Handle), P(Handle), V, U32, U32, V,
                                                         U32, V]
        lib.qwn_hip_ext_quantize_image_device.argtypes = [P(Handle), P(Handle), V, U32, U32, V,
                                                          U32, V, V, U32, V]
        lib.qwn_hip_ext_gemm_image_device.argtypes = [P(Handle), P(Handle), V, U32, V,
                                                      ctypes.c_float, V, U32, U32, V]
        lib.qwn_hip_ext_quantize_device.argtypes = [P(Handle), ctypes.c_void_p, ctypes.c_uint32,
                                                    ctypes.c_uint32, ctypes.c_uint32,
                                                    ctypes.c_void_p, ctypes.c_uint32,
                                                    ctypes.c_void_p, ctypes.c_void_p]
        lib.qwn_hip_ext_kv_append_device.argtypes = [P(Handle), P(Handle), ctypes.c_void_p,
                                                     ctypes.c_void_p, ctypes.c_uint32,
                                                     ctypes.c_void_p]
        lib.qwn_hip_ext_attention_workspace_bytes.argtypes = [P(Handle), ctypes.c_uint32,
                                                              ctypes.c_uint32]
        lib.qwn_hip_ext_attention_workspace_bytes.restype = ctypes.c_uint64
        lib.qwn_hip_ext_kv_attention_device.argtypes = [P(Handle), P(Handle), ctypes.c_void_p,
                                                        ctypes.c_void_p, ctypes.c_uint32,
                                                        ctypes.c_uint32, ctypes.c_float,
                                                        ctypes.c_void_p, ctypes.c_void_p]
        lib.qwn_hip_ext_kv_attention_device_noalloc.argtypes = [P(Handle), P(Handle), ctypes.c_void_p,
                                                                ctypes.c_void_p, ctypes.c_uint32,
                                                                ctypes.c_uint32, ctypes.c_float,
                                                                ctypes.c_void_p]
        lib.qwn_hip_ext_debug_int_sums.argtypes = [P(Handle), P(Handle), ctypes.c_void_p,
                                                   ctypes.c_void_p, ctypes.c_uint64]
        lib.qwn_hip_ext_debug_mfma_int_sums.argtypes = [P(Handle), P(Handle), V, U32, V, ctypes.c_uint64]
        lib.qwn_hip_ext_debug_kv_read.argtypes = [P(Handle), P(Handle), U32, U32, V, V, V, V]
        lib.qwn_hip_ext_gemv_group_partials.argtypes = [P(Handle), P(GemvGroupRequest)]
        lib.qwn_hip_ext_gemv_group_partials.restype = ctypes.c_uint32
        lib.qwn_hip_ext_gemv_group_device.argtypes = [P(Handle), P(GemvGroupRequest), V]
        lib.qwn_hip_ext_argmax_device.argtypes = [P(Handle), V, U32, V, V]
        lib.qwn_hip_ext_mfma_image_bytes.argtypes = [P(Handle)]
        lib.qwn_hip_ext_mfma_image_bytes.restype = ctypes.c_uint64
        lib.qwn_hip_ext_mfma_image_device.argtypes = [P(Handle), P(Handle), V, U32, U32, V, V]
        lib.qwn_hip_ext_gemm_mfma_device.argtypes = [P(Handle), P(Handle), V, V, V, U32, U32, V]
        lib.qwn_hip_ext_gemm_mfma_group_device.argtypes = [P(Handle), P(Handle), U32, V, V, V, U32, U32, U32, V]
        lib.qwn_hip_ext_upload_batch.argtypes = [P(Handle), P(TensorUpload), U32, P(Handle)]
        lib.qwn_hip_ext_plan_residency.argtypes = [V, V, V, V, U32, ctypes.c_uint64, ctypes.c_uint64, V, V]
        lib.qwn_hip_decoder_create.argtypes = [P(Handle), P(DecoderDesc), P(Handle)]
        lib.qwn_hip_decoder_destroy.argtypes = [P(Handle), P(Handle)]
        lib.qwn_hip_decoder_reset.argtypes = [P(Handle), P(Handle)]
        lib.qwn_hip_decoder_forward.argtypes = [P(Handle), P(Handle), ctypes.c_int32, V, V]
        lib.qwn_hip_decoder_generate.argtypes = [P(Handle), P(Handle), V, U32, U32, V, P(DecoderStats)]
        lib.qwn_hip_decoder_prefill.argtypes = [P(Handle), P(Handle), V, U32, V, V]
        lib.qwn_hip_decoder_debug_kv_read.argtypes = [P(Handle), P(Handle), U32, U32, U32, V, V, V, V]
        lib.qwn_hip_decoder_verify.argtypes = [P(Handle), P(Handle), V, U32, V, V]
        lib.qwn_hip_decoder_truncate.argtypes = [P(Handle), P(Handle), U32]
        lib.qwn_hip_decoder_verify_tree.argtypes = [P(Handle), P(Handle), V, V, U32, V, V]
        lib.qwn_hip_decoder_commit_path.argtypes = [P(Handle), P(Handle), V, U32]

    def last_error(self) -> str:
        buf = ctypes.create_string_buffer(512)
        self.lib.qwn_cuda_abi_last_error(buf, 512)
        return buf.value.decode(errors="replace")

    def check(self, fn: str, status: int) -> None:
        if status != 0:
            raise AbiError(fn, status, self.last_error())

    def call(self, fn: str, *args) -> int:
        return getattr(self.lib, fn)(*args)

    def query(self) -> AbiInfo:
        info = AbiInfo()
        self.check("query", self.lib.qwn_cuda_abi_query(ctypes.byref(info)))
        return info

    def devices(self) -> list[DeviceInfo]:
        arr = (DeviceInfo * 16)()
        for d in arr:
            d.header.struct_size = ctypes.sizeof(DeviceInfo)
            d.header.abi_version = ABI_VERSION
        count = ctypes.c_uint32(0)
        st = self.lib.qwn_cuda_abi_enumerate_devices(arr, 16, ctypes.byref(count))
        if st != 0:
            return []
        return [arr[i] for i in range(min(count.value, 16))]


class Context:
    """One qwn_hip context: resident tensors, KV caches, telemetry."""

    def __init__(self, lib: Library, device: int = 0, budget: int = 0):
        self.lib = lib
        opts = ContextOptions(device_id=device, memory_budget_bytes=budget)
        self.handle = Handle()
        lib.check("context_create",
                  lib.lib.qwn_cuda_abi_context_create(ctypes.byref(opts), ctypes.byref(self.handle)))
        self._h = ctypes.byref(self.handle)

    def close(self) -> None:
        if self.handle.opaque:
            self.lib.check("context_destroy", self.lib.lib.qwn_cuda_abi_context_destroy(self._h))

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- tensors --------------------------------------------------------------
    def upload(self, data: np.ndarray, dtype: str, rows: int, cols: int) -> Handle:
        code, block = DTYPES[dtype]
        data = np.ascontiguousarray(data)
        up = TensorUpload(host_data=_p(data), data_bytes=data.nbytes, dtype=code, rows=rows,
                          cols=cols, block_bytes=block)
        h = Handle()
        self.lib.check("upload_tensor", self.lib.lib.qwn_cuda_abi_upload_tensor(
            self._h, ctypes.byref(up), ctypes.byref(h)))
        return h

    def upload_batch(self, items) -> list:
        """Upload [(data, dtype, rows, cols), ...] through one pipelined call
        (qwn_hip_ext_upload_batch); returns the handles in order."""
        keep = [np.ascontiguousarray(d) for d, _, _, _ in items]
        n = len(items)
        ups = (TensorUpload * n)()
        hs = (Handle * n)()
        for i, (d, (_, dtype, rows, cols)) in enumerate(zip(keep, items)):
            code, block = DTYPES[dtype]
            ups[i] = TensorUpload(host_data=_p(d), data_bytes=d.nbytes, dtype=code, rows=rows, cols=cols,
                                  block_bytes=block)
            hs[i] = Handle()
        self.lib.check("upload_batch", self.lib.lib.qwn_hip_ext_upload_batch(self._h, ups, n, hs))
        return [hs[i] for i in range(n)]

    def release(self, h: Handle) -> None:
        self.lib.check("release_tensor",
                       self.lib.lib.qwn_cuda_abi_release_tensor(self._h, ctypes.byref(h)))

    def tensor_info(self, h: Handle) -> TensorInfo:
        info = TensorInfo()
        self.lib.check("tensor_info",
                       self.lib.lib.qwn_hip_ext_tensor_info(ctypes.byref(h), ctypes.byref(info)))
        return info

    def gemm(self, h: Handle, x: np.ndarray, rows: int, cols: int, scale=None, scales=None,
             gemv: bool = False, telemetry: Telemetry | None = None) -> np.ndarray:
        """y[batch][rows] for int8 x[batch][>=cols] (or fp32 x for F16 tensors)."""
        x = np.ascontiguousarray(x)
        if x.ndim == 1:
            x = x[None, :]
        batch, stride = x.shape
        out = np.zeros((batch, rows), dtype=np.float32)
        sc = None if scales is None else np.ascontiguousarray(scales, dtype=np.float32)
        req = GemmRequest(tensor=h, input_q8=_p(x), input_scale=float(scale or 0.0),
                          input_scales=_p(sc), output=_p(out), batch=batch, rows=rows, cols=cols,
                          input_stride=stride, output_stride=rows,
                          input_mode=INPUT_F32 if x.dtype == np.float32 else INPUT_Q8)
        tm = telemetry if telemetry is not None else Telemetry()
        fn = "qwn_cuda_abi_hypervsq2_gemv" if gemv else "qwn_cuda_abi_hypervsq2_gemm"
        self.lib.check(fn, getattr(self.lib.lib, fn)(self._h, ctypes.byref(req), ctypes.byref(tm)))
        return out

    def debug_int_sums(self, h: Handle, q8: np.ndarray, count: int) -> np.ndarray:
        out = np.zeros(count, dtype=np.int32)
        q8 = np.ascontiguousarray(q8, dtype=np.int8)
        self.lib.check("debug_int_sums", self.lib.lib.qwn_hip_ext_debug_int_sums(
            self._h, ctypes.byref(h), _p(q8), _p(out), count))
        return out

    def debug_mfma_sums(self, h: Handle, q8: np.ndarray, rows: int, nblk: int) -> np.ndarray:
        """Exact int32 block dots of the MFMA GEMM: [batch][rows][nblk]."""
        q8 = np.ascontiguousarray(q8, dtype=np.int8)
        batch = q8.shape[0]
        out = np.zeros((batch, rows, nblk), dtype=np.int32)
        self.lib.check("debug_mfma_int_sums", self.lib.lib.qwn_hip_ext_debug_mfma_int_sums(
            self._h, ctypes.byref(h), _p(q8), batch, _p(out), out.size))
        return out

    def kv_read(self, h: Handle, first: int, count: int, channels: int):
        """Cached tokens [first, first+count) token-major: (keys, values,
        key_scales, value_scales)."""
        groups = (channels + 63) // 64
        k = np.zeros((count, channels), dtype=np.int8)
        v = np.zeros((count, channels), dtype=np.int8)
        ks = np.zeros((count, groups), dtype=np.float32)
        vs = np.zeros((count, groups), dtype=np.float32)
        self.lib.check("debug_kv_read", self.lib.lib.qwn_hip_ext_debug_kv_read(
            self._h, ctypes.byref(h), first, count, _p(k), _p(v), _p(ks), _p(vs)))
        return k, v, ks, vs

    def image_bytes(self, h: Handle) -> int:
        """Bytes of one token's activation image for tensor h."""
        return int(self.lib.lib.qwn_hip_ext_activation_image_bytes(ctypes.byref(h)))

    def prepare_image_device(self, h: Handle, x_ptr: int, batch: int, x_stride: int,
                             image_ptr: int, image_stride: int, stream: int | None = None) -> None:
        self.lib.check("prepare_image_device", self.lib.lib.qwn_hip_ext_prepare_image_device(
            self._h, ctypes.byref(h), x_ptr, batch, x_stride, image_ptr, image_stride, stream))

    def quantize_image_device(self, h: Handle, x_ptr: int, batch: int, x_stride: int,
                              image_ptr: int | None, image_stride: int, scales_ptr: int,
                              q8_ptr: int | None = None, q8_stride: int = 0,
                              stream: int | None = None) -> None:
        self.lib.check("quantize_image_device", self.lib.lib.qwn_hip_ext_quantize_image_device(
            self._h, ctypes.byref(h), x_ptr, batch, x_stride, image_ptr, image_stride, scales_ptr,
            q8_ptr, q8_stride, stream))

    def gemm_image_device(self, h: Handle, image_ptr: int, image_stride: int, out_ptr: int,
                          batch: int, output_stride: int, scales_ptr: int | None = None,
                          scale: float = 0.0, stream: int | None = None) -> None:
        self.lib.check("gemm_image_device", self.lib.lib.qwn_hip_ext_gemm_image_device(
            self._h, ctypes.byref(h), image_ptr, image_stride, scales_ptr, scale, out_ptr, batch,
            output_stride, stream))

    def quantize_device(self, x_ptr: int, batch: int, cols: int, x_stride: int, q8_ptr: int,
                        q8_stride: int, scales_ptr: int, stream: int | None = None) -> None:
        self.lib.check("quantize_device", self.lib.lib.qwn_hip_ext_quantize_device(
            self._h, x_ptr, batch, cols, x_stride, q8_ptr, q8_stride, scales_ptr, stream))

    def gemv_group_request(self, handles: list, outputs: list[int], input_mode: str = "image",
                           output_mode: str = "store", batch: int = 1, image_ptr: int | None = None,
                           image_stride: int = 0, scales_ptr: int | None = None, scale: float = 0.0,
                           x_ptr: int | None = None, x2_ptr: int | None = None,
                           norm_ptr: int | None = None, eps: float = 0.0,
                           scale_out_ptr: int | None = None, partials_ptr: int | None = None,
                           output_stride: int = 0):
        """A QwnHipGemvGroupRequest plus the arrays it points into (keep both alive)."""
        hs = (Handle * len(handles))(*handles)
        outs = (ctypes.c_void_p * len(outputs))(*outputs)
        req = GemvGroupRequest(count=len(handles), input_mode=GEMV_INPUT[input_mode],
                               output_mode=GEMV_OUTPUT[output_mode], batch=batch,
                               tensors=ctypes.cast(hs, ctypes.c_void_p).value,
                               outputs=ctypes.cast(outs, ctypes.c_void_p).value,
                               output_stride=output_stride, image_stride=image_stride, image=image_ptr,
                               scales=scales_ptr, scale=scale, eps=eps, x=x_ptr, x2=x2_ptr, norm=norm_ptr,
                               scale_out=scale_out_ptr, argmax_partials=partials_ptr)
        return req, (hs, outs)

    def gemv_group_partials(self, req: GemvGroupRequest) -> int:
        return int(self.lib.lib.qwn_hip_ext_gemv_group_partials(self._h, ctypes.byref(req)))

    def gemv_group_device(self, req: GemvGroupRequest, stream: int | None = None) -> None:
        self.lib.check("gemv_group_device",
                       self.lib.lib.qwn_hip_ext_gemv_group_device(self._h, ctypes.byref(req), stream))

    def argmax_device(self, partials_ptr: int, count: int, index_ptr: int, stream: int | None = None) -> None:
        self.lib.check("argmax_device", self.lib.lib.qwn_hip_ext_argmax_device(
            self._h, partials_ptr, count, index_ptr, stream))

    def mfma_image_bytes(self, h: Handle) -> int:
        return int(self.lib.lib.qwn_hip_ext_mfma_image_bytes(ctypes.byref(h)))

    def mfma_image_device(self, h: Handle, q8_ptr: int, batch: int, q8_stride: int, image_ptr: int,
                          stream: int | None = None) -> None:
        self.lib.check("mfma_image_device", self.lib.lib.qwn_hip_ext_mfma_image_device(
            self._h, ctypes.byref(h), q8_ptr, batch, q8_stride, image_ptr, stream))

    def gemm_mfma_device(self, h: Handle, image_ptr: int, scales_ptr: int, out_ptr: int, batch: int,
                         output_stride: int = 0, stream: int | None = None) -> None:
        self.lib.check("gemm_mfma_device", self.lib.lib.qwn_hip_ext_gemm_mfma_device(
            self._h, ctypes.byref(h), image_ptr, scales_ptr, out_ptr, batch, output_stride, stream))

    def gemm_mfma_group_device(self, handles, image_ptr: int, scales_ptr: int, out_ptrs, batch: int,
                               output_stride: int = 0, stream: int | None = None,
                               accumulate: bool = False) -> None:
        """One MFMA launch over 1..4 tensors of equal columns sharing an image
        (accumulate: outputs += the product)."""
        n = len(handles)
        hs = (Handle * n)(*handles)
        outs = (ctypes.c_void_p * n)(*out_ptrs)
        self.lib.check("gemm_mfma_group_device", self.lib.lib.qwn_hip_ext_gemm_mfma_group_device(
            self._h, hs, n, image_ptr, scales_ptr, outs, batch, output_stride, int(accumulate), stream))

    # -- KV cache ---------------------------------------------------------------
    def kv_create(self, max_tokens: int, kv_heads: int, head_dim: int) -> Handle:
        opts = KvCacheOptions(max_tokens=max_tokens, kv_heads=kv_heads, head_dim=head_dim)
        h = Handle()
        self.lib.check("kv_cache_create", self.lib.lib.qwn_cuda_abi_kv_cache_create(
            self._h, ctypes.byref(opts), ctypes.byref(h)))
        return h

    def kv_destroy(self, h: Handle) -> None:
        self.lib.check("kv_cache_destroy",
                       self.lib.lib.qwn_cuda_abi_kv_cache_destroy(self._h, ctypes.byref(h)))

    def kv_reset(self, h: Handle) -> None:
        self.lib.check("kv_cache_reset",
                       self.lib.lib.qwn_cuda_abi_kv_cache_reset(self._h, ctypes.byref(h)))

    def kv_append(self, h: Handle, key: np.ndarray, value: np.ndarray, token: int,
                  telemetry: Telemetry | None = None) -> None:
        key = np.ascontiguousarray(key, dtype=np.float32)
        value = np.ascontiguousarray(value, dtype=np.float32)
        req = KvAppendRequest(cache=h, host_key=_p(key), host_value=_p(value),
                              n_channels=key.size, token=token)
        tm = telemetry if telemetry is not None else Telemetry()
        self.lib.check("kv_cache_append", self.lib.lib.qwn_cuda_abi_kv_cache_append(
            self._h, ctypes.byref(req), ctypes.byref(tm)))

    def kv_attention(self, h: Handle, query: np.ndarray, query_heads: int, kv_heads: int,
                     head_dim: int, position: int, scale: float,
                     telemetry: Telemetry | None = None) -> np.ndarray:
        query = np.ascontiguousarray(query, dtype=np.float32)
        out = np.zeros(query_heads * head_dim, dtype=np.float32)
        req = KvAttentionRequest(cache=h, host_query=_p(query), host_output=_p(out),
                                 query_heads=query_heads, kv_heads=kv_heads, head_dim=head_dim,
                                 position=position, scale=scale)
        tm = telemetry if telemetry is not None else Telemetry()
        self.lib.check("kv_cache_attention", self.lib.lib.qwn_cuda_abi_kv_cache_attention(
            self._h, ctypes.byref(req), ctypes.byref(tm)))
        return out

    def kv_append_device(self, h: Handle, k_ptr: int, v_ptr: int, count: int,
                         stream: int | None = None) -> None:
        self.lib.check("kv_append_device", self.lib.lib.qwn_hip_ext_kv_append_device(
            self._h, ctypes.byref(h), k_ptr, v_ptr, count, stream))

    def attention_workspace_bytes(self, h: Handle, query_heads: int, position: int) -> int:
        return int(self.lib.lib.qwn_hip_ext_attention_workspace_bytes(ctypes.byref(h),
                                                                     query_heads, position))

    def kv_attention_device(self, h: Handle, q_ptr: int, out_ptr: int, query_heads: int,
                            position: int, scale: float, work_ptr: int,
                            stream: int | None = None) -> None:
        self.lib.check("kv_attention_device", self.lib.lib.qwn_hip_ext_kv_attention_device(
            self._h, ctypes.byref(h), q_ptr, out_ptr, query_heads, position, scale, work_ptr,
            stream))

    # -- misc -----------------------------------------------------------------
    def telemetry(self) -> Telemetry:
        tm = Telemetry()
        self.lib.check("get_telemetry",
                       self.lib.lib.qwn_cuda_abi_get_telemetry(self._h, ctypes.byref(tm)))
        return tm

    def synchronize(self) -> None:
        self.lib.check("synchronize", self.lib.lib.qwn_cuda_abi_synchronize(self._h))


class ResidentDecoder:
    """The library's resident greedy decoder (include/qwn_hip_decoder.h) over a
    synth.decoder_model / qwn_file model dict: uploads the seven projections
    per layer, the F16 or BF16 embedding and an untied LM head if the model
    has one to `ctx`, then creates the decoder."""

    PROJ_ORDER = ("q", "k", "v", "o", "gate", "up", "down")

    def __init__(self, ctx: Context, model: dict):
        self.ctx = ctx
        cfg = model["cfg"]
        self.cfg = cfg
        dtype = model["dtype"]
        D, I = cfg["hidden"], cfg["intermediate"]
        Q, KV = cfg["heads"] * cfg["head_dim"], cfg["kv_heads"] * cfg["head_dim"]
        shapes = {"q": (Q, D), "k": (KV, D), "v": (KV, D), "o": (D, Q), "gate": (I, D), "up": (I, D),
                  "down": (D, I)}
        L = cfg["layers"]
        self._tensors = []
        for l in range(L):
            for p in self.PROJ_ORDER:
                rows, cols = shapes[p]
                self._tensors.append(ctx.upload(model["layers"][l][p], dtype, rows, cols))
        self._embed = ctx.upload(model["embed"], model.get("embed_dtype", "f16"), cfg["vocab"], D)
        self._head = None
        if "lm_head" in model:
            self._head = ctx.upload(model["lm_head"], model["lm_head_dtype"], cfg["vocab"], D)
        self._proj_arr = (Handle * len(self._tensors))(*self._tensors)
        self._norm_in = np.ascontiguousarray(np.stack([model["layers"][l]["input_norm"] for l in range(L)]),
                                             dtype=np.float32)
        self._norm_post = np.ascontiguousarray(np.stack([model["layers"][l]["post_norm"] for l in range(L)]),
                                               dtype=np.float32)
        self._final = np.ascontiguousarray(model["final_norm"], dtype=np.float32)
        self._qn = self._kn = None
        if "q_norm" in model["layers"][0]:
            self._qn = np.ascontiguousarray(np.stack([model["layers"][l]["q_norm"] for l in range(L)]),
                                            dtype=np.float32)
            self._kn = np.ascontiguousarray(np.stack([model["layers"][l]["k_norm"] for l in range(L)]),
                                            dtype=np.float32)
        # optional q/k/v/o biases, [layers][rows] per projection
        self._bias = {}
        for p in "qkvo":
            if all(p + "_bias" in model["layers"][l] for l in range(L)):
                self._bias[p] = np.ascontiguousarray(np.stack([model["layers"][l][p + "_bias"] for l in range(L)]),
                                                     dtype=np.float32)
            elif any(p + "_bias" in model["layers"][l] for l in range(L)):
                raise ValueError(f"{p}_proj.bias must be present in every layer or in none")
        desc = DecoderDesc(hidden=D, intermediate=I, layers=L, heads=cfg["heads"], kv_heads=cfg["kv_heads"],
                           head_dim=cfg["head_dim"], vocab=cfg["vocab"], max_ctx=cfg["max_ctx"],
                           rope_theta=cfg["rope_theta"], rms_eps=cfg["rms_eps"],
                           projections=ctypes.cast(self._proj_arr, ctypes.c_void_p).value,
                           embedding=ctypes.addressof(self._embed), input_norms=_p(self._norm_in),
                           post_norms=_p(self._norm_post), final_norm=_p(self._final),
                           q_norms=_p(self._qn), k_norms=_p(self._kn),
                           **{p + "_biases": _p(self._bias.get(p)) for p in "qkvo"},
                           lm_head=ctypes.addressof(self._head) if self._head is not None else None)
        self.handle = Handle()
        lib = ctx.lib
        lib.check("decoder_create", lib.lib.qwn_hip_decoder_create(ctx._h, ctypes.byref(desc),
                                                                   ctypes.byref(self.handle)))

    def verify(self, tokens, logits: bool = True):
        """One verify block: (logits [count][vocab] or None, greedy id after
        each token [count])."""
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        n = tokens.size
        out = np.zeros((n, self.cfg["vocab"]), dtype=np.float32) if logits else None
        ids = np.zeros(n, dtype=np.int32)
        lib = self.ctx.lib
        lib.check("decoder_verify", lib.lib.qwn_hip_decoder_verify(
            self.ctx._h, ctypes.byref(self.handle), _p(tokens), n, _p(out), _p(ids)))
        return out, ids

    def verify_tree(self, tokens, parents, logits: bool = True):
        """One draft tree (node i = tokens[i] under parents[i], -1 for a root)
        after the cached prefix: (logits after each node [count][vocab] or
        None, their first maxima [count])."""
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        parents = np.ascontiguousarray(parents, dtype=np.int32)
        n = tokens.size
        out = np.zeros((n, self.cfg["vocab"]), dtype=np.float32) if logits else None
        ids = np.zeros(n, dtype=np.int32)
        lib = self.ctx.lib
        lib.check("decoder_verify_tree", lib.lib.qwn_hip_decoder_verify_tree(
            self.ctx._h, ctypes.byref(self.handle), _p(tokens), _p(parents), n, _p(out), _p(ids)))
        return out, ids

    def commit_path(self, nodes) -> None:
        """Keep the root-to-node path `nodes` of the last verified tree."""
        nodes = np.ascontiguousarray(nodes, dtype=np.uint32)
        lib = self.ctx.lib
        lib.check("decoder_commit_path", lib.lib.qwn_hip_decoder_commit_path(
            self.ctx._h, ctypes.byref(self.handle), _p(nodes), nodes.size))

    def truncate(self, position: int) -> None:
        lib = self.ctx.lib
        lib.check("decoder_truncate", lib.lib.qwn_hip_decoder_truncate(self.ctx._h, ctypes.byref(self.handle),
                                                                       position))

    def kv_read(self, layer: int, first: int, count: int):
        """Layer `layer`'s cached tokens [first, first+count), token-major:
        (keys, values, key_scales, value_scales)."""
        C = self.cfg["kv_heads"] * self.cfg["head_dim"]
        groups = (C + 63) // 64
        k = np.zeros((count, C), dtype=np.int8)
        v = np.zeros((count, C), dtype=np.int8)
        ks = np.zeros((count, groups), dtype=np.float32)
        vs = np.zeros((count, groups), dtype=np.float32)
        lib = self.ctx.lib
        lib.check("decoder_debug_kv_read", lib.lib.qwn_hip_decoder_debug_kv_read(
            self.ctx._h, ctypes.byref(self.handle), layer, first, count, _p(k), _p(v), _p(ks), _p(vs)))
        return k, v, ks, vs

    def forward(self, token: int, logits: bool = True):
        """One step; returns (logits or None, greedy next token)."""
        out = np.zeros(self.cfg["vocab"], dtype=np.float32) if logits else None
        nxt = ctypes.c_int32(0)
        self.ctx.lib.check("decoder_forward", self.ctx.lib.lib.qwn_hip_decoder_forward(
            self.ctx._h, ctypes.byref(self.handle), int(token), _p(out), ctypes.addressof(nxt)))
        return out, nxt.value

    def prefill(self, tokens, logits: bool = True):
        """Prompt tokens in prefill blocks; returns (last logits or None,
        greedy next token)."""
        tk = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.zeros(self.cfg["vocab"], dtype=np.float32) if logits else None
        nxt = ctypes.c_int32(0)
        self.ctx.lib.check("decoder_prefill", self.ctx.lib.lib.qwn_hip_decoder_prefill(
            self.ctx._h, ctypes.byref(self.handle), _p(tk), tk.size, _p(out), ctypes.addressof(nxt)))
        return out, nxt.value

    def generate(self, prompt, max_new: int):
        """Greedy generation; returns (tokens[max_new], DecoderStats)."""
        pr = np.ascontiguousarray(prompt, dtype=np.int32)
        toks = np.zeros(max_new, dtype=np.int32)
        st = DecoderStats()
        self.ctx.lib.check("decoder_generate", self.ctx.lib.lib.qwn_hip_decoder_generate(
            self.ctx._h, ctypes.byref(self.handle), _p(pr), pr.size, max_new, _p(toks), ctypes.byref(st)))
        return toks, st

    def reset(self) -> None:
        self.ctx.lib.check("decoder_reset", self.ctx.lib.lib.qwn_hip_decoder_reset(
            self.ctx._h, ctypes.byref(self.handle)))

    def close(self) -> None:
        if self.handle.opaque:
            self.ctx.lib.check("decoder_destroy", self.ctx.lib.lib.qwn_hip_decoder_destroy(
                self.ctx._h, ctypes.byref(self.handle)))
        for t in self._tensors + [self._embed, self._head]:
            if t is not None:
                self.ctx.release(t)
        self._tensors, self._embed, self._head = [], None, None


_LIB: Library | None = None


def load() -> Library:
    """Load the library once per process.  When torch is importable it is
    imported first: torch bundles a HIP runtime with the same soname as the
    one the library links, and whichever loads first serves both, so loading
    torch first lets torch device tensors be passed as device buffers."""
    global _LIB
    if _LIB is None:
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        _LIB = Library()
    return _LIB
