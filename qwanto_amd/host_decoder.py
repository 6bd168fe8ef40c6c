"""ctypes front end of libqwn_host_decoder.so (include/qwn_host_decoder.h):
the host-side decoder that drives every projection, the LM head and the Q8
KV cache through the qwn_cuda ABI, as qwnrun's host does."""
from __future__ import annotations

import ctypes
import os

import numpy as np

from . import build

# QWN_HOST_DECODER_LIB names another build of the same source (the sanitizer run)
LIB_PATH = os.environ.get("QWN_HOST_DECODER_LIB") or build.HOST_DECODER
PROJ_ORDER = ("q", "k", "v", "o", "gate", "up", "down")


class QhdConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("hidden", "intermediate", "layers", "heads", "kv_heads",
                                            "head_dim", "vocab", "max_ctx")] + \
               [("rope_theta", ctypes.c_float), ("rms_eps", ctypes.c_float), ("proj_dtype", ctypes.c_int)]


class QhdModel(ctypes.Structure):
    _fields_ = [("cfg", QhdConfig), ("embed", ctypes.c_void_p), ("final_norm", ctypes.c_void_p),
                ("proj", ctypes.POINTER(ctypes.c_void_p)), ("norms", ctypes.POINTER(ctypes.c_void_p)),
                ("qk_norms", ctypes.POINTER(ctypes.c_void_p)), ("biases", ctypes.POINTER(ctypes.c_void_p)),
                ("embed_dtype", ctypes.c_int), ("lm_head", ctypes.c_void_p), ("lm_head_dtype", ctypes.c_int)]


# include/qwn_host_decoder.h QHD_DT_*
DT_CODES = {"f16": 1, "q4_0": 2, "bf16": 4, "hvsq2": 9}


class QhdMetrics(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in ("gpu_matmul_count", "cpu_fallback_count",
                                               "gpu_kernel_launch_count", "gpu_upload_bytes",
                                               "gpu_resident_bytes", "kv_cache_kernel_count", "abi_calls")] + \
               [(n, ctypes.c_double) for n in ("gpu_kernel_ms", "gpu_transfer_ms", "gpu_sync_ms", "prefill_ms",
                                               "decode_wall_ms")] + \
               [("prompt_tokens", ctypes.c_int), ("generated_tokens", ctypes.c_int),
                ("kernel_type", ctypes.c_char * 32), ("backend_reason", ctypes.c_char * 96)]


class OpenError(RuntimeError):
    """qhd_open refused: `reason` is the loader's backend_reason string."""

    def __init__(self, message: str, reason: str):
        super().__init__(f"host decoder open failed: {message} [{reason}]")
        self.reason = reason


def model_struct(model: dict):
    """QhdModel over a synth.decoder_model / qwn_file.read_decoder_model dict;
    returns the struct and the pointer tables it references."""
    cfg = model["cfg"]
    c = QhdConfig(hidden=cfg["hidden"], intermediate=cfg["intermediate"], layers=cfg["layers"],
                  heads=cfg["heads"], kv_heads=cfg["kv_heads"], head_dim=cfg["head_dim"], vocab=cfg["vocab"],
                  max_ctx=cfg["max_ctx"], rope_theta=cfg["rope_theta"], rms_eps=cfg["rms_eps"],
                  proj_dtype=2 if model["dtype"] == "q4_0" else 1)
    L = cfg["layers"]
    proj = (ctypes.c_void_p * (7 * L))(*[model["layers"][l][p].ctypes.data for l in range(L) for p in PROJ_ORDER])
    norms = (ctypes.c_void_p * (2 * L))(*[model["layers"][l][n].ctypes.data for l in range(L)
                                          for n in ("input_norm", "post_norm")])
    qk = None
    if "q_norm" in model["layers"][0]:
        qk = (ctypes.c_void_p * (2 * L))(*[model["layers"][l][n].ctypes.data for l in range(L)
                                           for n in ("q_norm", "k_norm")])
    bias = None
    names = ("q_bias", "k_bias", "v_bias", "o_bias")
    if any(b in layer for layer in model["layers"] for b in names):
        bias = (ctypes.c_void_p * (4 * L))(*[model["layers"][l][b].ctypes.data if b in model["layers"][l] else None
                                             for l in range(L) for b in names])
    P = ctypes.POINTER(ctypes.c_void_p)
    m = QhdModel(cfg=c, embed=model["embed"].ctypes.data, final_norm=model["final_norm"].ctypes.data,
                 proj=ctypes.cast(proj, P), norms=ctypes.cast(norms, P),
                 qk_norms=ctypes.cast(qk, P) if qk is not None else None,
                 biases=ctypes.cast(bias, P) if bias is not None else None,
                 embed_dtype=DT_CODES[model.get("embed_dtype", "f16")],
                 lm_head=model["lm_head"].ctypes.data if "lm_head" in model else None,
                 lm_head_dtype=DT_CODES[model["lm_head_dtype"]] if "lm_head" in model else 0)
    return m, (proj, norms, qk, bias)


class HostDecoder:
    def __init__(self, model: dict, abi_path: str | None = None, device: int = 0):
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} is not built (python qwanto_amd/build.py)")
        if abi_path is None:
            try:
                import torch  # noqa: F401  (one HIP runtime per process, see qwanto_amd.abi.load)
            except ImportError:
                pass
        lib = ctypes.CDLL(LIB_PATH)
        lib.qhd_open.argtypes = [ctypes.POINTER(QhdModel), ctypes.c_char_p, ctypes.c_int, ctypes.c_char_p,
                                 ctypes.c_int, ctypes.c_char_p]
        lib.qhd_open.restype = ctypes.c_void_p
        lib.qhd_close.argtypes = [ctypes.c_void_p]
        lib.qhd_forward.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_float)]
        lib.qhd_generate.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int32), ctypes.c_int, ctypes.c_int,
                                     ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_float)]
        lib.qhd_metrics.argtypes = [ctypes.c_void_p, ctypes.POINTER(QhdMetrics)]
        lib.qhd_last_error.argtypes = [ctypes.c_void_p]
        lib.qhd_last_error.restype = ctypes.c_char_p
        self.lib, self.model = lib, model
        self.struct, self._keep = model_struct(model)
        err = ctypes.create_string_buffer(256)
        reason = ctypes.create_string_buffer(96)
        self.h = lib.qhd_open(ctypes.byref(self.struct), abi_path.encode() if abi_path else None, device, err, 256,
                              reason)
        if not self.h:
            raise OpenError(err.value.decode(), reason.value.decode())
        self.vocab = model["cfg"]["vocab"]

    def _check(self, rc):
        if rc < 0:
            raise RuntimeError(self.lib.qhd_last_error(self.h).decode())
        return rc

    def forward(self, token: int) -> np.ndarray:
        logits = np.empty(self.vocab, dtype=np.float32)
        self._check(self.lib.qhd_forward(self.h, int(token),
                                         logits.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))
        return logits

    def generate(self, prompt, max_new: int):
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        tokens = np.zeros(max_new, dtype=np.int32)
        margins = np.zeros(max_new, dtype=np.float32)
        self._check(self.lib.qhd_generate(self.h, prompt.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), prompt.size,
                                          max_new, tokens.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                                          margins.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))
        return tokens, margins

    def metrics(self) -> QhdMetrics:
        m = QhdMetrics()
        self._check(self.lib.qhd_metrics(self.h, ctypes.byref(m)))
        return m

    def close(self):
        if self.h:
            self.lib.qhd_close(self.h)
            self.h = None

    def __del__(self):
        self.close()
