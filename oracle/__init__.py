"""ctypes bindings for the CPU oracle — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker or the timed CPU baseline.
The qwn_hip library never calls into it.

``load()`` returns the restatement (liboracle.so, built by oracle/Makefile);
``load_ref()`` returns the reference's own CPU kernels compiled in place
(oracle/_ref/libqwn_ref.so) or None when that build is absent.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# QWN_ORACLE_LIB names another build of the same sources (the sanitizer run)
ORACLE_SO = os.environ.get("QWN_ORACLE_LIB") or os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libqwn_ref.so")

_c_i8p = ctypes.POINTER(ctypes.c_int8)
_c_u8p = ctypes.POINTER(ctypes.c_uint8)
_c_u16p = ctypes.POINTER(ctypes.c_uint16)
_c_i32p = ctypes.POINTER(ctypes.c_int32)
_c_f32p = ctypes.POINTER(ctypes.c_float)


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def ptr(a: np.ndarray, ctype):
    assert a.flags["C_CONTIGUOUS"], "oracle buffers must be contiguous"
    return a.ctypes.data_as(ctypes.POINTER(ctype))


class QoModelConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("hidden", "intermediate", "layers", "heads",
                                            "kv_heads", "head_dim", "vocab", "max_ctx")] + \
               [("rope_theta", ctypes.c_float), ("rms_eps", ctypes.c_float),
                ("proj_dtype", ctypes.c_int)]


class QoModel(ctypes.Structure):
    _fields_ = [("cfg", QoModelConfig), ("embed", ctypes.c_void_p), ("final_norm", ctypes.c_void_p),
                ("proj", ctypes.POINTER(ctypes.c_void_p)), ("norms", ctypes.POINTER(ctypes.c_void_p)),
                ("qk_norms", ctypes.POINTER(ctypes.c_void_p)), ("biases", ctypes.POINTER(ctypes.c_void_p)),
                ("embed_dtype", ctypes.c_int), ("lm_head", ctypes.c_void_p), ("lm_head_dtype", ctypes.c_int)]


# qwn_oracle.h QO_DT_*: the embedding's and an untied LM head's dtype
DT_CODES = {"f16": 1, "bf16": 4, "q4_0": 2, "hvsq2": 9}


BIAS_ORDER = ("q_bias", "k_bias", "v_bias", "o_bias")


PROJ_ORDER = ("q", "k", "v", "o", "gate", "up", "down")


def model_struct(model: dict) -> tuple:
    """ctypes view of a qwanto_amd.synth.decoder_model dict (the arrays stay
    owned by the dict; keep it alive)."""
    cfg = model["cfg"]
    c = QoModelConfig(hidden=cfg["hidden"], intermediate=cfg["intermediate"], layers=cfg["layers"],
                      heads=cfg["heads"], kv_heads=cfg["kv_heads"], head_dim=cfg["head_dim"],
                      vocab=cfg["vocab"], max_ctx=cfg["max_ctx"], rope_theta=cfg["rope_theta"],
                      rms_eps=cfg["rms_eps"], proj_dtype=2 if model["dtype"] == "q4_0" else 1)
    L = cfg["layers"]
    proj = (ctypes.c_void_p * (7 * L))(*[model["layers"][l][p].ctypes.data
                                         for l in range(L) for p in PROJ_ORDER])
    norms = (ctypes.c_void_p * (2 * L))(*[model["layers"][l][n].ctypes.data
                                          for l in range(L) for n in ("input_norm", "post_norm")])
    qk = None
    if "q_norm" in model["layers"][0]:
        qk = (ctypes.c_void_p * (2 * L))(*[model["layers"][l][n].ctypes.data
                                           for l in range(L) for n in ("q_norm", "k_norm")])
    bias = None
    if any(b in layer for layer in model["layers"] for b in BIAS_ORDER):
        bias = (ctypes.c_void_p * (4 * L))(*[model["layers"][l][b].ctypes.data if b in model["layers"][l] else None
                                             for l in range(L) for b in BIAS_ORDER])
    m = QoModel(cfg=c, embed=model["embed"].ctypes.data, final_norm=model["final_norm"].ctypes.data,
                proj=ctypes.cast(proj, ctypes.POINTER(ctypes.c_void_p)),
                norms=ctypes.cast(norms, ctypes.POINTER(ctypes.c_void_p)),
                qk_norms=ctypes.cast(qk, ctypes.POINTER(ctypes.c_void_p)) if qk is not None else None,
                biases=ctypes.cast(bias, ctypes.POINTER(ctypes.c_void_p)) if bias is not None else None,
                embed_dtype=DT_CODES[model.get("embed_dtype", "f16")],
                lm_head=model["lm_head"].ctypes.data if "lm_head" in model else None,
                lm_head_dtype=DT_CODES[model["lm_head_dtype"]] if "lm_head" in model else 0)
    return m, (proj, norms, qk, bias)


class Decoder:
    """The oracle decoder (qwn_oracle_decoder.c) over a synthetic model."""

    def __init__(self, oracle: "Oracle", model: dict, threads: int = 0):
        self.o, self.model = oracle, model
        self.struct, self._keep = model_struct(model)
        self.h = oracle.lib.qo_decoder_create(ctypes.byref(self.struct), threads)
        if not self.h:
            raise MemoryError("qo_decoder_create failed")
        self.vocab = model["cfg"]["vocab"]

    def close(self):
        if self.h:
            self.o.lib.qo_decoder_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def perturb(self, seed: int) -> None:
        """Calibration mode: rounding-sized moves of half of every stage's
        outputs (seed 0: off, the reference's arithmetic)."""
        self.o.lib.qo_decoder_set_perturbation(self.h, seed)

    def forward(self, token: int) -> np.ndarray:
        logits = np.empty(self.vocab, dtype=np.float32)
        rc = self.o.lib.qo_decoder_forward(self.h, int(token), ptr(logits, ctypes.c_float))
        assert rc == 0, "oracle forward failed"
        return logits

    def generate(self, prompt: np.ndarray, max_new: int):
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        tokens = np.zeros(max_new, dtype=np.int32)
        margins = np.zeros(max_new, dtype=np.float32)
        rc = self.o.lib.qo_decoder_generate(self.h, ptr(prompt, ctypes.c_int32), prompt.size, max_new,
                                            ptr(tokens, ctypes.c_int32), ptr(margins, ctypes.c_float))
        assert rc == max_new, "oracle generate failed"
        return tokens, margins


class Oracle:
    """Typed numpy front end of liboracle.so."""

    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            build()
        lib = ctypes.CDLL(path)
        self.lib = lib
        lib.qo_half_to_float.argtypes = [ctypes.c_uint16]
        lib.qo_half_to_float.restype = ctypes.c_float
        lib.qo_quantize_tokens.argtypes = [_c_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                           _c_i8p, _c_f32p, _c_i32p, ctypes.c_int]
        lib.qo_gemv_q4_0_q8.argtypes = [_c_u8p, _c_i8p, ctypes.c_float, ctypes.c_int,
                                        ctypes.c_int, _c_f32p, ctypes.c_int]
        lib.qo_matmul_q4_0.argtypes = [_c_u8p, _c_f32p, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_int, _c_f32p, ctypes.c_int]
        lib.qo_q4_0_block_sums.argtypes = [_c_u8p, _c_i8p, ctypes.c_int, ctypes.c_int, _c_i32p]
        lib.qo_gemv_hvsq2_scalar.argtypes = [_c_u8p, _c_i8p, _c_i32p, ctypes.c_float,
                                             ctypes.c_int, ctypes.c_int, ctypes.c_size_t, _c_f32p]
        lib.qo_gemv_hvsq2_delayed.argtypes = [_c_u8p, _c_i8p, _c_i32p, ctypes.c_float,
                                              ctypes.c_int, ctypes.c_int, ctypes.c_size_t,
                                              _c_f32p, ctypes.c_int]
        lib.qo_matmul_hvsq2.argtypes = [_c_u8p, _c_f32p, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, _c_f32p, ctypes.c_int, ctypes.c_int]
        lib.qo_hvsq2_octant_sums.argtypes = [_c_u8p, _c_i8p, ctypes.c_int, ctypes.c_int,
                                             _c_i32p, _c_i32p]
        lib.qo_hvsq2_best_variant.restype = ctypes.c_int
        lib.qo_variant_name.argtypes = [ctypes.c_int]
        lib.qo_variant_name.restype = ctypes.c_char_p
        lib.qo_matmul_f16.argtypes = [_c_u16p, _c_f32p, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, _c_f32p, ctypes.c_int]
        lib.qo_matmul_bf16.argtypes = lib.qo_matmul_f16.argtypes
        lib.qo_bf16_to_float.argtypes = [ctypes.c_uint16]
        lib.qo_bf16_to_float.restype = ctypes.c_float
        lib.qo_q8_quantize_vector.argtypes = [_c_f32p, _c_i8p, _c_f32p, ctypes.c_int]
        lib.qo_q8_attention.argtypes = [_c_f32p, _c_i8p, _c_i8p, _c_f32p, _c_f32p,
                                        ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_float, _c_f32p, ctypes.c_int]
        lib.qo_q8_attention_abi.argtypes = lib.qo_q8_attention.argtypes[:-1]
        lib.qo_rmsnorm.argtypes = [_c_f32p, _c_f32p, _c_f32p, ctypes.c_int, ctypes.c_float]
        lib.qo_rope_table.argtypes = [_c_f32p, _c_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_float]
        lib.qo_rope_apply.argtypes = [_c_f32p, ctypes.c_int, ctypes.c_int, _c_f32p, _c_f32p]
        lib.qo_argmax.argtypes = [_c_f32p, ctypes.c_int]
        lib.qo_decoder_create.argtypes = [ctypes.POINTER(QoModel), ctypes.c_int]
        lib.qo_decoder_create.restype = ctypes.c_void_p
        lib.qo_decoder_free.argtypes = [ctypes.c_void_p]
        lib.qo_decoder_forward.argtypes = [ctypes.c_void_p, ctypes.c_int, _c_f32p]
        lib.qo_decoder_set_perturbation.argtypes = [ctypes.c_void_p, ctypes.c_uint32]
        lib.qo_decoder_generate.argtypes = [ctypes.c_void_p, _c_i32p, ctypes.c_int, ctypes.c_int,
                                            _c_i32p, _c_f32p]

    # -- decoder pieces -------------------------------------------------
    def rmsnorm(self, x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.float32)
        out = np.empty_like(x)
        self.lib.qo_rmsnorm(ptr(out, ctypes.c_float), ptr(x, ctypes.c_float), ptr(w, ctypes.c_float),
                            x.size, eps)
        return out

    def rope_table(self, max_ctx: int, half: int, theta: float):
        c = np.empty((max_ctx, half), dtype=np.float32)
        s = np.empty((max_ctx, half), dtype=np.float32)
        self.lib.qo_rope_table(ptr(c, ctypes.c_float), ptr(s, ctypes.c_float), max_ctx, half, theta)
        return c, s

    def decoder(self, model: dict, threads: int = 0) -> "Decoder":
        return Decoder(self, model, threads)

    # -- scalar helpers -------------------------------------------------
    def half_to_float(self, h: int) -> float:
        return self.lib.qo_half_to_float(h)

    def best_variant(self) -> int:
        return self.lib.qo_hvsq2_best_variant()

    def variant_name(self, v: int) -> str:
        return self.lib.qo_variant_name(v).decode()

    # -- a1 ---------------------------------------------------------------
    def quantize(self, x: np.ndarray, padded_k: int | None = None):
        """Per-token quantization; returns (q8 [M, padded_k], scales [M],
        sums [M, padded_k/32])."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.ndim == 1:
            x = x[None, :]
        M, K = x.shape
        padded = padded_k or (K + 255) // 256 * 256
        q8 = np.zeros((M, padded), dtype=np.int8)
        scales = np.zeros(M, dtype=np.float32)
        sums = np.zeros((M, padded // 32), dtype=np.int32)
        self.lib.qo_quantize_tokens(ptr(x, ctypes.c_float), M, K, padded, ptr(q8, ctypes.c_int8),
                                    ptr(scales, ctypes.c_float), ptr(sums, ctypes.c_int32),
                                    padded // 32)
        return q8, scales, sums

    # -- Q4_0 ---------------------------------------------------------------
    def gemv_q4_0_q8(self, w: np.ndarray, q8: np.ndarray, x_scale: float, K: int, N: int,
                     threads: int = 0) -> np.ndarray:
        y = np.zeros(N, dtype=np.float32)
        q8 = np.ascontiguousarray(q8, dtype=np.int8)
        self.lib.qo_gemv_q4_0_q8(ptr(w, ctypes.c_uint8), ptr(q8, ctypes.c_int8), x_scale, K, N,
                                 ptr(y, ctypes.c_float), threads)
        return y

    def matmul_q4_0(self, w: np.ndarray, x: np.ndarray, N: int, threads: int = 0) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        M, K = x.shape
        y = np.zeros((M, N), dtype=np.float32)
        rc = self.lib.qo_matmul_q4_0(ptr(w, ctypes.c_uint8), ptr(x, ctypes.c_float), M, K, N,
                                     ptr(y, ctypes.c_float), threads)
        assert rc == 0
        return y

    def q4_0_block_sums(self, w: np.ndarray, q8: np.ndarray, K: int, N: int) -> np.ndarray:
        raw = np.zeros((N, (K + 31) // 32), dtype=np.int32)
        q8 = np.ascontiguousarray(q8, dtype=np.int8)
        self.lib.qo_q4_0_block_sums(ptr(w, ctypes.c_uint8), ptr(q8, ctypes.c_int8), K, N,
                                    ptr(raw, ctypes.c_int32))
        return raw

    # -- HyperVSQ-2 ------------------------------------------------------------
    def gemv_hvsq2(self, w: np.ndarray, q8: np.ndarray, sums, x_scale: float, K: int, N: int,
                   variant: int = -1) -> np.ndarray:
        """variant -2 = scalar golden, otherwise the delayed kernel."""
        y = np.zeros(N, dtype=np.float32)
        q8 = np.ascontiguousarray(q8, dtype=np.int8)
        sp = ptr(np.ascontiguousarray(sums, dtype=np.int32), ctypes.c_int32) if sums is not None \
            else None
        row_bytes = (K + 255) // 256 * 74
        if variant == -2:
            self.lib.qo_gemv_hvsq2_scalar(ptr(w, ctypes.c_uint8), ptr(q8, ctypes.c_int8), sp,
                                          x_scale, K, N, row_bytes, ptr(y, ctypes.c_float))
        else:
            self.lib.qo_gemv_hvsq2_delayed(ptr(w, ctypes.c_uint8), ptr(q8, ctypes.c_int8), sp,
                                           x_scale, K, N, row_bytes, ptr(y, ctypes.c_float),
                                           variant)
        return y

    def matmul_hvsq2(self, w: np.ndarray, x: np.ndarray, N: int, threads: int = 0,
                     variant: int = -1) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        M, K = x.shape
        y = np.zeros((M, N), dtype=np.float32)
        rc = self.lib.qo_matmul_hvsq2(ptr(w, ctypes.c_uint8), ptr(x, ctypes.c_float), M, K, N,
                                      ptr(y, ctypes.c_float), threads, variant)
        assert rc == 0
        return y

    def hvsq2_octant_sums(self, w: np.ndarray, q8: np.ndarray, K: int, N: int):
        nb = (K + 255) // 256
        sq = np.zeros((N, nb * 8), dtype=np.int32)
        sa = np.zeros(nb * 8, dtype=np.int32)
        q8 = np.ascontiguousarray(q8, dtype=np.int8)
        self.lib.qo_hvsq2_octant_sums(ptr(w, ctypes.c_uint8), ptr(q8, ctypes.c_int8), K, N,
                                      ptr(sq, ctypes.c_int32), ptr(sa, ctypes.c_int32))
        return sq, sa

    # -- F16 -------------------------------------------------------------------
    def matmul_f16(self, w: np.ndarray, x: np.ndarray, threads: int = 1) -> np.ndarray:
        w = np.ascontiguousarray(w, dtype=np.float16)
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.ndim == 1:
            x = x[None, :]
        N, K = w.shape
        M = x.shape[0]
        y = np.zeros((M, N), dtype=np.float32)
        self.lib.qo_matmul_f16(w.view(np.uint16).ctypes.data_as(_c_u16p), ptr(x, ctypes.c_float),
                               M, K, N, ptr(y, ctypes.c_float), threads)
        return y

    def matmul_bf16(self, w: np.ndarray, x: np.ndarray, threads: int = 1) -> np.ndarray:
        """w: [N][K] bfloat16 bit patterns (uint16)."""
        w = np.ascontiguousarray(w, dtype=np.uint16)
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.ndim == 1:
            x = x[None, :]
        N, K = w.shape
        M = x.shape[0]
        y = np.zeros((M, N), dtype=np.float32)
        self.lib.qo_matmul_bf16(w.ctypes.data_as(_c_u16p), ptr(x, ctypes.c_float), M, K, N,
                                ptr(y, ctypes.c_float), threads)
        return y

    # -- Q8 KV -----------------------------------------------------------------
    def q8_quantize(self, v: np.ndarray):
        v = np.ascontiguousarray(v, dtype=np.float32)
        n = v.shape[-1]
        groups = (n + 63) // 64
        flat = v.reshape(-1, n)
        q = np.zeros(flat.shape, dtype=np.int8)
        s = np.zeros((flat.shape[0], groups), dtype=np.float32)
        for t in range(flat.shape[0]):
            self.lib.qo_q8_quantize_vector(ptr(flat[t], ctypes.c_float), ptr(q[t], ctypes.c_int8),
                                           ptr(s[t], ctypes.c_float), n)
        return q.reshape(v.shape), (s[0] if v.ndim == 1 else s.reshape(v.shape[:-1] + (groups,)))

    def q8_attention(self, query, kq, vq, ks, vs, query_heads, kv_heads, head_dim, pos, scale,
                     threads: int = 0) -> np.ndarray:
        out = np.zeros(query_heads * head_dim, dtype=np.float32)
        query = np.ascontiguousarray(query, dtype=np.float32)
        self.lib.qo_q8_attention(ptr(query, ctypes.c_float), ptr(kq, ctypes.c_int8),
                                 ptr(vq, ctypes.c_int8), ptr(ks, ctypes.c_float),
                                 ptr(vs, ctypes.c_float), query_heads, kv_heads, head_dim, pos,
                                 scale, ptr(out, ctypes.c_float), threads)
        return out

    def q8_attention_abi(self, query, kq, vq, ks, vs, query_heads, kv_heads, head_dim, pos,
                         scale) -> np.ndarray:
        """Attention with the GPU ABI's head mapping kv = h * HK // H (any ratio)."""
        out = np.zeros(query_heads * head_dim, dtype=np.float32)
        query = np.ascontiguousarray(query, dtype=np.float32)
        self.lib.qo_q8_attention_abi(ptr(query, ctypes.c_float), ptr(kq, ctypes.c_int8),
                                     ptr(vq, ctypes.c_int8), ptr(ks, ctypes.c_float),
                                     ptr(vs, ctypes.c_float), query_heads, kv_heads, head_dim,
                                     pos, scale, ptr(out, ctypes.c_float))
        return out


class Reference:
    """The reference's own CPU kernels (oracle/_ref), for pinning the oracle."""

    def __init__(self, path: str = REF_SO):
        lib = ctypes.CDLL(path)
        self.lib = lib
        for name in ("ref_matmul_q4_0", "ref_matmul_hvsq2", "ref_matmul_f16", "ref_matmul_bf16"):
            fn = getattr(lib, name)
            fn.argtypes = [ctypes.c_void_p, ctypes.c_uint64, _c_f32p, ctypes.c_int, ctypes.c_int,
                           ctypes.c_int, _c_f32p]
        lib.ref_quantize_token.argtypes = [_c_f32p, ctypes.c_int, _c_i8p, _c_f32p, _c_i32p]
        lib.ref_cpu_kernel_name.restype = ctypes.c_char_p
        lib.ref_q8_attention.argtypes = [_c_f32p, _c_f32p, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_int, _c_f32p, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_float, _c_f32p, _c_i8p, _c_i8p, _c_f32p,
                                         _c_f32p]
        lib.qwn_gemv_hypervsq2_scalar.argtypes = [_c_u8p, _c_i8p, _c_i32p, ctypes.c_float,
                                                  ctypes.c_int, ctypes.c_int, ctypes.c_size_t,
                                                  _c_f32p]
        lib.qwn_gemv_hypervsq2_vnni_delayed.argtypes = lib.qwn_gemv_hypervsq2_scalar.argtypes

    def cpu_kernel_name(self) -> str:
        return self.lib.ref_cpu_kernel_name().decode()

    def plan_residency(self, path: str, gpu_budget: int, ram_budget: int, capacity: int):
        """The reference's qwn_plan_residency of a .qwn file: ([(name_hash,
        byte_offset, byte_size, tensor_index, tier, priority)] in plan order,
        (gpu, ram, file bytes))."""
        class Placement(ctypes.Structure):
            _fields_ = [("name_hash", ctypes.c_uint64), ("byte_offset", ctypes.c_uint64),
                        ("byte_size", ctypes.c_uint64), ("tensor_index", ctypes.c_uint32),
                        ("tier", ctypes.c_uint8), ("priority", ctypes.c_uint8),
                        ("reserved", ctypes.c_uint16)]
        fn = self.lib.qrh_plan_residency
        fn.argtypes = [ctypes.c_char_p, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint32,
                       ctypes.c_void_p]
        items = (Placement * capacity)()
        totals = (ctypes.c_uint64 * 3)()
        n = fn(path.encode(), int(gpu_budget), int(ram_budget), items, capacity, totals)
        assert n >= 0, "reference residency plan failed"
        rows = [(p.name_hash, p.byte_offset, p.byte_size, p.tensor_index, p.tier, p.priority)
                for p in items[:n]]
        return rows, (totals[0], totals[1], totals[2])

    def _matmul(self, fn, w: np.ndarray, x: np.ndarray, N: int) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        M, K = x.shape
        y = np.zeros((M, N), dtype=np.float32)
        rc = fn(w.ctypes.data, w.nbytes, ptr(x, ctypes.c_float), M, K, N, ptr(y, ctypes.c_float))
        assert rc == 0, "reference matmul rejected its input"
        return y

    def matmul_q4_0(self, w, x, N):
        return self._matmul(self.lib.ref_matmul_q4_0, w, x, N)

    def matmul_hvsq2(self, w, x, N):
        return self._matmul(self.lib.ref_matmul_hvsq2, w, x, N)

    def matmul_f16(self, w, x):
        w = np.ascontiguousarray(w, dtype=np.float16)
        return self._matmul(self.lib.ref_matmul_f16, w, x, w.shape[0])

    def matmul_bf16(self, w, x):
        """w: [N][K] bfloat16 bit patterns (uint16)."""
        w = np.ascontiguousarray(w, dtype=np.uint16)
        return self._matmul(self.lib.ref_matmul_bf16, w, x, w.shape[0])

    def quantize_token(self, x: np.ndarray):
        x = np.ascontiguousarray(x, dtype=np.float32)
        K = x.shape[0]
        padded = (K + 255) // 256 * 256
        q8 = np.zeros(padded, dtype=np.int8)
        scale = np.zeros(1, dtype=np.float32)
        sums = np.zeros(padded // 32, dtype=np.int32)
        rc = self.lib.ref_quantize_token(ptr(x, ctypes.c_float), K, ptr(q8, ctypes.c_int8),
                                         ptr(scale, ctypes.c_float), ptr(sums, ctypes.c_int32))
        assert rc == 0
        return q8, float(scale[0]), sums

    def gemv_hvsq2(self, w, q8, sums, x_scale, K, N, delayed=True):
        y = np.zeros(N, dtype=np.float32)
        fn = self.lib.qwn_gemv_hypervsq2_vnni_delayed if delayed else \
            self.lib.qwn_gemv_hypervsq2_scalar
        sp = ptr(np.ascontiguousarray(sums, dtype=np.int32), ctypes.c_int32) if sums is not None \
            else None
        fn(ptr(w, ctypes.c_uint8), ptr(np.ascontiguousarray(q8, dtype=np.int8), ctypes.c_int8), sp,
           x_scale, K, N, (K + 255) // 256 * 74, ptr(y, ctypes.c_float))
        return y

    def q8_attention(self, keys, values, kv_heads, head_dim, query, query_heads, pos, scale):
        keys = np.ascontiguousarray(keys, dtype=np.float32)
        values = np.ascontiguousarray(values, dtype=np.float32)
        query = np.ascontiguousarray(query, dtype=np.float32)
        tokens = keys.shape[0]
        channels = kv_heads * head_dim
        groups = (channels + 63) // 64
        out = np.zeros(query_heads * head_dim, dtype=np.float32)
        kq = np.zeros((tokens, channels), dtype=np.int8)
        vq = np.zeros((tokens, channels), dtype=np.int8)
        ks = np.zeros((tokens, groups), dtype=np.float32)
        vs = np.zeros((tokens, groups), dtype=np.float32)
        rc = self.lib.ref_q8_attention(ptr(keys, ctypes.c_float), ptr(values, ctypes.c_float),
                                       tokens, kv_heads, head_dim, ptr(query, ctypes.c_float),
                                       query_heads, pos, scale, ptr(out, ctypes.c_float),
                                       ptr(kq, ctypes.c_int8), ptr(vq, ctypes.c_int8),
                                       ptr(ks, ctypes.c_float), ptr(vs, ctypes.c_float))
        assert rc == 0
        return out, kq, vq, ks, vs


def load() -> Oracle:
    return Oracle()


def load_ref():
    return Reference() if os.path.exists(REF_SO) else None


REF_DECODER_SO = os.path.join(HERE, "_ref", "libqwn_ref_decoder.so")


class RefDecoder:
    """The reference decoder (c/qwanto_decode.c) compiled in place, CPU
    backend with the Q8 KV cache, over a .qwn file."""

    def __init__(self, path: str, context: int, threads: int = 0):
        lib = ctypes.CDLL(REF_DECODER_SO)
        lib.qrd_open.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.c_char_p,
                                 ctypes.c_int]
        lib.qrd_open.restype = ctypes.c_void_p
        lib.qrd_forward.argtypes = [ctypes.c_void_p, ctypes.c_int, _c_f32p, ctypes.c_int]
        lib.qrd_close.argtypes = [ctypes.c_void_p]
        lib.qrd_cpu_fallback_count.argtypes = [ctypes.c_void_p]
        lib.qrd_cpu_fallback_count.restype = ctypes.c_uint64
        self.lib = lib
        err = ctypes.create_string_buffer(256)
        self.h = lib.qrd_open(path.encode(), context, threads, err, 256)
        if not self.h:
            raise RuntimeError(f"reference decoder open failed: {err.value.decode()}")

    def forward(self, token: int, vocab: int) -> np.ndarray:
        logits = np.empty(vocab, dtype=np.float32)
        rc = self.lib.qrd_forward(self.h, int(token), ptr(logits, ctypes.c_float), vocab)
        assert rc == 0, f"reference forward failed ({rc})"
        return logits

    def close(self):
        if self.h:
            self.lib.qrd_close(self.h)
            self.h = None

    def __del__(self):
        self.close()


def load_ref_decoder(path: str, context: int, threads: int = 0):
    return RefDecoder(path, context, threads) if os.path.exists(REF_DECODER_SO) else None
