"""Seeded synthetic inputs for the quantized decode path.

Byte layouts follow the reference writers: Q4_0 blocks are
``[fp16 d][16 bytes of nibbles, element 2j = low nibble of byte j]``
(c/qwanto_native.h:35, c/tools/qwn_convert.py:65-110) and HyperVSQ-2 blocks
are ``[fp16 d_base][fp16 m_base][4 bytes of octant multipliers][2 reserved]
[64 bytes of 2-bit codes]`` (c/qwanto_native.h:96-103,
c/tools/qwn_convert.py:365-469).  Values are random rather than quantized
from real weights; the distributions are the ones the benchmark
configurations name:

* Q4_0: ``d = fp16(|N(0, 0.02)|)``, uniform random nibble bytes.
* HyperVSQ-2: ``d_base = fp16(|N(0, 0.02)|)``, ``m_base = fp16(N(0, 0.02))``,
  octant multipliers uniform in 1..8 (the converter's range,
  c/tools/qwn_convert.py:397), random reserved bytes (they must be ignored),
  uniform random code bytes.
* activations ``x ~ N(0, 1)`` in fp32; fp16 tensors ``N(0, 0.02)``.
"""
from __future__ import annotations

import numpy as np

Q4_0_BLOCK_BYTES = 18
Q4_0_BLOCK_ELEMS = 32
HVSQ2_BLOCK_BYTES = 74
HVSQ2_BLOCK_ELEMS = 256

# Qwen2-1.5B projection shapes (rows N x cols K)
QWEN2_1P5B_SHAPES = {
    "q": (1536, 1536), "k": (256, 1536), "v": (256, 1536), "o": (1536, 1536),
    "gate": (8960, 1536), "up": (8960, 1536), "down": (1536, 8960),
}
# Qwen3-4B projection shapes (rows N x cols K)
QWEN3_4B_SHAPES = {
    "q": (4096, 2560), "k": (1024, 2560), "v": (1024, 2560), "o": (2560, 4096),
    "gate": (9728, 2560), "up": (9728, 2560), "down": (2560, 9728),
}
PROJECTIONS = ("q", "k", "v", "o", "gate", "up", "down")


def q4_0_row_bytes(cols: int) -> int:
    return (cols + 31) // 32 * Q4_0_BLOCK_BYTES


def hvsq2_row_bytes(cols: int) -> int:
    return (cols + 255) // 256 * HVSQ2_BLOCK_BYTES


def _half_bytes(values: np.ndarray) -> np.ndarray:
    return values.astype(np.float16).view(np.uint8).reshape(values.shape + (2,))


def q4_0_weights(rng: np.random.Generator, rows: int, cols: int, std: float = 0.02,
                 zero_mean: bool = False) -> np.ndarray:
    """Row-major Q4_0 matrix as a flat uint8 array (block scales |N(0, std)|;
    codes uniform over 0..15, or over 1..15 with zero_mean: weights (code-8)
    with mean 0 instead of -scale/2)."""
    blocks = rows * ((cols + 31) // 32)
    out = np.empty((blocks, Q4_0_BLOCK_BYTES), dtype=np.uint8)
    out[:, 0:2] = _half_bytes(np.abs(rng.normal(0.0, std, blocks)).astype(np.float32))
    if zero_mean:
        nib = rng.integers(1, 16, (blocks, 32), dtype=np.uint8)
        out[:, 2:] = nib[:, :16] | (nib[:, 16:] << 4)
    else:
        out[:, 2:] = rng.integers(0, 256, (blocks, 16), dtype=np.uint8)
    return out.reshape(-1)


def hvsq2_weights(rng: np.random.Generator, rows: int, cols: int, std: float = 0.02) -> np.ndarray:
    """Row-major HyperVSQ-2 matrix as a flat uint8 array (d_base |N(0, std)|,
    m_base N(0, std))."""
    blocks = rows * ((cols + 255) // 256)
    out = np.empty((blocks, HVSQ2_BLOCK_BYTES), dtype=np.uint8)
    out[:, 0:2] = _half_bytes(np.abs(rng.normal(0.0, std, blocks)).astype(np.float32))
    out[:, 2:4] = _half_bytes(rng.normal(0.0, std, blocks).astype(np.float32))
    sub = rng.integers(1, 9, (blocks, 8), dtype=np.uint8)
    out[:, 4:8] = sub[:, 0::2] | (sub[:, 1::2] << 4)
    out[:, 8:10] = rng.integers(0, 256, (blocks, 2), dtype=np.uint8)
    out[:, 10:] = rng.integers(0, 256, (blocks, 64), dtype=np.uint8)
    return out.reshape(-1)


def f16_weights(rng: np.random.Generator, rows: int, cols: int,
                std: float = 0.02) -> np.ndarray:
    return rng.normal(0.0, std, (rows, cols)).astype(np.float16)


def to_bf16_bits(values: np.ndarray) -> np.ndarray:
    """fp32 -> bfloat16 bit patterns (uint16), rounded to nearest even."""
    b = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


def bf16_weights(rng: np.random.Generator, rows: int, cols: int, std: float = 0.02) -> np.ndarray:
    """[rows][cols] bfloat16 bit patterns (uint16) of N(0, std) draws."""
    return to_bf16_bits(rng.normal(0.0, std, (rows, cols)).astype(np.float32))


def activations(rng: np.random.Generator, batch: int, cols: int) -> np.ndarray:
    return rng.standard_normal((batch, cols), dtype=np.float32)


def weights(dtype: str, rng: np.random.Generator, rows: int, cols: int, std: float = 0.02,
            zero_mean: bool = False) -> np.ndarray:
    if dtype == "q4_0":
        return q4_0_weights(rng, rows, cols, std, zero_mean)
    if dtype == "hvsq2":
        return hvsq2_weights(rng, rows, cols, std)
    if dtype == "f16":
        return f16_weights(rng, rows, cols, std)
    if dtype == "bf16":
        return bf16_weights(rng, rows, cols, std)
    raise ValueError(f"unknown weight dtype {dtype!r}")


def weight_bytes(dtype: str, rows: int, cols: int) -> int:
    """Algorithmic (on-disk) bytes of one matrix."""
    if dtype == "q4_0":
        return rows * q4_0_row_bytes(cols)
    if dtype == "hvsq2":
        return rows * hvsq2_row_bytes(cols)
    if dtype in ("f16", "bf16"):
        return rows * cols * 2
    raise ValueError(dtype)


# ---- synthetic decoder models ------------------------------------------------

# Qwen2-1.5B shaped dense decoder (the Q4_0 decode workload): tied F16
# embedding / LM head, no biases, no q/k norms, F32 norm weights of 1.
QWEN2_1P5B_CONFIG = {
    "hidden": 1536, "intermediate": 8960, "layers": 28, "heads": 12, "kv_heads": 2,
    "head_dim": 128, "vocab": 151936, "max_ctx": 512, "rope_theta": 1.0e6, "rms_eps": 1.0e-6,
}
# the Qwen3-4B layer shapes of the HyperVSQ-2 GEMV workload as a decoder
# (per-head q/k norms with decoder_model(..., qk_norm=True)), tied F16
# embedding
QWEN3_4B_SHAPED_CONFIG = {
    "hidden": 2560, "intermediate": 9728, "layers": 36, "heads": 32, "kv_heads": 8,
    "head_dim": 128, "vocab": 151936, "max_ctx": 512, "rope_theta": 1.0e6, "rms_eps": 1.0e-6,
}


def decoder_model(rng: np.random.Generator, cfg: dict, dtype: str = "q4_0", qk_norm: bool = False,
                  weight_std: float = 0.02, embed_std: float = 0.02, zero_mean: bool = False,
                  biases: str = "", embed_dtype: str = "f16", lm_head: str | None = None,
                  head_std: float = 0.02) -> dict:
    """Random decoder weights with the layout of a .qwn dense model: per layer
    q, k, v, o, gate, up, down quantized matrices ([out][in] row-major
    blocks), input/post norm vectors (and, with qk_norm, per-head q/k norm
    weights [head_dim] as Qwen3's self_attn.q_norm / k_norm, drawn
    1 + 0.2 N(0,1)); a tied F16 embedding [vocab][hidden] and the final
    norm.  weight_std / embed_std: the scale distributions' sigma (0.02 is
    the benchmark models' draw); zero_mean: Q4_0 codes drawn from 1..15 so
    the weights carry no common offset (with codes 0..15 every row's mean
    weight is -scale/2, which drives the residual stream of a random model
    toward one direction and its greedy output toward one token).  biases:
    the projections among "qkvo" that get an F32 bias drawn 0.5 N(0,1)
    (Qwen2 checkpoints carry q/k/v biases), as self_attn.*_proj.bias.
    embed_dtype: "f16" (the benchmark models) or "bf16" (bit patterns as
    uint16).  lm_head: None (the embedding is the LM head), or the dtype of a
    separate lm_head.weight [vocab][hidden] ("f16", "bf16", "q4_0",
    "hvsq2"), drawn after everything else with scale sigma head_std."""
    D, I = cfg["hidden"], cfg["intermediate"]
    Q, KV = cfg["heads"] * cfg["head_dim"], cfg["kv_heads"] * cfg["head_dim"]
    shapes = {"q": (Q, D), "k": (KV, D), "v": (KV, D), "o": (D, Q),
              "gate": (I, D), "up": (I, D), "down": (D, I)}
    layers = []
    for _ in range(cfg["layers"]):
        layer = {p: weights(dtype, rng, *shapes[p], std=weight_std, zero_mean=zero_mean) for p in PROJECTIONS}
        layer["input_norm"] = np.ones(D, dtype=np.float32)
        layer["post_norm"] = np.ones(D, dtype=np.float32)
        for p in biases:
            layer[p + "_bias"] = (0.5 * rng.standard_normal(shapes[p][0])).astype(np.float32)
        if qk_norm:
            for n in ("q_norm", "k_norm"):
                layer[n] = (1.0 + 0.2 * rng.standard_normal(cfg["head_dim"])).astype(np.float32)
        layers.append(layer)
    embed = (f16_weights if embed_dtype == "f16" else bf16_weights)(rng, cfg["vocab"], D, embed_std)
    model = {"cfg": dict(cfg), "dtype": dtype, "shapes": shapes, "layers": layers,
             "embed": embed, "embed_dtype": embed_dtype, "final_norm": np.ones(D, dtype=np.float32)}
    if lm_head is not None:
        model["lm_head"] = weights(lm_head, rng, cfg["vocab"], D, std=head_std)
        model["lm_head_dtype"] = lm_head
    return model


def prompt_tokens(rng: np.random.Generator, vocab: int, count: int = 32) -> np.ndarray:
    return rng.integers(0, vocab, count, dtype=np.int32)
