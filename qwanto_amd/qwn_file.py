"""Reader and writer of the Qwanto native model container (.qwn).

The on-disk format is the reference's (c/qwanto_native.h:14-136,
c/qwanto_native.c:86-177, writer c/tools/qwn_convert.py:566-645), kept
byte-compatible so the same file opens in qwnrun and here:

* a 4 KiB header: 112-byte prefix (magic ``QWANTO_NATIVE_V1``, version 1,
  flags, arch code, tensor count, inline count, reserved, parameter count,
  eight architecture dims), up to 29 inline 136-byte tensor descriptors,
  then the explicit q/k/v projection dims;
* tensor payloads, each at a 4 KiB aligned offset, sizes padded to 64;
* a tail: overflow header (count, descriptor size, descriptor offset, index
  offset, reserved), the overflow descriptors, an index of (FNV-1a 64 name
  hash, descriptor offset) sorted by hash, and finally the tail offset as
  the file's last 8 bytes.

A 2-D tensor's shape is (in, out): shape[0] is the fastest-varying
dimension, so a quantized [out][in] matrix is stored row by row.
"""
from __future__ import annotations

import json
import mmap
import os
import struct

import numpy as np

MAGIC = b"QWANTO_NATIVE_V1"
VERSION = 1
HEADER_SIZE = 0x1000
ALIGN = 0x1000
INLINE_MAX = 29
DESC_FMT = "<64sIII4Q3QI"
DESC_SIZE = struct.calcsize(DESC_FMT)
PREFIX_FMT = "<16sIIIIIIQ8Q"
PREFIX_SIZE = struct.calcsize(PREFIX_FMT)
EXT_OFFSET = PREFIX_SIZE + INLINE_MAX * DESC_SIZE
TAIL_FMT = "<IIQQQ"
TAIL_SIZE = struct.calcsize(TAIL_FMT)
assert DESC_SIZE == 136 and PREFIX_SIZE == 112

DT_F32, DT_F16, DT_Q4_0, DT_Q8_0, DT_BF16, DT_BYTES = 0, 1, 2, 3, 4, 5
DT_HYPER_VSQ2 = 9


def _align(n: int, a: int = ALIGN) -> int:
    return (n + a - 1) & ~(a - 1)


def fnv1a64(name: str) -> int:
    h = 0xCBF29CE484222325
    for b in name.encode("utf-8"):
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def payload_bytes(dtype: int, shape: tuple) -> int:
    numel = int(np.prod(shape))
    if dtype == DT_F32:
        return numel * 4
    if dtype in (DT_F16, DT_BF16):
        return numel * 2
    if dtype == DT_BYTES:
        return numel
    if dtype == DT_Q4_0:
        rows = numel // shape[0] if len(shape) == 2 else 1
        return rows * ((shape[0] + 31) // 32) * 18
    if dtype == DT_HYPER_VSQ2:
        rows = numel // shape[0] if len(shape) == 2 else 1
        return rows * ((shape[0] + 255) // 256) * 74
    raise ValueError(f"unsupported dtype {dtype}")


def _block_q(dtype: int) -> int:
    return 32 if dtype in (DT_Q4_0, DT_Q8_0) else 0


def write_qwn(path: str, tensors: list, arch_dims=(0,) * 8, qkv_dims=(0, 0, 0), arch_code: int = 1) -> int:
    """tensors: list of (name, dtype, shape, payload) with payload a bytes-like
    or numpy array of exactly payload_bytes(dtype, shape) bytes."""
    layout = []
    cursor = HEADER_SIZE
    for name, dtype, shape, payload in tensors:
        enc = name.encode("utf-8")
        if not 1 <= len(enc) <= 63:
            raise ValueError(f"tensor name must be 1..63 bytes: {name!r}")
        shape = tuple(int(s) for s in shape)
        data = memoryview(np.ascontiguousarray(payload) if isinstance(payload, np.ndarray) else payload).cast("B")
        size = payload_bytes(dtype, shape)
        if data.nbytes != size:
            raise ValueError(f"{name}: payload {data.nbytes} B, expected {size} B")
        cursor = _align(cursor)
        layout.append({"name": name, "enc": enc, "dtype": dtype, "shape": shape,
                       "numel": int(np.prod(shape)), "offset": cursor,
                       "size": (size + 63) & ~63, "data": data})
        cursor += layout[-1]["size"]
    inline = layout[:INLINE_MAX]
    overflow = layout[INLINE_MAX:]
    tail = _align(cursor)
    desc_off = tail + TAIL_SIZE
    index_off = desc_off + len(overflow) * DESC_SIZE
    file_size = index_off + len(overflow) * 16 + 8

    def desc(t):
        shape = list(t["shape"]) + [0] * (4 - len(t["shape"]))
        return struct.pack(DESC_FMT, t["enc"], len(t["enc"]), t["dtype"], len(t["shape"]), *shape,
                           t["numel"], t["offset"], t["size"], _block_q(t["dtype"]))

    header = bytearray(HEADER_SIZE)
    dims = (tuple(int(x) for x in arch_dims) + (0,) * 8)[:8]
    struct.pack_into(PREFIX_FMT, header, 0, MAGIC, VERSION, 0, arch_code, len(layout), len(inline), 0,
                     sum(t["numel"] for t in layout), *dims)
    for i, t in enumerate(inline):
        header[PREFIX_SIZE + i * DESC_SIZE:PREFIX_SIZE + (i + 1) * DESC_SIZE] = desc(t)
    struct.pack_into("<3Q", header, EXT_OFFSET, *[int(x) for x in qkv_dims])
    tmp = path + ".partial"
    with open(tmp, "wb") as f:
        f.write(header)
        for t in layout:
            f.seek(t["offset"])
            f.write(t["data"])
            pad = t["size"] - t["data"].nbytes
            if pad:
                f.write(b"\0" * pad)
        f.seek(tail)
        f.write(struct.pack(TAIL_FMT, len(overflow), DESC_SIZE, desc_off, index_off, 0))
        offs = []
        for i, t in enumerate(overflow):
            offs.append(desc_off + i * DESC_SIZE)
            f.write(desc(t))
        for h, off in sorted((fnv1a64(t["name"]), offs[i]) for i, t in enumerate(overflow)):
            f.write(struct.pack("<QQ", h, off))
        f.write(struct.pack("<Q", tail))
        f.truncate(file_size)
    os.replace(tmp, path)
    return file_size


class QwnFile:
    """Memory-mapped .qwn reader: tensors by name as numpy views."""

    def __init__(self, path: str):
        self._f = open(path, "rb")
        self.mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        prefix = struct.unpack_from(PREFIX_FMT, self.mm, 0)
        if prefix[0] != MAGIC or prefix[1] != VERSION:
            raise ValueError("not a version-1 .qwn file")
        self.arch_dims = prefix[8:16]
        n_tensors, inline_count = prefix[4], prefix[5]
        self.qkv_dims = struct.unpack_from("<3Q", self.mm, EXT_OFFSET)
        descs = [struct.unpack_from(DESC_FMT, self.mm, PREFIX_SIZE + i * DESC_SIZE)
                 for i in range(inline_count)]
        tail = struct.unpack_from("<Q", self.mm, len(self.mm) - 8)[0]
        count, dsize, doff, index_off, _ = struct.unpack_from(TAIL_FMT, self.mm, tail)
        # overflow tensors in the order of the hash-sorted index, as the
        # reference enumerates them (c/qwanto_native.c:286-305, 374-378), so
        # tensor indices agree with qwn_tensor_at
        for i in range(count):
            _, off = struct.unpack_from("<QQ", self.mm, index_off + 16 * i)
            descs.append(struct.unpack_from(DESC_FMT, self.mm, off))
        if len(descs) != n_tensors:
            raise ValueError("descriptor count mismatch")
        self.tensors = {}
        for d in descs:
            name = d[0][:d[1]].decode("utf-8")
            n_dims = d[3]
            self.tensors[name] = {"dtype": d[2], "shape": tuple(d[4:4 + n_dims]), "numel": d[8],
                                  "offset": d[9], "size": d[10]}

    def close(self):
        """Release the mapping; if array views of it are still alive it is
        released when the last of them goes away."""
        try:
            self.mm.close()
        except BufferError:
            pass
        self._f.close()

    def raw(self, name: str) -> np.ndarray:
        t = self.tensors[name]
        n = payload_bytes(t["dtype"], t["shape"])
        return np.frombuffer(self.mm, dtype=np.uint8, count=n, offset=t["offset"])

    def array(self, name: str) -> np.ndarray:
        t = self.tensors[name]
        raw = self.raw(name)
        if t["dtype"] == DT_F32:
            return raw.view(np.float32).reshape(t["shape"][::-1])
        if t["dtype"] == DT_F16:
            return raw.view(np.float16).reshape(t["shape"][::-1])
        if t["dtype"] == DT_BF16:  # bit patterns
            return raw.view(np.uint16).reshape(t["shape"][::-1])
        return raw

    def json(self, name: str):
        return json.loads(bytes(self.raw(name)).decode("utf-8"))


# ---- decoder models -------------------------------------------------------------

_HEAD_DT = {"f16": DT_F16, "bf16": DT_BF16, "q4_0": DT_Q4_0, "hvsq2": DT_HYPER_VSQ2}
_PROJ_NAMES = {"q": "self_attn.q_proj.weight", "k": "self_attn.k_proj.weight",
               "v": "self_attn.v_proj.weight", "o": "self_attn.o_proj.weight",
               "gate": "mlp.gate_proj.weight", "up": "mlp.up_proj.weight",
               "down": "mlp.down_proj.weight"}


def write_decoder_model(path: str, model: dict) -> int:
    """Write a synthetic dense decoder (qwanto_amd.synth.decoder_model) as a
    .qwn file the reference decoder opens: __qwn.config (HF-style JSON),
    a minimal __qwn.tokenizer, the F16 or BF16 embedding, F32 norms, the
    quantized projections and, for an untied model, lm_head.weight
    (c/qwanto_decode.c:1074-1076)."""
    cfg = model["cfg"]
    D, V = cfg["hidden"], cfg["vocab"]
    qdt = DT_Q4_0 if model["dtype"] == "q4_0" else DT_HYPER_VSQ2
    hf = {"hidden_size": D, "intermediate_size": cfg["intermediate"],
          "num_hidden_layers": cfg["layers"], "num_attention_heads": cfg["heads"],
          "num_key_value_heads": cfg["kv_heads"], "head_dim": cfg["head_dim"], "vocab_size": V,
          "max_position_embeddings": cfg["max_ctx"], "rms_norm_eps": cfg["rms_eps"],
          "rope_theta": cfg["rope_theta"], "bos_token_id": -1, "eos_token_id": -1,
          "tie_word_embeddings": "lm_head" not in model}
    tok = {"model": {"type": "BPE", "vocab": {f"t{i}": i for i in range(V)}, "merges": []},
           "added_tokens": []}
    cj, tj = json.dumps(hf).encode(), json.dumps(tok).encode()
    tensors = [("__qwn.config", DT_BYTES, (len(cj),), cj), ("__qwn.tokenizer", DT_BYTES, (len(tj),), tj),
               ("model.embed_tokens.weight", DT_BF16 if model.get("embed_dtype") == "bf16" else DT_F16, (D, V),
                model["embed"])]
    for l, layer in enumerate(model["layers"]):
        pre = f"model.layers.{l}."
        tensors.append((pre + "input_layernorm.weight", DT_F32, (D,), layer["input_norm"]))
        tensors.append((pre + "post_attention_layernorm.weight", DT_F32, (D,), layer["post_norm"]))
        if "q_norm" in layer:  # Qwen3 per-head q/k norms (c/qwanto_decode.c:975-976)
            tensors.append((pre + "self_attn.q_norm.weight", DT_F32, (cfg["head_dim"],), layer["q_norm"]))
            tensors.append((pre + "self_attn.k_norm.weight", DT_F32, (cfg["head_dim"],), layer["k_norm"]))
        for p, suffix in _PROJ_NAMES.items():
            out, inp = model["shapes"][p]
            tensors.append((pre + suffix, qdt, (inp, out), layer[p]))
        for p in ("q", "k", "v", "o"):  # optional biases (c/qwanto_decode.c:970-973)
            if p + "_bias" in layer:
                tensors.append((pre + f"self_attn.{p}_proj.bias", DT_F32, (model["shapes"][p][0],),
                                layer[p + "_bias"]))
    tensors.append(("model.norm.weight", DT_F32, (D,), model["final_norm"]))
    if "lm_head" in model:
        tensors.append(("lm_head.weight", _HEAD_DT[model["lm_head_dtype"]], (D, V), model["lm_head"]))
    dims = (D, cfg["intermediate"], cfg["heads"], cfg["kv_heads"], cfg["head_dim"], cfg["layers"], V,
            cfg["max_ctx"])
    return write_qwn(path, tensors, arch_dims=dims,
                     qkv_dims=(cfg["heads"] * cfg["head_dim"], cfg["kv_heads"] * cfg["head_dim"],
                               cfg["kv_heads"] * cfg["head_dim"]))


def read_decoder_model(path: str) -> dict:
    """The inverse of write_decoder_model (arrays are views of the mapping)."""
    f = QwnFile(path)
    hf = f.json("__qwn.config")
    cfg = {"hidden": hf["hidden_size"], "intermediate": hf["intermediate_size"],
           "layers": hf["num_hidden_layers"], "heads": hf["num_attention_heads"],
           "kv_heads": hf["num_key_value_heads"], "head_dim": hf["head_dim"], "vocab": hf["vocab_size"],
           "max_ctx": hf["max_position_embeddings"], "rope_theta": hf["rope_theta"],
           "rms_eps": hf["rms_norm_eps"]}
    layers, shapes, dtype = [], {}, None
    for l in range(cfg["layers"]):
        pre = f"model.layers.{l}."
        layer = {"input_norm": f.array(pre + "input_layernorm.weight"),
                 "post_norm": f.array(pre + "post_attention_layernorm.weight")}
        if pre + "self_attn.q_norm.weight" in f.tensors:
            layer["q_norm"] = f.array(pre + "self_attn.q_norm.weight")
            layer["k_norm"] = f.array(pre + "self_attn.k_norm.weight")
        for p in ("q", "k", "v", "o"):
            if pre + f"self_attn.{p}_proj.bias" in f.tensors:
                layer[p + "_bias"] = f.array(pre + f"self_attn.{p}_proj.bias")
        for p, suffix in _PROJ_NAMES.items():
            t = f.tensors[pre + suffix]
            dtype = "q4_0" if t["dtype"] == DT_Q4_0 else "hvsq2"
            shapes[p] = (t["shape"][1], t["shape"][0])
            layer[p] = f.raw(pre + suffix)
        layers.append(layer)
    model = {"cfg": cfg, "dtype": dtype, "shapes": shapes, "layers": layers,
             "embed": f.array("model.embed_tokens.weight"),
             "embed_dtype": "bf16" if f.tensors["model.embed_tokens.weight"]["dtype"] == DT_BF16 else "f16",
             "final_norm": f.array("model.norm.weight"), "file": f}
    if "lm_head.weight" in f.tensors:
        dt = {v: k for k, v in _HEAD_DT.items()}[f.tensors["lm_head.weight"]["dtype"]]
        model["lm_head"] = f.array("lm_head.weight") if dt in ("f16", "bf16") else f.raw("lm_head.weight")
        model["lm_head_dtype"] = dt
    return model
