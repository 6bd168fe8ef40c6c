"""The oracle decoder (oracle/qwn_oracle_decoder.c) against the reference's
own decoder compiled in place (oracle/_ref/libqwn_ref_decoder.so from
c/qwanto_decode.c and its library sources), and the .qwn container writer
against the reference's reader: the same synthetic model is written as a
.qwn file, opened by qwn_decoder_open_with_config (CPU backend, Q8 KV
cache) and stepped token by token; the logits must be bit-identical."""
import os

import numpy as np
import pytest

import oracle
from qwanto_amd import qwn_file, synth

SMALL = dict(hidden=256, intermediate=512, layers=2, heads=4, kv_heads=2, head_dim=64, vocab=1000,
             max_ctx=64, rope_theta=1e6, rms_eps=1e-6)
# head_dim 128 and GQA 6:1 as the 1.5B shape, fewer/narrower layers
QWEN2_LIKE = dict(hidden=768, intermediate=1024, layers=3, heads=6, kv_heads=1, head_dim=128, vocab=4096,
                  max_ctx=64, rope_theta=1e6, rms_eps=1e-6)


def ref_decoder_or_skip(path, ctx):
    if not os.path.exists(oracle.REF_DECODER_SO):
        pytest.skip("reference decoder build (oracle/_ref) absent")
    return oracle.load_ref_decoder(path, ctx)


@pytest.mark.parametrize("cfg,dtype,steps,qk,bias", [
    (SMALL, "q4_0", 12, False, ""), (SMALL, "hvsq2", 8, False, ""), (QWEN2_LIKE, "q4_0", 10, False, ""),
    (SMALL, "hvsq2", 8, True, ""), (QWEN2_LIKE, "q4_0", 10, True, ""),
    (QWEN2_LIKE, "q4_0", 10, False, "qkv"), (SMALL, "hvsq2", 8, True, "qkvo"), (SMALL, "q4_0", 8, False, "o")])
def test_oracle_decoder_matches_reference_decoder(tmp_path, oracle_lib, cfg, dtype, steps, qk, bias):
    """qk: Qwen3-style per-head q/k RMSNorm weights in the file
    (self_attn.q_norm / k_norm, c/qwanto_decode.c:975-976, 1652-1655).
    bias: the projections carrying self_attn.*_proj.bias (q/k/v as Qwen2,
    c/qwanto_decode.c:1649-1651; o, :1722)."""
    rng = np.random.default_rng(11)
    model = synth.decoder_model(rng, cfg, dtype, qk_norm=qk, biases=bias)
    path = str(tmp_path / "m.qwn")
    qwn_file.write_decoder_model(path, model)
    ref = ref_decoder_or_skip(path, cfg["max_ctx"])
    dec = oracle_lib.decoder(model)
    token = 3
    for step in range(steps):
        a = ref.forward(token, cfg["vocab"])
        b = dec.forward(token)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), \
            f"step {step}: logits differ by up to {np.abs(a - b).max()}"
        token = int(np.argmax(a))
    ref.close()
    dec.close()
    if bias:
        # the biases matter: the same model without them gives other logits
        plain = {**model, "layers": [{k: v for k, v in layer.items() if not k.endswith("_bias")}
                                     for layer in model["layers"]]}
        d2, d3 = oracle_lib.decoder(plain), oracle_lib.decoder(model)
        assert not np.array_equal(d2.forward(3), d3.forward(3))
        d2.close()
        d3.close()


@pytest.mark.parametrize("embed,head,cfg_name,dtype", [
    ("bf16", None, "SMALL", "q4_0"), ("f16", "f16", "SMALL", "hvsq2"), ("f16", "bf16", "SMALL", "q4_0"),
    ("bf16", "q4_0", "SMALL", "q4_0"), ("f16", "hvsq2", "SMALL", "hvsq2"), ("bf16", "bf16", "QWEN2_LIKE", "q4_0"),
    ("f16", "q4_0", "QWEN2_LIKE", "q4_0")])
def test_untied_head_and_bf16_embedding_match_reference(tmp_path, oracle_lib, embed, head, cfg_name, dtype):
    """A BF16 embedding (c/qwanto_decode.c:561; qwn_row_f32,
    c/qwanto_kernels.c:1508-1527) and an untied lm_head.weight in each dtype
    the LM head matmul takes (c/qwanto_decode.c:1074-1076, 2007; F16/BF16 rows
    and the Q4_0 / HyperVSQ-2 quantized matmuls): the oracle's logits are the
    reference decoder's bit for bit, and the head is really used (the same
    model with the head dropped, i.e. tied, gives other logits)."""
    cfg = {"SMALL": SMALL, "QWEN2_LIKE": QWEN2_LIKE}[cfg_name]
    rng = np.random.default_rng(21)
    model = synth.decoder_model(rng, cfg, dtype, embed_dtype=embed, lm_head=head)
    path = str(tmp_path / "m.qwn")
    qwn_file.write_decoder_model(path, model)
    back = qwn_file.read_decoder_model(path)
    assert back["embed_dtype"] == embed and back.get("lm_head_dtype") == head
    assert np.array_equal(np.asarray(back["embed"]).view(np.uint16), model["embed"].view(np.uint16))
    if head is not None:
        assert np.array_equal(np.asarray(back["lm_head"]).view(np.uint8).ravel(), model["lm_head"].view(np.uint8).ravel())
    back["file"].close()
    ref = ref_decoder_or_skip(path, cfg["max_ctx"])
    dec = oracle_lib.decoder(model)
    token = 5
    for step in range(6):
        a = ref.forward(token, cfg["vocab"])
        b = dec.forward(token)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), \
            f"step {step}: logits differ by up to {np.abs(a - b).max()}"
        token = int(np.argmax(a))
    ref.close()
    dec.close()
    if head is not None:
        tied = {k: v for k, v in model.items() if k not in ("lm_head", "lm_head_dtype")}
        d1, d2 = oracle_lib.decoder(tied), oracle_lib.decoder(model)
        assert not np.array_equal(d1.forward(5), d2.forward(5))
        d1.close()
        d2.close()


def test_qwn_roundtrip_biases(tmp_path):
    rng = np.random.default_rng(4)
    model = synth.decoder_model(rng, SMALL, "q4_0", biases="qkvo")
    path = str(tmp_path / "b.qwn")
    qwn_file.write_decoder_model(path, model)
    back = qwn_file.read_decoder_model(path)
    for l in range(SMALL["layers"]):
        for p in "qkvo":
            assert np.array_equal(back["layers"][l][p + "_bias"], model["layers"][l][p + "_bias"])
    back["file"].close()


def test_qwn_roundtrip(tmp_path):
    rng = np.random.default_rng(2)
    model = synth.decoder_model(rng, SMALL, "hvsq2")
    path = str(tmp_path / "m.qwn")
    size = qwn_file.write_decoder_model(path, model)
    assert os.path.getsize(path) == size
    back = qwn_file.read_decoder_model(path)
    assert back["cfg"] == {k: SMALL[k] for k in back["cfg"]}
    assert back["dtype"] == "hvsq2" and back["shapes"] == model["shapes"]
    for l in range(SMALL["layers"]):
        for p in synth.PROJECTIONS:
            assert np.array_equal(back["layers"][l][p], model["layers"][l][p])
    assert np.array_equal(back["embed"], model["embed"])
    f = back["file"]
    # 2 + 2 norms*layers + 7*layers + embed + final norm descriptors; 29 inline, rest in the tail
    assert len(f.tensors) == 2 + 9 * SMALL["layers"] + 2
    assert all(t["offset"] % 4096 == 0 and t["size"] % 64 == 0 for t in f.tensors.values())
    f.close()


def test_fnv1a64_known_values():
    # FNV-1a 64 test vectors (offset basis for "", published values for "a", "foobar")
    assert qwn_file.fnv1a64("") == 0xCBF29CE484222325
    assert qwn_file.fnv1a64("a") == 0xAF63DC4C8601EC8C
    assert qwn_file.fnv1a64("foobar") == 0x85944171F73967E8


def test_rmsnorm_closed_form(oracle_lib):
    rng = np.random.default_rng(3)
    x = rng.standard_normal(1536).astype(np.float32) * 3
    w = rng.uniform(0.5, 1.5, 1536).astype(np.float32)
    got = oracle_lib.rmsnorm(x, w, 1e-6)
    ref = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * w
    assert np.allclose(got, ref, rtol=3e-7, atol=0)
    # constant input: x * 1/sqrt(x^2 + eps)
    c = np.full(16, 2.0, dtype=np.float32)
    assert np.allclose(oracle_lib.rmsnorm(c, np.ones(16, np.float32), 0.0), 1.0, rtol=0, atol=1e-7)


def test_rope_table_closed_form(oracle_lib):
    c, s = oracle_lib.rope_table(64, 64, 1e6)
    # angle = (float)pos * powf(theta, -2i/dim), both steps in fp32
    pos = np.arange(64, dtype=np.float32)[:, None]
    freq = np.power(np.float32(1e6), (-2.0 * np.arange(64) / 128.0).astype(np.float32))
    ang = (pos * freq).astype(np.float64)
    assert np.allclose(c, np.cos(ang), atol=2e-6) and np.allclose(s, np.sin(ang), atol=2e-6)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)


def test_greedy_is_first_maximum(oracle_lib):
    import ctypes
    logits = np.array([0.5, 2.0, -1.0, 2.0, 1.0], dtype=np.float32)
    assert oracle_lib.lib.qo_argmax(logits.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), 5) == 1
