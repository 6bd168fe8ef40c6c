"""The host decoder (libqwn_host_decoder.so, every projection, the LM head
and the Q8 KV cache through the qwn_cuda ABI on the GPU) against the
oracle decoder, which is bit-identical to the reference decoder (see
test_decoder_oracle.py).

GEMV outputs differ from the CPU's in fp32 rounding only (the integer sums
are exact); where an activation sits within that rounding of an int8
boundary its quantized value moves by one and the difference travels
through the later layers.  Logits are held to the oracle's own sensitivity
to such differences on the same model and tokens (parity.within_envelope),
and greedy ids must agree unless the best two logits are within the step's
error."""
import numpy as np
import pytest

import decode_golden
from parity import oracle_envelope, step_errors, within_envelope
from qwanto_amd import synth
from qwanto_amd.host_decoder import HostDecoder

pytestmark = pytest.mark.gpu

SMALL = dict(hidden=256, intermediate=512, layers=2, heads=4, kv_heads=2, head_dim=64, vocab=1000,
             max_ctx=64, rope_theta=1e6, rms_eps=1e-6)
QWEN2_LIKE = dict(hidden=768, intermediate=1024, layers=3, heads=6, kv_heads=1, head_dim=128, vocab=4096,
                  max_ctx=64, rope_theta=1e6, rms_eps=1e-6)


def run_against_oracle(oracle_lib, model, steps=20, token=7):
    """`steps` host-decoder steps fed the oracle's greedy ids; returns the
    metrics after the run."""
    gpu = HostDecoder(model)
    ref = oracle_lib.decoder(model)
    inputs, gpu_steps, ref_steps = [], [], []
    try:
        for step in range(steps):
            a = gpu.forward(token)
            b = ref.forward(token)
            inputs.append(token)
            gpu_steps.append(a)
            ref_steps.append(b)
            ta, tb = int(np.argmax(a)), int(np.argmax(b))
            if ta != tb:
                err = step_errors([a], [b])[0]
                top2 = np.sort(b)[-2:]
                assert top2[1] - top2[0] <= 2 * err * np.max(np.abs(b)), \
                    f"step {step}: greedy ids differ with margin {top2[1] - top2[0]:.3g}"
            token = tb
        m = gpu.metrics()
    finally:
        gpu.close()
        ref.close()
    ok, msg = within_envelope(step_errors(gpu_steps, ref_steps),
                              oracle_envelope(oracle_lib, model, inputs, ref_steps))
    assert ok, msg
    return m


@pytest.mark.parametrize("cfg,dtype", [(SMALL, "q4_0"), (SMALL, "hvsq2"), (QWEN2_LIKE, "q4_0")])
def test_host_decoder_matches_oracle(oracle_lib, cfg, dtype):
    rng = np.random.default_rng(21)
    model = synth.decoder_model(rng, cfg, dtype)
    m = run_against_oracle(oracle_lib, model)
    assert m.cpu_fallback_count == 0
    assert m.gpu_matmul_count == 20 * (7 * cfg["layers"] + 1)


@pytest.mark.parametrize("cfg,dtype,qk,bias", [(SMALL, "q4_0", True, "qkv"), (QWEN2_LIKE, "hvsq2", False, "qkvo"),
                                               (SMALL, "hvsq2", True, ""), (QWEN2_LIKE, "q4_0", False, "qkv")])
def test_host_decoder_norms_and_biases(oracle_lib, cfg, dtype, qk, bias):
    """Per-head q/k RMSNorm (c/qwanto_decode.c:654-684, 1652-1655) and
    q/k/v/o biases (:926-929, 1649-1651, 1722) in the host decoder."""
    rng = np.random.default_rng(41)
    model = synth.decoder_model(rng, cfg, dtype, qk_norm=qk, biases=bias)
    run_against_oracle(oracle_lib, model, steps=16, token=5)


@pytest.mark.parametrize("cfg,dtype,embed,head", [(SMALL, "q4_0", "bf16", None), (SMALL, "hvsq2", "f16", "bf16"),
                                                  (QWEN2_LIKE, "q4_0", "bf16", "q4_0"),
                                                  (SMALL, "hvsq2", "f16", "hvsq2"), (QWEN2_LIKE, "q4_0", "f16", "f16")])
def test_host_decoder_untied_head_and_bf16_embedding(oracle_lib, cfg, dtype, embed, head):
    """A BF16 embedding (c/qwanto_decode.c:561) and an untied lm_head.weight in
    each dtype (:1074-1076, 2007) through the ABI: the BF16 GEMV with fp32
    input, or the head's activation quantized on the host as every
    projection's."""
    rng = np.random.default_rng(43)
    model = synth.decoder_model(rng, cfg, dtype, embed_dtype=embed, lm_head=head)
    m = run_against_oracle(oracle_lib, model, steps=12, token=9)
    assert m.cpu_fallback_count == 0 and m.gpu_matmul_count == 12 * (7 * cfg["layers"] + 1)


@pytest.mark.parametrize("name", decode_golden.NAMES)
def test_host_decoder_qwen2_1p5b_golden(name):
    """Config-2 shape through the ABI as qwnrun drives it (one synchronous
    call per projection and KV operation): the prompt, then the 128 golden
    ids teacher-forced, every step's logits against the golden step within
    the golden's envelope; then a free-running greedy generation against the
    golden ids (decode_golden.check_greedy_ids: every id on the successor
    golden)."""
    loaded = decode_golden.load(name)
    if loaded is None:
        pytest.skip("golden decode fixture absent")
    g, model, prompt = loaded
    gpu = HostDecoder(model)
    try:
        for t in prompt:
            a = gpu.forward(int(t))
        errs = [decode_golden.step_error(a, g["steps"][0])]
        for s, tok in enumerate(g["tokens"][:-1]):
            errs.append(decode_golden.step_error(gpu.forward(tok), g["steps"][s + 1]))
    finally:
        gpu.close()
    ok, msg = within_envelope(errs, g["envelope"])
    gpu = HostDecoder(model)
    tokens, _ = gpu.generate(prompt, len(g["tokens"]))
    m = gpu.metrics()
    gpu.close()
    print(f"host decoder {name}: {m.generated_tokens / (m.decode_wall_ms / 1e3):.1f} tok/s, {m.abi_calls} ABI calls, "
          f"{msg}")
    assert ok, msg
    print(decode_golden.check_greedy_ids(name, g, tokens.tolist(), errs))
    assert m.cpu_fallback_count == 0 and m.gpu_matmul_count > 0
    assert m.backend_reason.decode() == "versioned_abi_1_loaded_device_0"
