"""The host decoder (libqwn_host_decoder.so, every projection, the LM head
and the Q8 KV cache through the qwn_cuda ABI on the GPU) against the
oracle decoder, which is bit-identical to the reference decoder (see
test_decoder_oracle.py).

GEMV outputs differ from the CPU's in fp32 rounding only (the integer sums
are exact), so per-step logits agree to ~1e-6 of their scale at most steps;
where an activation sits within that rounding of an int8 boundary its
quantized value moves by one and the step's logits move by up to a few
1e-3 of their scale.  So: every step within 5e-3, the median step within
1e-5, and greedy ids equal unless the best two logits are within the step's
error (reported with that margin)."""
import json
import os

import numpy as np
import pytest

from qwanto_amd import synth
from qwanto_amd.host_decoder import HostDecoder

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "decode_qwen2_1p5b_q4_0.json")
SMALL = dict(hidden=256, intermediate=512, layers=2, heads=4, kv_heads=2, head_dim=64, vocab=1000,
             max_ctx=64, rope_theta=1e6, rms_eps=1e-6)
QWEN2_LIKE = dict(hidden=768, intermediate=1024, layers=3, heads=6, kv_heads=1, head_dim=128, vocab=4096,
                  max_ctx=64, rope_theta=1e6, rms_eps=1e-6)
STEP_RTOL = 5e-3     # any step, of the logit vector's max magnitude
MEDIAN_RTOL = 1e-5   # the median step


@pytest.mark.parametrize("cfg,dtype", [(SMALL, "q4_0"), (SMALL, "hvsq2"), (QWEN2_LIKE, "q4_0")])
def test_host_decoder_matches_oracle(oracle_lib, cfg, dtype):
    rng = np.random.default_rng(21)
    model = synth.decoder_model(rng, cfg, dtype)
    gpu = HostDecoder(model)
    ref = oracle_lib.decoder(model)
    token = 7
    steps = 20
    errs = []
    for step in range(steps):
        a = gpu.forward(token)
        b = ref.forward(token)
        scale = float(np.max(np.abs(b)))
        err = float(np.max(np.abs(a - b))) / scale
        errs.append(err)
        assert err <= STEP_RTOL, f"step {step}: logits differ by {err:.3g} of their scale"
        ta, tb = int(np.argmax(a)), int(np.argmax(b))
        if ta != tb:
            top2 = np.sort(b)[-2:]
            assert top2[1] - top2[0] <= 2 * err * scale, f"step {step}: greedy ids differ with margin " \
                                                         f"{top2[1] - top2[0]:.3g}"
        token = tb
    assert float(np.median(errs)) <= MEDIAN_RTOL, f"median step error {np.median(errs):.3g}"
    m = gpu.metrics()
    assert m.cpu_fallback_count == 0
    assert m.gpu_matmul_count == steps * (7 * cfg["layers"] + 1)
    gpu.close()
    ref.close()


def test_host_decoder_qwen2_1p5b_greedy_128():
    """Config-2 shape: 28 layers of Q4_0, tied F16 LM head (151936 x 1536),
    Q8 KV; 32-token prompt, 128 greedy steps, ids compared with the golden
    ids the oracle and the reference decoder produced."""
    if not os.path.exists(GOLDEN):
        pytest.skip("golden decode fixture absent")
    g = json.load(open(GOLDEN))
    rng = np.random.default_rng(g["seed"])
    model = synth.decoder_model(rng, g["config"], g["dtype"])
    prompt = synth.prompt_tokens(rng, g["config"]["vocab"], len(g["prompt"]))
    assert prompt.tolist() == g["prompt"]
    gpu = HostDecoder(model)
    tokens, margins = gpu.generate(prompt, len(g["tokens"]))
    m = gpu.metrics()
    gpu.close()
    first_diff = next((i for i, (a, b) in enumerate(zip(tokens.tolist(), g["tokens"])) if a != b), None)
    print(f"host decoder: {m.generated_tokens} tokens in {m.decode_wall_ms:.0f} ms "
          f"({m.generated_tokens / (m.decode_wall_ms / 1e3):.1f} tok/s), {m.abi_calls} ABI calls, "
          f"min golden margin {min(g['margins']):.4g}, first divergence {first_diff}")
    if first_diff is not None:
        assert g["margins"][first_diff] < 1e-2, \
            f"greedy ids diverge at step {first_diff} with golden margin {g['margins'][first_diff]:.4g}"
    assert m.cpu_fallback_count == 0 and m.gpu_matmul_count > 0
