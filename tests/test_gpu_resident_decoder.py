"""The resident decoder (include/qwn_hip_decoder.h: the whole step on the
device, one HIP graph per token) against the oracle decoder, which is
bit-identical to the reference decoder (test_decoder_oracle.py), and
against the golden greedy decodes of the Qwen2-1.5B-shaped Q4_0 model.

On the device the RMSNorm sums, the SwiGLU exp and the GEMV combination run
in another fp32 order than the CPU's.  Where an activation lands within that
rounding of an int8 boundary its quantized value moves by one; the
difference travels through the later layers and stays in the KV cache.
The logits are therefore held to the oracle's own sensitivity to
rounding-sized differences, measured on the same model and tokens
(parity.oracle_envelope / parity.within_envelope): the GPU's median and
worst step within ENV_K times the perturbed oracle's.  The caches written
by a prefill block and by token-by-token steps are compared entry by
entry: the first layer's may differ only by one int8 step where such a
flip happened.
"""
import numpy as np
import pytest

import decode_golden
from parity import ENV_K, oracle_envelope, step_errors, within_envelope
from qwanto_amd import abi, synth

pytestmark = pytest.mark.gpu

SMALL = dict(hidden=256, intermediate=512, layers=2, heads=4, kv_heads=2, head_dim=64, vocab=1000,
             max_ctx=64, rope_theta=1e6, rms_eps=1e-6)
QWEN2_LIKE = dict(hidden=768, intermediate=1024, layers=3, heads=6, kv_heads=1, head_dim=128, vocab=4096,
                  max_ctx=80, rope_theta=1e6, rms_eps=1e-6)
# a context of more than one split: RoPE/append kernel + MFMA split attention
LONG_CTX = dict(SMALL, max_ctx=1500)
# contexts of one split past the first 256-token chunk(s) of the fused
# decode attention (head_dim 64, 128 and 256)
MID_CTX = dict(SMALL, max_ctx=640)
MID_QWEN2 = dict(hidden=768, intermediate=1024, layers=3, heads=6, kv_heads=1, head_dim=128, vocab=4096,
                 max_ctx=640, rope_theta=1e6, rms_eps=1e-6)
MID_HD256 = dict(SMALL, heads=2, kv_heads=1, head_dim=256, max_ctx=640)
# a hidden size whose block GEMMs split K over waves (HyperVSQ-2 and Q4_0
# gate/up pairs with two or more K-split waves per job)
WIDE = dict(QWEN2_LIKE, hidden=1536, intermediate=2048, layers=2)


def with_norms(rng, model):
    """Non-trivial norm weights (the synthetic models default to ones)."""
    D = model["cfg"]["hidden"]
    for layer in model["layers"]:
        layer["input_norm"] = (1.0 + 0.2 * rng.standard_normal(D)).astype(np.float32)
        layer["post_norm"] = (1.0 + 0.2 * rng.standard_normal(D)).astype(np.float32)
    model["final_norm"] = (1.0 + 0.2 * rng.standard_normal(D)).astype(np.float32)
    return model


@pytest.mark.parametrize("cfg,dtype,qk,bias", [(SMALL, "q4_0", False, ""), (SMALL, "hvsq2", False, ""),
                                               (QWEN2_LIKE, "q4_0", False, ""), (QWEN2_LIKE, "hvsq2", False, ""),
                                               (LONG_CTX, "q4_0", False, ""), (SMALL, "hvsq2", True, ""),
                                               (QWEN2_LIKE, "q4_0", True, ""), (LONG_CTX, "hvsq2", True, ""),
                                               (QWEN2_LIKE, "q4_0", False, "qkv"), (SMALL, "hvsq2", False, "qkvo"),
                                               (LONG_CTX, "q4_0", False, "qkvo")])
def test_resident_decoder_matches_oracle(gpu_ctx, oracle_lib, cfg, dtype, qk, bias):
    """24 steps, each fed the oracle's greedy token.  qk: Qwen3-style
    per-head q/k RMSNorm before RoPE (in the fused decode attention kernel,
    and for LONG_CTX in the RoPE/append kernel).  bias: q/k/v(/o) projection
    biases, added in the GEMV epilogues (c/qwanto_decode.c:1649-1651, 1722)."""
    rng = np.random.default_rng(31)
    model = with_norms(rng, synth.decoder_model(rng, cfg, dtype, qk_norm=qk, biases=bias))
    dec = abi.ResidentDecoder(gpu_ctx, model)
    ref = oracle_lib.decoder(model)
    try:
        token, inputs, gpu_steps, ref_steps = 11, [], [], []
        for step in range(24):
            a, greedy = dec.forward(token)
            b = ref.forward(token)
            assert greedy == int(np.argmax(a)), "device argmax is not the first maximum of its logits"
            inputs.append(token)
            gpu_steps.append(a)
            ref_steps.append(b)
            err = step_errors([a], [b])[0]
            tb = int(np.argmax(b))
            if greedy != tb:
                top2 = np.sort(b)[-2:]
                assert top2[1] - top2[0] <= 2 * err * np.max(np.abs(b)), \
                    f"step {step}: greedy ids differ with margin {top2[1] - top2[0]:.3g}"
            token = tb
    finally:
        dec.close()
        ref.close()
    errs = step_errors(gpu_steps, ref_steps)
    ok, msg = within_envelope(errs, oracle_envelope(oracle_lib, model, inputs, ref_steps))
    assert ok, msg


@pytest.mark.parametrize("cfg,dtype,embed,head", [
    (SMALL, "q4_0", "bf16", None), (SMALL, "hvsq2", "f16", "f16"), (QWEN2_LIKE, "q4_0", "bf16", "bf16"),
    (QWEN2_LIKE, "q4_0", "f16", "q4_0"), (SMALL, "hvsq2", "bf16", "hvsq2"), (LONG_CTX, "q4_0", "f16", "hvsq2")])
def test_untied_head_and_bf16_embedding(gpu_ctx, oracle_lib, cfg, dtype, embed, head):
    """A BF16 embedding (c/qwanto_decode.c:561) and an untied lm_head.weight
    (c/qwanto_decode.c:1074-1076, 2007) in each dtype, one token's head
    normalizing x in its own GEMV prologue (F16/BF16 rows on fp32 values,
    Q4_0/HyperVSQ-2 on the quantized image).  Stepping (the device argmax
    epilogue on the head), a prefill block and a verify block (the batched
    head on every token) against the oracle, which is bit-identical to the
    reference decoder on the same model (test_decoder_oracle.py)."""
    rng = np.random.default_rng(47)
    model = with_norms(rng, synth.decoder_model(rng, cfg, dtype, embed_dtype=embed, lm_head=head))
    prompt = synth.prompt_tokens(rng, cfg["vocab"], 6)
    draft = synth.prompt_tokens(rng, cfg["vocab"], 5)
    dec = abi.ResidentDecoder(gpu_ctx, model)
    ref = oracle_lib.decoder(model)
    try:
        token, inputs, gpu_steps, ref_steps = 11, [], [], []
        for step in range(12):
            a, greedy = dec.forward(token)
            b = ref.forward(token)
            assert greedy == int(np.argmax(a)), "device argmax is not the first maximum of its logits"
            inputs.append(token)
            gpu_steps.append(a)
            ref_steps.append(b)
            token = int(np.argmax(b))
        # a prefill block, then a verify block, continuing the same context
        a, greedy = dec.prefill(prompt)
        assert greedy == int(np.argmax(a))
        inputs += [int(t) for t in prompt]
        ref_prompt = [ref.forward(int(t)) for t in prompt]
        gpu_steps.append(a)
        ref_steps += ref_prompt
        vl, ids = dec.verify(draft)
        assert ids.tolist() == [int(np.argmax(r)) for r in vl]
        inputs += [int(t) for t in draft]
        ref_steps += [ref.forward(int(t)) for t in draft]
        gpu_steps += list(vl)
    finally:
        dec.close()
        ref.close()
    env = oracle_envelope(oracle_lib, model, inputs, ref_steps)
    # the compared steps: the 12 forwards, the prefill's last token, the 5 verify rows
    keep = list(range(12)) + [12 + len(prompt) - 1] + list(range(12 + len(prompt), len(inputs)))
    ref_kept = [ref_steps[i] for i in keep]
    ok, msg = within_envelope(step_errors(gpu_steps, ref_kept), env[:, keep])
    assert ok, msg


def read_caches(dec, layers, count):
    return [dec.kv_read(l, 0, count) for l in range(layers)]


@pytest.mark.parametrize("cfg,dtype,P,qk,bias", [
    (SMALL, "q4_0", 21, False, ""), (SMALL, "hvsq2", 16, False, ""), (QWEN2_LIKE, "q4_0", 37, False, ""),
    (QWEN2_LIKE, "hvsq2", 37, False, ""), (QWEN2_LIKE, "hvsq2", 5, False, ""), (LONG_CTX, "q4_0", 18, False, ""),
    (SMALL, "q4_0", 1, False, ""), (QWEN2_LIKE, "hvsq2", 20, True, ""), (LONG_CTX, "q4_0", 18, True, ""),
    (LONG_CTX, "q4_0", 24, True, ""),
    # biases through the MFMA GEMM epilogue (6+-token Q4_0 and 3+-token HyperVSQ-2 blocks) and the dot8 GEMV
    (QWEN2_LIKE, "q4_0", 37, False, "qkv"), (QWEN2_LIKE, "hvsq2", 20, False, "qkvo"),
    (SMALL, "q4_0", 5, False, "qkvo"),
    # prompts past the fused decode attention's 256-token chunks: the block
    # prefill and the token-by-token steps both cross chunk boundaries
    (MID_CTX, "q4_0", 270, False, ""), (MID_CTX, "hvsq2", 520, True, ""), (MID_QWEN2, "q4_0", 300, False, ""),
    (MID_HD256, "q4_0", 270, True, ""),
    (WIDE, "hvsq2", 40, False, ""), (WIDE, "q4_0", 40, False, "")])
def test_prefill_matches_stepwise_and_oracle(gpu_ctx, oracle_lib, cfg, dtype, P, qk, bias):
    check_prefill(gpu_ctx, oracle_lib, cfg, dtype, P, qk, bias)


@pytest.mark.parametrize("cfg,dtype,P", [(QWEN2_LIKE, "q4_0", 70), (QWEN2_LIKE, "hvsq2", 70), (SMALL, "q4_0", 37)])
def test_prefill_without_mfma_copy(gpu_ctx, oracle_lib, monkeypatch, cfg, dtype, P):
    """The same checks with the weights uploaded without the MFMA-order copy
    (QWN_HIP_MFMA_COPY=0): a block's GEMMs take the staged MFMA kernels
    (weights read from the wave tiles), over 16-token groups in one launch
    (a 64-token block and a 6-token one; a 37-token block)."""
    monkeypatch.setenv("QWN_HIP_MFMA_COPY", "0")
    check_prefill(gpu_ctx, oracle_lib, cfg, dtype, P, False, "")


def check_prefill(gpu_ctx, oracle_lib, cfg, dtype, P, qk, bias):
    """qwn_hip_decoder_prefill (prompt blocks of up to 64 tokens: the int8
    MFMA GEMM over 16-token groups from 3 (Q4_0) / 2 (HyperVSQ-2) tokens,
    the batched GEMV below; block RoPE/append, causal attention per token;
    the split-attention path for LONG_CTX): the last prompt token's
    logits and eight forward() steps that read the cache the prefill wrote.

    Against the oracle (prompt and the oracle's greedy ids): within the
    oracle's envelope.  Against the same decoder stepping the prompt token
    by token: the two differ in the fp32 order of the RMSNorm sums and, for
    blocks on the MFMA GEMM, of the GEMM sums, so within twice the envelope.
    Their Q8 caches: layer 0, whose input is the embedding itself, holds the
    same int8 values except where a value sits at a rounding boundary (one
    int8 step, at most 2% of the entries); deeper layers carry those flips'
    effects forward, so at most 5% of their entries may differ -- 8% past
    128 prompt tokens, where each position's attention mixes more flipped
    entries (3 layers at head_dim 128 and 300 tokens: 5.3-5.6% in layer 2,
    with this decode attention and with the one before it)."""
    rng = np.random.default_rng(77 + P)
    model = with_norms(rng, synth.decoder_model(rng, cfg, dtype, qk_norm=qk, biases=bias))
    prompt = synth.prompt_tokens(rng, cfg["vocab"], P)
    dec = abi.ResidentDecoder(gpu_ctx, model)
    ref = oracle_lib.decoder(model)
    try:
        ref_all = [ref.forward(int(t)) for t in prompt]
        oracle_steps, tokens = [ref_all[-1]], []
        for _ in range(8):
            tokens.append(int(np.argmax(oracle_steps[-1])))
            oracle_steps.append(ref.forward(tokens[-1]))
        ref_all += oracle_steps[1:]
        a, greedy = dec.prefill(prompt)
        assert greedy == int(np.argmax(a)), "device argmax is not the first maximum of its logits"
        prefill_caches = read_caches(dec, cfg["layers"], P)
        prefill_steps = [a] + [dec.forward(t)[0] for t in tokens]
        dec.reset()
        for t in prompt:
            a, _ = dec.forward(int(t))
        step_caches = read_caches(dec, cfg["layers"], P)
        step_steps = [a] + [dec.forward(t)[0] for t in tokens]
    finally:
        dec.close()
        ref.close()
    env_all = oracle_envelope(oracle_lib, model, list(prompt) + tokens, ref_all)
    env = env_all[:, P - 1:]   # the steps compared: the last prompt token and the eight after it
    ok, msg = within_envelope(step_errors(prefill_steps, oracle_steps), env)
    assert ok, "prefill vs oracle: " + msg
    ok, msg = within_envelope(step_errors(prefill_steps, step_steps), env, k=2 * ENV_K)
    assert ok, "prefill vs token-by-token: " + msg
    for l, (pc, sc) in enumerate(zip(prefill_caches, step_caches)):
        for name, x, y in (("keys", pc[0], sc[0]), ("values", pc[1], sc[1])):
            d = np.abs(x.astype(np.int32) - y.astype(np.int32))
            frac = float(np.mean(d > 0))
            print(f"layer {l} {name}: {frac:.3%} of entries differ, by at most {d.max()}")
            if l == 0:
                assert d.max() <= 1 and frac <= 0.02, f"layer 0 {name}: {frac:.3%} differ, by up to {d.max()}"
            else:
                deep = 0.05 if P < 128 else 0.08
                assert frac <= deep, f"layer {l} {name}: {frac:.3%} of entries differ (by up to {d.max()})"
        for name, x, y in (("key scales", pc[2], sc[2]), ("value scales", pc[3], sc[3])):
            rel = np.abs(x.astype(np.float64) - y) / np.abs(y)
            bound = 1.0 / 127 if l == 0 else 0.1
            assert rel.max() <= bound, f"layer {l} {name}: relative difference {rel.max():.3g}"


def test_decoder_cache_matches_oracle_quantization(gpu_ctx, oracle_lib):
    """The resident decoder's layer-0 cache after its first token: the Q8
    quantization (c/qwanto_turboquant.c:555-600) of the k and v projections
    of the normalized embedding row (RoPE is the identity at position 0),
    recomputed with the oracle: int8 entries equal except where the GEMV's
    fp32 combination moved a value across a rounding boundary (one step, a
    handful of entries), scales within an ulp or so."""
    rng = np.random.default_rng(12)
    cfg = SMALL
    model = with_norms(rng, synth.decoder_model(rng, cfg, "q4_0"))
    dec = abi.ResidentDecoder(gpu_ctx, model)
    try:
        dec.forward(7)
        k, v, ks, vs = dec.kv_read(0, 0, 1)
    finally:
        dec.close()
    KV = cfg["kv_heads"] * cfg["head_dim"]
    x = model["embed"][7].astype(np.float32)
    xn = oracle_lib.rmsnorm(x, model["layers"][0]["input_norm"], cfg["rms_eps"])
    kf = oracle_lib.matmul_q4_0(model["layers"][0]["k"], xn[None, :], KV)[0]
    vf = oracle_lib.matmul_q4_0(model["layers"][0]["v"], xn[None, :], KV)[0]
    kq, kss = oracle_lib.q8_quantize(kf)
    vq, vss = oracle_lib.q8_quantize(vf)
    assert np.abs(k[0].astype(int) - kq).max() <= 1 and np.mean(k[0] != kq) <= 0.02
    assert np.abs(v[0].astype(int) - vq).max() <= 1 and np.mean(v[0] != vq) <= 0.02
    assert np.allclose(ks[0], kss, rtol=1e-6, atol=0) and np.allclose(vs[0], vss, rtol=1e-6, atol=0)


def test_generate_equals_stepwise(gpu_ctx):
    """generate() (prefill blocks, then graph replays with no host sync
    between tokens, the device's own argmax fed back) gives the ids of
    prefill() followed by step-by-step forward() calls."""
    rng = np.random.default_rng(5)
    model = with_norms(rng, synth.decoder_model(rng, SMALL, "q4_0"))
    dec = abi.ResidentDecoder(gpu_ctx, model)
    try:
        prompt = synth.prompt_tokens(rng, SMALL["vocab"], 19)
        toks, st = dec.generate(prompt, 20)
        assert st.generated_tokens == 20 and st.position == 39 and st.graph == 1
        assert st.prefill_block_tokens == 64   # int8 MFMA GEMMs over 16-token groups
        dec.reset()
        _, nxt = dec.prefill(prompt, logits=False)
        step = []
        for _ in range(20):
            step.append(nxt)
            _, nxt = dec.forward(nxt, logits=False)
        assert toks.tolist() == step
        with pytest.raises(abi.AbiError):           # context full
            dec.generate(prompt, SMALL["max_ctx"])
    finally:
        dec.close()


@pytest.mark.parametrize("name", decode_golden.NAMES)
def test_resident_decoder_qwen2_1p5b_golden(gpu_ctx, name):
    """Config-2 shape: 28 Q4_0 layers, F16 LM head (151936 x 1536; tied, or
    the successor golden's untied head), Q8 KV; 32-token prompt, 128 greedy steps of the golden decode (the oracle's,
    bit-identical to the reference decoder's).

    Teacher-forced: the prompt as one 32-token prefill block, then the
    golden ids one forward() at a time; every step's logits against the
    golden step (decode_golden.step_error: the top-16 logits, nothing else
    above them), within the golden's stored envelope.  Free-running:
    generate() gives the golden ids (decode_golden.check_greedy_ids): all
    128 on the successor golden (128 distinct ids, every margin far above
    the error); on the others none may differ before a step whose golden
    top-two margin is within twice that step's measured error."""
    loaded = decode_golden.load(name)
    if loaded is None:
        pytest.skip("golden decode fixture absent")
    g, model, prompt = loaded
    dec = abi.ResidentDecoder(gpu_ctx, model)
    try:
        a, greedy = dec.prefill(prompt)
        errs = [decode_golden.step_error(a, g["steps"][0])]
        for s, tok in enumerate(g["tokens"][:-1]):
            a, greedy = dec.forward(tok)
            errs.append(decode_golden.step_error(a, g["steps"][s + 1]))
        dec.reset()
        toks, st = dec.generate(prompt, len(g["tokens"]))
    finally:
        dec.close()
    ok, msg = within_envelope(errs, g["envelope"])
    print(f"{name}: {msg}, {st.generated_tokens / (st.decode_ms / 1e3):.1f} tok/s")
    assert ok, msg
    print(decode_golden.check_greedy_ids(name, g, toks.tolist(), errs))
    assert st.graph == 1


@pytest.mark.parametrize("cfg,dtype,P,M,embed,head", [
    (QWEN2_LIKE, "q4_0", 20, 16, "f16", None), (SMALL, "hvsq2", 5, 8, "f16", None),
    (SMALL, "q4_0", 3, 4, "f16", None), (QWEN2_LIKE, "hvsq2", 1, 1, "f16", None),
    (LONG_CTX, "q4_0", 30, 16, "f16", None),
    # untied heads: BF16 and F16 rows on the matrix cores, a Q4_0 head on the batched GEMV
    (QWEN2_LIKE, "q4_0", 20, 16, "bf16", "bf16"), (SMALL, "hvsq2", 5, 11, "f16", "f16"),
    (QWEN2_LIKE, "hvsq2", 3, 16, "bf16", "q4_0")])
def test_verify_block_matches_oracle_steps(gpu_ctx, oracle_lib, cfg, dtype, P, M, embed, head):
    """qwn_hip_decoder_verify: M draft tokens after a P-token prompt as one
    block, logits for every token (the [nodes x vocab] a draft verifier
    scores, c/qwanto_jetspec.c:160-205), against the oracle stepping the
    same tokens one at a time; each token's greedy id is the first maximum
    of its logits.  Then truncate() to keep two of the drafts and step the
    third token again: its logits agree with the verify block's.  F16/BF16
    heads (tied or untied) run as matrix-core products of the head with the
    tokens' narrow activation pieces (qwn_head.hip)."""
    rng = np.random.default_rng(900 + P + M)
    model = with_norms(rng, synth.decoder_model(rng, cfg, dtype, embed_dtype=embed, lm_head=head))
    prompt = synth.prompt_tokens(rng, cfg["vocab"], P)
    draft = synth.prompt_tokens(rng, cfg["vocab"], M)
    dec = abi.ResidentDecoder(gpu_ctx, model)
    ref = oracle_lib.decoder(model)
    try:
        ref_all = [ref.forward(int(t)) for t in list(prompt) + list(draft)]
        dec.prefill(prompt, logits=False)
        logits, ids = dec.verify(draft)
        assert ids.tolist() == [int(np.argmax(row)) for row in logits]
        again = None
        if M >= 3:
            dec.truncate(P + 2)
            again, _ = dec.forward(int(draft[2]))
    finally:
        dec.close()
        ref.close()
    env = oracle_envelope(oracle_lib, model, list(prompt) + list(draft), ref_all)[:, P:]
    ok, msg = within_envelope(step_errors(list(logits), ref_all[P:]), env)
    assert ok, "verify vs oracle: " + msg
    if again is not None:
        ok, msg = within_envelope(step_errors([again], [logits[2]]), env[:, 2:3], k=2 * ENV_K)
        assert ok, "step after truncate vs verify: " + msg
