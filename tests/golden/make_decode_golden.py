"""Golden greedy decodes of the Qwen2-1.5B shaped synthetic Q4_0 model.

Three models, each from the seeded generator (qwanto_amd.synth):
  decode_qwen2_1p5b_q4_0.json         the benchmark draw (block scales and
      the F16 embedding N(0, 0.02), codes uniform over 0..15); its greedy
      output settles on one token, as random models with biased weights do
  decode_qwen2_1p5b_q4_0_varied.json  zero-mean codes (1..15), block scales
      |N(0, 0.01)|, embedding N(0, 0.05): a greedy sequence that keeps
      changing token, but whose logits are small and nearly tied, so
      rounding-sized differences move them far (a loose envelope)
  decode_qwen2_1p5b_q4_0_successor.json  zero-mean codes with block
      scales |N(0, 0.002)|, embedding N(0, 2) and an untied F16 LM head
      whose row perm[t] is embedding row t (perm a seeded permutation of
      the vocabulary): the embedding dominates the residual stream, so the
      greedy id after token t is perm[t] by a wide margin (128 distinct ids,
      every top-two margin above 0.8 of the largest logit) while the 28
      layers still move every logit by 1-2% of the largest (against the same
      model with its projections zeroed), about 40 times the envelope; a
      random model with a tied head either settles on one token (codes
      0..15 give every row a common offset that the residual stream
      amplifies layer after layer) or is chaotic (zero-mean codes at the
      benchmark scale)
For each: the oracle decoder (oracle/qwn_oracle_decoder.c) runs a 32-token
prompt and 128 greedy steps; every step's logits are summarised (the 16
largest with their ids, the largest magnitude, the top-two margin, a
SHA-256 of the whole vector).  The sensitivity envelope: the same run
teacher-forced on those ids with the oracle's calibration perturbation
(rounding-sized moves of half the outputs of every RMSNorm, projection,
attention and SwiGLU, four seeds),
each step's distance from the exact logits measured as the GPU tests
measure theirs (tests/decode_golden.step_error) -- how far rounding-sized
differences travel through 28 layers of this model.  Where the reference decoder is built in
place (oracle/_ref/libqwn_ref_decoder.so, from c/qwanto_decode.c) the same
prompt and ids are replayed through it from a .qwn file, requiring
bit-identical logits at every step.

    python tests/golden/make_decode_golden.py [--steps 128] [--threads 8]
"""
import argparse
import hashlib
import json
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from qwanto_amd import qwn_file, synth  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
VARIANTS = {
    "decode_qwen2_1p5b_q4_0.json": dict(seed=2026, weight_std=0.02, embed_std=0.02, zero_mean=False),
    "decode_qwen2_1p5b_q4_0_varied.json": dict(seed=2028, weight_std=0.01, embed_std=0.05, zero_mean=True),
    "decode_qwen2_1p5b_q4_0_successor.json": dict(seed=2031, weight_std=0.002, embed_std=2.0, zero_mean=True,
                                                  successor_head=True),
}
SPEC_KEYS = ("seed", "weight_std", "embed_std", "zero_mean", "successor_head")
TOP = 16
ENVELOPE_SEEDS = (1, 2, 3, 4)


def build_model(spec: dict):
    """The model and prompt a golden file describes (tests rebuild them from
    the same fields).  successor_head: an untied F16 LM head whose row
    perm[t] is embedding row t (perm drawn after the prompt)."""
    rng = np.random.default_rng(spec["seed"])
    model = synth.decoder_model(rng, synth.QWEN2_1P5B_CONFIG, "q4_0", weight_std=spec["weight_std"],
                                embed_std=spec["embed_std"], zero_mean=spec["zero_mean"])
    prompt = synth.prompt_tokens(rng, synth.QWEN2_1P5B_CONFIG["vocab"], 32)
    if spec.get("successor_head"):
        perm = rng.permutation(synth.QWEN2_1P5B_CONFIG["vocab"])
        head = np.empty_like(model["embed"])
        head[perm] = model["embed"]
        model["lm_head"], model["lm_head_dtype"] = head, "f16"
    return model, prompt


def summarise(logits: np.ndarray) -> dict:
    # 16 largest, ordered by value then index (the first-maximum rule)
    ids = np.lexsort((np.arange(logits.size), -logits.astype(np.float64)))[:TOP]
    srt = np.partition(logits, -2)[-2:]
    return {"ids": [int(i) for i in ids], "logits": [float(logits[i]) for i in ids],
            "max_abs": float(np.max(np.abs(logits))), "margin": float(srt[1] - srt[0]),
            "sha256": hashlib.sha256(logits.tobytes()).hexdigest()}


def envelope(name, model, prompt, tokens, summaries, threads) -> dict:
    """The perturbed oracle's per-step distances from the golden steps."""
    sys.path.insert(0, os.path.dirname(HERE))
    import decode_golden
    o = oracle.load()
    env = []
    for seed in ENVELOPE_SEEDS:
        d = o.decoder(model, threads=threads)
        d.perturb(seed)
        for tok in prompt:
            logits = d.forward(int(tok))
        errs = [decode_golden.step_error(logits, summaries[0])]
        for s in range(len(tokens) - 1):
            errs.append(decode_golden.step_error(d.forward(tokens[s]), summaries[s + 1]))
        d.close()
        env.append(errs)
    env = np.array(env)
    print(f"{name}: envelope median {np.median(env, axis=1).max():.3g}, max {env.max():.3g}", flush=True)
    return {"seeds": list(ENVELOPE_SEEDS), "median": float(np.median(env, axis=1).max()), "max": float(env.max()),
            "per_step": [float(v) for v in env.max(axis=0)]}


def layer_signal(model, prompt, tokens, summaries, threads) -> dict:
    """How far the layers move the logits: the same prompt and ids through
    the model with every projection's block scales zeroed (the layers add
    nothing), each step's distance from the golden step as step_error
    measures it.  A decoder whose layers computed nothing, or computed
    something else, would be off by this much."""
    sys.path.insert(0, os.path.dirname(HERE))
    import decode_golden
    zero = dict(model)
    zero["layers"] = []
    for layer in model["layers"]:
        z = dict(layer)
        for p in synth.PROJECTIONS:
            blocks = layer[p].copy().reshape(-1, synth.Q4_0_BLOCK_BYTES)
            blocks[:, :2] = 0
            z[p] = blocks.reshape(-1)
        zero["layers"].append(z)
    d = oracle.load().decoder(zero, threads=threads)
    for tok in prompt:
        logits = d.forward(int(tok))
    sig = [decode_golden.step_error(logits, summaries[0])]
    for s in range(len(tokens) - 1):
        sig.append(decode_golden.step_error(d.forward(tokens[s]), summaries[s + 1]))
    d.close()
    return {"median": float(np.median(sig)), "min": float(np.min(sig))}


def refresh_envelope(name: str, threads: int):
    """Recompute only the envelope of an existing golden file."""
    path = os.path.join(HERE, name)
    g = json.load(open(path))
    model, prompt = build_model({k: g[k] for k in SPEC_KEYS if k in g})
    g["envelope"] = envelope(name, model, prompt, g["tokens"], g["steps"], threads)
    with open(path, "w") as f:
        json.dump(g, f)


def run(name: str, spec: dict, steps: int, threads: int):
    t0 = time.time()
    model, prompt = build_model(spec)
    o = oracle.load()
    dec = o.decoder(model, threads=threads)
    for tok in prompt:
        logits = dec.forward(int(tok))
    tokens, summaries = [], []
    for _ in range(steps):
        summaries.append(summarise(logits))
        tokens.append(summaries[-1]["ids"][0])
        logits = dec.forward(tokens[-1])
    dec.close()
    print(f"{name}: oracle {steps} steps in {time.time() - t0:.1f}s, {len(set(tokens))} distinct ids", flush=True)
    checked = False
    if os.path.exists(oracle.REF_DECODER_SO):
        with tempfile.TemporaryDirectory() as tmp:
            path = os.path.join(tmp, "m.qwn")
            qwn_file.write_decoder_model(path, model)
            ref = oracle.load_ref_decoder(path, synth.QWEN2_1P5B_CONFIG["max_ctx"], threads)
            V = synth.QWEN2_1P5B_CONFIG["vocab"]
            for tok in prompt:
                rl = ref.forward(int(tok), V)
            for s in range(steps):
                assert hashlib.sha256(rl.tobytes()).hexdigest() == summaries[s]["sha256"], f"step {s}: logits differ"
                rl = ref.forward(tokens[s], V)
            ref.close()
        print(f"{name}: reference decoder agrees bit for bit", flush=True)
        checked = True
    out = {"config": synth.QWEN2_1P5B_CONFIG, "dtype": "q4_0", **spec,
           "prompt": [int(t) for t in prompt], "tokens": tokens,
           "margins": [s["margin"] for s in summaries], "steps": summaries,
           "envelope": envelope(name, model, prompt, tokens, summaries, threads),
           "checked_against_reference_decoder": checked}
    if spec.get("successor_head"):
        out["layer_signal"] = layer_signal(model, prompt, tokens, summaries, threads)
        print(f"{name}: layer signal median {out['layer_signal']['median']:.3g}, "
              f"min {out['layer_signal']['min']:.3g}", flush=True)
    with open(os.path.join(HERE, name), "w") as f:
        json.dump(out, f)
    print(f"wrote {name}; min margin {min(out['margins']):.4g}", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--threads", type=int, default=8)
    ap.add_argument("--only", default=None, help="one output file name")
    ap.add_argument("--envelope-only", action="store_true",
                    help="recompute only the sensitivity envelope of the existing files")
    args = ap.parse_args()
    for name, spec in VARIANTS.items():
        if args.only in (None, name):
            if args.envelope_only:
                refresh_envelope(name, args.threads)
            else:
                run(name, spec, args.steps, args.threads)


if __name__ == "__main__":
    main()
