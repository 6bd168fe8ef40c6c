"""Golden greedy decode of the Qwen2-1.5B shaped synthetic Q4_0 model.

Builds the model from the seeded generator (qwanto_amd.synth), runs the
oracle decoder (oracle/qwn_oracle_decoder.c) over a 32-token prompt and 128
greedy steps, and -- where the reference decoder is built in place
(oracle/_ref/libqwn_ref_decoder.so, from c/qwanto_decode.c) -- replays the
same prompt and generated ids through it from a .qwn file and requires the
same ids and bit-identical logits.  Writes decode_qwen2_1p5b_q4_0.json:
seed, prompt, generated ids, logit margins, and the logit vector of the
first generated step (as a checksum source).

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

SEED = 2026
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "decode_qwen2_1p5b_q4_0.json")


def build_model():
    rng = np.random.default_rng(SEED)
    model = synth.decoder_model(rng, synth.QWEN2_1P5B_CONFIG, "q4_0")
    prompt = synth.prompt_tokens(rng, synth.QWEN2_1P5B_CONFIG["vocab"], 32)
    return model, prompt


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--threads", type=int, default=8)
    args = ap.parse_args()
    t0 = time.time()
    model, prompt = build_model()
    print(f"model built in {time.time() - t0:.1f}s", flush=True)
    o = oracle.load()
    dec = o.decoder(model, threads=args.threads)
    logits_steps = []
    for tok in prompt:
        logits = dec.forward(int(tok))
    tokens, margins = [], []
    first_logits = None
    t1 = time.time()
    for s in range(args.steps):
        t = int(np.argmax(logits))
        srt = np.partition(logits, -2)[-2:]
        tokens.append(t)
        margins.append(float(logits[t] - srt[0] if srt[1] == logits[t] else logits[t] - srt[1]))
        if first_logits is None:
            first_logits = logits.copy()
        logits_steps.append(hashlib.sha256(logits.tobytes()).hexdigest())
        logits = dec.forward(t)
    print(f"oracle decode {args.steps} steps in {time.time() - t1:.1f}s", flush=True)
    checked = False
    if os.path.exists(oracle.REF_DECODER_SO):
        with tempfile.TemporaryDirectory() as tmp:
            path = os.path.join(tmp, "m.qwn")
            qwn_file.write_decoder_model(path, model)
            ref = oracle.load_ref_decoder(path, synth.QWEN2_1P5B_CONFIG["max_ctx"], args.threads)
            V = synth.QWEN2_1P5B_CONFIG["vocab"]
            t2 = time.time()
            for tok in prompt:
                rl = ref.forward(int(tok), V)
            for s in range(args.steps):
                assert hashlib.sha256(rl.tobytes()).hexdigest() == logits_steps[s], f"step {s}: logits differ"
                assert int(np.argmax(rl)) == tokens[s]
                rl = ref.forward(tokens[s], V)
            ref.close()
            print(f"reference decoder agrees bit for bit ({time.time() - t2:.1f}s)", flush=True)
            checked = True
    out = {"config": synth.QWEN2_1P5B_CONFIG, "dtype": "q4_0", "seed": SEED,
           "prompt": [int(t) for t in prompt], "tokens": tokens, "margins": margins,
           "first_step_logits_sha256": logits_steps[0],
           "checked_against_reference_decoder": checked}
    with open(OUT, "w") as f:
        json.dump(out, f)
    print(f"wrote {OUT}; min margin {min(margins):.4g}")


if __name__ == "__main__":
    main()
