"""The golden greedy decodes of the Qwen2-1.5B shaped Q4_0 model
(tests/golden/make_decode_golden.py) and the per-step logit distance the
GPU decoders are measured with (held to each golden's stored envelope,
parity.within_envelope)."""
import importlib.util
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
NAMES = ("decode_qwen2_1p5b_q4_0.json", "decode_qwen2_1p5b_q4_0_varied.json",
         "decode_qwen2_1p5b_q4_0_successor.json")
# goldens whose every greedy step has a top-two margin far above the
# envelope: the decoders must reproduce all their ids, with no margin escape
STRICT = ("decode_qwen2_1p5b_q4_0_successor.json",)


def _maker():
    spec = importlib.util.spec_from_file_location("make_decode_golden",
                                                  os.path.join(HERE, "golden", "make_decode_golden.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def load(name: str):
    """(golden dict, model, prompt) or None when the fixture is absent."""
    path = os.path.join(HERE, "golden", name)
    if not os.path.exists(path):
        return None
    g = json.load(open(path))
    mk = _maker()
    model, prompt = mk.build_model({k: g[k] for k in mk.SPEC_KEYS if k in g})
    assert prompt.tolist() == g["prompt"]
    return g, model, prompt


def step_error(logits: np.ndarray, step: dict) -> float:
    """Distance of one step's logits from the golden step, in units of the
    golden logits' largest magnitude: at the golden top-16 ids, and no other
    id may rise above the golden 16th value by more than that."""
    ids = np.array(step["ids"])
    ref = np.array(step["logits"], dtype=np.float64)
    a = logits.astype(np.float64)
    err = float(np.max(np.abs(a[ids] - ref)))
    rest = np.delete(a, ids)
    err = max(err, float(np.max(rest)) - ref[-1])
    return err / step["max_abs"]


def check_greedy_ids(name: str, g: dict, tokens, errs) -> str:
    """The free-running greedy ids against the golden's.  STRICT goldens: all
    identical.  Others: the first divergence may not come before the first
    step whose golden top-two margin is within twice that step's measured
    (teacher-forced) error -- before it the ids are fixed to well within
    the rounding differences.  Returns a note for the log; raises
    AssertionError on failure."""
    tokens = list(tokens)
    first_diff = next((i for i, (x, y) in enumerate(zip(tokens, g["tokens"])) if x != y), None)
    close = [i for i, (m, e, st) in enumerate(zip(g["margins"], errs, g["steps"])) if m <= 2 * e * st["max_abs"]]
    first_close = close[0] if close else None
    note = (f"{len(set(g['tokens']))} distinct golden ids, first divergence {first_diff}, "
            f"first step with margin within 2x its error {first_close}")
    if name in STRICT:
        assert first_diff is None, f"{name}: greedy ids diverge at step {first_diff} ({note})"
    elif first_diff is not None:
        assert first_close is not None and first_diff >= first_close, \
            f"{name}: greedy ids diverge at step {first_diff}, before any near-tied step ({note})"
    return note
