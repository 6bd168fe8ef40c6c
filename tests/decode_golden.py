"""The golden greedy decodes of the Qwen2-1.5B shaped Q4_0 model
(tests/golden/make_decode_golden.py) and the per-step logit distance the
GPU decoders are measured with (held to each golden's stored envelope,
parity.within_envelope)."""
import importlib.util
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
NAMES = ("decode_qwen2_1p5b_q4_0.json", "decode_qwen2_1p5b_q4_0_varied.json")


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
    model, prompt = _maker().build_model({k: g[k] for k in ("seed", "weight_std", "embed_std", "zero_mean")})
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
