"""Shared parity helpers for the tests."""
import numpy as np

# fp32 GEMV tolerance: |y - ref| <= 1e-4 * max(|ref|, rms(ref)) per element
GEMV_RTOL = 1e-4
# attention tolerance (reference test c/tests/test_cuda_q8_kv.cu:158)
ATTN_ATOL = 1e-4


def gemv_close(y, ref, rtol=GEMV_RTOL):
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    rms = np.sqrt(np.mean(ref ** 2, axis=-1, keepdims=True)) if ref.size else 0.0
    bound = rtol * np.maximum(np.abs(ref), rms)
    err = np.abs(y - ref)
    ok = bool(np.all(err <= bound))
    worst = float(np.max(err / np.maximum(bound, 1e-30))) if ref.size else 0.0
    return ok, worst


# ---- decoders: rounding differences through the layers --------------------
#
# A decoder step on the GPU sums RMSNorm, SwiGLU and the GEMV combination in
# another fp32 order than the CPU; wherever an activation lands within that
# rounding of an int8 boundary its quantized value moves by one, and the
# difference travels through the later layers and stays in the KV cache.
# How far it travels depends on the model, so decoder logits are held to
# the oracle's own sensitivity: the same tokens through the oracle with its
# calibration perturbation (rounding-sized moves of half the outputs of every
# RMSNorm, projection, attention and SwiGLU: one ulp of an element-wise
# result, 2^-23 of the largest output of a sum; oracle/qwn_oracle_decoder.c),
# sixteen seeds.  The GPU's per-step
# distance from the exact oracle must stay within ENV_K times that envelope
# (its largest step and its median step), or within ENV_FLOOR of the logit
# scale where the envelope is smaller still.
# An int8 flip is a rare event in a small model (a few of 16 perturbed runs
# of 24 steps show one) and a frequent one in a deep model; 16 seeds make it
# unlikely that the GPU shows one while no perturbed run does.
ENV_K = 4.0
ENV_FLOOR = 1e-5
ENV_SEEDS = tuple(range(1, 17))


def step_errors(a_steps, b_steps) -> np.ndarray:
    """Per step max |a - b| in units of max |b|."""
    return np.array([float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64)))) /
                     float(np.max(np.abs(b))) for a, b in zip(a_steps, b_steps)])


def oracle_envelope(oracle_lib, model, inputs, ref_steps, seeds=ENV_SEEDS) -> np.ndarray:
    """[seed][step] distances of the perturbed oracle from ref_steps, the
    exact oracle's logits after each token of `inputs` (prompt and
    teacher-forced ids, one forward each)."""
    out = []
    for seed in seeds:
        d = oracle_lib.decoder(model)
        d.perturb(seed)
        steps = [d.forward(int(t)) for t in inputs]
        d.close()
        out.append(step_errors(steps, ref_steps))
    return np.array(out)


def within_envelope(errs, env, k: float = ENV_K):
    """(ok, message): errs [step] against env [seed][step] (or a dict with
    'median' and 'max'): the GPU's median step within k times the largest
    per-seed median, its worst step within k times the worst step of any
    seed."""
    errs = np.asarray(errs)
    if isinstance(env, dict):
        env_med, env_max = env["median"], env["max"]
    else:
        env = np.asarray(env)
        env_med, env_max = float(np.median(env, axis=1).max()), float(env.max())
    med_bound = max(ENV_FLOOR, k * env_med)
    max_bound = max(ENV_FLOOR, k * env_max)
    med, mx = float(np.median(errs)), float(errs.max())
    msg = (f"median step {med:.3g} (bound {med_bound:.3g}), worst step {mx:.3g} at {int(errs.argmax())} "
           f"(bound {max_bound:.3g}); oracle envelope median {env_med:.3g}, max {env_max:.3g}")
    return med <= med_bound and mx <= max_bound, msg
