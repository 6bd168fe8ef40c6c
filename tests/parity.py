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
