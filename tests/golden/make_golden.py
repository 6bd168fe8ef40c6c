"""Writes the golden vectors in tests/golden/*.npz from the reference's own
CPU kernels (c/qwanto_kernels.c, c/qwanto_turboquant.c), compiled in place by
oracle/Makefile into oracle/_ref/libqwn_ref.so.  Each file holds seeded
inputs and the reference outputs; the tests check the oracle against them
wherever the reference build is absent.  Run in the build container:

    make -C oracle && python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from qwanto_amd import synth  # noqa: E402


def main() -> None:
    ref = oracle.load_ref()
    if ref is None:
        raise SystemExit("oracle/_ref/libqwn_ref.so missing: run make -C oracle first")
    rng = np.random.default_rng(20261201)
    kernel = ref.cpu_kernel_name()

    # HyperVSQ-2: full and tail blocks; matmul (production dispatch) and the
    # scalar golden on the same quantized token.
    for name, (N, K, M) in {"hvsq2_small": (5, 513, 2), "hvsq2_k2560": (8, 2560, 1)}.items():
        w = synth.hvsq2_weights(rng, N, K)
        x = synth.activations(rng, M, K)
        y = ref.matmul_hvsq2(w, x, N)
        q8, xs, sums = ref.quantize_token(x[0])
        y_scalar = ref.gemv_hvsq2(w, q8, sums, xs, K, N, delayed=False)
        np.savez_compressed(os.path.join(HERE, name + ".npz"), w=w, x=x, y=y, q8=q8,
                            xs=np.float32(xs), sums=sums, y_scalar=y_scalar, N=N, K=K,
                            kernel=kernel)

    for name, (N, K, M) in {"q4_0_small": (7, 100, 2), "q4_0_k1536": (6, 1536, 1)}.items():
        w = synth.q4_0_weights(rng, N, K)
        x = synth.activations(rng, M, K)
        y = ref.matmul_q4_0(w, x, N)
        np.savez_compressed(os.path.join(HERE, name + ".npz"), w=w, x=x, y=y, N=N, K=K)

    w = synth.f16_weights(rng, 5, 70)
    x = synth.activations(rng, 1, 70)
    np.savez_compressed(os.path.join(HERE, "f16_small.npz"), w=w, x=x, y=ref.matmul_f16(w, x))

    # per-token quantization with planted ties (x * inv lands on k + 0.5)
    x = synth.activations(rng, 1, 2600)[0]
    x[0] = 4.0          # amax -> scale 4/127, x*inv = 127 exactly
    x[1:9] = (np.arange(8) + 0.5) * np.float32(4.0 / 127.0)
    q8, xs, sums = ref.quantize_token(x)
    np.savez_compressed(os.path.join(HERE, "quantize.npz"), x=x, q8=q8, xs=np.float32(xs),
                        sums=sums)

    # Q8 KV cache + attention, with a 65-wide head (64-channel groups span
    # heads) and non-finite inputs in the last token.
    T, HK, D, H = 20, 2, 65, 4
    k = rng.standard_normal((T, HK * D), dtype=np.float32)
    v = rng.standard_normal((T, HK * D), dtype=np.float32)
    k[-1, 0], k[-1, 1], v[-1, 0], v[-1, 1] = np.nan, np.inf, -np.inf, np.nan
    q = rng.standard_normal(H * D, dtype=np.float32)
    out, kq, vq, ks, vs = ref.q8_attention(k, v, HK, D, q, H, T - 2, np.float32(1 / np.sqrt(D)))
    np.savez_compressed(os.path.join(HERE, "q8_attention.npz"), k=k, v=v, q=q, out=out, kq=kq,
                        vq=vq, ks=ks, vs=vs, T=T, HK=HK, D=D, H=H, pos=T - 2)
    print("golden vectors written with reference kernel", kernel)


if __name__ == "__main__":
    main()
