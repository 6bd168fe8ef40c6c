"""Pins the CPU oracle (oracle/qwn_oracle.c) before it is trusted as the
checker of the GPU library.

Each oracle function is checked three ways where possible:
  * bit for bit against the reference's own CPU kernels, compiled in place
    (oracle/_ref; skipped when that build is absent) and against the golden
    vectors those kernels wrote (tests/golden/*.npz, always run);
  * against the reference's known-answer tests, restated
    (c/tests/test_qwn_hypervsq2_cuda_abi.cu:84-149, test_qwn_hypervsq2_cuda.cu:9-23,
    test_cuda_q8_kv.cu:107-158, test_kv_cache.c:29-59);
  * against closed forms / brute force in numpy, with a planted mistake
    showing that the check can fail.
"""
import os

import numpy as np
import pytest

from qwanto_amd import synth

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def golden(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"))


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


# ---------------------------------------------------------------------------
# numpy brute-force decoders (independent of the C code)
# ---------------------------------------------------------------------------

def np_hvsq2_codes(w, N, K):
    """codes [N][nb*256] in element order (c/qwanto_native.h:96-103)."""
    nb = (K + 255) // 256
    blk = w.reshape(N, nb, 74)
    codes = blk[:, :, 10:].reshape(N, nb, 8, 8)            # octant, byte
    shifts = np.array([0, 2, 4, 6], dtype=np.uint8)
    c = (codes[..., None] >> shifts) & 3                   # octant, byte, field
    return c.reshape(N, nb * 256).astype(np.int64)


def np_hvsq2_subs(w, N, K):
    nb = (K + 255) // 256
    sb = w.reshape(N, nb, 74)[:, :, 4:8]
    sub = np.stack([sb & 0x0F, sb >> 4], axis=-1).reshape(N, nb, 8)
    return sub.astype(np.int64)


def np_q4_codes(w, N, K):
    nb = (K + 31) // 32
    blk = w.reshape(N, nb, 18)[:, :, 2:]
    c = np.stack([blk & 0x0F, blk >> 4], axis=-1).reshape(N, nb * 32)
    return c.astype(np.int64)


def np_half(w, N, nb, block, off):
    return w.reshape(N, nb, block)[:, :, off:off + 2].copy().view(np.float16)[..., 0].astype(np.float64)


# ---------------------------------------------------------------------------
# fp16 conversion and activation quantization
# ---------------------------------------------------------------------------

def test_half_to_float_all_patterns(oracle_lib):
    pats = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    expect = pats.view(np.float16).astype(np.float32)
    got = np.array([oracle_lib.half_to_float(int(h)) for h in pats], dtype=np.float32)
    finite = np.isfinite(expect) | np.isinf(expect)
    assert np.array_equal(bits(got)[finite], bits(expect)[finite])
    assert np.all(np.isnan(got[~finite]))
    # subnormal halves keep their value (c/qwanto_kernels.c:264-285)
    assert oracle_lib.half_to_float(0x0001) == np.float32(2.0 ** -24)


def test_quantize_golden(oracle_lib):
    g = golden("quantize")
    q8, xs, sums = oracle_lib.quantize(g["x"])
    assert np.array_equal(q8[0], g["q8"])
    assert bits(xs[0]) == bits(g["xs"])
    assert np.array_equal(sums[0], g["sums"])


def test_quantize_closed_forms(oracle_lib):
    # amax == 127 gives scale 1.0 and inv 1.0 exactly: q = rint-half-even(x)
    x = np.array([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, 3.49], dtype=np.float32)
    q8, xs, sums = oracle_lib.quantize(x)
    assert xs[0] == 1.0
    assert list(q8[0, :9]) == [127, 0, 2, 2, 0, -2, -2, 126, 3]
    assert np.all(q8[0, 9:] == 0)                  # zero padding to 256
    assert sums[0, 0] == sum([127, 0, 2, 2, 0, -2, -2, 126, 3])
    # all-zero token: scale 1
    q8, xs, _ = oracle_lib.quantize(np.zeros(40, dtype=np.float32))
    assert xs[0] == 1.0 and not q8.any()
    # planted mistake: round-half-away-from-zero would give 1 and 3 for 0.5, 2.5
    assert list(np.round(x[[1, 3]] + 1e-7 * np.sign(x[[1, 3]])).astype(int)) != list(q8[0, [1, 3]])


# ---------------------------------------------------------------------------
# HyperVSQ-2
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("name", ["hvsq2_small", "hvsq2_k2560"])
def test_hvsq2_golden(oracle_lib, name):
    g = golden(name)
    N, K = int(g["N"]), int(g["K"])
    y = oracle_lib.matmul_hvsq2(g["w"], g["x"], N)
    assert np.array_equal(bits(y), bits(g["y"])), "delayed restatement vs reference"
    for v in (0, 1, 2, 3):
        yv = oracle_lib.gemv_hvsq2(g["w"], g["q8"], g["sums"], float(g["xs"]), K, N, variant=v)
        assert np.array_equal(bits(yv), bits(g["y"][0])), oracle_lib.variant_name(v)
    ys = oracle_lib.gemv_hvsq2(g["w"], g["q8"], g["sums"], float(g["xs"]), K, N, variant=-2)
    assert np.array_equal(bits(ys), bits(g["y_scalar"])), "scalar golden vs reference"


@pytest.mark.parametrize("N,K", [(3, 513), (4, 256), (2, 1), (5, 300), (3, 2560), (2, 9728)])
def test_hvsq2_octant_sums_brute_force(oracle_lib, N, K):
    rng = np.random.default_rng(N * 1000 + K)
    w = synth.hvsq2_weights(rng, N, K)
    q8, xs, sums = oracle_lib.quantize(synth.activations(rng, 1, K))
    sq, sa = oracle_lib.hvsq2_octant_sums(w, q8[0], K, N)
    nb = (K + 255) // 256
    a = q8[0, :nb * 256].astype(np.int64)
    codes = np_hvsq2_codes(w, N, K)
    expect_q = ((codes - 1) * a).reshape(N, nb * 8, 32).sum(-1)
    expect_a = a.reshape(nb * 8, 32).sum(-1)
    assert np.array_equal(sq, expect_q) and np.array_equal(sa, expect_a)
    # planted mistake: reading codes high-bits-first changes the sums
    wrong = (((codes.reshape(N, -1, 4)[..., ::-1]).reshape(N, -1) - 1) * a).reshape(N, nb * 8, 32).sum(-1)
    assert not np.array_equal(sq, wrong)
    # fp32 output vs an fp64 sum of the exact integer terms
    d = np_half(w, N, nb, 74, 0)
    m = np_half(w, N, nb, 74, 2)
    sub = np_hvsq2_subs(w, N, K)
    exact = (d[:, :, None] * sub / 8.0 * expect_q.reshape(N, nb, 8)).sum((1, 2)) \
        + (m * expect_a.reshape(nb, 8).sum(-1)).sum(-1)
    exact *= float(xs[0])
    y = oracle_lib.gemv_hvsq2(w, q8[0], sums[0], float(xs[0]), K, N)
    rms = np.sqrt(np.mean(exact ** 2))
    assert np.all(np.abs(y - exact) <= 1e-5 * np.maximum(np.abs(exact), rms))


def abi_known_answer_case():
    """c/tests/test_qwn_hypervsq2_cuda_abi.cu:84-119: patterned 3x513 weights,
    batch 2, input (i*13)%127-63, scale 0.03125."""
    rows, cols, batch = 3, 513, 2
    blocks = (cols + 255) // 256
    w = np.zeros((rows, blocks, 74), dtype=np.uint8)
    for r in range(rows):
        for b in range(blocks):
            w[r, b, 0:2] = np.frombuffer(np.uint16(0x3800 + r * 0x200).tobytes(), np.uint8)
            w[r, b, 2:4] = np.frombuffer(np.uint16(0x1000 + b * 0x200).tobytes(), np.uint8)
            for i in range(4):
                w[r, b, 4 + i] = 0x18 + i * 0x11
            w[r, b, 8], w[r, b, 9] = 0xFF, 0x55
            for i in range(64):
                w[r, b, 10 + i] = ((i + r + b) & 3) * 0x55
    i = np.arange(batch * cols)
    x = ((i * 13) % 127 - 63).astype(np.int8).reshape(batch, cols)
    return w.reshape(-1), x, np.float32(0.03125), rows, cols


def abi_known_answer_expected(w, x, scale, rows, cols):
    """Exact per-octant integer sums combined in fp64."""
    nb = (cols + 255) // 256
    codes = np_hvsq2_codes(w, rows, cols)[:, :cols]
    sub = np_hvsq2_subs(w, rows, cols)
    d = np_half(w, rows, nb, 74, 0)
    m = np_half(w, rows, nb, 74, 2)
    out = np.zeros((x.shape[0], rows))
    for t in range(x.shape[0]):
        a = np.zeros(nb * 256, dtype=np.int64)
        a[:cols] = x[t]
        c = np.zeros((rows, nb * 256), dtype=np.int64)
        c[:, :cols] = codes
        sq = ((c - 1) * a).reshape(rows, nb, 8, 32)
        sq[:, :, :, :] = sq  # noqa
        # octant sums only count valid elements (tails have a == 0)
        sq = sq.sum(-1)
        sa = a.reshape(nb, 8, 32).sum(-1)
        out[t] = ((d[:, :, None] * sub / 8.0 * sq) + m[:, :, None] * sa).sum((1, 2)) * float(scale)
    return out


def test_hvsq2_abi_known_answer(oracle_lib):
    w, x, scale, rows, cols = abi_known_answer_case()
    expect = abi_known_answer_expected(w, x, scale, rows, cols)
    for t in range(x.shape[0]):
        q8 = np.zeros(768, dtype=np.int8)
        q8[:cols] = x[t]
        for v in (-2, -1):
            y = oracle_lib.gemv_hvsq2(w, q8, None, float(scale), cols, rows, variant=v)
            assert np.all(np.abs(y - expect[t]) <= 1e-3), (t, v, y, expect[t])


def test_hvsq2_single_block_closed_form(oracle_lib):
    """c/tests/test_qwn_hypervsq2_cuda.cu:9-23: d = 1, multipliers 8, m = 0,
    code(i) = i % 4, so y = xs * sum((i%4) - 1) * a_i."""
    w = np.zeros(74, dtype=np.uint8)
    w[0:2] = np.frombuffer(np.uint16(0x3C00).tobytes(), np.uint8)
    w[4:8] = 0x88
    for i in range(256):
        w[10 + i // 4] |= (i % 4) << ((i % 4) * 2)
    a = (np.arange(256) % 17 - 8).astype(np.int8)
    y = oracle_lib.gemv_hvsq2(w, a, None, 0.125, 256, 1, variant=-2)
    assert y[0] == np.float32(0.125 * np.sum(((np.arange(256) % 4) - 1) * a.astype(np.int64)))


def test_hvsq2_matches_reference_random(oracle_lib, ref_lib):
    rng = np.random.default_rng(7)
    for N, K, M in [(64, 2560, 1), (70, 4096, 2), (9, 9728, 1), (33, 1000, 3), (1, 1, 1)]:
        w = synth.hvsq2_weights(rng, N, K)
        x = synth.activations(rng, M, K)
        assert np.array_equal(bits(oracle_lib.matmul_hvsq2(w, x, N)), bits(ref_lib.matmul_hvsq2(w, x, N)))


# ---------------------------------------------------------------------------
# Q4_0
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("name", ["q4_0_small", "q4_0_k1536"])
def test_q4_0_golden(oracle_lib, name):
    g = golden(name)
    y = oracle_lib.matmul_q4_0(g["w"], g["x"], int(g["N"]))
    assert np.array_equal(bits(y), bits(g["y"]))


@pytest.mark.parametrize("N,K", [(3, 32), (4, 100), (2, 1), (5, 1536), (2, 8960)])
def test_q4_0_block_sums_brute_force(oracle_lib, N, K):
    rng = np.random.default_rng(N * 7 + K)
    w = synth.q4_0_weights(rng, N, K)
    q8, xs, _ = oracle_lib.quantize(synth.activations(rng, 1, K))
    raw = oracle_lib.q4_0_block_sums(w, q8[0], K, N)
    nb = (K + 31) // 32
    a = np.zeros(nb * 32, dtype=np.int64)
    a[:K] = q8[0, :K]
    codes = np_q4_codes(w, N, K)
    expect = ((codes - 8) * a).reshape(N, nb, 32).sum(-1)
    # elements past K do not count even though their nibbles are read
    assert np.array_equal(raw, expect)
    wrong = ((np_q4_codes(w, N, K).reshape(N, -1, 2)[..., ::-1].reshape(N, -1) - 8) * a).reshape(N, nb, 32).sum(-1)
    assert not np.array_equal(raw, wrong)  # high-nibble-first would be caught
    d = np_half(w, N, nb, 18, 0)
    exact = (d * expect).sum(-1) * float(xs[0])
    y = oracle_lib.gemv_q4_0_q8(w, q8[0], float(xs[0]), K, N)
    rms = np.sqrt(np.mean(exact ** 2))
    assert np.all(np.abs(y - exact) <= 1e-5 * np.maximum(np.abs(exact), rms))


def test_q4_0_matches_reference_random(oracle_lib, ref_lib):
    rng = np.random.default_rng(11)
    for N, K, M in [(64, 1536, 1), (37, 8960, 2), (7, 100, 1), (256, 1536, 1)]:
        w = synth.q4_0_weights(rng, N, K)
        x = synth.activations(rng, M, K)
        assert np.array_equal(bits(oracle_lib.matmul_q4_0(w, x, N)), bits(ref_lib.matmul_q4_0(w, x, N)))


# ---------------------------------------------------------------------------
# F16 generic matmul (LM head)
# ---------------------------------------------------------------------------

def test_f16_golden(oracle_lib):
    g = golden("f16_small")
    assert np.array_equal(bits(oracle_lib.matmul_f16(g["w"], g["x"])), bits(g["y"]))


def test_f16_closed_form_and_reference(oracle_lib, ref_lib):
    rng = np.random.default_rng(5)
    for K in (1, 7, 12, 70, 1536):
        w = synth.f16_weights(rng, 9, K)
        w[0, 0] = np.float16(6e-8)  # subnormal weight
        x = synth.activations(rng, 2, K)
        y = oracle_lib.matmul_f16(w, x)
        exact = x.astype(np.float64) @ w.astype(np.float64).T
        assert np.all(np.abs(y - exact) <= 1e-5 * (np.abs(x) @ np.abs(w.astype(np.float64)).T) + 1e-12)
        assert np.array_equal(bits(y), bits(ref_lib.matmul_f16(w, x)))


def test_bf16_conversion_all_patterns(oracle_lib):
    """bfloat16 -> fp32 is the 16 bits placed high (c/qwanto_kernels.c:287-290):
    every one of the 65536 patterns, NaN payloads and subnormals included,
    against the same bits built by integer arithmetic."""
    pats = np.arange(65536, dtype=np.uint32)
    want = (pats << 16).astype(np.uint32)
    got = np.array([oracle_lib.lib.qo_bf16_to_float(int(p)) for p in pats[::257]], dtype=np.float32)
    assert np.array_equal(got.view(np.uint32), want[::257])
    # the conversion the synthetic generator uses rounds to nearest even
    assert synth.to_bf16_bits(np.array([1.0 + 2.0 ** -8], np.float32))[0] == 0x3F80  # tie -> even
    assert synth.to_bf16_bits(np.array([1.0 + 3 * 2.0 ** -9], np.float32))[0] == 0x3F81


def test_bf16_closed_form_and_reference(oracle_lib, ref_lib):
    """qwn_matmul_f32 on BF16 rows (c/qwanto_kernels.c:1508-1527, 1605-1614):
    within fp32 rounding of the fp64 product of the decoded weights, and
    bit-identical to the reference build."""
    rng = np.random.default_rng(15)
    for K in (1, 7, 12, 70, 1536):
        w = synth.bf16_weights(rng, 9, K)
        w[0, 0] = 0x0001  # subnormal weight
        x = synth.activations(rng, 2, K)
        y = oracle_lib.matmul_bf16(w, x)
        wf = synth.bf16_to_f32(w).astype(np.float64)
        exact = x.astype(np.float64) @ wf.T
        assert np.all(np.abs(y - exact) <= 1e-5 * (np.abs(x) @ np.abs(wf).T) + 1e-12)
        assert np.array_equal(bits(y), bits(ref_lib.matmul_bf16(w, x)))
        # a dropped conversion (the raw bits read as F16) would differ
        assert not np.array_equal(bits(y), bits(oracle_lib.matmul_f16(w.view(np.float16), x)))


# ---------------------------------------------------------------------------
# Q8 KV cache
# ---------------------------------------------------------------------------

def np_q8_attention(q, kq, vq, ks, vs, H, HK, D, pos, scale):
    """fp64 softmax attention over the dequantized cache."""
    C = HK * D
    ch = np.arange(C)
    kf = kq[:pos + 1].astype(np.float64) * ks[:pos + 1][:, ch // 64]
    vf = vq[:pos + 1].astype(np.float64) * vs[:pos + 1][:, ch // 64]
    out = np.zeros(H * D)
    for h in range(H):
        kh = h * HK // H
        s = kf[:, kh * D:(kh + 1) * D] @ q[h * D:(h + 1) * D].astype(np.float64) * scale
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h * D:(h + 1) * D] = p @ vf[:, kh * D:(kh + 1) * D]
    return out


def test_q8_golden(oracle_lib):
    g = golden("q8_attention")
    kq, ks = oracle_lib.q8_quantize(g["k"])
    vq, vs = oracle_lib.q8_quantize(g["v"])
    assert np.array_equal(kq, g["kq"]) and np.array_equal(vq, g["vq"])
    assert np.array_equal(bits(ks), bits(g["ks"])) and np.array_equal(bits(vs), bits(g["vs"]))
    H, HK, D, pos = int(g["H"]), int(g["HK"]), int(g["D"]), int(g["pos"])
    out = oracle_lib.q8_attention(g["q"], kq, vq, ks, vs, H, HK, D, pos, np.float32(1 / np.sqrt(D)))
    assert np.array_equal(bits(out), bits(g["out"]))


def test_q8_known_answer(oracle_lib):
    """c/tests/test_cuda_q8_kv.cu:107-158: 2 tokens, 4 query heads, 2 KV heads,
    head_dim 4, scale 0.5, 1e-4 absolute."""
    T, H, HK, D = 2, 4, 2, 4
    i = np.arange(T * HK * D)
    k = ((i - 3) * np.float32(0.17)).astype(np.float32).reshape(T, HK * D)
    v = ((i + 2) * np.float32(-0.11)).astype(np.float32).reshape(T, HK * D)
    q = ((np.arange(H * D) - 5) * np.float32(0.09)).astype(np.float32)
    kq, ks = oracle_lib.q8_quantize(k)
    vq, vs = oracle_lib.q8_quantize(v)
    # closed-form quantization of token 0 of K: amax = 4*0.17, scale = amax/127
    s0 = np.float32(np.float32(4 * 0.17) / np.float32(127.0))
    assert abs(ks[0, 0] - s0) <= 1e-9
    out = oracle_lib.q8_attention(q, kq, vq, ks, vs, H, HK, D, T - 1, 0.5)
    expect = np_q8_attention(q, kq, vq, ks, vs, H, HK, D, T - 1, 0.5)
    assert np.max(np.abs(out - expect)) <= 1e-6
    # planted mistake: a wrong GQA mapping (h % HK) is caught
    bad = np_q8_attention(q, kq, vq, ks, vs, H, HK, D, T - 1, 0.5).copy()
    bad[D:2 * D], bad[2 * D:3 * D] = bad[2 * D:3 * D].copy(), bad[D:2 * D].copy()
    assert np.max(np.abs(out - bad)) > 1e-3


def test_q8_special_values(oracle_lib):
    """c/tests/test_kv_cache.c:29-59: a 65-wide head (groups span heads) and
    NaN/Inf inputs quantize to 0 with finite scales."""
    key = ((np.arange(130) - 65) * np.float32(0.03125)).astype(np.float32)
    value = np.sin(np.arange(130, dtype=np.float32) * np.float32(0.07)).astype(np.float32)
    kq, ks = oracle_lib.q8_quantize(key)
    vq, vs = oracle_lib.q8_quantize(value)
    assert ks.shape == (3,)
    assert abs(vq[0] * vs[0] - value[0]) <= 0.02 and abs(vq[64] * vs[1] - value[64]) <= 0.02
    key[0], key[1], value[0], value[1] = np.nan, np.inf, -np.inf, np.nan
    kq, ks = oracle_lib.q8_quantize(key)
    vq, vs = oracle_lib.q8_quantize(value)
    assert np.all(np.isfinite(ks)) and np.all(np.isfinite(vs))
    assert kq[0] == kq[1] == vq[0] == vq[1] == 0


def test_q8_attention_matches_reference_random(oracle_lib, ref_lib):
    rng = np.random.default_rng(9)
    for T, HK, D, H in [(50, 2, 65, 4), (300, 8, 128, 32), (17, 2, 128, 12)]:
        k = rng.standard_normal((T, HK * D), dtype=np.float32)
        v = rng.standard_normal((T, HK * D), dtype=np.float32)
        q = rng.standard_normal(H * D, dtype=np.float32)
        sc = np.float32(1 / np.sqrt(D))
        out_r, kq, vq, ks, vs = ref_lib.q8_attention(k, v, HK, D, q, H, T - 1, sc)
        kq2, ks2 = oracle_lib.q8_quantize(k)
        vq2, vs2 = oracle_lib.q8_quantize(v)
        assert np.array_equal(kq, kq2) and np.array_equal(vq, vq2)
        out = oracle_lib.q8_attention(q, kq2, vq2, ks2, vs2, H, HK, D, T - 1, sc)
        assert np.array_equal(bits(out), bits(out_r))
        expect = np_q8_attention(q, kq, vq, ks, vs, H, HK, D, T - 1, sc)
        assert np.max(np.abs(out - expect)) <= 1e-5
