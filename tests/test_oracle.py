"""Pins the CPU oracle (oracle/oracle.py, oracle/qk_oracle.c) against hand-
derived known answers, closed forms, brute force and invariants, so that a
plausible mistake (a dropped term, a wrong sign or index, a swapped nibble)
fails here before it is trusted as the checker of the HIP kernels.
"""

import math

import numpy as np
import pytest
import torch

import oracle as O

# ---------------------------------------------------------------------------
# bf16 rounding


def test_bf16_bits_known_answers():
    cases = [
        (1.0, 0x3F80),
        (-2.0, 0xC000),
        # 1 + 2^-8 is exactly halfway between 1 and 1 + 2^-7: ties to even.
        (1.0 + 2.0 ** -8, 0x3F80),
        # 1 + 3*2^-8 is halfway between 1+2^-7 (odd) and 1+2^-6: up.
        (1.0 + 3 * 2.0 ** -8, 0x3F82),
        # just above the tie rounds up
        (1.0 + 2.0 ** -8 + 2.0 ** -20, 0x3F81),
        (float("inf"), 0x7F80),
        (-float("inf"), 0xFF80),
        (0.0, 0x0000),
        (-0.0, 0x8000),
        (3.4e38, 0x7F80),  # overflows to inf after rounding
    ]
    for v, want in cases:
        got = int(O.bf16_bits(np.float32(v)).reshape(-1)[0])
        assert got == want, (v, hex(got), hex(want))
    nan = O.bf16_bits(np.float32("nan")).reshape(-1)[0]
    assert (int(nan) & 0x7F80) == 0x7F80 and (int(nan) & 0x7F) != 0


def test_bf16_matches_torch_rne():
    r = np.random.default_rng(0)
    x = np.concatenate([
        r.standard_normal(100000).astype(np.float32),
        (r.standard_normal(1000) * 1e-39).astype(np.float32),  # subnormals
        (r.standard_normal(1000) * 1e30).astype(np.float32),
    ])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy()
    assert np.array_equal(O.bf16_bits(x), want.view(np.uint16))


# ---------------------------------------------------------------------------
# activations and the GEMM reference


def test_activation_closed_forms():
    assert math.isnan(float(O.act_relu(np.nan)))  # ReLU keeps NaN
    assert float(O.act_relu(-3.0)) == 0.0 and float(O.act_relu(2.5)) == 2.5
    # SiLU(0) = 0, SiLU(x) - SiLU(-x) = x, SiLU(large) ~ x
    x = np.linspace(-8, 8, 101)
    assert np.allclose(O.act_silu(x) - O.act_silu(-x), x, atol=1e-12)
    assert float(O.act_silu(0.0)) == 0.0
    assert abs(float(O.act_silu(40.0)) - 40.0) < 1e-12
    # GELU(tanh): GELU(x) - GELU(-x) = x; GELU(0) = 0; sqrt(2/pi) constant
    assert np.allclose(O.act_gelu(x) - O.act_gelu(-x), x, atol=1e-12)
    assert abs(O.GELU_K - math.sqrt(2 / math.pi)) < 1e-15
    # tanh form differs from the erf form by < 1e-3 (known bound).
    erf_gelu = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2)))
                         for v in x])
    assert np.max(np.abs(O.act_gelu(x) - erf_gelu)) < 1e-3


def test_gemm_ref_matches_bruteforce():
    r = np.random.default_rng(1)
    for m, n, k in [(1, 1, 1), (3, 5, 7), (4, 2, 9)]:
        a = r.standard_normal((m, k))
        b = r.standard_normal((k, n))
        bias = r.standard_normal(n)
        c = r.standard_normal((m, n))
        want = O.gemm_bruteforce(a, b) * 0.5 - 1.5 * c + bias
        _, v = O.gemm_ref(a, b, c, bias, alpha=0.5, beta=-1.5)
        assert np.allclose(v, want, rtol=0, atol=1e-12)
        d, v = O.gemm_ref(a, b, bias=bias, act=3)
        assert np.allclose(d, v / (1 + np.exp(-v)), atol=1e-15)


def test_gemm_ref_exact_products():
    # The reference gtest's inputs (metal_blas_lt_test.cc:125-130): multiples
    # of 1/4, so every product and sum is exact in float64.
    m, n, k = 5, 7, 3
    a = np.array([((i * 7) % 9) * 0.25 - 1.0 for i in range(m * k)])
    b = np.array([((i * 5) % 11) * 0.25 - 1.25 for i in range(k * n)])
    a, b = a.reshape(m, k), b.reshape(k, n)
    _, v = O.gemm_ref(a, b)
    assert v[0, 0] == a[0] @ b[:, 0]
    # D[0,0] by hand:
    # a row 0 = ((0,7,14)%9)*.25-1 = (0,7,5)*.25-1 = (-1, .75, .25)
    # b col 0 = ((0,35,70)%11)*.25-1.25 = (0,2,4)*.25-1.25 = (-1.25,-.75,-.25)
    assert v[0, 0] == (-1 * -1.25) + (0.75 * -0.75) + (0.25 * -0.25)


def test_epilogue_table_matches_names():
    # DecodeEpilogue: (bias, act, aux) for the 12 BlasLt epilogues.
    names = ["Default", "ReLU", "Bias", "BiasThenReLU", "GELU", "GELUWithAux",
             "BiasThenGELU", "BiasThenGELUWithAux", "SILU", "SILUWithAux",
             "BiasThenSILU", "BiasThenSILUWithAux"]
    for i, name in enumerate(names):
        bias, act, aux = O.EPILOGUES[i]
        assert bias == name.startswith("Bias")
        assert aux == name.endswith("WithAux")
        want_act = 1 if "ReLU" in name else 2 if "GELU" in name else \
            3 if "SILU" in name else 0
        assert act == want_act


# ---------------------------------------------------------------------------
# quantizers


def test_quantize_int4_known_answer_positive_anchor():
    # A group 0, 1/15, ..., 1 (repeated): anchored at hi = 1, step -1/15,
    # so the code of j/15 is 15 - j (derived by hand from qwen3.py:177-196).
    j = np.arange(64) % 16
    w = (j / 15.0).astype(np.float32)[None, :]
    codes, s, b = O.quantize_int4(w)
    assert np.array_equal(codes[0, 0], (15 - j).astype(np.uint8))
    assert b[0, 0, 0] == np.float32(1.0)
    assert np.isclose(s[0, 0, 0], -1.0 / 15, rtol=1e-7)


def test_quantize_int4_known_answer_negative_anchor():
    # lo = -1, hi = 0.2: |lo| > |hi|, step 1.2/15 = 0.08, q0 = rint(-1/0.08)
    # = rint(-12.5) = -12 (the float32 quotient is within an ulp of the tie,
    # and either way rounds to -12), so s = 1/12 and b = -1. Then
    # w = 0.2 -> rint(14.4) = 14, w = 0.1 -> rint(13.2) = 13, w = 0 -> 12.
    w = np.full((1, 64), 0.0, np.float32)
    w[0, 0], w[0, 1], w[0, 2] = -1.0, 0.2, 0.1
    codes, s, b = O.quantize_int4(w)
    assert b[0, 0, 0] == np.float32(-1.0)
    assert np.isclose(s[0, 0, 0], 1.0 / 12, rtol=1e-6)
    assert codes[0, 0, 0] == 0 and codes[0, 0, 1] == 14
    assert codes[0, 0, 2] == 13
    assert np.all(codes[0, 0, 3:] == 12)  # zero is on the grid
    deq = O.dequantize_f32(codes, s, b)
    assert np.all(deq[0, 3:] == 0.0)


def test_quantize_int4_bruteforce_properties():
    r = np.random.default_rng(2)
    w = (r.standard_normal((32, 256)) * r.uniform(0.01, 3, (32, 1))).astype(
        np.float32)
    codes, s, b = O.quantize_int4(w)
    assert codes.max() <= 15
    deq = O.dequantize_f32(codes, s, b).reshape(32, -1, 64)
    wg = w.reshape(32, -1, 64)
    # the anchored grid covers [lo, hi] to within half a step... except the
    # stretched step may leave the far end up to one step (clipped) away.
    err = np.abs(deq - wg)
    assert np.all(err <= np.abs(s) * 1.0 + 1e-6)
    # the anchor (largest-magnitude weight) is reproduced exactly
    idx = np.argmax(np.abs(wg), axis=-1)
    anchors = np.take_along_axis(wg, idx[..., None], -1)
    got = np.take_along_axis(deq, idx[..., None], -1)
    assert np.allclose(got, anchors, rtol=1e-6, atol=1e-7)
    # zero lies on the grid: -b/s is an integer in 0..15
    z = -b / s
    assert np.allclose(z, np.rint(z), atol=1e-3)


def test_quantize_int4_brute_force_code_choice():
    # For each weight, the chosen code is the nearest of the 16 grid points
    # (or clipped): brute force over all codes on small groups.
    r = np.random.default_rng(3)
    w = r.standard_normal((8, 64)).astype(np.float32)
    codes, s, b = O.quantize_int4(w)
    grid = np.arange(16, dtype=np.float64)
    for row in range(8):
        sv, bv = float(s[row, 0, 0]), float(b[row, 0, 0])
        pts = grid * sv + bv
        for j in range(64):
            best = np.argmin(np.abs(pts - float(w[row, j])))
            assert abs(pts[codes[row, 0, j]] - w[row, j]) <= \
                abs(pts[best] - w[row, j]) + abs(sv) * 1e-5


def test_quantize_int8_properties():
    r = np.random.default_rng(4)
    w = r.standard_normal((16, 128)).astype(np.float32)
    q, s = O.quantize_int8(w)
    assert q.dtype == np.int8 and np.abs(q).max(axis=-1).min() == 127
    deq = q.astype(np.float64) * s
    assert np.all(np.abs(deq - w.reshape(16, -1, 64)) <= s / 2 + 1e-7)
    # all-zero group: scale floor 1e-12/127, codes zero
    q0, s0 = O.quantize_int8(np.zeros((1, 64), np.float32))
    assert np.all(q0 == 0) and np.isclose(s0[0, 0, 0], 1e-12 / 127)


def test_packings_known_bits_and_round_trips():
    codes = np.arange(64, dtype=np.uint8)[None, :] % 16  # 0..15,0..15,...
    words = O.pack_u32x8(codes)
    # word 0 holds elements 0..7 = nibbles 0..7 -> 0x76543210
    assert words[0, 0] == 0x76543210 and words[0, 1] == 0xFEDCBA98
    assert np.array_equal(O.unpack_u32x8(words), codes)
    hs = O.pack_halfsplit(codes.reshape(1, 1, 64))
    # byte j = element j | element j+32 << 4; element j+32 = (j+32)%16 = j%16
    assert hs[0, 0, 1] == (1 | (1 << 4))
    r = np.random.default_rng(5)
    c = r.integers(0, 16, (7, 256), dtype=np.uint8)
    p = O.pack_halfsplit(c.reshape(7, -1, 64))
    assert np.array_equal(O.unpack_halfsplit(p).reshape(7, -1), c)
    c2 = c.copy()
    c2[3, 40] ^= 1  # one flipped bit changes exactly one word
    assert np.sum(O.pack_u32x8(c2) != O.pack_u32x8(c)) == 1


def test_dequantize_exact_closed_form():
    # power-of-two scales and offsets: s*q + b exact in f32 and bf16
    q = np.arange(64, dtype=np.uint8).reshape(1, 1, 64) % 16
    s = np.array([[[0.25]]], np.float32)
    b = np.array([[[-2.0]]], np.float32)
    w = O.dequantize_f32(q, s, b)
    assert np.array_equal(w[0], (q[0, 0] * 0.25 - 2.0).astype(np.float32))
    bits = O.dequantize_bf16_bits(q, s, b)
    assert np.array_equal(O.bf16_to_f32(bits), w)


def test_dequantize_rounding_is_unfused():
    # f32 scale with 24 significant bits: q*s rounds in f32 before + b.
    q = np.full((1, 1, 64), 15, np.uint8)
    s = np.array([[[1.0 + 2.0 ** -23]]], np.float32)
    b = np.array([[[2.0 ** -22]]], np.float32)
    w = O.dequantize_f32(q, s, b)[0, 0]
    prod = np.float32(np.float32(15.0) * s[0, 0, 0])
    assert w == np.float32(prod + b[0, 0, 0])


def test_matvec_reference_forms_equal_dot_product():
    r = np.random.default_rng(6)
    n, k, m = 24, 256, 3
    w = r.standard_normal((n, k)).astype(np.float32)
    codes, s, b = O.quantize_int4(w)
    packed = O.pack_halfsplit(codes)
    x = r.standard_normal((m, k)).astype(np.float32)
    want = O.matvec_f64(x, O.dequantize_f32(codes, s, b))
    got = O.matvec_int4_reference_form(x, packed, s, b)
    assert O.rel_fro(got, want) < 1e-5
    q8, s8 = O.quantize_int8(w)
    want8 = O.matvec_f64(x, O.dequantize_f32(q8, s8))
    assert O.rel_fro(O.matvec_int8_reference_form(x, q8, s8), want8) < 1e-5


def test_c_port_matvecs():
    r = np.random.default_rng(7)
    n, k, m = 37, 512, 2
    codes, s, b = O.config_affine(n, k, bits=4, seed=7)
    x = O.bf16_round(r.standard_normal((m, k)).astype(np.float32))
    w = O.dequantize_f32(codes.reshape(n, -1, 64), s[..., None], b[..., None])
    want = O.matvec_f64(x, w)
    got = O.c_matvec_int4_u32x8(O.bf16_bits(x), O.pack_u32x8(codes),
                                O.bf16_bits(s), O.bf16_bits(b), threads=2)
    assert O.rel_fro(got, want) < 1e-5
    codes8, s8, b8 = O.config_affine(n, k, bits=8, seed=8)
    w8 = O.dequantize_f32(codes8.reshape(n, -1, 64), s8[..., None],
                          b8[..., None])
    got8 = O.c_matvec_u8(O.bf16_bits(x), codes8, O.bf16_bits(s8),
                         O.bf16_bits(b8), threads=2)
    assert O.rel_fro(got8, O.matvec_f64(x, w8)) < 1e-5
    # a dropped offset term would be caught:
    w_nob = O.dequantize_f32(codes.reshape(n, -1, 64), s[..., None])
    assert O.rel_fro(O.matvec_f64(x, w_nob), want) > 1e-2
    # the magnitude output is sum_k |x||w| (numpy closed form), and the
    # values returned with it are the same as without it
    got_m, mag = O.c_matvec_int4_u32x8(O.bf16_bits(x), O.pack_u32x8(codes),
                                       O.bf16_bits(s), O.bf16_bits(b),
                                       threads=3, with_mag=True)
    assert np.array_equal(got_m, got)
    want_mag = np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T
    assert np.allclose(mag, want_mag, rtol=1e-12)
    got8m, mag8 = O.c_matvec_u8(O.bf16_bits(x), codes8, O.bf16_bits(s8),
                                O.bf16_bits(b8), threads=1, with_mag=True)
    assert np.array_equal(got8m, got8)
    assert np.allclose(mag8, np.abs(x).astype(np.float64) @
                       np.abs(w8).astype(np.float64).T, rtol=1e-12)
    # each output row depends only on its own row of x (row order of the
    # decode-once loop): swapping x's rows swaps y's rows exactly
    got_sw = O.c_matvec_int4_u32x8(O.bf16_bits(x[::-1].copy()),
                                   O.pack_u32x8(codes), O.bf16_bits(s),
                                   O.bf16_bits(b), threads=2)
    assert np.array_equal(got_sw, got[::-1])


# ---------------------------------------------------------------------------
# row normalisation


def test_rownorm_invariants():
    r = np.random.default_rng(9)
    # constant row c: rms_norm gives sign(c) * g (for eps << c^2)
    x = np.full((1, 128), -3.0)
    g = r.standard_normal(128)
    assert np.allclose(O.rms_norm(x, g, eps=0.0), -g, atol=1e-15)
    x = r.standard_normal((4, 1000)) * 5 + 2
    y = O.layer_norm(x, eps=0.0)
    assert np.allclose(y.mean(-1), 0, atol=1e-12)
    assert np.allclose(y.var(-1), 1, atol=1e-12)
    s = O.softmax(x)
    assert np.allclose(s.sum(-1), 1, atol=1e-14)
    assert np.allclose(O.softmax(x + 100.0), s, atol=1e-14)
    # softmax of two elements is a logistic function
    t = O.softmax(np.array([[0.3, -1.1]]))
    assert np.isclose(t[0, 0], 1 / (1 + math.exp(-1.4)), atol=1e-15)
    # layer_norm with gain and beta: an affine map of the plain output,
    # pinned by closed forms -- a constant row gives exactly beta (x - mean
    # = 0), and a row of +-a (mean 0, variance a^2) gives gain * (+-a /
    # sqrt(a^2 + eps)) + beta, which catches (y + beta) * gain.
    gain = r.standard_normal(6) + 2.0
    beta = r.standard_normal(6)
    xc = np.full((2, 6), 7.5)
    assert np.array_equal(O.layer_norm(xc, eps=1e-5, gain=gain, beta=beta),
                          np.broadcast_to(beta, (2, 6)))
    a, eps = 3.0, 0.25
    xs = np.array([[a, -a, a, -a, a, -a]])
    sign = np.array([1, -1, 1, -1, 1, -1], dtype=np.float64)
    want = gain * sign * a / math.sqrt(a * a + eps) + beta
    assert np.allclose(O.layer_norm(xs, eps=eps, gain=gain, beta=beta), want,
                       atol=1e-14)
    assert not np.allclose((O.layer_norm(xs, eps=eps) + beta) * gain, want)
    # gain alone scales and beta alone shifts the plain output
    y0 = O.layer_norm(x, eps=1e-5)
    g1 = r.standard_normal(1000)
    assert np.allclose(O.layer_norm(x, eps=1e-5, gain=g1), y0 * g1, atol=1e-14)
    assert np.allclose(O.layer_norm(x, eps=1e-5, beta=g1), y0 + g1, atol=1e-14)
    # rms_norm's defining identity: mean(y^2) = mean(x^2)/(mean(x^2)+eps)
    y = O.rms_norm(x, eps=0.5)
    ms = (x * x).mean(-1)
    assert np.allclose((y * y).mean(-1), ms / (ms + 0.5), atol=1e-12)


def test_config_generators_deterministic():
    a1, b1 = O.config_gemm_f32(0, 64)
    a2, b2 = O.config_gemm_f32(0, 64)
    assert np.array_equal(a1, a2) and np.array_equal(b1, b2)
    c, s, b = O.config_affine(16, 128, bits=4, seed=3)
    assert c.max() <= 15 and s.min() >= 0.001 * 0.99 and s.max() <= 0.02 * 1.01
    # scale and offset are bf16-representable
    assert np.array_equal(O.bf16_round(s), s)
    assert np.array_equal(O.bf16_round(b), b)


@pytest.mark.parametrize("group", [32, 64, 128])
def test_quantize_groups(group):
    r = np.random.default_rng(group)
    w = r.standard_normal((4, 256)).astype(np.float32)
    codes, s, b = O.quantize_int4(w, group)
    assert codes.shape == (4, 256 // group, group)
    assert O.rel_fro(O.dequantize_f32(codes, s, b), w) < 0.2


# ---------------------------------------------------------------------------
# decode attention


def attention_bruteforce(q, k, v, pos, scale, window):
    """Loops over heads and slots (pins O.decode_attention on tiny
    shapes): explicit max-subtracted exponentials and weighted sums."""
    B, KV, G, D = q.shape
    out = np.zeros((B, KV, G, D))
    for b in range(B):
        for h in range(KV):
            for g in range(G):
                slots = [s for s in range(window) if s <= pos]
                t = [scale * sum(float(q[b, h, g, d]) * float(k[b, h, s, d])
                                 for d in range(D)) for s in slots]
                m = max(t)
                e = [math.exp(x - m) for x in t]
                z = sum(e)
                for d in range(D):
                    out[b, h, g, d] = sum(e[i] * float(v[b, h, d, s])
                                          for i, s in enumerate(slots)) / z
    return out


def test_decode_attention_oracle():
    r = np.random.default_rng(21)
    B, KV, G, D, Smax = 2, 2, 3, 4, 8
    q = r.standard_normal((B, KV, G, D))
    k = r.standard_normal((B, KV, Smax, D))
    v = r.standard_normal((B, KV, D, Smax))
    for pos, window in [(0, 8), (3, 8), (7, 8), (9, 6), (4, 5)]:
        got = O.decode_attention(q, k, v, pos, 0.7, window)
        want = attention_bruteforce(q, k, v, pos, 0.7, window)
        assert np.allclose(got, want, atol=1e-12), (pos, window)
    # closed forms: one attended slot returns that slot's values; equal
    # keys (or scale 0) give the mean of the attended values; a key far
    # more aligned than the rest selects its slot
    one = O.decode_attention(q, k, v, 0, 0.5)
    assert np.allclose(one, np.broadcast_to(v[:, :, None, :, 0], one.shape))
    kc = np.broadcast_to(k[:, :, :1], k.shape)
    mean = O.decode_attention(q, kc, v, 5, 0.9)
    assert np.allclose(mean, np.broadcast_to(
        v[:, :, None, :, :6].mean(-1), mean.shape), atol=1e-12)
    assert np.allclose(O.decode_attention(q, k, v, 5, 0.0), mean, atol=1e-12)
    kb = k.copy()
    kb[:, :, 2] = 50.0 * q[:, :, 0]  # slot 2 aligned with head 0
    sel = O.decode_attention(q, kb, v, 7, 1.0)
    assert np.allclose(sel[:, :, 0], v[:, :, :, 2], atol=1e-9)
    # a transposed value cache (the [B, KV, S, D] layout of keys) or a
    # dropped scale would be caught
    assert not np.allclose(O.decode_attention(q, k, v, 7, 0.7),
                           O.decode_attention(q, k, v, 7, 1.0))


def test_embed_gathers_dequantized_rows_and_clamps():
    # qwen3.embed gathers the q4, s and b rows, then dequantizes
    # (qwen3.py:270-274): the same as picking rows of the dequantized table
    rng = np.random.default_rng(3)
    v, k = 9, 128
    codes = rng.integers(0, 16, size=(v, k)).astype(np.float32)
    s = O.bf16_round(rng.uniform(0.001, 0.02, (v, k // 64)).astype(np.float32))
    b = O.bf16_round(0.05 * rng.standard_normal((v, k // 64)).astype(np.float32))
    tokens = np.array([[3, 0, 8], [8, 8, 1]])
    gathered = O.dequantize_f32(codes[tokens.reshape(-1)].reshape(-1, 2, 64),
                                s[tokens.reshape(-1)][..., None],
                                b[tokens.reshape(-1)][..., None])
    table = O.dequantize_f32(codes.reshape(v, 2, 64), s[..., None],
                             b[..., None])
    got = O.embed(table, tokens)
    assert got.shape == (2, 3, k)
    assert np.array_equal(got.reshape(-1, k), gathered)
    # identity gather, and clamping of indices outside [0, V)
    assert np.array_equal(O.embed(table, np.arange(v)), table)
    assert np.array_equal(O.embed(table, [-5, v, 10 ** 6]),
                          table[[0, v - 1, v - 1]])
