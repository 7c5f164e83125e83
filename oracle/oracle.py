"""CPU oracle for the qkern hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker (or the timed CPU baseline),
never as a product path.

Each function restates the reference's algorithm (file:line cited) in
numpy, float64 where the reference's semantics is a real-number value and
in the reference's own float32 steps where bits matter. How each one is
pinned (tests/test_oracle.py):

  bf16_round            bit patterns of hand-picked values (ties, NaN, inf,
                        subnormals) and torch's RNE cast.
  act_*                 closed forms: relu(NaN) is NaN, gelu/silu special
                        values, odd/even identities, math.erf-free limits.
  gemm_ref              brute-force triple loop on tiny shapes; the
                        reference gtest's exact-product inputs
                        (metal_blas_lt_test.cc:125-130) give integer-exact
                        results.
  quantize_int4         brute force over all 16-level grids on tiny groups:
                        every weight lands within s/2 of its code, zero is
                        on the grid when q0 != 0, codes within 0..15.
  quantize_int8         |w - q s| <= s/2, max |q| == 127 per group.
  pack_* / unpack_*     round trips and hand-computed bit patterns.
  dequantize            closed form s*q + b on exact cases (power-of-two
                        scales) and brute force against float64.
  matvec_*              float64 dot product of the dequantized matrix vs
                        the reference's per-group factoring (exact identity).
  rms_norm/layer_norm/  invariants: constant rows, softmax sums to 1 and
  softmax               is shift invariant, layernorm mean 0 / var 1.

Parity unpinned (no reference golden vectors exist; JAX is not installed):
the bitwise behaviour of XLA:CPU's bf16 dequantize rounding sequence and
its reduction order. The canonical dequant rounding is fixed here as
bf16(f32(f32(q)*f32(s)) + f32(b)).
"""

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))

# ---------------------------------------------------------------------------
# bf16 / f16 rounding.


def bf16_bits(x):
    """Round-to-nearest-even float32 -> bf16 bit patterns (uint16); NaN
    stays a quiet NaN."""
    f = np.ascontiguousarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16).astype(np.uint32)
    r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint32), r)
    return r.astype(np.uint16)


def bf16_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(
        np.float32)


def bf16_round(x):
    """float32 values of round-to-nearest-even bf16(x)."""
    return bf16_to_f32(bf16_bits(x))


def round_to(x, dtype):
    """Round float64/float32 values to 'float32' | 'float16' | 'bfloat16'
    (returned as float64)."""
    x32 = np.asarray(x, dtype=np.float64).astype(np.float32)
    if dtype == "float32":
        return x32.astype(np.float64)
    if dtype == "float16":
        return x32.astype(np.float16).astype(np.float64)
    if dtype == "bfloat16":
        return bf16_round(x32).astype(np.float64)
    raise ValueError(dtype)


# ---------------------------------------------------------------------------
# GEMM with the cuBLASLt epilogue.
# Reference: metal_pjrt/blas/blas_lt_support.h:20-38 (semantics),
# kernels/steel_gemm.metal:57-66 and 215-225 (activations, one rounding),
# metal_blas.cc:133-171 (f32 second pass: same formulas).

GELU_K = 0.7978845608028654  # sqrt(2/pi)


def act_relu(x):
    x = np.asarray(x, dtype=np.float64)
    return np.where(np.isnan(x), x, np.where(x > 0, x, 0.0))


def act_gelu(x):
    x = np.asarray(x, dtype=np.float64)
    return 0.5 * x * (1.0 + np.tanh(GELU_K * (x + 0.044715 * x * x * x)))


def act_silu(x):
    x = np.asarray(x, dtype=np.float64)
    with np.errstate(over="ignore"):
        return x / (1.0 + np.exp(-x))


ACTS = {0: lambda x: np.asarray(x, dtype=np.float64), 1: act_relu,
        2: act_gelu, 3: act_silu}

# Epilogue id (qkern.Epilogue order) -> (bias, act, aux); reference
# DecodeEpilogue, metal_pjrt/blas/blas_lt_support.cc:25-83.
EPILOGUES = {
    0: (False, 0, False), 1: (False, 1, False), 2: (True, 0, False),
    3: (True, 1, False), 4: (False, 2, False), 5: (False, 2, True),
    6: (True, 2, False), 7: (True, 2, True), 8: (False, 3, False),
    9: (False, 3, True), 10: (True, 3, False), 11: (True, 3, True),
}


def gemm_ref(a, b, c=None, bias=None, alpha=1.0, beta=0.0, act=0):
    """Row-major (batched) v = alpha*a@b + beta*c + bias[col], returned as
    (act(v), v) in float64. Inputs are taken at their stored values (pass
    arrays already rounded to the operand dtype)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    v = alpha * np.matmul(a, b)
    if c is not None and beta != 0.0:
        v = v + beta * np.asarray(c, dtype=np.float64)
    if bias is not None:
        v = v + np.asarray(bias, dtype=np.float64)
    return ACTS[act](v), v


def gemm_bruteforce(a, b):
    """Triple loop in float64 for tiny 2-D shapes (pins gemm_ref)."""
    m, k = a.shape
    n = b.shape[1]
    out = np.zeros((m, n), dtype=np.float64)
    for i in range(m):
        for j in range(n):
            s = 0.0
            for t in range(k):
                s += float(a[i, t]) * float(b[t, j])
            out[i, j] = s
    return out


def rel_fro(got, want):
    """Relative Frobenius error ||got - want|| / ||want||."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    den = np.linalg.norm(want)
    return float(np.linalg.norm(got - want) / (den if den > 0 else 1.0))


# ---------------------------------------------------------------------------
# Quantizers and packings. Reference: examples/llm/qwen3.py:151-207.

GROUP = 64


def quantize_int8(w, group=GROUP):
    """Symmetric int8 per `group` inputs (qwen3.py:154-166), float32 steps.
    Returns q int8 [N, K/g, g] and s float32 [N, K/g, 1]."""
    w32 = np.asarray(w, dtype=np.float32).reshape(np.shape(w)[0], -1, group)
    amax = np.abs(w32).max(axis=-1, keepdims=True)
    s = np.maximum(amax, np.float32(1e-12)) / np.float32(127.0)
    q = np.clip(np.rint(w32 / s), -127, 127).astype(np.int8)
    return q, s.astype(np.float32)


def quantize_int4(w, group=GROUP):
    """Affine 4-bit grid anchored at the largest-magnitude weight
    (qwen3.py:169-196: MLX's affine_quantize), float32 steps.
    Returns codes uint8 [N, K/g, g] (0..15, unpacked), s and b float32
    [N, K/g, 1]."""
    w32 = np.asarray(w, dtype=np.float32).reshape(np.shape(w)[0], -1, group)
    lo = w32.min(axis=-1, keepdims=True)
    hi = w32.max(axis=-1, keepdims=True)
    neg = np.abs(lo) > np.abs(hi)
    step = np.maximum(hi - lo, np.float32(1e-12)) / np.float32(15.0)
    step = np.where(neg, step, -step).astype(np.float32)
    edge = np.where(neg, lo, hi).astype(np.float32)
    q0 = np.rint(edge / step)
    nz = q0 != 0
    step = np.where(nz, edge / np.where(nz, q0, np.float32(1.0)), step)
    step = step.astype(np.float32)
    off = np.where(nz, edge, np.float32(0.0)).astype(np.float32)
    codes = np.clip(np.rint((w32 - off) / step), 0, 15).astype(np.uint8)
    return codes, step, off


def pack_halfsplit(codes, group=GROUP):
    """codes [N, K/g, g] (0..15) -> bytes [N, K/g, g/2]: element j in the low
    nibble of byte j, element j + g/2 in its high nibble (qwen3.py:195)."""
    c = np.asarray(codes, dtype=np.uint8).reshape(np.shape(codes)[0], -1,
                                                  group)
    half = group // 2
    return (c[..., :half] | (c[..., half:] << 4)).astype(np.uint8)


def unpack_halfsplit(p):
    """bytes [N, K/g, g/2] -> codes [N, K/g, g] (qwen3.py:202)."""
    p = np.asarray(p, dtype=np.uint8)
    return np.concatenate([p & 0xF, p >> 4], axis=-1)


def pack_u32x8(codes):
    """codes [N, K] (0..15) -> uint32 [N, K/8]; element 8i+j in bits
    4j..4j+3 of word i."""
    # byte t of a little-endian word holds elements 2t (bits 8t..8t+3) and
    # 2t+1 (bits 8t+4..8t+7)
    c = np.asarray(codes, dtype=np.uint8).reshape(np.shape(codes)[0], -1)
    pairs = np.ascontiguousarray(c[:, 0::2] | (c[:, 1::2] << 4))
    return pairs.view("<u4").astype(np.uint32, copy=False)


def unpack_u32x8(words):
    """uint32 [N, K/8] -> codes uint8 [N, K]."""
    w = np.asarray(words, dtype=np.uint32)[..., None]
    shifts = (4 * np.arange(8, dtype=np.uint32))
    return ((w >> shifts) & 0xF).astype(np.uint8).reshape(w.shape[0], -1)


def dequantize_f32(q, s, b=None):
    """f32(f32(q)*f32(s)) + f32(b) per element (unfused float32 steps).
    q [N, K/g, g] numbers, s/b [N, K/g, 1] float32 values. Returns float32
    [N, K]."""
    q32 = np.asarray(q).astype(np.float32)
    w = (q32 * np.asarray(s, dtype=np.float32)).astype(np.float32)
    if b is not None:
        w = (w + np.asarray(b, dtype=np.float32)).astype(np.float32)
    return w.reshape(w.shape[0], -1)


def dequantize_bf16_bits(q, s, b=None):
    """Canonical bf16 dequant bits: bf16(f32(f32(q)*f32(s)) + f32(b))."""
    return bf16_bits(dequantize_f32(q, s, b))


def matvec_f64(x, w):
    """sum_k x[m,k] w[o,k] in float64 (x [M, K], w [N, K] float values)."""
    return np.asarray(x, dtype=np.float64) @ np.asarray(w,
                                                        dtype=np.float64).T


def matvec_int4_reference_form(x, packed, s, b):
    """_matvec_int4 (qwen3.py:243-267) in float32: per byte,
    (x_lo*lo + x_hi*hi)*s + (x_lo + x_hi)*b, summed over groups and bytes.
    x [M, K] float32 values; packed [N, K/g, g/2] (half-split bytes);
    s, b [N, K/g, 1] float32."""
    p = np.asarray(packed, dtype=np.uint8)
    n, groups, half = p.shape
    xg = np.asarray(x, dtype=np.float32).reshape(-1, 1, groups, 2, half)
    lo = (p & 0xF).astype(np.float32)
    hi = (p >> 4).astype(np.float32)
    xlo, xhi = xg[:, :, :, 0], xg[:, :, :, 1]
    s32 = np.asarray(s, dtype=np.float32)
    b32 = np.asarray(b, dtype=np.float32)
    t = (xlo * lo + xhi * hi) * s32 + (xlo + xhi) * b32
    return t.sum(axis=(2, 3), dtype=np.float32)


def matvec_int8_reference_form(x, q, s):
    """_matvec_int8 (qwen3.py:233-240) in float32: sum x*q*s."""
    q = np.asarray(q)
    n, groups, g = q.shape
    xg = np.asarray(x, dtype=np.float32).reshape(-1, 1, groups, g)
    t = xg * q.astype(np.float32) * np.asarray(s, dtype=np.float32)
    return t.sum(axis=(2, 3), dtype=np.float32)


# ---------------------------------------------------------------------------
# Row normalisation. Reference: qwen3.py:294-297 (rms_norm), jax.nn.softmax
# (qwen3.py:325,330), bench/jax_bench.py:44-46 (layernorm: biased variance).


def embed(table, tokens):
    """qwen3.embed (examples/llm/qwen3.py:270-274): the rows of `table`
    picked by `tokens`, shaped [*tokens.shape, K]. For a quantized table the
    reference gathers the q4/q, s and b rows and dequantizes them
    (qwen3.py:271); dequantization is per row, so that equals the rows of
    the dequantized table, which is what `table` is here. Indices outside
    [0, V) are clamped, as a JAX gather clamps them."""
    table = np.asarray(table)
    idx = np.clip(np.asarray(tokens, np.int64), 0, table.shape[0] - 1)
    return table[idx.reshape(-1)].reshape(*np.shape(tokens), table.shape[1])


def rms_norm(x, w=None, eps=1e-6):
    x = np.asarray(x, dtype=np.float64)
    y = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    if w is not None:
        y = y * np.asarray(w, dtype=np.float64)
    return y


def layer_norm(x, eps=1e-5, gain=None, beta=None):
    x = np.asarray(x, dtype=np.float64)
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    y = (x - mu) / np.sqrt(var + eps)
    if gain is not None:
        y = y * np.asarray(gain, dtype=np.float64)
    if beta is not None:
        y = y + np.asarray(beta, dtype=np.float64)
    return y


def softmax(x):
    x = np.asarray(x, dtype=np.float64)
    e = np.exp(x - x.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def decode_attention(q, k, v, pos, scale, window=None):
    """The one-query branch of qwen3.attention (examples/llm/qwen3.py:
    322-326) with forward()'s decode mask (qwen3.py:357-358), in float64:
    q [B, KV, G, D], k [B, KV, Smax, D], v [B, KV, D, Smax]; slots
    s < window (default Smax) with s <= pos are attended:
      t = scale * q.k,  p = softmax(t over attended slots),  o = p.v
    Returns [B, KV, G, D]."""
    q = np.asarray(q, dtype=np.float64)
    S = window or np.shape(k)[2]
    k = np.asarray(k, dtype=np.float64)[:, :, :S]
    v = np.asarray(v, dtype=np.float64)[..., :S]
    t = np.einsum("bkgd,bksd->bkgs", q, k) * scale
    t = np.where(np.arange(S) <= pos, t, -np.inf)
    with np.errstate(invalid="ignore"):
        p = softmax(t)
    return np.einsum("bkgs,bkds->bkgd", p, v)


# ---------------------------------------------------------------------------
# Seeded inputs of the benchmark configs (numpy default_rng(seed)).


def config_gemm_f32(seed=0, n=1024):
    r = np.random.default_rng(seed)
    return (r.standard_normal((n, n), dtype=np.float32),
            r.standard_normal((n, n), dtype=np.float32))


def config_affine(n, k, group=GROUP, bits=4, seed=0):
    """Codes uniform over the full range, scale U(0.001, 0.02) and bias
    N(0, 0.05) per group, both rounded to bf16 (float32 values)."""
    r = np.random.default_rng(seed)
    hi = 16 if bits == 4 else 256
    codes = r.integers(0, hi, size=(n, k), dtype=np.uint8)
    s = bf16_round(r.uniform(0.001, 0.02, size=(n, k // group)).astype(
        np.float32))
    b = bf16_round((0.05 * r.standard_normal((n, k // group))).astype(
        np.float32))
    return codes, s, b


# ---------------------------------------------------------------------------
# C port (oracle/qk_oracle.c): the matvecs in the reference's float32
# form, multithreaded; the CPU baseline of the benchmark.

_clib = None


def clib():
    global _clib
    if _clib is None:
        path = os.path.join(_HERE, "_build", "libqk_oracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run make -C oracle")
        l = ctypes.CDLL(path)
        vp, i64 = ctypes.c_void_p, ctypes.c_int64
        l.qo_matvec_int4_u32x8.argtypes = [vp, vp, vp, vp, vp, vp, i64, i64,
                                          i64, ctypes.c_int, ctypes.c_int]
        l.qo_matvec_int4_u32x8.restype = None
        l.qo_matvec_u8.argtypes = [vp, vp, vp, vp, vp, vp, i64, i64, i64,
                                   ctypes.c_int, ctypes.c_int]
        l.qo_matvec_u8.restype = None
        l.qo_num_threads.restype = ctypes.c_int
        l.qo_num_threads.argtypes = [ctypes.c_int]
        _clib = l
    return _clib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def c_matvec_int4_u32x8(x_bf16_bits, words, s_bits, b_bits, group=GROUP,
                        threads=0, with_mag=False):
    """y (float32 [M, N]) = sum over groups of s*sum(x q) + b*sum(x) with
    bf16 inputs given as uint16 bit arrays; words uint32 [N, K/8]. With
    `with_mag`, returns (y, mag) where mag[m, o] = sum_k |x||s q + b|
    (float64), the scale of an f32 product's rounding error."""
    x = np.ascontiguousarray(x_bf16_bits, dtype=np.uint16)
    w = np.ascontiguousarray(words, dtype=np.uint32)
    s = np.ascontiguousarray(s_bits, dtype=np.uint16)
    b = np.ascontiguousarray(b_bits, dtype=np.uint16)
    m, k = x.shape
    n = w.shape[0]
    y = np.zeros((m, n), dtype=np.float32)
    mag = np.zeros((m, n), dtype=np.float64) if with_mag else None
    clib().qo_matvec_int4_u32x8(_ptr(x), _ptr(w), _ptr(s), _ptr(b), _ptr(y),
                                None if mag is None else _ptr(mag),
                                m, n, k, group, threads)
    return (y, mag) if with_mag else y


def c_matvec_u8(x_bf16_bits, codes, s_bits, b_bits, group=GROUP, threads=0,
                with_mag=False):
    """As c_matvec_int4_u32x8 for affine uint8 codes [N, K]."""
    x = np.ascontiguousarray(x_bf16_bits, dtype=np.uint16)
    c = np.ascontiguousarray(codes, dtype=np.uint8)
    s = np.ascontiguousarray(s_bits, dtype=np.uint16)
    b = np.ascontiguousarray(b_bits, dtype=np.uint16)
    m, k = x.shape
    n = c.shape[0]
    y = np.zeros((m, n), dtype=np.float32)
    mag = np.zeros((m, n), dtype=np.float64) if with_mag else None
    clib().qo_matvec_u8(_ptr(x), _ptr(c), _ptr(s), _ptr(b), _ptr(y),
                        None if mag is None else _ptr(mag), m, n, k, group,
                        threads)
    return (y, mag) if with_mag else y


def c_threads(requested=0):
    """Threads the C port uses for `requested` (0: all available)."""
    return clib().qo_num_threads(requested)


