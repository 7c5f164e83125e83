"""GPU parity of qk$rownorm (rownorm.hip) against the float64 oracle.

Tolerances: 1e-5 for f32 and 8e-3 for bf16 (2e-3 for f16),
relative to each element, with a floor of tol * 1e-3 * max|row| for
elements near zero. Shapes cover one element, ragged and unaligned rows,
the register kernels' size classes, rows long enough for the looping
kernel, and the [4096, 4096] configs.
"""

import numpy as np
import pytest
import torch

import oracle as O
import qkern
from qkern.ffi import RownormKind
from helpers import TORCH

pytestmark = pytest.mark.gpu

TOL = {"float32": 1e-5, "bfloat16": 8e-3, "float16": 2e-3}


def check(got, want, dtype, beta=None, extra=None):
    """extra: magnitude of intermediate terms whose rounding reaches the
    output (layer norm: (|x| + |mean|) / std * |gain|, since x - mean
    carries the rounding error of the mean)."""
    tol = TOL[dtype]
    floor = tol * 1e-3 * np.max(np.abs(want), axis=-1, keepdims=True)
    err = np.abs(got - want)
    # with a layer-norm offset the output's error scales with the terms
    # that are added, not with their (possibly cancelling) sum
    mag = np.abs(want) if beta is None else \
        np.abs(want - beta) + np.abs(beta)
    if extra is not None:
        mag = mag + extra
    # f16 outputs below 2^-14 are subnormal: one subnormal step is 2^-24
    sub = 2.0 ** -24 if dtype == "float16" else 0.0
    bound = tol * mag + floor + sub
    assert np.all(err <= bound), float(np.max(err / np.maximum(bound, 1e-30)))


def run(dev, kind, x, dtype, gain=None, beta=None, eps=1e-6, pdtype=None):
    """pdtype: storage type of gain and beta (default float32); the oracle
    gets the stored values."""
    dx = torch.from_numpy(x.astype(np.float32)).to(TORCH[dtype]).to(dev)
    xr = dx.float().cpu().numpy().astype(np.float64)  # values as stored
    pt = TORCH[pdtype or "float32"]
    dg = None if gain is None else torch.from_numpy(gain).to(pt).to(dev)
    dbeta = None if beta is None else torch.from_numpy(beta).to(pt).to(dev)
    gain = None if gain is None else dg.float().cpu().numpy()
    beta = None if beta is None else dbeta.float().cpu().numpy()
    y = qkern.rownorm(dx, kind, eps=eps, gain=dg, beta=dbeta)
    torch.cuda.synchronize()
    got = y.float().cpu().numpy().astype(np.float64)
    if kind == RownormKind.RMS:
        want = O.rms_norm(xr, gain, eps)
    elif kind == RownormKind.LAYER:
        want = O.layer_norm(xr, eps, gain, beta)
        mu = xr.mean(axis=-1, keepdims=True)
        inv = 1.0 / np.sqrt(((xr - mu) ** 2).mean(axis=-1, keepdims=True) + eps)
        extra = (np.abs(xr) + np.abs(mu)) * inv * \
            (1.0 if gain is None else np.abs(gain))
    else:
        want = O.softmax(xr)
    # compare against the oracle rounded once to the output type
    check(got, O.round_to(want, dtype) if dtype != "float32" else want, dtype,
          beta, extra if kind == RownormKind.LAYER else None)


SHAPES = [(1, 1), (3, 7), (5, 64), (7, 1000), (2, 129), (4, 4096),
          (3, 8192), (2, 16384), (2, 50000), (9, 33000)]


@pytest.mark.parametrize("kind", list(RownormKind))
@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
def test_rownorm_shapes(dev, kind, dtype):
    rng = np.random.default_rng(int(kind))
    for rows, n in SHAPES:
        x = rng.standard_normal((rows, n)) * (2.0 if kind == 2 else 1.0) + 0.3
        gain = beta = None
        if kind != RownormKind.SOFTMAX:
            gain = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        if kind == RownormKind.LAYER:
            beta = (0.1 * rng.standard_normal(n)).astype(np.float32)
        run(dev, kind, x, dtype, gain, beta, 1e-6 if kind == 0 else 1e-5)


@pytest.mark.parametrize("kind", list(RownormKind))
@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
def test_rownorm_many_rows(dev, kind, dtype):
    """Enough rows for the persistent streaming kernel (several rows per
    wave, a ragged last round), for each register size class (rows of up
    to 16 vectors per lane shared by two waves; 16-bit layer norm rows of
    up to 8 vectors per lane on two waves of 4), with gains and offsets of
    the row type and of f32."""
    rng = np.random.default_rng(10 + int(kind))
    cases = [(4099, 1000, "float32"), (4101, 4096, dtype),
             (4097, 8192 if dtype != "float32" else 4104, "float32"),
             # two waves per row with a partly filled second half
             (4103, 3000 if dtype == "float32" else 6000, dtype),
             # 16-bit layer norm: two waves of four vectors per lane
             (4099, 2500, dtype)]
    for rows, n, pdtype in cases:
        x = rng.standard_normal((rows, n)) * (2.0 if kind == 2 else 1.0) + 0.3
        gain = beta = None
        if kind != RownormKind.SOFTMAX:
            gain = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        if kind == RownormKind.LAYER:
            beta = (0.1 * rng.standard_normal(n)).astype(np.float32)
        run(dev, kind, x, dtype, gain, beta, 1e-6 if kind == 0 else 1e-5,
            pdtype)


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_layer_norm_packed_parameters(dev, dtype):
    """16-bit layer norm rows of up to 8 vectors per lane whose gain and
    offset are absent (the reference's layernorm, bench/jax_bench.py:44-46)
    or of the row's type, singly or together: one wave per row with the
    parameters held packed (a partly filled last vector per lane at
    n = 3000)."""
    rng = np.random.default_rng(77)
    for n in (4096, 3000):
        x = rng.standard_normal((4100, n)) + 0.3
        gain = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        beta = (0.1 * rng.standard_normal(n)).astype(np.float32)
        for g, b in ((None, None), (gain, None), (None, beta), (gain, beta)):
            run(dev, RownormKind.LAYER, x, dtype, g, b, 1e-5, dtype)


def test_rownorm_no_gain_and_leading_dims(dev):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 3, 5, 96))
    run(dev, RownormKind.RMS, x, "float32")
    run(dev, RownormKind.LAYER, x, "bfloat16", eps=1e-5)
    run(dev, RownormKind.SOFTMAX, x, "float32")


def test_rownorm_special_rows(dev):
    # constant rows: RMS gives sign * gain, layer norm gives 0, softmax 1/n
    x = np.full((2, 512), -3.0)
    x[1] = 2.5
    g = np.linspace(0.5, 1.5, 512).astype(np.float32)
    run(dev, RownormKind.RMS, x, "float32", gain=g, eps=0.0)
    run(dev, RownormKind.SOFTMAX, x, "float32")
    # huge logits: softmax stays finite (max subtraction)
    x = np.array([[1000.0, 999.0, -1000.0] * 100])
    run(dev, RownormKind.SOFTMAX, x, "float32")
    # -inf (masked) entries get probability 0
    x = np.zeros((1, 256))
    x[0, ::2] = -np.inf
    dx = torch.from_numpy(x.astype(np.float32)).to(dev)
    y = qkern.softmax(dx).cpu().numpy()
    assert np.all(y[0, ::2] == 0) and np.allclose(y[0, 1::2], 1 / 128)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_config_rmsnorm_4096(dev, dtype):
    rng = np.random.default_rng(0)
    x = rng.standard_normal((4096, 4096)).astype(np.float32)
    g = (1 + 0.1 * np.random.default_rng(1).standard_normal(4096)).astype(
        np.float32)
    run(dev, RownormKind.RMS, x, dtype, gain=g, eps=1e-6)


def test_config_softmax_4096(dev):
    x = 2.0 * np.random.default_rng(2).standard_normal((4096, 4096))
    run(dev, RownormKind.SOFTMAX, x, "float32")
