"""Shared helpers for the GPU parity tests: operand construction in the
reference's steel-test style (metal_pjrt/blas/steel_gemm_test.cc:111-125)
and tolerance checks."""

import numpy as np
import torch

import oracle as O

TORCH = {"float32": torch.float32, "float16": torch.float16,
         "bfloat16": torch.bfloat16}

# Steel test epsilon of the output type (steel_gemm_test.cc:68-75).
EPS = {"float32": 1e-5, "float16": 1.0 / 1024, "bfloat16": 1.0 / 128}


def to_dev(values, dtype, dev):
    """float values (already representable in `dtype`) -> device tensor."""
    return torch.tensor(np.asarray(values, np.float32)).to(TORCH[dtype]).to(dev)


def from_dev(t):
    return t.float().cpu().numpy().astype(np.float64)


def rand_values(rng, n, dtype, lo=-1.0, hi=1.0):
    return O.round_to(rng.uniform(lo, hi, n), dtype)


class StoredMatrix:
    """A strided operand as the steel test allocates it: rows x cols per
    batch with `pad` extra elements per stored row, exactly sized (no
    padding after the last row), batch stride 0 when broadcast."""

    def __init__(self, rng, rows, cols, pad, batches, dtype, broadcast=False):
        self.rows, self.cols = rows, cols
        self.ld = cols + pad
        self.stride = 0 if broadcast else rows * self.ld
        nb = 1 if broadcast else batches
        self.elems = max(1, (nb - 1) * self.stride +
                         ((rows - 1) * self.ld + cols if rows > 0 else 0))
        self.values = rand_values(rng, self.elems, dtype)
        self.batches = batches

    def matrix(self, b):
        """The stored rows x cols matrix of batch b (float64)."""
        base = b * self.stride
        out = np.zeros((self.rows, self.cols))
        for i in range(self.rows):
            s = base + i * self.ld
            out[i] = self.values[s:s + self.cols]
        return out
