"""The BlasLt matmul plan, mirroring the reference's MetalBlasLt interface.

Reference: metal_pjrt/blas/metal_blas.h:51-104 (GetMatmulPlan /
MatmulPlan::ExecuteOnStream), metal_pjrt/blas/blas_lt_support.{h,cc}
(ValidateMatmul, epilogue semantics). A plan is created from a GemmConfig
of four MatrixLayouts plus alpha/beta and an Epilogue, then executed on a
stream with MemoryArgs (device buffers). Validation and the kernels are in
libqkern.so; this module only marshals.
"""

import ctypes
import enum

from . import _lib
from ._lib import check, lib


class Order(enum.IntEnum):
    kRowMajor = 0
    kColumnMajor = 1


class Epilogue(enum.IntEnum):
    """gpu::BlasLt::Epilogue names (values are the C ABI's own)."""
    kDefault = 0
    kReLU = 1
    kBias = 2
    kBiasThenReLU = 3
    kGELU = 4
    kGELUWithAux = 5
    kBiasThenGELU = 6
    kBiasThenGELUWithAux = 7
    kSILU = 8
    kSILUWithAux = 9
    kBiasThenSILU = 10
    kBiasThenSILUWithAux = 11


_DT = {"float32": _lib.F32, "float16": _lib.F16, "bfloat16": _lib.BF16}


def dtype_code(dtype):
    """qk_dtype of a torch/numpy dtype or name ('float32', 'bfloat16' ...)."""
    name = str(dtype).replace("torch.", "")
    if name not in _DT:
        raise ValueError(f"unsupported GEMM dtype {dtype}")
    return _DT[name]


class MatrixLayout:
    """gpu::MatrixLayout: dtype, rows, cols, order, batch, ld, batch stride.

    Defaults follow XLA: ld is the row length of the stored order and the
    batch stride is rows*cols.
    """

    def __init__(self, dtype, num_rows, num_cols, order=Order.kRowMajor,
                 batch_size=1, leading_dim_stride=None, batch_stride=None,
                 transpose=False):
        self.dtype = dtype_code(dtype) if not isinstance(dtype, int) else dtype
        self.num_rows = int(num_rows)
        self.num_cols = int(num_cols)
        self.order = Order(order)
        self.batch_size = int(batch_size)
        if leading_dim_stride is None:
            leading_dim_stride = (num_cols if self.order == Order.kRowMajor
                                  else num_rows)
        if batch_stride is None:
            batch_stride = num_rows * num_cols
        self.leading_dim_stride = int(leading_dim_stride)
        self.batch_stride = int(batch_stride)
        self.transpose = bool(transpose)

    def to_c(self):
        return _lib.MatrixLayoutC(self.dtype, int(self.order), self.num_rows,
                                  self.num_cols, self.batch_size,
                                  self.leading_dim_stride, self.batch_stride,
                                  int(self.transpose), 0)


class GemmConfig:
    """gpu::GemmConfig fields the plan reads: D = alpha*A*B + beta*C."""

    def __init__(self, lhs_layout, rhs_layout, c_layout, output_layout,
                 alpha=1.0, beta=0.0):
        self.lhs_layout = lhs_layout
        self.rhs_layout = rhs_layout
        self.c_layout = c_layout
        self.output_layout = output_layout
        self.alpha = complex(alpha)
        self.beta = float(beta)

    def to_c(self):
        return _lib.GemmConfigC(self.lhs_layout.to_c(), self.rhs_layout.to_c(),
                                self.c_layout.to_c(),
                                self.output_layout.to_c(), self.alpha.real,
                                self.alpha.imag, self.beta)


def _ptr_size(t):
    if t is None:
        return None, 0
    return t.data_ptr(), t.numel() * t.element_size()


class MemoryArgs:
    """gpu::BlasLt::MemoryArgs: device tensors a, b, c, d, bias, aux."""

    def __init__(self, a, b, c=None, d=None, bias=None, aux=None):
        self.a, self.b, self.c, self.d = a, b, c, d
        self.bias, self.aux = bias, aux

    def to_c(self):
        vals = []
        for t in (self.a, self.b, self.c, self.d, self.bias, self.aux):
            vals.extend(_ptr_size(t))
        return _lib.MemoryArgsC(*vals)


def stream_handle(stream):
    """hipStream_t of a torch stream (None: torch's current stream)."""
    import torch
    if stream is None:
        if not torch.cuda.is_available():
            return None  # host-only calls (argument checks) launch nothing
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


class MatmulPlan:
    """An immutable plan (MetalBlasLt::MatmulPlan)."""

    def __init__(self, handle):
        self._h = handle
        self._destroy = lib().qk_gemm_plan_destroy  # outlives module teardown

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._destroy(h)
            self._h = None

    def describe(self):
        return lib().qk_gemm_plan_describe(self._h).decode()

    def execute_on_stream(self, stream, args):
        """Runs D = act(alpha*A*B + beta*C + bias) on `stream` (torch stream
        or None for the current one). Raises QkError on failure."""
        margs = args.to_c()
        check(lib().qk_gemm_execute(self._h, stream_handle(stream),
                                    ctypes.byref(margs)))

    # Same spelling as the reference's C++ method.
    ExecuteOnStream = execute_on_stream


class BlasLt:
    """MetalBlasLt::GetMatmulPlan."""

    @staticmethod
    def get_matmul_plan(cfg, epilogue=Epilogue.kDefault):
        c = cfg.to_c()
        h = ctypes.c_void_p()
        check(lib().qk_gemm_plan_create(ctypes.byref(c), int(epilogue),
                                        ctypes.byref(h)))
        return MatmulPlan(h)

    GetMatmulPlan = get_matmul_plan


def matmul(a, b, bias=None, epilogue=None, out_dtype=None, stream=None,
           alpha=1.0):
    """Convenience: row-major (batched) D = act(alpha*a @ b + bias).

    a [..., m, k], b [k, n] or [..., k, n] (torch device tensors, contiguous,
    one dtype). The epilogue defaults to kBias when bias is given.
    """
    import torch
    if epilogue is None:
        epilogue = Epilogue.kBias if bias is not None else Epilogue.kDefault
    out_dtype = out_dtype or a.dtype
    m, k = a.shape[-2:]
    n = b.shape[-1]
    batch = 1
    for s in a.shape[:-2]:
        batch *= s
    a_bs = m * k if batch > 1 else 0
    b_batch = 1
    for s in b.shape[:-2]:
        b_batch *= s
    lhs = MatrixLayout(a.dtype, m, k, Order.kRowMajor, batch, k, a_bs)
    rhs = MatrixLayout(b.dtype, k, n, Order.kRowMajor, b_batch, n,
                       k * n if b_batch > 1 else 0)
    out = MatrixLayout(out_dtype, m, n, Order.kRowMajor, batch, n, m * n)
    d = torch.empty(*a.shape[:-2], m, n, dtype=out_dtype, device=a.device)
    aux = None
    if epilogue in (Epilogue.kGELUWithAux, Epilogue.kBiasThenGELUWithAux,
                    Epilogue.kSILUWithAux, Epilogue.kBiasThenSILUWithAux):
        aux = torch.empty_like(d)
    plan = BlasLt.get_matmul_plan(GemmConfig(lhs, rhs, out, out, alpha, 0.0),
                                  epilogue)
    plan.execute_on_stream(stream, MemoryArgs(a, b, None, d, bias, aux))
    return (d, aux) if aux is not None else d
