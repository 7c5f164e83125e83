"""qkern: the MI355X (gfx950) hot path of the metal-pjrt-plugin JAX plugin.

Three kernel families behind a C ABI (include/qkern.h, libqkern.so):
  - blas:  BlasLt matmul plans, f32/f16/bf16 with the cuBLASLt epilogue;
  - ffi:   qk$qmatvec / qk$dequantize (int4 / int8 group-affine weights)
           qk$rownorm (RMSNorm, LayerNorm, softmax) and
           qk$decode_attention (one query against the KV cache);
  - quant: host-side quantizers and packers for the weight formats;
  - weights: safetensors reading and quantization on the device
           (qk_quantize).
Every compute call runs a HIP kernel; there is no CPU fallback.
"""

from ._lib import QkError, lib  # noqa: F401
from .blas import (BlasLt, Epilogue, GemmConfig, MatmulPlan,  # noqa: F401
                   MatrixLayout, MemoryArgs, Order, matmul)
from .ffi import (Packing, RownormKind, decode_attention,  # noqa: F401
                  decode_attention_noalloc,
                  decode_attention_workspace_size, dequantize, embed,
                  layer_norm,
                  qmatvec, quantize, rms_norm, rownorm, softmax)
from .weights import load_quantized, read_safetensors  # noqa: F401


def version():
    return lib().qk_version().decode()


def device_error():
    """0, or the sticky device error code."""
    return lib().qk_device_error()


def reset_device_error():
    lib().qk_reset_device_error()
