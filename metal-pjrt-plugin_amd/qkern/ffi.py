"""Typed-FFI style targets: qk$qmatvec, qk$dequantize, qk$rownorm,
qk$decode_attention.

The reference has no custom-call target for these (XLA fuses the JAX code
of examples/llm/qwen3.py into reduction kernels). They follow the
reference's convention for a new target (metal_pjrt/ffi/scan_ffi.cc:
112-133): operands then results as FFI AnyBuffers (data, element type,
dimensions), then attributes. Buffers here are torch device tensors.
"""

import ctypes
import enum

import torch

from . import _lib
from ._lib import check, lib
from .blas import stream_handle


class Packing(enum.IntEnum):
    U32X8 = 0            # 4-bit, 8 codes per uint32 along K
    BYTE_HALFSPLIT = 1   # 4-bit, qwen3.quantize_int4's byte layout
    U8 = 2               # 8-bit unsigned affine
    S8_SYM = 3           # 8-bit signed symmetric (qwen3.quantize_int8)


class RownormKind(enum.IntEnum):
    RMS = 0
    LAYER = 1
    SOFTMAX = 2


_TORCH_DT = {
    torch.float32: _lib.F32, torch.float16: _lib.F16,
    torch.bfloat16: _lib.BF16, torch.uint8: _lib.U8, torch.int8: _lib.S8,
    torch.int32: _lib.U32, torch.uint32: _lib.U32,
}


def any_buffer(t):
    """An FFI AnyBuffer descriptor of a contiguous torch tensor (or None)."""
    if t is None:
        return None
    if not t.is_contiguous():
        raise ValueError("qkern buffers must be contiguous")
    if t.dtype not in _TORCH_DT:
        raise ValueError(f"unsupported buffer dtype {t.dtype}")
    if t.dim() > _lib.MAX_RANK or t.dim() == 0:
        raise ValueError(f"buffer rank {t.dim()} not in 1..{_lib.MAX_RANK}")
    b = _lib.BufferC()
    b.data = t.data_ptr()
    b.dtype = _TORCH_DT[t.dtype]
    b.rank = t.dim()
    for i, s in enumerate(t.shape):
        b.dims[i] = s
    return b


def _ref(b):
    return ctypes.byref(b) if b is not None else None


def _attrs(packing, group_size, has_bias):
    packing = Packing(packing)
    bits = 4 if packing in (Packing.U32X8, Packing.BYTE_HALFSPLIT) else 8
    return _lib.QuantAttrsC(bits, group_size, int(packing), int(bool(has_bias)))


def qmatvec(x, codes, scales, biases=None, *, packing=Packing.U32X8,
            group_size=64, out=None, stream=None):
    """qk$qmatvec: y[..., o] = sum_k x[..., k] * (scale*q + bias)[o, k].

    x [..., K] f32/f16/bf16; codes per `packing`; scales/biases [N, K/g].
    Returns y [..., N] in x's dtype.
    """
    n = codes.shape[0]
    if out is None:
        out = torch.empty(*x.shape[:-1], n, dtype=x.dtype, device=x.device)
    bx, bc, bs, bb, by = (any_buffer(t) for t in (x, codes, scales, biases,
                                                   out))
    attrs = _attrs(packing, group_size, biases is not None)
    check(lib().qk_qmatvec(stream_handle(stream), _ref(bx), _ref(bc),
                           _ref(bs), _ref(bb), _ref(by), ctypes.byref(attrs)))
    return out


def dequantize(codes, scales, biases=None, *, k, packing=Packing.U32X8,
               group_size=64, dtype=torch.bfloat16, out=None, stream=None):
    """qk$dequantize: the [N, K] weights, each f32(q)*f32(s) + f32(b)
    rounded once to `dtype`."""
    n = codes.shape[0]
    if out is None:
        out = torch.empty(n, k, dtype=dtype, device=codes.device)
    bc, bs, bb, bw = (any_buffer(t) for t in (codes, scales, biases, out))
    attrs = _attrs(packing, group_size, biases is not None)
    check(lib().qk_dequantize(stream_handle(stream), _ref(bc), _ref(bs),
                              _ref(bb), _ref(bw), ctypes.byref(attrs)))
    return out


def quantize(w, *, packing=Packing.U32X8, group_size=64,
             scale_dtype=torch.float32, stream=None):
    """qk_quantize: the codes, scales and offsets of w [N, K] (f32 / f16 /
    bf16 on the device) on the reference's grids (examples/llm/qwen3.py:
    154-196): int4 affine for U32X8 / BYTE_HALFSPLIT, symmetric int8 for
    S8_SYM. Returns (codes, scales, offsets or None) laid out as qmatvec
    takes them: U32X8 int32 [N, K/8], BYTE_HALFSPLIT uint8 [N, K/g, g/2],
    S8_SYM int8 [N, K]; scales / offsets [N, K/g] in scale_dtype."""
    packing = Packing(packing)
    n, k = w.shape
    g = group_size
    dev = w.device
    if packing == Packing.U32X8:
        codes = torch.empty(n, k // 8, dtype=torch.int32, device=dev)
    elif packing == Packing.BYTE_HALFSPLIT:
        codes = torch.empty(n, k // g, g // 2, dtype=torch.uint8, device=dev)
    else:
        codes = torch.empty(n, k, dtype=torch.int8 if packing ==
                            Packing.S8_SYM else torch.uint8, device=dev)
    scales = torch.empty(n, k // g, dtype=scale_dtype, device=dev)
    int4 = packing in (Packing.U32X8, Packing.BYTE_HALFSPLIT)
    biases = torch.empty_like(scales) if int4 else None
    bw, bc, bs, bb = (any_buffer(t) for t in (w, codes, scales, biases))
    attrs = _attrs(packing, group_size, int4)
    check(lib().qk_quantize(stream_handle(stream), _ref(bw), _ref(bc),
                            _ref(bs), _ref(bb), ctypes.byref(attrs)))
    return codes, scales, biases


def embed(table, tokens, scales=None, biases=None, *, k=None,
          packing=Packing.U32X8, group_size=64, dtype=None, out=None,
          stream=None):
    """qk$embed: qwen3.embed (examples/llm/qwen3.py:270-274), the rows of
    `table` picked by int32 `tokens`, [*tokens.shape, K]. With scales the
    table holds codes (k: the row length, required) and each row is
    dequantized to `dtype` (default: the scales' type, as the reference
    does); without, it is a dense [V, K] table copied in its own type.
    Tokens outside the table are clamped."""
    if scales is None:
        k = table.shape[1]
        dtype = table.dtype
    elif dtype is None:
        dtype = scales.dtype
    if out is None:
        out = torch.empty(*tokens.shape, k, dtype=dtype, device=table.device)
    bt, bw, bs, bb, bo = (any_buffer(t) for t in (tokens, table, scales,
                                                   biases, out))
    attrs = _attrs(packing, group_size, biases is not None)
    check(lib().qk_embed(stream_handle(stream), _ref(bt), _ref(bw), _ref(bs),
                         _ref(bb), _ref(bo), ctypes.byref(attrs)))
    return out


def rownorm(x, kind, *, eps=1e-6, gain=None, beta=None, out=None,
            stream=None):
    """qk$rownorm over the last dimension of x (RMS, LAYER or SOFTMAX)."""
    if out is None:
        out = torch.empty_like(x)
    bx, bg, bb, by = (any_buffer(t) for t in (x, gain, beta, out))
    attrs = _lib.RownormAttrsC(int(RownormKind(kind)), float(eps),
                               int(gain is not None), int(beta is not None))
    check(lib().qk_rownorm(stream_handle(stream), _ref(bx), _ref(bg),
                           _ref(bb), _ref(by), ctypes.byref(attrs)))
    return out


def rms_norm(x, w, eps):
    """qwen3.rms_norm (examples/llm/qwen3.py:294-297) on the GPU."""
    return rownorm(x, RownormKind.RMS, eps=eps, gain=w)


def softmax(x):
    """jax.nn.softmax(x, axis=-1) on the GPU."""
    return rownorm(x, RownormKind.SOFTMAX)


def layer_norm(x, eps=1e-5, gain=None, beta=None):
    """(x - mean) / sqrt(var + eps) [* gain + beta] over the last axis
    (bench/jax_bench.py:44-46 without the affine terms)."""
    return rownorm(x, RownormKind.LAYER, eps=eps, gain=gain, beta=beta)


def decode_attention_workspace_size(q, k_cache, *, scale=None, window=0):
    """Bytes of workspace qk$decode_attention takes for these shapes."""
    attrs = _attn_attrs(q, scale, window)
    n = ctypes.c_uint64()
    check(lib().qk_decode_attention_workspace_size(
        _ref(any_buffer(q)), _ref(any_buffer(k_cache)), ctypes.byref(attrs),
        ctypes.byref(n)))
    return n.value


def _attn_attrs(q, scale, window):
    if scale is None:
        scale = q.shape[-1] ** -0.5
    return _lib.AttentionAttrsC(float(scale), int(window or 0))


def decode_attention(q, k_cache, v_cache, position, *, scale=None, window=0,
                     workspace=None, out=None, stream=None):
    """qk$decode_attention: qwen3.attention for one query
    (examples/llm/qwen3.py:322-326) with the decode mask s <= position over
    cache slots s < window (0: all). q [B, KV, G, D] or [B, 1, KV, G, D],
    k_cache [B, KV, Smax, D], v_cache [B, KV, D, Smax], position an int32
    device tensor of one element. scale defaults to D ** -0.5 (the
    reference's). A workspace is allocated when none is given."""
    attrs = _attn_attrs(q, scale, window)
    if out is None:
        out = torch.empty_like(q, dtype=v_cache.dtype)
    if workspace is None:
        need = decode_attention_workspace_size(q, k_cache, scale=scale,
                                               window=window)
        workspace = torch.empty(max(need, 16), dtype=torch.uint8,
                                device=q.device)
    pos = position.reshape(1) if position.dim() == 0 else position
    bq, bk, bv, bp, bo = (any_buffer(t) for t in (q, k_cache, v_cache, pos,
                                                   out))
    check(lib().qk_decode_attention(
        stream_handle(stream), _ref(bq), _ref(bk), _ref(bv), _ref(bp),
        _ref(bo), ctypes.byref(attrs), workspace.data_ptr(),
        workspace.numel() * workspace.element_size()))
    return out


def decode_attention_noalloc(q, k_cache, v_cache, position, *, out,
                             scale=None, window=0, stream=None):
    """qk$decode_attention through the entry point that allocates nothing
    (qk_decode_attention_noalloc): the partials go to the library's fixed
    per-device scratch. `out` is required (the caller owns every buffer).
    Calls that overlap on one device race on that scratch."""
    attrs = _attn_attrs(q, scale, window)
    pos = position.reshape(1) if position.dim() == 0 else position
    bq, bk, bv, bp, bo = (any_buffer(t) for t in (q, k_cache, v_cache, pos,
                                                   out))
    check(lib().qk_decode_attention_noalloc(
        stream_handle(stream), _ref(bq), _ref(bk), _ref(bv), _ref(bp),
        _ref(bo), ctypes.byref(attrs)))
    return out
