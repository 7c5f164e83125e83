"""Host-side weight formats for qk$qmatvec / qk$dequantize (numpy).

One-time preprocessing, as the reference's loader does it
(examples/llm/qwen3.py:113-128 quantizes each matrix when the checkpoint is
loaded). Both 4-bit packings are supported:
  - BYTE_HALFSPLIT: the reference's own layout (qwen3.py:169-196);
  - U32X8: 8 codes per uint32 along K (MLX-style word packing).
"""

import numpy as np

GROUP = 64


def quantize_int4(w, group=GROUP):
    """MLX-style affine 4-bit grid per `group` inputs (qwen3.py:169-196).

    The grid is anchored at the group's largest-magnitude weight (the
    offset) and its step stretched so that zero falls on the grid. float32
    arithmetic throughout. Returns codes uint8 [N, K] (0..15) and scale,
    offset float32 [N, K/group]."""
    w = np.asarray(w, dtype=np.float32)
    n = w.shape[0]
    g = w.reshape(n, -1, group)
    lo = g.min(axis=-1, keepdims=True)
    hi = g.max(axis=-1, keepdims=True)
    anchor_lo = np.abs(lo) > np.abs(hi)
    width = np.maximum(hi - lo, np.float32(1e-12)) / np.float32(15)
    scale = np.where(anchor_lo, width, -width).astype(np.float32)
    anchor = np.where(anchor_lo, lo, hi).astype(np.float32)
    steps = np.rint(anchor / scale)
    on_grid = steps != 0
    scale = np.where(on_grid, anchor / np.where(on_grid, steps,
                                                np.float32(1)),
                     scale).astype(np.float32)
    offset = np.where(on_grid, anchor, np.float32(0)).astype(np.float32)
    codes = np.clip(np.rint((g - offset) / scale), 0, 15).astype(np.uint8)
    return (codes.reshape(n, -1), scale.reshape(n, -1),
            offset.reshape(n, -1))


def quantize_int8(w, group=GROUP):
    """Symmetric int8 per `group` inputs (qwen3.py:154-166): codes int8
    [N, K] in -127..127 and scale float32 [N, K/group]."""
    w = np.asarray(w, dtype=np.float32)
    n = w.shape[0]
    g = w.reshape(n, -1, group)
    scale = np.maximum(np.abs(g).max(axis=-1, keepdims=True),
                       np.float32(1e-12)) / np.float32(127)
    codes = np.clip(np.rint(g / scale), -127, 127).astype(np.int8)
    return codes.reshape(n, -1), scale.reshape(n, -1).astype(np.float32)


def pack_u32x8(codes):
    """codes [N, K] (0..15) -> uint32 [N, K/8]: element 8i + j in bits
    4j..4j+3 of word i."""
    c = np.asarray(codes, dtype=np.uint32)
    n, k = c.shape
    c = c.reshape(n, k // 8, 8)
    out = np.zeros((n, k // 8), dtype=np.uint32)
    for j in range(8):
        out |= c[:, :, j] << np.uint32(4 * j)
    return out


def pack_halfsplit(codes, group=GROUP):
    """codes [N, K] (0..15) -> uint8 [N, K/group, group/2]: byte j of a
    group holds element j (low nibble) and element j + group/2 (high)."""
    c = np.asarray(codes, dtype=np.uint8)
    n = c.shape[0]
    g = c.reshape(n, -1, group)
    h = group // 2
    return (g[..., :h] | (g[..., h:] << 4)).astype(np.uint8)


def halfsplit_to_u32x8(packed):
    """Re-pack the reference's byte layout into U32X8 words."""
    p = np.asarray(packed, dtype=np.uint8)
    n = p.shape[0]
    codes = np.concatenate([p & 0xF, p >> 4], axis=-1).reshape(n, -1)
    return pack_u32x8(codes)


def to_bf16_bits(x):
    """float32 -> bf16 bit patterns (uint16), round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    u = u.astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
