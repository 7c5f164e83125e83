"""Checkpoint reading for the quantized decode path: safetensors files into
torch tensors (host, memory-mapped, no copy), and matrices quantized on
the GPU with qk_quantize.

read_safetensors restates the reference's reader (examples/llm/qwen3.py:
75-96): an 8-byte little-endian header length, a JSON header of
{name: {dtype, shape, data_offsets}} (plus an optional "__metadata__"),
then the raw tensor bytes; BF16, F16 and F32 tensors only, any other dtype
refused with the tensor's name. torch holds bfloat16 natively, so the
tensors are views of one read-only memory map of the file.

load_quantized does what the reference's load_params does per matrix
(qwen3.py:113-128: quantize every 2-D weight in groups of 64 along its
input dimension) with the quantization on the device: each matrix is
copied to HBM once and qk_quantize writes its codes, scales and offsets
there, bit-identical to the reference's float32 quantizers.
"""

import json
import mmap
import struct
import warnings

import torch

from .ffi import Packing, quantize

_DTYPES = {"BF16": torch.bfloat16, "F16": torch.float16, "F32": torch.float32}


def read_safetensors(path):
    """{name: torch.Tensor} viewing a read-only memory map of the file."""
    with open(path, "rb") as f:
        buf = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
    if len(buf) < 8:
        raise ValueError(f"{path}: not a safetensors file (shorter than 8 "
                         "bytes)")
    (n,) = struct.unpack("<Q", buf[:8])
    if 8 + n > len(buf):
        raise ValueError(f"{path}: header length {n} runs past the end of "
                         f"the file ({len(buf)} bytes)")
    header = json.loads(bytes(buf[8:8 + n]))
    header.pop("__metadata__", None)
    data = memoryview(buf)[8 + n:]
    out = {}
    for name, info in header.items():
        if info["dtype"] not in _DTYPES:
            raise ValueError(f"{path}: tensor {name} has dtype "
                             f"{info['dtype']}; only "
                             f"{', '.join(_DTYPES)} checkpoints are "
                             "supported")
        dt = _DTYPES[info["dtype"]]
        start, end = info["data_offsets"]
        shape = [int(d) for d in info["shape"]]
        count = 1
        for d in shape:
            count *= d
        esz = torch.empty(0, dtype=dt).element_size()
        if end - start != count * esz or end > len(data):
            raise ValueError(f"{path}: tensor {name} spans bytes "
                             f"{start}..{end}, not {count} x {esz}")
        with warnings.catch_warnings():
            # a read-only map: the tensor must not be written
            warnings.simplefilter("ignore", UserWarning)
            t = torch.frombuffer(data, dtype=dt, count=count,
                                 offset=start) if count else \
                torch.empty(0, dtype=dt)
        out[name] = t.reshape(shape)
    return out


def load_quantized(tensors, device, packing=Packing.U32X8, group_size=64,
                   scale_dtype=torch.bfloat16, keep=lambda name, t: False):
    """Every 2-D tensor (unless keep(name, t)) quantized on `device` into
    {"codes", "scales", "biases" (None for S8_SYM), "k"}; other tensors
    copied to the device as they are. The matrices keep the checkpoint's
    [out, in] layout, as the reference's loader does."""
    out = {}
    for name, t in tensors.items():
        w = t.to(device)
        if w.dim() == 2 and not keep(name, t) and w.shape[1] % group_size == 0:
            codes, scales, biases = quantize(w.contiguous(), packing=packing,
                                             group_size=group_size,
                                             scale_dtype=scale_dtype)
            out[name] = {"codes": codes, "scales": scales, "biases": biases,
                         "k": w.shape[1]}
            del w
        else:
            out[name] = w
    return out
