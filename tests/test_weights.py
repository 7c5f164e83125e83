"""Checkpoint reading (qkern.weights.read_safetensors, the reference's
read_safetensors, examples/llm/qwen3.py:75-96) and the argument checks of
qk_quantize; CPU only."""

import json
import struct

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import qkern
from qkern import _lib


def test_read_safetensors_round_trip(tmp_path):
    """bf16 / f16 / f32 tensors of several ranks (and an empty one) come
    back bit for bit, the metadata entry is skipped, and the tensors view
    the file without a copy (read-only)."""
    torch.manual_seed(0)
    d = {"w": torch.randn(48, 64).to(torch.bfloat16),
         "b": torch.arange(10, dtype=torch.float32),
         "h": torch.randn(2, 3, 4).half(),
         "e": torch.zeros(0, 5, dtype=torch.float32)}
    f = tmp_path / "m.safetensors"
    save_file(d, str(f), metadata={"format": "pt"})
    r = qkern.read_safetensors(str(f))
    assert set(r) == set(d)
    for k, v in d.items():
        assert r[k].dtype == v.dtype and tuple(r[k].shape) == tuple(v.shape)
        assert torch.equal(r[k].view(torch.uint8) if v.numel() else r[k],
                           v.contiguous().view(torch.uint8)
                           if v.numel() else v)


def _write(path, header, payload):
    h = json.dumps(header).encode()
    path.write_bytes(struct.pack("<Q", len(h)) + h + payload)


def test_read_safetensors_refusals(tmp_path):
    """A dtype the reference does not read (named in the message), a
    tensor whose byte span does not match its shape, a header running past
    the file, and a file shorter than the length field."""
    f = tmp_path / "i8.safetensors"
    _write(f, {"q": {"dtype": "I8", "shape": [4], "data_offsets": [0, 4]}},
           bytes(4))
    with pytest.raises(ValueError, match="tensor q has dtype I8"):
        qkern.read_safetensors(str(f))
    f = tmp_path / "span.safetensors"
    _write(f, {"x": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}},
           bytes(8))
    with pytest.raises(ValueError, match="spans bytes"):
        qkern.read_safetensors(str(f))
    f = tmp_path / "long.safetensors"
    f.write_bytes(struct.pack("<Q", 1000) + b"{}")
    with pytest.raises(ValueError, match="runs past the end"):
        qkern.read_safetensors(str(f))
    f = tmp_path / "short.safetensors"
    f.write_bytes(b"abc")
    with pytest.raises(ValueError, match="shorter than 8"):
        qkern.read_safetensors(str(f))


def test_quantize_argument_checks():
    # shapes and types are checked before any launch (host tensors stand in
    # for device buffers)
    def status(fn):
        try:
            fn()
            return _lib.OK, ""
        except qkern.QkError as e:
            return e.status, e.message

    w = torch.zeros(8, 128, dtype=torch.bfloat16)
    st, msg = status(lambda: qkern.quantize(w, packing=qkern.Packing.U8))
    assert st == _lib.UNIMPLEMENTED and "8-bit affine" in msg
    with pytest.raises(ValueError):  # [N, K] only
        qkern.quantize(w.reshape(8, 2, 64))
    st, msg = status(lambda: qkern.quantize(w, group_size=48))
    assert st == _lib.UNIMPLEMENTED and "group size" in msg
    st, msg = status(lambda: qkern.quantize(torch.zeros(8, 100,
                                                        dtype=torch.float32)))
    assert st == _lib.INVALID_ARGUMENT and "multiple of the group" in msg
    # empty matrices launch nothing
    qkern.quantize(w[:0])
