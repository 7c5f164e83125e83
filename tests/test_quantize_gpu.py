"""GPU parity of qk_quantize (quantize.hip) and of a checkpoint loaded
through it: codes, scales and offsets bit-identical to the oracle's float32
restatements of the reference's quantizers (examples/llm/qwen3.py:154-196),
which tests/test_oracle.py pins by known answers and brute force."""

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import oracle as O
import qkern
from qkern.ffi import Packing
from helpers import TORCH

pytestmark = pytest.mark.gpu


def weights(rng, n, k, group):
    """Normal weights with the grid's special groups planted: all zeros
    (the 1e-12 floor), constant, a negative anchor, an anchor whose first
    step rounds to zero (offset 0), exact ties, and one huge outlier."""
    w = (0.02 * rng.standard_normal((n, k))).astype(np.float32)
    gpr = k // group
    if n >= 1 and gpr >= 6:
        w[0, 0:group] = 0.0
        w[0, group:2 * group] = 0.375
        w[0, 2 * group:3 * group] = -rng.random(group) - 1.0
        w[0, 3 * group:4 * group] = np.linspace(-1.0, 0.03, group)
        w[0, 4 * group:5 * group] = np.arange(group) % 16 * 0.125
        w[0, 5 * group] = 300.0
    if n >= 2 and gpr >= 2:
        # quotients on and a hair off half-integers: 127 (int8) and 15
        # (int4) steps with weights at k + 1/2 steps and their neighbours
        t = (np.arange(group) % 126 + 0.5).astype(np.float32)
        w[1, 0:group] = t / 127.0
        w[1, group - 1] = 1.0
        w[1, group:2 * group] = np.nextafter(t, np.float32(0)) / 15.0
        w[1, 2 * group - 1] = -1.0
    return w


@pytest.mark.parametrize("wdt", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("group", [32, 64, 128])
def test_quantize_int4_bit_exact(dev, wdt, group):
    rng = np.random.default_rng(group + len(wdt))
    n, k = 37, 8 * group
    w = O.round_to(weights(rng, n, k, group), wdt).astype(np.float32)
    codes, s, b = O.quantize_int4(w, group)
    codes = codes.reshape(n, -1)
    dw = torch.from_numpy(w).to(TORCH[wdt]).to(dev)
    for packing in (Packing.U32X8, Packing.BYTE_HALFSPLIT):
        for sdt in (torch.float32, torch.bfloat16):
            dc, ds, db = qkern.quantize(dw, packing=packing, group_size=group,
                                        scale_dtype=sdt)
            torch.cuda.synchronize()
            if packing == Packing.U32X8:
                got = dc.cpu().numpy().view(np.uint32)
                assert np.array_equal(got, O.pack_u32x8(codes))
            else:
                got = dc.cpu().numpy()
                assert np.array_equal(got.reshape(n, -1),
                                      O.pack_halfsplit(codes, group)
                                      .reshape(n, -1))
            want_s, want_b = s.reshape(n, -1), b.reshape(n, -1)
            if sdt == torch.float32:
                assert np.array_equal(ds.cpu().numpy().view(np.uint32),
                                      want_s.view(np.uint32))
                assert np.array_equal(db.cpu().numpy().view(np.uint32),
                                      want_b.view(np.uint32))
            else:
                assert np.array_equal(ds.view(torch.int16).cpu().numpy()
                                      .view(np.uint16), O.bf16_bits(want_s))
                assert np.array_equal(db.view(torch.int16).cpu().numpy()
                                      .view(np.uint16), O.bf16_bits(want_b))


@pytest.mark.parametrize("wdt", ["float32", "bfloat16"])
@pytest.mark.parametrize("group", [32, 64, 128])
def test_quantize_int8_bit_exact(dev, wdt, group):
    rng = np.random.default_rng(7 * group)
    n, k = 29, 8 * group
    w = O.round_to(weights(rng, n, k, group), wdt).astype(np.float32)
    q, s = O.quantize_int8(w, group)
    dw = torch.from_numpy(w).to(TORCH[wdt]).to(dev)
    dc, ds, db = qkern.quantize(dw, packing=Packing.S8_SYM, group_size=group)
    torch.cuda.synchronize()
    assert db is None
    assert np.array_equal(dc.cpu().numpy(), q.reshape(n, -1))
    assert np.array_equal(ds.cpu().numpy().view(np.uint32),
                          s.reshape(n, -1).view(np.uint32))


def test_quantize_large_matrix(dev):
    """A Qwen3-8B-sized projection (12288 x 4096, bf16, 786432 groups in
    one launch): 256 rows spread over the matrix checked bit for bit
    (codes, scales, offsets) against the oracle."""
    torch.manual_seed(0)
    w = (0.02 * torch.randn(12288, 4096, device=dev)).to(torch.bfloat16)
    dc, ds, db = qkern.quantize(w)
    torch.cuda.synchronize()
    rows = np.random.default_rng(1).choice(12288, 256, replace=False)
    rows.sort()
    wr = w[torch.from_numpy(rows).to(dev)].float().cpu().numpy()
    codes, s, b = O.quantize_int4(wr)
    r = torch.from_numpy(rows).to(dev)
    assert np.array_equal(dc[r].cpu().numpy().view(np.uint32),
                          O.pack_u32x8(codes.reshape(len(rows), -1)))
    assert np.array_equal(ds[r].cpu().numpy(), s.reshape(len(rows), -1))
    assert np.array_equal(db[r].cpu().numpy(), b.reshape(len(rows), -1))


def test_load_quantized_checkpoint_end_to_end(dev, tmp_path):
    """A safetensors checkpoint (bf16 projections, an f32 norm vector)
    read by qkern.read_safetensors and quantized on the device by
    load_quantized (as the reference's load_params quantizes each matrix);
    the loaded matrices drive qk$qmatvec against the oracle's matvec of the
    oracle's own quantization of the same weights."""
    rng = np.random.default_rng(3)
    mats = {"layers.0.q_proj.weight": (512, 1024),
            "layers.0.down_proj.weight": (1024, 768)}
    d = {name: torch.from_numpy((0.02 * rng.standard_normal(shape))
                                .astype(np.float32)).to(torch.bfloat16)
         for name, shape in mats.items()}
    d["layers.0.norm.weight"] = torch.ones(1024, dtype=torch.float32)
    f = tmp_path / "model.safetensors"
    save_file(d, str(f))
    loaded = qkern.load_quantized(qkern.read_safetensors(str(f)), dev)
    assert loaded["layers.0.norm.weight"].device.type == "cuda"
    for name, (n, k) in mats.items():
        entry = loaded[name]
        w = d[name].float().numpy()
        codes, s, b = O.quantize_int4(w)
        assert np.array_equal(entry["codes"].cpu().numpy().view(np.uint32),
                              O.pack_u32x8(codes.reshape(n, -1)))
        x = O.round_to(rng.standard_normal((3, k)), "bfloat16").astype(
            np.float32)
        y = qkern.qmatvec(torch.from_numpy(x).to(torch.bfloat16).to(dev),
                          entry["codes"], entry["scales"], entry["biases"])
        torch.cuda.synchronize()
        sb = O.bf16_round(s.reshape(n, -1))
        bb = O.bf16_round(b.reshape(n, -1))
        wq = O.dequantize_f32(codes, sb[..., None], bb[..., None]).reshape(n, k)
        want = O.matvec_f64(x, wq)
        assert O.rel_fro(y.float().cpu().numpy().astype(np.float64),
                         want) <= 1e-2
