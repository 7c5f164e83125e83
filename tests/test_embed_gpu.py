"""GPU parity of qk$embed (the dequantize kernel of qmatvec.hip with a row
gather, and a dense row gather) against oracle.embed, the restatement of
qwen3.embed (examples/llm/qwen3.py:270-274).

Bit-exact: a gathered row of a quantized table is the canonical
dequantization (f32(q)*f32(s) + f32(b), rounded once) of that table row, in
every packing and output type; a dense gather copies rows. Cases: token
arrays of rank 1 and 2, repeated tokens, indices outside the table
(clamped), empty token arrays, Qwen3-8B's int4 vocabulary table.
"""

import numpy as np
import pytest
import torch

import oracle as O
import qkern
from qkern.ffi import Packing
from helpers import TORCH
from test_qmatvec_gpu import make_weights

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("packing", list(Packing))
@pytest.mark.parametrize("odt", ["bfloat16", "float16", "float32"])
def test_embed_quantized_bit_exact(dev, packing, odt):
    rng = np.random.default_rng(int(packing) * 7 + len(odt))
    v, k = 50, 256
    dc, ds, db, w, *_ = make_weights(rng, v, k, packing, 64)
    tokens = np.array([[0, 49, 7, 7], [13, 2, 49, 0]], dtype=np.int32)
    got = qkern.embed(dc.to(dev), torch.from_numpy(tokens).to(dev),
                      ds.to(dev), None if db is None else db.to(dev), k=k,
                      packing=packing, dtype=TORCH[odt])
    torch.cuda.synchronize()
    want = O.round_to(O.embed(w, tokens), odt)
    assert got.shape == (2, 4, k)
    assert np.array_equal(got.float().cpu().numpy(), want.astype(np.float32))


def test_embed_default_type_clamps_and_empty(dev):
    rng = np.random.default_rng(11)
    v, k = 40, 512
    dc, ds, db, w, *_ = make_weights(rng, v, k, Packing.U32X8, 64)
    dc, ds, db = dc.to(dev), ds.to(dev), db.to(dev)
    tokens = np.array([-3, 0, 39, 40, 2 ** 30], dtype=np.int32)
    got = qkern.embed(dc, torch.from_numpy(tokens).to(dev), ds, db, k=k)
    torch.cuda.synchronize()
    assert got.dtype == torch.bfloat16  # the scales' type, as the reference
    want = O.round_to(O.embed(w, tokens), "bfloat16")
    assert np.array_equal(got.float().cpu().numpy(), want.astype(np.float32))
    empty = qkern.embed(dc, torch.zeros(0, dtype=torch.int32, device=dev),
                        ds, db, k=k)
    torch.cuda.synchronize()
    assert empty.shape == (0, k)


@pytest.mark.parametrize("dt", ["bfloat16", "float16", "float32"])
def test_embed_dense_table(dev, dt):
    rng = np.random.default_rng(12)
    v, k = 1000, 1024
    table = O.round_to(rng.standard_normal((v, k)), dt).astype(np.float32)
    tokens = rng.integers(-10, v + 10, size=(3, 17)).astype(np.int32)
    got = qkern.embed(torch.from_numpy(table).to(TORCH[dt]).to(dev),
                      torch.from_numpy(tokens).to(dev))
    torch.cuda.synchronize()
    assert got.shape == (3, 17, k)
    assert np.array_equal(got.float().cpu().numpy(), O.embed(table, tokens))


def test_embed_qwen3_8b_vocabulary(dev):
    # the int4 token embedding of Qwen3-8B: 151936 x 4096, group 64
    n, k = 151936, 4096
    codes, s, b = O.config_affine(n, k, bits=4, seed=0)
    dc = torch.from_numpy(O.pack_u32x8(codes).view(np.int32)).to(dev)
    ds = torch.from_numpy(s).to(torch.bfloat16).to(dev)
    db = torch.from_numpy(b).to(torch.bfloat16).to(dev)
    tokens = np.array([0, 1, 151935, 77777, 123, 151935], dtype=np.int32)
    got = qkern.embed(dc, torch.from_numpy(tokens).to(dev), ds, db, k=k)
    torch.cuda.synchronize()
    sel = np.clip(tokens, 0, n - 1)
    want = O.round_to(O.dequantize_f32(
        codes[sel].reshape(len(sel), -1, 64).astype(np.float32),
        O.bf16_round(s[sel])[..., None], O.bf16_round(b[sel])[..., None]),
        "bfloat16")
    assert np.array_equal(got.float().cpu().numpy(), want.astype(np.float32))
