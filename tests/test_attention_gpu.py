"""GPU parity of qk$decode_attention (attention.hip) against the float64
oracle (oracle.decode_attention, the one-query branch of
examples/llm/qwen3.py:322-326 with the decode mask of :357-358).

The reference computes the scores, softmax and weighted sum in float32 and
rounds once to the cache type; the bar here is the bf16/f16 one: relative
Frobenius error <= 1e-2 and, elementwise, |got - want| <= 1e-2 |want| +
2e-3 sum_s p_s |v_s| (the output's rounding scale). Cases cover the
cache layouts at Qwen3-8B's decode shape (KV = 8, G = 4, D = 128), other
head counts and dims, windows shorter than the cache, positions before,
inside and past the window, ragged window ends, both cache types, and the
runs of several chunks per wave that long windows take.
"""

import numpy as np
import pytest
import torch

import oracle as O
import qkern

pytestmark = pytest.mark.gpu

TORCH = {"bfloat16": torch.bfloat16, "float16": torch.float16}


def make_case(rng, b, kv, g, d, smax, dtype):
    q = O.round_to(rng.standard_normal((b, kv, g, d)), dtype)
    k = O.round_to(rng.standard_normal((b, kv, smax, d)), dtype)
    v = O.round_to(rng.standard_normal((b, kv, d, smax)), dtype)
    return q, k, v


def to_dev(a, dtype, dev):
    return torch.from_numpy(np.asarray(a, np.float32)).to(TORCH[dtype]).to(dev)


def check_attention(got, q, k, v, pos, scale, window):
    want = O.decode_attention(q, k, v, pos, scale, window)
    # magnitude: sum_s p_s |v_s| with the oracle's p
    S = window or k.shape[2]
    t = np.einsum("bkgd,bksd->bkgs", q.astype(np.float64),
                  k[:, :, :S].astype(np.float64)) * scale
    t = np.where(np.arange(S) <= pos, t, -np.inf)
    p = O.softmax(t)
    mag = np.einsum("bkgs,bkds->bkgd", p, np.abs(v[..., :S]).astype(
        np.float64))
    got = np.asarray(got, np.float64)
    assert np.all(np.isfinite(got))
    assert O.rel_fro(got, want) <= 1e-2
    over = np.abs(got - want) - (1e-2 * np.abs(want) + 2e-3 * mag)
    assert np.all(over <= 0), float(over.max())


def run(dev, q, k, v, pos, dtype, scale=None, window=0, workspace=None):
    dq, dk, dv = (to_dev(a, dtype, dev) for a in (q, k, v))
    dpos = torch.tensor([pos], dtype=torch.int32, device=dev)
    out = qkern.decode_attention(dq, dk, dv, dpos, scale=scale, window=window,
                                 workspace=workspace)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


CASES = [
    # (b, kv, g, d, smax, pos, window)
    (1, 1, 1, 128, 8, 0, 0),
    (1, 2, 4, 128, 64, 63, 0),
    (2, 3, 5, 64, 136, 100, 0),     # ragged last chunk, odd head counts
    (1, 2, 16, 128, 200, 199, 0),   # 16 query heads per KV head
    (3, 1, 2, 64, 1024, 500, 0),    # slots past pos never read
    (1, 4, 4, 128, 512, 700, 300),  # pos past the window
    (1, 2, 8, 128, 4096, 77, 4096),
    (2, 2, 4, 64, 520, 519, 513),   # window end inside an 8-slot group
]


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_decode_attention_small(dev, dtype):
    rng = np.random.default_rng(31 + len(dtype))
    for (b, kv, g, d, smax, pos, window) in CASES:
        q, k, v = make_case(rng, b, kv, g, d, smax, dtype)
        got = run(dev, q, k, v, pos, dtype, window=window)
        check_attention(got, q, k, v, pos, d ** -0.5, window)


@pytest.mark.parametrize("smax,pos,b", [(4096, 4095, 1), (4096, 1000, 4),
                                        (32768, 20000, 1)])
def test_decode_attention_qwen3_8b(dev, smax, pos, b):
    # Qwen3-8B decode: 32 query heads over 8 KV heads of dim 128; the
    # 32768-slot window takes runs of two chunks per wave.
    rng = np.random.default_rng(smax + pos)
    q, k, v = make_case(rng, b, 8, 4, 128, smax, "bfloat16")
    got = run(dev, q, k, v, pos, "bfloat16")
    check_attention(got, q, k, v, pos, 128 ** -0.5, 0)


def test_decode_attention_short_prefix_of_long_window(dev):
    # the window's parts are cut from the position read on the device: a
    # short attended prefix of a 32768-slot cache still splits over them
    rng = np.random.default_rng(9)
    q, k, v = make_case(rng, 1, 8, 4, 128, 32768, "bfloat16")
    for pos in (0, 100, 4095, 20001):
        got = run(dev, q, k, v, pos, "bfloat16")
        check_attention(got, q, k, v, pos, 128 ** -0.5, 0)


@pytest.mark.parametrize("pos", [467, 500, 503, 511])
def test_decode_attention_slots_past_position_take_no_part(dev, pos):
    # NaN keys and values in every slot past the position (also inside the
    # last 8-slot unit the values are fetched in, in either half of the
    # last chunk: 467 and 500 end in its first and second half) leave the
    # output finite
    rng = np.random.default_rng(10 + pos)
    q, k, v = make_case(rng, 2, 2, 4, 128, 1024, "bfloat16")
    kp, vp = k.copy(), v.copy()
    kp[:, :, pos + 1:] = np.nan
    vp[..., pos + 1:] = np.nan
    got = run(dev, q, kp, vp, pos, "bfloat16")
    check_attention(got, q, k, v, pos, 128 ** -0.5, 0)


def test_decode_attention_peaked_scores(dev):
    # scores up to ~1e3 (unscaled keys far larger than the queries): the
    # running maximum must keep the exponentials finite
    rng = np.random.default_rng(5)
    q, k, v = make_case(rng, 1, 2, 4, 128, 512, "bfloat16")
    k = O.round_to(k * 30.0, "bfloat16")
    got = run(dev, q, k, v, 511, "bfloat16", scale=1.0)
    check_attention(got, q, k, v, 511, 1.0, 0)


def test_decode_attention_layouts_and_position_on_device(dev):
    # the reference's q [B, 1, KV, G, D]; the position is read on the
    # device, so one set of buffers serves consecutive decode steps
    rng = np.random.default_rng(6)
    q, k, v = make_case(rng, 2, 2, 4, 128, 256, "bfloat16")
    dq = to_dev(q, "bfloat16", dev).unsqueeze(1)
    dk, dv = to_dev(k, "bfloat16", dev), to_dev(v, "bfloat16", dev)
    dpos = torch.zeros(1, dtype=torch.int32, device=dev)
    ws = torch.empty(qkern.decode_attention_workspace_size(dq, dk),
                     dtype=torch.uint8, device=dev)
    out = torch.empty_like(dq)
    for pos in (3, 130, 255, 17):
        dpos.fill_(pos)
        qkern.decode_attention(dq, dk, dv, dpos, workspace=ws, out=out)
        torch.cuda.synchronize()
        assert out.shape == (2, 1, 2, 4, 128)
        check_attention(out[:, 0].float().cpu().numpy(), q, k, v, pos,
                        128 ** -0.5, 0)


def test_decode_attention_nothing_attended_is_nan(dev):
    # a negative position masks every slot: softmax over -inf only is NaN
    rng = np.random.default_rng(8)
    q, k, v = make_case(rng, 1, 1, 4, 64, 64, "bfloat16")
    dq, dk, dv = (to_dev(a, "bfloat16", dev) for a in (q, k, v))
    out = qkern.decode_attention(dq, dk, dv, torch.tensor(
        [-1], dtype=torch.int32, device=dev))
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all()
