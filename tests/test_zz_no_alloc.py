"""GPU parity of qk_decode_attention_noalloc (the decode-attention entry
point that allocates nothing and keeps its partials in the library's fixed
per-device scratch) against qk_decode_attention with a caller workspace.

Both run the same kernels over the same split of the cache window, so the
outputs must be bit-identical; each is also checked against the float64
oracle (oracle.decode_attention, examples/llm/qwen3.py:322-326). Two calls
in a row, the second smaller than the first, show that what the first call
left in the scratch does not leak into the second.
"""

import numpy as np
import pytest
import torch

import qkern
from test_attention_gpu import check_attention, make_case, to_dev

pytestmark = pytest.mark.gpu


def both(dev, q, k, v, pos, dtype, window=0):
    dq, dk, dv = (to_dev(a, dtype, dev) for a in (q, k, v))
    dpos = torch.tensor([pos], dtype=torch.int32, device=dev)
    want = qkern.decode_attention(dq, dk, dv, dpos, window=window)
    out = torch.full_like(dq, float("nan"))
    qkern.decode_attention_noalloc(dq, dk, dv, dpos, out=out, window=window)
    torch.cuda.synchronize()
    assert qkern.device_error() == 0
    assert torch.equal(out, want)
    return out.float().cpu().numpy()


def test_noalloc_matches_workspace_entry_two_calls(dev):
    rng = np.random.default_rng(11)
    # 1: Qwen3-8B decode over a 32768-slot cache (4.3 MB of partials)
    q, k, v = make_case(rng, 1, 8, 4, 128, 32768, "bfloat16")
    got = both(dev, q, k, v, 20000, "bfloat16")
    check_attention(got, q, k, v, 20000, 128 ** -0.5, 0)
    # 2: a smaller problem right after, in the same scratch
    q, k, v = make_case(rng, 2, 3, 5, 64, 136, "float16")
    got = both(dev, q, k, v, 100, "float16")
    check_attention(got, q, k, v, 100, 64 ** -0.5, 0)


def test_noalloc_position_on_device_and_window(dev):
    rng = np.random.default_rng(12)
    q, k, v = make_case(rng, 1, 4, 4, 128, 512, "bfloat16")
    for pos, window in ((700, 300), (77, 0), (511, 513 - 1)):
        got = both(dev, q, k, v, pos, "bfloat16", window=window)
        check_attention(got, q, k, v, pos, 128 ** -0.5, window)


def test_noalloc_refuses_shapes_past_the_scratch(dev):
    # 1024 (batch, KV head) pairs x 16 query heads, one partial each:
    # 8.5 MB > 8 MiB
    q = torch.zeros(16, 64, 16, 128, dtype=torch.bfloat16, device=dev)
    k = torch.zeros(16, 64, 64, 128, dtype=torch.bfloat16, device=dev)
    v = torch.zeros(16, 64, 128, 64, dtype=torch.bfloat16, device=dev)
    pos = torch.zeros(1, dtype=torch.int32, device=dev)
    assert qkern.decode_attention_workspace_size(q, k) > 8 << 20
    with pytest.raises(qkern.QkError) as e:
        qkern.decode_attention_noalloc(q, k, v, pos, out=torch.empty_like(q))
    assert "fixed scratch" in e.value.message
    assert qkern.device_error() == 0
