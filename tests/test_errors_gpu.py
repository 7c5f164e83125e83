"""Failure handling (reference: tests/test_gpu_errors.py, the sticky device
error of metal_pjrt/runtime/metal_runtime.h:43-53 and the
METAL_PJRT_FAIL_COMMAND_BUFFER hook). The failure is injected on the host
(QK_FAIL_LAUNCH=n marks the n-th launch failed after it was issued), so
every kernel still runs to completion: a failed call raises, later calls
keep raising until the error is reset, and values are never silently
wrong.
"""

import os

import pytest
import torch

import qkern
from qkern import _lib

pytestmark = pytest.mark.gpu


def test_injected_launch_failure_is_sticky(dev):
    x = torch.randn(4, 256, device=dev)
    try:
        os.environ["QK_FAIL_LAUNCH"] = "2"
        qkern.reset_device_error()  # re-reads the environment
        y1 = qkern.softmax(x)  # launch 1: fine
        torch.cuda.synchronize()
        assert torch.allclose(y1.sum(-1), torch.ones(4, device=dev))
        with pytest.raises(qkern.QkError) as e:
            qkern.softmax(x)  # launch 2: injected failure
        assert e.value.status == _lib.INTERNAL
        assert "QK_FAIL_LAUNCH" in e.value.message
        assert qkern.device_error() == _lib.INTERNAL
        with pytest.raises(qkern.QkError) as e:  # sticky, other target too
            qkern.matmul(x, x.T.contiguous())
        assert "earlier GPU launch failed" in e.value.message
    finally:
        os.environ.pop("QK_FAIL_LAUNCH", None)
        qkern.reset_device_error()
    torch.cuda.synchronize()
    assert qkern.device_error() == 0
    y = qkern.softmax(x)
    torch.cuda.synchronize()
    assert torch.allclose(y, torch.softmax(x, -1), atol=1e-6)


def test_host_argument_errors_are_not_sticky(dev):
    x = torch.randn(2, 100, device=dev, dtype=torch.bfloat16)
    words = torch.zeros(8, 32, dtype=torch.int32, device=dev)
    s = torch.zeros(8, 4, dtype=torch.bfloat16, device=dev)
    with pytest.raises(qkern.QkError):
        qkern.qmatvec(x, words, s, s)
    assert qkern.device_error() == 0
    y = qkern.rms_norm(x, None, 1e-6)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all()


@pytest.mark.parametrize("m,n", [(16, 4096), (64, 4096), (8, 151936)],
                         ids=["ws", "wsmid", "wsp"])
def test_wait_timeout_is_an_error_not_wrong_values(dev, m, n, monkeypatch):
    # The producer / consumer kernels (rows 5..16, 33..128 and the
    # persistent lm_head form) wait on LDS flags with a bounded spin. A wait
    # that gives up must surface as the sticky device error with NaN
    # outputs, never as plausible values. QK_SPIN_LIMIT=0 makes every wait
    # give up at once from the host side: no wait is left unbounded and
    # every kernel still ends normally. QK_QSTREAM=0 keeps the lm_head
    # shape on the persistent kernel (the streamed kernel that serves it
    # otherwise has no waits).
    monkeypatch.setenv("QK_QSTREAM", "0")
    k = 4096
    g = torch.Generator().manual_seed(7)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16).to(dev)
    words = torch.randint(-2**31, 2**31 - 1, (n, k // 8), dtype=torch.int32,
                          generator=g).to(dev)
    s = (torch.rand(n, k // 64, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    b = (torch.randn(n, k // 64, generator=g) * 0.05).to(torch.bfloat16).to(dev)
    want = qkern.qmatvec(x, words, s, b)
    torch.cuda.synchronize()
    assert qkern.device_error() == 0
    assert torch.isfinite(want.float()).all()
    try:
        os.environ["QK_SPIN_LIMIT"] = "0"
        qkern.reset_device_error()  # re-reads the environment
        y = qkern.qmatvec(x, words, s, b)  # the launch itself succeeds
        torch.cuda.synchronize()
        assert qkern.device_error() == _lib.INTERNAL
        assert torch.isnan(y.float()).any()
        # no finite output differs from the true one by more than rounding:
        # a workgroup that gave up stores NaN for all its outputs
        fin = torch.isfinite(y.float())
        assert torch.equal(y[fin], want[fin])
        with pytest.raises(qkern.QkError) as e:  # sticky
            qkern.qmatvec(x, words, s, b)
        assert "gave up waiting" in e.value.message
    finally:
        os.environ.pop("QK_SPIN_LIMIT", None)
        torch.cuda.synchronize()
        qkern.reset_device_error()
    assert qkern.device_error() == 0
    y = qkern.qmatvec(x, words, s, b)
    torch.cuda.synchronize()
    assert qkern.device_error() == 0
    assert torch.equal(y, want)
