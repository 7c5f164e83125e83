"""C ABI checks that need no GPU: the library loads, exports every symbol
include/qkern.h declares, and the host-side validation behaves as the
reference's ValidateMatmul (metal_pjrt/blas/blas_lt_support.cc:103-201) and
the FFI argument checks do. No kernel is launched here.
"""

import ctypes
import os
import re

import pytest
import torch

import qkern
from qkern import _lib
from qkern.blas import (BlasLt, Epilogue, GemmConfig, MatrixLayout, Order)
from qkern import quant

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    text = open(os.path.join(ROOT, "include", "qkern.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qk_[a-z_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    syms = header_symbols()
    assert len(syms) >= 10
    for s in syms:
        assert hasattr(lib, s), s
    # and the ctypes binding covers exactly the declared set
    assert sorted(_lib.SIGNATURES) == syms


def test_version_and_clean_state():
    assert "gfx950" in qkern.version()
    qkern.reset_device_error()
    assert qkern.device_error() == 0


def plan_status(cfg, epi=Epilogue.kDefault):
    try:
        BlasLt.get_matmul_plan(cfg, epi)
        return _lib.OK, ""
    except qkern.QkError as e:
        return e.status, e.message


def simple_cfg(dt="bfloat16", m=4, n=5, k=6, out_dt=None, order=Order.kRowMajor):
    out = MatrixLayout(out_dt or dt, m, n, order)
    return GemmConfig(MatrixLayout(dt, m, k), MatrixLayout(dt, k, n), out, out)


def test_plan_ok_for_all_types_and_epilogues():
    for dt, out in [("float32", None), ("float16", None), ("bfloat16", None),
                    ("float16", "float32"), ("bfloat16", "float32")]:
        for e in Epilogue:
            st, msg = plan_status(simple_cfg(dt, out_dt=out), e)
            assert st == _lib.OK, (dt, out, e, msg)


def test_plan_refusals_match_reference_classes():
    # unsupported epilogue value -> Unimplemented
    cfg = simple_cfg()
    h = ctypes.c_void_p()
    c = cfg.to_c()
    st = _lib.lib().qk_gemm_plan_create(ctypes.byref(c), 99, ctypes.byref(h))
    assert st == _lib.UNIMPLEMENTED
    assert b"epilogue 99" in _lib.lib().qk_last_error_message()
    # complex alpha -> Unimplemented
    cfg = simple_cfg()
    cfg.alpha = 1 + 1j
    assert plan_status(cfg)[0] == _lib.UNIMPLEMENTED
    # transposed layout -> Unimplemented
    cfg = simple_cfg()
    cfg.lhs_layout.transpose = True
    st, msg = plan_status(cfg)
    assert st == _lib.UNIMPLEMENTED and "transposed layout" in msg
    # mixed operand types -> Unimplemented with the reference's advice
    cfg = GemmConfig(MatrixLayout("bfloat16", 4, 6), MatrixLayout("float16", 6, 5),
                     MatrixLayout("bfloat16", 4, 5), MatrixLayout("bfloat16", 4, 5))
    st, msg = plan_status(cfg)
    assert st == _lib.UNIMPLEMENTED and "Cast the operands" in msg
    # f32 inputs with a bf16 output -> Unimplemented
    st, _ = plan_status(simple_cfg("float32", out_dt="bfloat16"))
    assert st == _lib.UNIMPLEMENTED
    # inconsistent shapes -> InvalidArgument
    cfg = GemmConfig(MatrixLayout("float32", 4, 6), MatrixLayout("float32", 7, 5),
                     MatrixLayout("float32", 4, 5), MatrixLayout("float32", 4, 5))
    st, msg = plan_status(cfg)
    assert st == _lib.INVALID_ARGUMENT and "inconsistent shapes" in msg
    # batch mismatch -> InvalidArgument
    cfg = GemmConfig(MatrixLayout("float32", 4, 6, batch_size=3),
                     MatrixLayout("float32", 6, 5),
                     MatrixLayout("float32", 4, 5, batch_size=2),
                     MatrixLayout("float32", 4, 5, batch_size=2))
    st, msg = plan_status(cfg)
    assert st == _lib.INVALID_ARGUMENT and "batch mismatch" in msg
    # beta != 0 with C laid out unlike D -> Unimplemented
    out = MatrixLayout("float32", 4, 5)
    cfg = GemmConfig(MatrixLayout("float32", 4, 6), MatrixLayout("float32", 6, 5),
                     MatrixLayout("float32", 4, 5, leading_dim_stride=8), out,
                     beta=1.0)
    st, msg = plan_status(cfg)
    assert st == _lib.UNIMPLEMENTED and "laid out unlike" in msg
    # ... but the same C is fine with beta == 0
    cfg.beta = 0.0
    assert plan_status(cfg)[0] == _lib.OK


def test_half_index_limit_like_reference():
    # metal_blas_lt_test.cc SteelOnlyShapeLimit: lda > INT32_MAX/256 is
    # refused for f16/bf16 (Unimplemented, naming the leading dimension) and
    # accepted for f32.
    k = (1 << 23) + 16
    for dt in ("bfloat16", "float16", "float32"):
        out = MatrixLayout(dt, 2, 2)
        cfg = GemmConfig(MatrixLayout(dt, 2, k), MatrixLayout(dt, k, 2), out, out)
        st, msg = plan_status(cfg)
        if dt == "float32":
            assert st == _lib.OK
        else:
            assert st == _lib.UNIMPLEMENTED and "leading dimension" in msg


def test_f32_sizes_beyond_int32_refused():
    # The f32 kernels take 32-bit sizes: a dimension or leading dimension
    # above INT32_MAX is refused (Unimplemented), never truncated.
    big = (1 << 31) + 64
    out = MatrixLayout("float32", 2, 2)
    cfg = GemmConfig(MatrixLayout("float32", 2, 8, leading_dim_stride=big),
                     MatrixLayout("float32", 8, 2), out, out)
    st, msg = plan_status(cfg)
    assert st == _lib.UNIMPLEMENTED and "leading dimension" in msg
    cfg = GemmConfig(MatrixLayout("float32", 2, big), MatrixLayout("float32", big, 2),
                     out, out)
    st, msg = plan_status(cfg)
    assert st == _lib.UNIMPLEMENTED and "dimension" in msg
    for e in (Epilogue.kDefault, Epilogue.kBiasThenSILU):
        out = MatrixLayout("float32", big, 2)
        cfg = GemmConfig(MatrixLayout("float32", big, 4), MatrixLayout("float32", 4, 2),
                         out, out)
        st, msg = plan_status(cfg, e)
        assert st == _lib.UNIMPLEMENTED and "f32 matmul too large" in msg
    # just inside the limit is accepted
    lim = (1 << 31) - 1
    out = MatrixLayout("float32", 2, 2)
    cfg = GemmConfig(MatrixLayout("float32", 2, 8, leading_dim_stride=lim),
                     MatrixLayout("float32", 8, 2), out, out)
    assert plan_status(cfg)[0] == _lib.OK


def test_column_major_output_swaps_operands():
    out = MatrixLayout("bfloat16", 6, 10, Order.kColumnMajor)
    cfg = GemmConfig(MatrixLayout("bfloat16", 6, 4), MatrixLayout("bfloat16", 4, 10),
                     out, out)
    plan = BlasLt.get_matmul_plan(cfg, Epilogue.kBiasThenGELU)
    d = plan.describe()
    # D^T (10 x 6) = B^T A^T: m and n exchange, both operands transposed
    assert "m=10 n=6 k=4" in d and "swap=1" in d and "bias=1" in d


def test_execute_refuses_bad_buffers_before_launch():
    cfg = simple_cfg("float32", 4, 5, 6)
    plan = BlasLt.get_matmul_plan(cfg, Epilogue.kBias)
    a = torch.zeros(4, 6)
    b = torch.zeros(6, 5)
    d = torch.zeros(4, 5)
    # host tensors are fine for the checks that run before any launch
    with pytest.raises(qkern.QkError) as e:
        margs = qkern.MemoryArgs(a, b, None, d, None)
        _lib.check(_lib.lib().qk_gemm_execute(plan._h, None,
                                              ctypes.byref(margs.to_c())))
    assert e.value.status == _lib.INVALID_ARGUMENT and "bias" in e.value.message
    with pytest.raises(qkern.QkError) as e:
        margs = qkern.MemoryArgs(a, b, None, torch.zeros(3, 5), torch.zeros(5))
        _lib.check(_lib.lib().qk_gemm_execute(plan._h, None,
                                              ctypes.byref(margs.to_c())))
    assert "D has" in e.value.message
    with pytest.raises(qkern.QkError) as e:
        margs = qkern.MemoryArgs(None, b, None, d, torch.zeros(5))
        _lib.check(_lib.lib().qk_gemm_execute(plan._h, None,
                                              ctypes.byref(margs.to_c())))
    assert "operand A is null" in e.value.message


def test_empty_problem_launches_nothing():
    cfg = simple_cfg("float32", 0, 5, 6)
    plan = BlasLt.get_matmul_plan(cfg)
    margs = qkern.MemoryArgs(torch.zeros(1), torch.zeros(30), None,
                             torch.zeros(1), None)
    _lib.check(_lib.lib().qk_gemm_execute(plan._h, None,
                                          ctypes.byref(margs.to_c())))


def test_ffi_argument_checks():
    from qkern import ffi
    x = torch.zeros(1, 256, dtype=torch.bfloat16)
    words = torch.zeros(8, 32, dtype=torch.int32)
    s = torch.zeros(8, 4, dtype=torch.bfloat16)
    with pytest.raises(qkern.QkError) as e:  # bad group size
        ffi.qmatvec(x, words, s, s, group_size=48)
    assert e.value.status == _lib.UNIMPLEMENTED
    with pytest.raises(qkern.QkError) as e:  # codes too short for K
        ffi.qmatvec(x, words[:, :16].contiguous(), s, s)
    assert e.value.status == _lib.INVALID_ARGUMENT and "codes" in e.value.message
    with pytest.raises(qkern.QkError) as e:  # wrong scale shape
        ffi.qmatvec(x, words, s[:, :2].contiguous(), s)
    assert "scales" in e.value.message
    with pytest.raises(qkern.QkError) as e:  # K not a multiple of the group
        ffi.qmatvec(torch.zeros(1, 100, dtype=torch.bfloat16), words, s, s)
    assert "multiple of the group" in e.value.message
    with pytest.raises(qkern.QkError) as e:  # symmetric int8 with a bias
        ffi.qmatvec(x, torch.zeros(8, 256, dtype=torch.int8), s, s,
                    packing=ffi.Packing.S8_SYM)
    assert "symmetric" in e.value.message
    with pytest.raises(qkern.QkError) as e:  # softmax takes no gain
        ffi.rownorm(torch.zeros(2, 8), ffi.RownormKind.SOFTMAX,
                    gain=torch.zeros(8))
    assert "softmax" in e.value.message
    with pytest.raises(qkern.QkError) as e:  # gain of the wrong length
        ffi.rownorm(torch.zeros(2, 8), ffi.RownormKind.RMS, gain=torch.zeros(7))
    assert "gain" in e.value.message
    # empty inputs are a no-op (no launch)
    ffi.rownorm(torch.zeros(0, 8), ffi.RownormKind.RMS)
    ffi.qmatvec(torch.zeros(0, 256, dtype=torch.bfloat16), words, s, s)


def test_ffi_huge_dims_refused_without_overflow():
    # Dimensions whose product overflows int64 are refused as invalid
    # arguments, never wrapped into a count that passes the shape checks.
    from qkern import ffi

    def buf(dtype, dims, data=16):
        b = _lib.BufferC()
        b.data, b.dtype, b.rank = data, dtype, len(dims)
        for i, d in enumerate(dims):
            b.dims[i] = d
        return b

    attrs = _lib.QuantAttrsC(4, 64, int(ffi.Packing.U32X8), 1)
    huge = 1 << 40
    # x [2^40, 2^40] (2^80 elements, wraps to 0 in int64)
    x = buf(_lib.BF16, [huge, huge])
    codes = buf(_lib.U32, [8, huge // 8])
    s = buf(_lib.BF16, [8, huge // 64])
    y = buf(_lib.BF16, [huge, 8])
    st = _lib.lib().qk_qmatvec(None, ctypes.byref(x), ctypes.byref(codes),
                               ctypes.byref(s), ctypes.byref(s),
                               ctypes.byref(y), ctypes.byref(attrs))
    assert st == _lib.INVALID_ARGUMENT
    assert b"2^56" in _lib.lib().qk_last_error_message()
    # N * K overflows int64 while each buffer is in range: codes
    # [2^35, 1] against K = 2^30 must not pass the element-count check.
    x = buf(_lib.BF16, [1, 1 << 30])
    codes = buf(_lib.U32, [1 << 35, 1])
    st = _lib.lib().qk_qmatvec(None, ctypes.byref(x), ctypes.byref(codes),
                               ctypes.byref(s), ctypes.byref(s),
                               ctypes.byref(y), ctypes.byref(attrs))
    assert st == _lib.INVALID_ARGUMENT
    assert b"codes" in _lib.lib().qk_last_error_message()
    # a zero dimension makes an empty buffer, whatever the others
    r = buf(_lib.F32, [0, 1 << 62], data=0)
    ra = _lib.RownormAttrsC(0, 1e-6, 0, 0)
    assert _lib.lib().qk_rownorm(None, ctypes.byref(r), None, None,
                                 ctypes.byref(r), ctypes.byref(ra)) == _lib.OK


def test_unknown_dtype_refused_everywhere():
    # A binding maps element types with no qk_dtype to -1 (INTEGRATION's
    # ToQk); every target must refuse such a buffer, not reinterpret it.
    from qkern import ffi
    x = torch.zeros(1, 256, dtype=torch.bfloat16)
    words = torch.zeros(8, 32, dtype=torch.int32)
    s = torch.zeros(8, 4, dtype=torch.bfloat16)
    y = torch.zeros(1, 8, dtype=torch.bfloat16)
    attrs = _lib.QuantAttrsC(4, 64, int(ffi.Packing.U32X8), 1)
    for pos in range(5):
        bufs = [ffi.any_buffer(t) for t in (x, words, s, s, y)]
        bufs[pos].dtype = -1
        st = _lib.lib().qk_qmatvec(None, *[ctypes.byref(b) for b in bufs],
                                   ctypes.byref(attrs))
        assert st in (_lib.INVALID_ARGUMENT, _lib.UNIMPLEMENTED), pos
    r = ffi.any_buffer(torch.zeros(2, 8))
    r.dtype = -1
    ra = _lib.RownormAttrsC(0, 1e-6, 0, 0)
    assert _lib.lib().qk_rownorm(None, ctypes.byref(r), None, None,
                                 ctypes.byref(r), ctypes.byref(ra)) == \
        _lib.UNIMPLEMENTED
    out = MatrixLayout("float32", 2, 2)
    cfg = GemmConfig(MatrixLayout("float32", 2, 2), MatrixLayout("float32", 2, 2),
                     out, out)
    c = cfg.to_c()
    c.lhs.dtype = c.rhs.dtype = -1
    h = ctypes.c_void_p()
    assert _lib.lib().qk_gemm_plan_create(ctypes.byref(c), 0, ctypes.byref(h)) \
        == _lib.UNIMPLEMENTED


def test_host_quantizer_matches_oracle():
    import numpy as np
    import oracle as O
    r = np.random.default_rng(11)
    w = r.standard_normal((24, 512)).astype(np.float32)
    codes, s, b = quant.quantize_int4(w)
    oc, os_, ob = O.quantize_int4(w)
    assert np.array_equal(codes, oc.reshape(24, -1))
    assert np.array_equal(s, os_.reshape(24, -1))
    assert np.array_equal(b, ob.reshape(24, -1))
    assert np.array_equal(quant.pack_u32x8(codes), O.pack_u32x8(codes))
    hs = quant.pack_halfsplit(codes)
    assert np.array_equal(hs, O.pack_halfsplit(oc))
    assert np.array_equal(quant.halfsplit_to_u32x8(hs), O.pack_u32x8(codes))
    q8, s8 = quant.quantize_int8(w)
    oq8, os8 = O.quantize_int8(w)
    assert np.array_equal(q8, oq8.reshape(24, -1))
    assert np.array_equal(s8, os8.reshape(24, -1))
    assert np.array_equal(quant.to_bf16_bits(w), O.bf16_bits(w))


def test_decode_attention_argument_checks():
    # shapes, types and workspace are checked before any launch (host
    # tensors stand in for device buffers here)
    q = torch.zeros(1, 8, 4, 128, dtype=torch.bfloat16)
    k = torch.zeros(1, 8, 64, 128, dtype=torch.bfloat16)
    v = torch.zeros(1, 8, 128, 64, dtype=torch.bfloat16)
    pos = torch.zeros(1, dtype=torch.int32)
    need = qkern.decode_attention_workspace_size(q, k)
    # one partial per 64-slot chunk: (D accumulators + max + sum) f32 per
    # query head
    assert need == 8 * 1 * 4 * (128 + 2) * 4

    def status(fn):
        try:
            fn()
            return _lib.OK, ""
        except qkern.QkError as e:
            return e.status, e.message

    ws = torch.zeros(need, dtype=torch.uint8)
    st, msg = status(lambda: qkern.decode_attention(
        q, k, v, pos, workspace=ws[:need - 4]))
    assert st == _lib.INVALID_ARGUMENT and "workspace" in msg
    st, msg = status(lambda: qkern.decode_attention(
        q, k, v.transpose(2, 3).contiguous(), pos, workspace=ws))
    assert st == _lib.INVALID_ARGUMENT and "v_cache" in msg
    st, msg = status(lambda: qkern.decode_attention(
        q.float(), k.float(), v.float(), pos, workspace=ws))
    assert st == _lib.UNIMPLEMENTED
    st, msg = status(lambda: qkern.decode_attention(
        q, k, v, pos.float(), workspace=ws))
    assert st == _lib.INVALID_ARGUMENT and "position" in msg
    st, msg = status(lambda: qkern.decode_attention(
        q, k, v, pos, window=65, workspace=ws))
    assert st == _lib.INVALID_ARGUMENT and "window" in msg
    q96 = torch.zeros(1, 8, 4, 96, dtype=torch.bfloat16)
    st, msg = status(lambda: qkern.decode_attention_workspace_size(
        q96, torch.zeros(1, 8, 64, 96, dtype=torch.bfloat16)))
    assert st == _lib.UNIMPLEMENTED and "head dim" in msg
    st, msg = status(lambda: qkern.decode_attention_workspace_size(
        q, torch.zeros(1, 8, 60, 128, dtype=torch.bfloat16)))
    assert st == _lib.UNIMPLEMENTED and "multiple of 8" in msg
    # long windows run several chunks per wave: about 512 partials in all
    # (64 per KV head here)
    kl = torch.zeros(1, 8, 32768, 128, dtype=torch.bfloat16)
    assert qkern.decode_attention_workspace_size(q, kl) == \
        8 * 64 * 4 * (128 + 2) * 4
    # an empty batch launches nothing
    qkern.decode_attention(q[:0], k[:0], v[:0], pos,
                           workspace=torch.zeros(16, dtype=torch.uint8))


def test_embed_argument_checks():
    # shapes and types are checked before any launch (host tensors stand in
    # for device buffers)
    def status(fn):
        try:
            fn()
            return _lib.OK, ""
        except qkern.QkError as e:
            return e.status, e.message

    codes = torch.zeros(10, 64, dtype=torch.int32)  # [V, K/8], K = 512
    s = torch.zeros(10, 8, dtype=torch.bfloat16)
    tok = torch.zeros(3, dtype=torch.int32)
    st, msg = status(lambda: qkern.embed(codes, tok.float(), s, k=512))
    assert st == _lib.INVALID_ARGUMENT and "int32" in msg
    st, msg = status(lambda: qkern.embed(
        codes, tok, s, k=512, out=torch.zeros(4, 512, dtype=torch.bfloat16)))
    assert st == _lib.INVALID_ARGUMENT and "tokens" in msg
    st, msg = status(lambda: qkern.embed(codes, tok, s, k=256))
    assert st == _lib.INVALID_ARGUMENT
    table = torch.zeros(10, 64, dtype=torch.bfloat16)
    st, msg = status(lambda: qkern.embed(
        table, tok, out=torch.zeros(3, 64, dtype=torch.float32)))
    assert st == _lib.INVALID_ARGUMENT and "dense embedding table" in msg
    # empty token arrays launch nothing
    qkern.embed(table, tok[:0])
