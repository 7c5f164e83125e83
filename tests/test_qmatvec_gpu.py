"""GPU parity of qk$qmatvec and qk$dequantize (qmatvec.hip).

Dequantized weights must match the oracle bit-exactly (canonical rounding
bf16/f16/f32 of f32(f32(q)*f32(s)) + f32(b)). The matvec must be within
1e-2 relative error (Frobenius over the output, and elementwise against
1e-2*|want| + 1e-3*sum_k |x w|) of the float64 product of the dequantized
float32 weights. At the BASELINE.json shapes the reference is the oracle's
C port (float32, the reference's per-group factoring).

The reference ships no test for its quantized path (its only check is a
KL-divergence run that downloads Qwen3 weights), so the cases here cover
the layouts (both 4-bit packings, affine u8, symmetric s8), the activation
types, group sizes, ragged N, single-group K, and M from 1 (decode) to 512
(prefill).
"""

import numpy as np
import pytest
import torch

import oracle as O
import qkern
from qkern import quant
from qkern.ffi import Packing
from helpers import TORCH

pytestmark = pytest.mark.gpu


def make_weights(rng, n, k, packing, group, sdt="bfloat16", has_bias=True):
    """Random codes + scale/offset; returns (device codes, device s, device
    b or None, float32 dequantized weights [N, K])."""
    bits = 4 if packing in (Packing.U32X8, Packing.BYTE_HALFSPLIT) else 8
    if packing == Packing.S8_SYM:
        codes = rng.integers(-127, 128, size=(n, k)).astype(np.int8)
        has_bias = False
    else:
        codes = rng.integers(0, 16 if bits == 4 else 256, size=(n, k)).astype(
            np.uint8)
    s = O.round_to(rng.uniform(0.001, 0.02, (n, k // group)), sdt).astype(
        np.float32)
    b = O.round_to(0.05 * rng.standard_normal((n, k // group)), sdt).astype(
        np.float32) if has_bias else None
    w = O.dequantize_f32(codes.reshape(n, -1, group).astype(np.float32),
                         s[..., None], None if b is None else b[..., None])
    if packing == Packing.U32X8:
        dc = torch.from_numpy(quant.pack_u32x8(codes).view(np.int32))
    elif packing == Packing.BYTE_HALFSPLIT:
        dc = torch.from_numpy(quant.pack_halfsplit(codes, group))
    else:
        dc = torch.from_numpy(codes)
    ds = torch.from_numpy(s).to(TORCH[sdt])
    db = None if b is None else torch.from_numpy(b).to(TORCH[sdt])
    return dc, ds, db, w, codes, s, b


def check_matvec(got, x, w, tol=1e-2):
    want = O.matvec_f64(x, w)
    mag = np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T
    err = np.abs(got - want)
    assert O.rel_fro(got, want) <= tol
    bound = tol * np.abs(want) + 1e-3 * mag
    assert np.all(err <= bound), float(np.max(err - bound))


CASES = [
    # (m, n, k, group)
    (1, 1, 64, 64), (1, 13, 256, 64), (2, 64, 512, 32), (3, 257, 256, 128),
    (4, 100, 4096, 64), (5, 37, 1024, 64), (8, 64, 2048, 64),
    (16, 48, 512, 64), (33, 20, 256, 64), (128, 24, 512, 64),
]


@pytest.mark.parametrize("packing", list(Packing))
@pytest.mark.parametrize("xdt", ["bfloat16", "float16", "float32"])
def test_qmatvec_small(dev, packing, xdt):
    rng = np.random.default_rng(int(packing) * 10 + len(xdt))
    for (m, n, k, group) in CASES:
        if packing == Packing.BYTE_HALFSPLIT and group < 32:
            continue
        dc, ds, db, w, *_ = make_weights(rng, n, k, packing, group)
        x = O.round_to(rng.standard_normal((m, k)), xdt).astype(np.float32)
        dx = torch.from_numpy(x).to(TORCH[xdt]).to(dev)
        y = qkern.qmatvec(dx, dc.to(dev), ds.to(dev),
                          None if db is None else db.to(dev), packing=packing,
                          group_size=group)
        torch.cuda.synchronize()
        assert y.shape == (m, n) and y.dtype == TORCH[xdt]
        check_matvec(y.float().cpu().numpy().astype(np.float64), x, w)


@pytest.mark.parametrize("packing", list(Packing))
@pytest.mark.parametrize("k", [4096, 8192, 12288, 16384])
def test_qmatvec_single_row_paths(dev, packing, k):
    """M = 1, bf16 x, group 64: the int4 and int8 decode kernels for every
    chunks-per-lane count (the general streaming kernel beyond), ragged N,
    with and without offsets; an x that is not 16-byte aligned is
    rejected."""
    rng = np.random.default_rng(k + int(packing))
    for n, has_bias in ((300, True), (77, False)):
        dc, ds, db, w, *_ = make_weights(rng, n, k, packing, 64,
                                         has_bias=has_bias)
        x = O.round_to(rng.standard_normal((1, k)), "bfloat16").astype(
            np.float32)
        base = torch.zeros(k + 8, dtype=torch.bfloat16, device=dev)
        for off in (0, 1):
            dx = base[off:off + k].view(1, k)
            dx.copy_(torch.from_numpy(x).to(torch.bfloat16))
            call = lambda: qkern.qmatvec(dx, dc.to(dev), ds.to(dev),
                                         None if db is None else db.to(dev),
                                         packing=packing, group_size=64)
            if off:
                with pytest.raises(qkern.QkError, match="16-byte aligned"):
                    call()
                continue
            y = call()
            torch.cuda.synchronize()
            check_matvec(y.float().cpu().numpy().astype(np.float64), x, w)


@pytest.mark.parametrize("mnk", [(5, 300, 4096), (8, 77, 1024),
                                 (16, 4096, 4096), (16, 6000, 1024),
                                 (12, 9000, 3072), (16, 12400, 1024),
                                 (7, 12500, 4096), (9, 12400, 5120),
                                 (32, 1000, 512), (27, 9000, 2048),
                                 (33, 64, 1024), (40, 520, 12288),
                                 (64, 2048, 2048)])
@pytest.mark.parametrize("packing", [Packing.U32X8, Packing.U8,
                                     Packing.S8_SYM])
def test_qmatvec_few_rows(dev, mnk, packing):
    """5..64 rows of bf16 x with group-64 int4 u32x8 or int8 codes (the
    streaming MFMA kernels up to 32 rows, the dequantizing paths
    beyond): ragged N, one to four 16-row blocks, long K, with and without
    offsets, elementwise against the float64 oracle. For int4 and at most
    16 rows: the streamed kernel with 16, 32 and 48 weight rows per
    workgroup (N = 4096, 6000, 9000; the last two with a partly filled
    workgroup), the streamed MFMA kernel with x in registers where 48-row
    blocks outnumber the CUs and K <= 4096 (N = 12400, 12500) and the
    register-staged kernel beyond (K = 5120); for
    int4 and 17..32 rows the streamed kernel with two row blocks of x
    (M = 32, 27)."""
    m, n, k = mnk
    rng = np.random.default_rng(m * 7 + n)
    for has_bias in (True, False):
        dc, ds, db, w, *_ = make_weights(rng, n, k, packing, 64,
                                         has_bias=has_bias)
        x = O.round_to(rng.standard_normal((m, k)), "bfloat16").astype(
            np.float32)
        y = qkern.qmatvec(torch.from_numpy(x).to(torch.bfloat16).to(dev),
                          dc.to(dev), ds.to(dev),
                          None if db is None else db.to(dev),
                          packing=packing)
        torch.cuda.synchronize()
        check_matvec(y.float().cpu().numpy().astype(np.float64), x, w)


@pytest.mark.parametrize("mnk", [(65, 64, 256), (100, 1000, 1024),
                                 (128, 3000, 4096), (128, 12288, 512),
                                 (80, 8192, 768), (33, 4100, 2048)])
@pytest.mark.parametrize("packing", [Packing.U32X8, Packing.U8,
                                     Packing.S8_SYM])
def test_qmatvec_mid_rows(dev, mnk, packing):
    """33..128 rows (int8 beyond 32, int4 beyond 64): the kernel that
    dequantizes in registers with K split over the waves of a workgroup —
    16, 32 and 48 weight rows per workgroup (by N), 5..8 row blocks,
    ragged M and N, one to sixteen groups per wave, with and without
    offsets, elementwise against the float64 oracle (the weights rounded
    to bf16 as the reference's dequantize does)."""
    m, n, k = mnk
    rng = np.random.default_rng(m * 13 + n + k)
    for has_bias in (True, False):
        dc, ds, db, w, *_ = make_weights(rng, n, k, packing, 64,
                                         has_bias=has_bias)
        x = O.round_to(rng.standard_normal((m, k)), "bfloat16").astype(
            np.float32)
        y = qkern.qmatvec(torch.from_numpy(x).to(torch.bfloat16).to(dev),
                          dc.to(dev), ds.to(dev),
                          None if db is None else db.to(dev),
                          packing=packing)
        torch.cuda.synchronize()
        check_matvec(y.float().cpu().numpy().astype(np.float64), x,
                     O.round_to(w, "bfloat16"))


@pytest.mark.parametrize("case", [
    (256, 384, 1024, Packing.U32X8, "bfloat16"),
    (512, 1024, 2048, Packing.U8, "bfloat16"),
    (256, 512, 1024, Packing.S8_SYM, "bfloat16"),
    (256, 256, 512, Packing.U32X8, "float16"),
    (2048, 8192, 256, Packing.U32X8, "bfloat16"),  # 256 x 256 tiles
    (512, 12288, 256, Packing.U32X8, "bfloat16"),  # 256 x 128 tiles
    (384, 1024, 512, Packing.U8, "bfloat16"),      # 128 x 128, M % 256 != 0
])
def test_qmatvec_prefill_tiles(dev, case):
    """Row counts that are multiples of 128 (the interior-tile GEMM with
    the dequantizing B loader: 128 x 128, 256 x 128 and 256 x 256 tiles,
    chosen by how many tiles one round of CUs takes), each packing it
    takes, bf16 and f16 x, with and without offsets. Like the reference's linear() for more than
    four rows (examples/llm/qwen3.py:215-230), the weights are dequantized
    to x's type first, so the float64 oracle multiplies by those rounded
    weights."""
    m, n, k, packing, xdt = case
    rng = np.random.default_rng(m + n + k)
    for has_bias in (True, False):
        dc, ds, db, w, *_ = make_weights(rng, n, k, packing, 64,
                                         has_bias=has_bias)
        x = O.round_to(rng.standard_normal((m, k)), xdt).astype(np.float32)
        y = qkern.qmatvec(torch.from_numpy(x).to(TORCH[xdt]).to(dev),
                          dc.to(dev), ds.to(dev),
                          None if db is None else db.to(dev),
                          packing=packing)
        torch.cuda.synchronize()
        check_matvec(y.float().cpu().numpy().astype(np.float64), x,
                     O.round_to(w, xdt))


@pytest.mark.parametrize("case", [
    (2000, 8192, 128, Packing.U32X8, "bfloat16"),  # 256 x 256, 208-row tail
    (1100, 4096, 128, Packing.U8, "bfloat16"),     # 256 x 128, 76-row tail
    (300, 1024, 512, Packing.S8_SYM, "float16"),   # 128 x 128, 44-row tail
    (129, 256, 256, Packing.U32X8, "bfloat16"),    # 128 x 128, one-row tail
    (300, 12288, 256, Packing.U32X8, "bfloat16"),  # 256 x 96, 44-row tail
    (700, 384, 512, Packing.U32X8, "float16"),     # 256 x 128 or 96, f16
])
def test_qmatvec_prefill_ragged_rows(dev, case):
    """Row counts that are not multiples of the interior-tile GEMM's tile
    height: the last M tile is partly filled (x rows past M read as zeros,
    their outputs are not stored). The output is a view into a larger
    buffer whose rows past M must keep their sentinel."""
    m, n, k, packing, xdt = case
    rng = np.random.default_rng(m + 3 * n + k)
    for has_bias in (True, False):
        dc, ds, db, w, *_ = make_weights(rng, n, k, packing, 64,
                                         has_bias=has_bias)
        x = O.round_to(rng.standard_normal((m, k)), xdt).astype(np.float32)
        big = torch.full((m + 300, n), 7.0, dtype=TORCH[xdt], device=dev)
        y = qkern.qmatvec(torch.from_numpy(x).to(TORCH[xdt]).to(dev),
                          dc.to(dev), ds.to(dev),
                          None if db is None else db.to(dev),
                          packing=packing, out=big[:m])
        torch.cuda.synchronize()
        assert bool((big[m:] == 7.0).all()), "rows past M were written"
        check_matvec(y.float().cpu().numpy().astype(np.float64), x,
                     O.round_to(w, xdt))


@pytest.mark.parametrize("packing", [Packing.U32X8, Packing.U8,
                                     Packing.S8_SYM])
def test_qgemm_dma_tiles_and_k_splits(dev, packing, monkeypatch):
    """The register-dequantizing GEMM (qgemm_dma.h) under every tile shape
    (256 x 128, 128 x 256, and 128 x 128 with two wave rows) and K split
    (1, 2, 4, 8: the partial tiles summed in K order by the last workgroup
    of each tile, whichever contributor that is) that fits the packing,
    forced through QK_QGEMM_DMA. M = 100 leaves a ragged last row tile. Every case
    runs twice, so the second call finds the arrival counters the first
    left behind (they must be zero again), and an f16 x case runs once per
    split."""
    m, n, k = 100, 768, 4096
    rng = np.random.default_rng(41 + int(packing))
    dc, ds, db, w, *_ = make_weights(rng, n, k, packing, 64)
    x = O.round_to(rng.standard_normal((m, k)), "bfloat16").astype(np.float32)
    want_w = O.round_to(w, "bfloat16")
    xd = torch.from_numpy(x).to(torch.bfloat16).to(dev)
    args = (dc.to(dev), ds.to(dev), None if db is None else db.to(dev))
    ran = 0
    for cfg in range(3):
        for split in (1, 2, 4, 8):
            monkeypatch.setenv("QK_QGEMM_DMA", f"{cfg},{split}")
            for _ in range(2):
                y = qkern.qmatvec(xd, *args, packing=packing)
                torch.cuda.synchronize()
                check_matvec(y.float().cpu().numpy().astype(np.float64), x,
                             want_w)
            ran += 1
    monkeypatch.delenv("QK_QGEMM_DMA")
    assert ran == 12
    xh = O.round_to(x, "float16").astype(np.float32)
    for split in (1, 4):
        monkeypatch.setenv("QK_QGEMM_DMA", f"2,{split}")
        y = qkern.qmatvec(torch.from_numpy(xh).to(torch.float16).to(dev),
                          *args, packing=packing)
        torch.cuda.synchronize()
        check_matvec(y.float().cpu().numpy().astype(np.float64), xh,
                     O.round_to(w, "float16"))


@pytest.mark.parametrize("packing", [Packing.U32X8, Packing.U8])
def test_qgemm_dma_routing_edges(dev, packing):
    """Row counts at the routing boundary (64: the K-split kernel of the
    workgroup's waves where it applies, 65: the register-dequantizing
    GEMM), one 512-wide K block (no K split possible), a single 128-column
    tile, and many rows (256 x 128 tiles), against the float64 oracle."""
    for m, n, k in ((64, 384, 1024), (65, 384, 1024), (70, 128, 512),
                    (300, 256, 512), (130, 4096, 512)):
        rng = np.random.default_rng(m + n + k)
        dc, ds, db, w, *_ = make_weights(rng, n, k, packing, 64)
        x = O.round_to(rng.standard_normal((m, k)), "bfloat16").astype(
            np.float32)
        y = qkern.qmatvec(torch.from_numpy(x).to(torch.bfloat16).to(dev),
                          dc.to(dev), ds.to(dev), db.to(dev), packing=packing)
        torch.cuda.synchronize()
        check_matvec(y.float().cpu().numpy().astype(np.float64), x,
                     O.round_to(w, "bfloat16"))


def test_qgemm_dma_split_workspace_growth_and_graph(dev, monkeypatch):
    """The K split's library workspace: a small split problem, then one
    needing a larger workspace (a new allocation), then the small one again
    on the same stream; then the larger problem captured into a HIP graph
    on a fresh stream (whose workspace is made first by an eager call on
    it) and replayed three times with eager work between the replays,
    every replay checked against the eager result bit for bit."""
    rng = np.random.default_rng(5)
    cases = []
    for n in (512, 4096):
        dc, ds, db, w, *_ = make_weights(rng, n, 4096, Packing.U32X8, 64)
        x = O.round_to(rng.standard_normal((128, 4096)),
                       "bfloat16").astype(np.float32)
        cases.append((torch.from_numpy(x).to(torch.bfloat16).to(dev),
                      (dc.to(dev), ds.to(dev), db.to(dev)), x,
                      O.round_to(w, "bfloat16")))
    monkeypatch.setenv("QK_QGEMM_DMA", "2,8")  # 128 x 128 tiles, K split 8
    for i in (0, 1, 0):
        xd, args, x, want_w = cases[i]
        y = qkern.qmatvec(xd, *args)
        torch.cuda.synchronize()
        check_matvec(y.float().cpu().numpy().astype(np.float64), x, want_w)
    xd, args, x, want_w = cases[1]
    eager = qkern.qmatvec(xd, *args)
    torch.cuda.synchronize()
    out = torch.empty_like(eager)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        qkern.qmatvec(xd, *args, out=out)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            qkern.qmatvec(xd, *args, out=out)
    torch.cuda.synchronize()
    for _ in range(3):
        out.fill_(7.0)
        qkern.qmatvec(cases[0][0], *cases[0][1])  # eager work between
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_qgemm_dma_split_on_concurrent_streams(dev, monkeypatch):
    """Two streams running K-split problems at the same time (each stream
    has its own workspace and arrival counters): five launches on each,
    interleaved without synchronization, every output equal bit for bit to
    the same problem run alone."""
    rng = np.random.default_rng(9)
    monkeypatch.setenv("QK_QGEMM_DMA", "2,4")  # 128 x 128 tiles, K split 4
    probs = []
    for n in (1024, 2048):
        dc, ds, db, w, *_ = make_weights(rng, n, 4096, Packing.U32X8, 64)
        x = O.round_to(rng.standard_normal((100, 4096)),
                       "bfloat16").astype(np.float32)
        probs.append((torch.from_numpy(x).to(torch.bfloat16).to(dev),
                      (dc.to(dev), ds.to(dev), db.to(dev))))
    alone = [qkern.qmatvec(x, *a) for x, a in probs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [[torch.empty_like(alone[i]) for _ in range(5)] for i in range(2)]
    for st in streams:
        st.wait_stream(torch.cuda.current_stream())
    for r in range(5):
        for i, st in enumerate(streams):
            with torch.cuda.stream(st):
                x, a = probs[i]
                qkern.qmatvec(x, *a, out=outs[i][r])
    torch.cuda.synchronize()
    for i in range(2):
        for o in outs[i]:
            assert torch.equal(o, alone[i])


def test_qmatvec_leading_dims_and_no_bias(dev):
    rng = np.random.default_rng(5)
    dc, ds, _, w, *_ = make_weights(rng, 40, 256, Packing.U32X8, 64,
                                    has_bias=False)
    x = O.round_to(rng.standard_normal((2, 3, 256)), "bfloat16").astype(
        np.float32)
    y = qkern.qmatvec(torch.from_numpy(x).to(torch.bfloat16).to(dev),
                      dc.to(dev), ds.to(dev), None)
    torch.cuda.synchronize()
    assert y.shape == (2, 3, 40)
    check_matvec(y.float().cpu().numpy().reshape(6, 40), x.reshape(6, 256), w)


def test_qmatvec_f32_scales(dev):
    rng = np.random.default_rng(6)
    dc, ds, db, w, *_ = make_weights(rng, 33, 512, Packing.U8, 64,
                                     sdt="float32")
    x = O.round_to(rng.standard_normal((3, 512)), "bfloat16").astype(
        np.float32)
    y = qkern.qmatvec(torch.from_numpy(x).to(torch.bfloat16).to(dev),
                      dc.to(dev), ds.to(dev), db.to(dev), packing=Packing.U8)
    torch.cuda.synchronize()
    check_matvec(y.float().cpu().numpy(), x, w)


def test_qmatvec_reference_quantizer_end_to_end(dev):
    # The reference's own pipeline: quantize_int4 -> half-split bytes, s/b
    # cast to bf16 by put() (qwen3.py:113-128), then _matvec_int4.
    rng = np.random.default_rng(7)
    wf = rng.standard_normal((96, 1024)).astype(np.float32) * 0.05
    codes, s, b = quant.quantize_int4(wf)
    sb, bb = O.bf16_round(s), O.bf16_round(b)
    packed = quant.pack_halfsplit(codes)
    x = O.bf16_round(rng.standard_normal((1, 1024)).astype(np.float32))
    y = qkern.qmatvec(torch.from_numpy(x).to(torch.bfloat16).to(dev),
                      torch.from_numpy(packed).to(dev),
                      torch.from_numpy(sb).to(torch.bfloat16).to(dev),
                      torch.from_numpy(bb).to(torch.bfloat16).to(dev),
                      packing=Packing.BYTE_HALFSPLIT)
    torch.cuda.synchronize()
    want_ref_form = O.matvec_int4_reference_form(
        x, packed.reshape(96, -1, 32), sb.reshape(96, -1, 1),
        bb.reshape(96, -1, 1))
    got = y.float().cpu().numpy()
    assert O.rel_fro(got, want_ref_form) <= 1e-2
    # symmetric int8 path of the same weights
    q8, s8 = quant.quantize_int8(wf)
    s8b = O.bf16_round(s8)
    y8 = qkern.qmatvec(torch.from_numpy(x).to(torch.bfloat16).to(dev),
                       torch.from_numpy(q8).to(dev),
                       torch.from_numpy(s8b).to(torch.bfloat16).to(dev), None,
                       packing=Packing.S8_SYM)
    torch.cuda.synchronize()
    want8 = O.matvec_int8_reference_form(x, q8.reshape(96, -1, 64),
                                         s8b.reshape(96, -1, 1))
    assert O.rel_fro(y8.float().cpu().numpy(), want8) <= 1e-2


@pytest.mark.parametrize("mnk", [(2, 300, 4096), (3, 77, 1024),
                                 (4, 4100, 2048), (2, 12400, 1024),
                                 (4, 13000, 4096), (3, 520, 12288)])
@pytest.mark.parametrize("packing", [Packing.U32X8, Packing.U8,
                                     Packing.S8_SYM])
def test_qmatvec_two_to_four_rows_both_paths(dev, mnk, packing, monkeypatch):
    """2..4 rows of bf16 x (the reference's matvec range, ROWS_MAX = 4,
    qwen3.py:215-230) with group-64 codes: the MFMA streaming kernels (the
    skinny kernel; for int4 over wide N with K <= 4096 the streamed kernel)
    and, with QK_QMV_MFMA_MIN_M=5, the dot-product streams they replace;
    ragged N, with and without offsets, each against the float64 oracle."""
    m, n, k = mnk
    rng = np.random.default_rng(m * 11 + n + int(packing))
    for has_bias in (True, False):
        dc, ds, db, w, *_ = make_weights(rng, n, k, packing, 64,
                                         has_bias=has_bias)
        x = O.round_to(rng.standard_normal((m, k)), "bfloat16").astype(
            np.float32)
        args = (torch.from_numpy(x).to(torch.bfloat16).to(dev), dc.to(dev),
                ds.to(dev), None if db is None else db.to(dev))
        for floor in ("2", "5"):
            monkeypatch.setenv("QK_QMV_MFMA_MIN_M", floor)
            y = qkern.qmatvec(*args, packing=packing)
            torch.cuda.synchronize()
            check_matvec(y.float().cpu().numpy().astype(np.float64), x, w)
        monkeypatch.delenv("QK_QMV_MFMA_MIN_M")


@pytest.mark.parametrize("mnk", [(5, 16400, 512), (16, 12400, 1024),
                                 (9, 20000, 2048), (16, 13000, 4096),
                                 (12, 18990, 4096), (16, 40000, 4096)])
def test_qmatvec_wide_few_rows_both_paths(dev, mnk, monkeypatch):
    """int4, 5..16 rows, N above 48 rows per CU: the streamed MFMA kernel
    with x in registers (K / 512 waves per 16-row block: 1, 2, 4 and 8;
    one ring slot for short runs, four for long ones; ragged last block)
    and the skinny kernels it replaces on long runs (QK_QSTREAM=0), each
    against the float64 oracle."""
    m, n, k = mnk
    rng = np.random.default_rng(n + k)
    for has_bias in (True, False):
        dc, ds, db, w, *_ = make_weights(rng, n, k, Packing.U32X8, 64,
                                         has_bias=has_bias)
        x = O.round_to(rng.standard_normal((m, k)), "bfloat16").astype(
            np.float32)
        args = (torch.from_numpy(x).to(torch.bfloat16).to(dev), dc.to(dev),
                ds.to(dev), None if db is None else db.to(dev))
        for off in ("2", "0"):  # the streamed kernel forced, then off
            monkeypatch.setenv("QK_QSTREAM", off)
            y = qkern.qmatvec(*args)
            torch.cuda.synchronize()
            check_matvec(y.float().cpu().numpy().astype(np.float64), x, w)
        monkeypatch.delenv("QK_QSTREAM")


@pytest.mark.parametrize("packing", list(Packing))
@pytest.mark.parametrize("odt", ["bfloat16", "float16", "float32"])
def test_dequantize_bit_exact(dev, packing, odt):
    rng = np.random.default_rng(8)
    for (n, k, group) in [(7, 64, 64), (33, 512, 32), (16, 1024, 128)]:
        dc, ds, db, w, codes, s, b = make_weights(rng, n, k, packing, group)
        out = qkern.dequantize(dc.to(dev), ds.to(dev),
                               None if db is None else db.to(dev), k=k,
                               packing=packing, group_size=group,
                               dtype=TORCH[odt])
        torch.cuda.synchronize()
        if odt == "bfloat16":
            want = O.bf16_bits(w)
            got = out.view(torch.int16).cpu().numpy().view(np.uint16)
        elif odt == "float16":
            want = w.astype(np.float16).view(np.uint16)
            got = out.view(torch.int16).cpu().numpy().view(np.uint16)
        else:
            want = w.view(np.uint32)
            got = out.view(torch.int32).cpu().numpy().view(np.uint32)
        assert np.array_equal(got, want), (n, k, group)


@pytest.mark.parametrize("packing", list(Packing))
@pytest.mark.parametrize("odt", ["bfloat16", "float32"])
def test_dequantize_into_unaligned_output(dev, packing, odt):
    # an output that is not 16-byte aligned takes element-wise stores: the
    # same bits as the 16-byte stores into an aligned output
    rng = np.random.default_rng(12)
    n, k, group = 9, 256, 32
    dc, ds, db, *_ = make_weights(rng, n, k, packing, group)
    args = (dc.to(dev), ds.to(dev), None if db is None else db.to(dev))
    kw = dict(k=k, packing=packing, group_size=group, dtype=TORCH[odt])
    want = qkern.dequantize(*args, **kw)
    buf = torch.zeros(n * k + 1, dtype=TORCH[odt], device=dev)
    out = buf[1:].view(n, k)
    qkern.dequantize(*args, out=out, **kw)
    torch.cuda.synchronize()
    assert out.data_ptr() % 16 != 0
    assert torch.equal(out, want)
    assert buf[0].item() == 0


def test_dequantize_f32_scale_rounding_unfused(dev):
    # f32 scales: q*s must round in f32 before + b (no fused multiply-add).
    n, k = 4, 64
    codes = np.full((n, k), 15, np.uint8)
    s = np.full((n, 1), 1.0 + 2.0 ** -23, np.float32)
    b = np.full((n, 1), 2.0 ** -22, np.float32)
    out = qkern.dequantize(torch.from_numpy(codes).to(dev),
                           torch.from_numpy(s).to(dev),
                           torch.from_numpy(b).to(dev), k=k,
                           packing=Packing.U8, dtype=torch.float32)
    torch.cuda.synchronize()
    want = O.dequantize_f32(codes.reshape(n, 1, k), s[..., None], b[..., None])
    assert np.array_equal(out.cpu().numpy(), want)


# ---------------------------------------------------------------------------
# BASELINE.json shapes (C4 int8 affine, C5 int4 u32x8) against the C port.

QWEN3_8B = [(4096, 4096), (12288, 4096), (4096, 12288), (151936, 4096)]

_CONFIG_CACHE = {}


def config_weights(dev, n, k, bits):
    """BASELINE config weights (seed 0) as host bit arrays for the C port
    and device tensors for qkern, built once per shape (the lm_head's
    codes take seconds to draw)."""
    key = (n, k, bits)
    if key not in _CONFIG_CACHE:
        if len(_CONFIG_CACHE) >= 2:  # bound host and device memory
            _CONFIG_CACHE.pop(next(iter(_CONFIG_CACHE)))
        codes, s, b = O.config_affine(n, k, bits=bits, seed=0)
        host = O.pack_u32x8(codes) if bits == 4 else codes
        dcodes = torch.from_numpy(host.view(np.int32) if bits == 4 else host)
        _CONFIG_CACHE[key] = dict(
            host=host, s_bits=O.bf16_bits(s), b_bits=O.bf16_bits(b),
            dcodes=dcodes.to(dev),
            ds=torch.from_numpy(s).to(torch.bfloat16).to(dev),
            db=torch.from_numpy(b).to(torch.bfloat16).to(dev))
    return _CONFIG_CACHE[key]


def check_config(got, want, mag, tol=1e-2):
    """Elementwise bound against the C port (float32, the reference's
    factoring): |got - want| <= tol |want| + 1e-3 sum_k |x||w| for every
    checked output, plus the relative Frobenius error."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert np.all(np.isfinite(got))
    assert O.rel_fro(got, want) <= tol
    err = np.abs(got - want)
    bound = tol * np.abs(want) + 1e-3 * mag
    bad = np.argwhere(err > bound)
    assert bad.size == 0, (bad[:5].tolist(), float(np.max(err - bound)))


def run_config_int4(dev, m, n, k, rows, seed):
    wts = config_weights(dev, n, k, 4)
    rng = np.random.default_rng(seed)
    x = O.bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    y = qkern.qmatvec(torch.from_numpy(x).to(torch.bfloat16).to(dev),
                      wts["dcodes"], wts["ds"], wts["db"])
    torch.cuda.synchronize()
    want, mag = O.c_matvec_int4_u32x8(O.bf16_bits(x[rows]), wts["host"],
                                      wts["s_bits"], wts["b_bits"],
                                      with_mag=True)
    check_config(y.float().cpu().numpy()[rows], want, mag)


def config_rows(m):
    """Rows checked at a config: all of them up to 128; beyond, one full
    128-row block that crosses the 256-row tile boundary, plus the first
    and last rows."""
    if m <= 128:
        return np.arange(m)
    return np.r_[0, 192:320, m - 1]


@pytest.mark.parametrize("m", [1, 4, 16, 512])
@pytest.mark.parametrize("nk", QWEN3_8B, ids=[f"{n}x{k}" for n, k in QWEN3_8B])
def test_config_int4(dev, nk, m):
    # every shape at M = 1 (decode), 16 and 512
    # (prefill; the lm_head at M = 512 is a 637 GFLOP fused dequantize +
    # MFMA GEMM).
    n, k = nk
    run_config_int4(dev, m, n, k, config_rows(m), seed={1: 1}.get(m, 2))


def test_config_int4_lm_head_128_rows(dev):
    # 128 rows against the lm_head: N = 151936 is not a multiple of 256, so
    # the GEMM runs 128 x 128 tiles (no 256-row tile, half of whose rows
    # would be padding); rows from the start, middle and end of the tile
    run_config_int4(dev, 128, 151936, 4096, np.r_[0:8, 60:68, 120:128],
                    seed=4)


@pytest.mark.parametrize("m", [1, 4, 8, 128])
def test_config_int8_affine(dev, m):
    n, k = 12288, 4096
    wts = config_weights(dev, n, k, 8)
    rng = np.random.default_rng(3)
    x = O.bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    y = qkern.qmatvec(torch.from_numpy(x).to(torch.bfloat16).to(dev),
                      wts["dcodes"], wts["ds"], wts["db"], packing=Packing.U8)
    torch.cuda.synchronize()
    rows = config_rows(m)
    want, mag = O.c_matvec_u8(O.bf16_bits(x[rows]), wts["host"],
                              wts["s_bits"], wts["b_bits"], with_mag=True)
    check_config(y.float().cpu().numpy()[rows], want, mag)
