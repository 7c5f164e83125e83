"""GPU parity of the BlasLt GEMM (gemm.hip) against the float64 oracle.

Cases follow the reference's device tests:
  - metal_pjrt/blas/steel_gemm_test.cc:225-330 (transposes, unaligned
    shapes, dtype/output combinations, alpha/beta, K = 0, batched/strided/
    broadcast, leading-dimension padding left untouched, tile configs,
    K = 4096), with its tolerance
      |got - want| <= eps(out)*|want| + (1e-5 + 1e-6 K)*sum|a b| + 1e-6;
  - metal_pjrt/blas/metal_blas_lt_test.cc:96-330 (all 12 epilogues x
    f32/f16/bf16 x row/column-major output x {5x7x3, 64x96x36}, batch 2, on
    exact-product inputs), tolerance tol*(1 + |want|), tol = 1e-5 / 4e-3 /
    2e-2 for f32 / f16 / bf16;
  - f32 1024^3 within 1e-5 relative Frobenius error of
    the float64 product; bf16 + bias + SiLU at the Qwen3-8B MLP shapes
    within 1e-2 relative error.
"""

import numpy as np
import pytest
import torch

import oracle as O
import qkern
from qkern.blas import (BlasLt, Epilogue, GemmConfig, MatrixLayout,
                        MemoryArgs, Order)
from helpers import EPS, StoredMatrix, from_dev, to_dev

pytestmark = pytest.mark.gpu


def run_case(dev, m, n, k, batch=1, tin="bfloat16", tout=None, ta=False,
             tb=False, alpha=1.0, beta=0.0, pad=0, broadcast_b=False,
             epilogue=Epilogue.kDefault, separate_c=False, seed=1234):
    tout = tout or tin
    rng = np.random.default_rng(seed)
    A = StoredMatrix(rng, k, m, pad, batch, tin) if ta else \
        StoredMatrix(rng, m, k, pad, batch, tin)
    B = StoredMatrix(rng, n, k, pad, batch, tin, broadcast_b) if tb else \
        StoredMatrix(rng, k, n, pad, batch, tin, broadcast_b)
    D = StoredMatrix(rng, m, n, pad, batch, tout)
    bias_v = O.round_to(rng.uniform(-1, 1, n), tout)
    has_bias, act, has_aux = O.EPILOGUES[int(epilogue)]

    order = lambda t: Order.kColumnMajor if t else Order.kRowMajor
    lhs = MatrixLayout(tin, m, k, order(ta), batch, A.ld, A.stride)
    rhs = MatrixLayout(tin, k, n, order(tb), 1 if broadcast_b else batch, B.ld,
                       B.stride)
    out = MatrixLayout(tout, m, n, Order.kRowMajor, batch, D.ld, D.stride)
    plan = BlasLt.get_matmul_plan(GemmConfig(lhs, rhs, out, out, alpha, beta),
                                  epilogue)
    da, db = to_dev(A.values, tin, dev), to_dev(B.values, tin, dev)
    dd = to_dev(D.values, tout, dev)
    dc = to_dev(D.values, tout, dev) if separate_c else None
    if separate_c:
        dd = to_dev(O.round_to(rng.uniform(-1, 1, D.elems), tout), tout, dev)
    dbias = to_dev(bias_v, tout, dev) if has_bias else None
    daux = torch.full_like(dd, 7.0) if has_aux else None
    plan.execute_on_stream(None, MemoryArgs(da, db, dc, dd, dbias, daux))
    torch.cuda.synchronize()
    got = from_dev(dd)
    aux = from_dev(daux) if has_aux else None

    bad = []
    for bt in range(batch):
        a = A.matrix(bt).T if ta else A.matrix(bt)
        b = B.matrix(bt if not broadcast_b else 0)
        b = b.T if tb else b
        c0 = D.matrix(bt)
        want_act, want = O.gemm_ref(a, b, c0, bias_v if has_bias else None,
                                    alpha, beta, act)
        mag = abs(alpha) * (np.abs(a) @ np.abs(b)) + abs(beta) * np.abs(c0)
        if has_bias:
            mag = mag + np.abs(bias_v)
        tol = EPS[tout] * np.abs(want) + (1e-5 + 1e-6 * k) * mag + 1e-6
        gm = np.zeros((m, n))
        for i in range(m):
            gm[i] = got[bt * D.stride + i * D.ld: bt * D.stride + i * D.ld + n]
        # the activation is at most 1.13-Lipschitz (GELU), 1.1 (SiLU)
        tol_act = EPS[tout] * np.abs(want_act) + 1.2 * tol
        err = np.abs(gm - want_act)
        nan_ok = np.isnan(gm) & np.isnan(want_act)
        if not np.all((err <= tol_act) | nan_ok):
            i, j = np.unravel_index(np.argmax(err - tol_act), err.shape)
            bad.append(f"batch {bt} ({i},{j}): got {gm[i, j]} want "
                       f"{want_act[i, j]}")
        if has_aux:
            am = np.array([aux[bt * D.stride + i * D.ld:
                               bt * D.stride + i * D.ld + n] for i in range(m)])
            if not np.all(np.abs(am - want) <= tol):
                bad.append(f"aux batch {bt}")
        # padding between rows untouched (steel_gemm_test.cc:203-211)
        for i in range(m - 1):
            s = bt * D.stride + i * D.ld
            if not separate_c and not np.array_equal(
                    got[s + n:s + D.ld], D.values[s + n:s + D.ld]):
                bad.append(f"padding clobbered in row {i}")
    assert not bad, (plan.describe(), bad[:5])
    return plan


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
def test_aligned_all_transposes(dev, ta, tb):
    run_case(dev, 128, 128, 64, ta=ta, tb=tb)


UNALIGNED = [(1, 1, 1), (3, 5, 7), (65, 63, 17), (100, 37, 50), (33, 129, 8),
             (130, 70, 300), (7, 200, 1), (64, 64, 15), (257, 31, 33)]


@pytest.mark.parametrize("shape", UNALIGNED)
@pytest.mark.parametrize("tin", ["bfloat16", "float32"])
def test_unaligned_shapes(dev, shape, tin):
    for ta in (False, True):
        for tb in (False, True):
            run_case(dev, *shape, tin=tin, ta=ta, tb=tb)


@pytest.mark.parametrize("combo", [("bfloat16", "bfloat16"),
                                   ("bfloat16", "float32"),
                                   ("float16", "float16"),
                                   ("float16", "float32"),
                                   ("float32", "float32")])
def test_dtypes_and_outputs(dev, combo):
    for m in (64, 77):
        run_case(dev, m, 96, 40, tin=combo[0], tout=combo[1], tb=True)


def test_alpha_beta(dev):
    for tout in ("bfloat16", "float32"):
        for alpha, beta in ((2.0, 0.0), (1.0, 1.0), (0.5, -1.5)):
            for m in (64, 45):
                run_case(dev, m, 64, 32, tout=tout, alpha=alpha, beta=beta)
    # distinct C buffer (D = alpha AB + beta C, C not overwritten)
    run_case(dev, 70, 33, 20, alpha=1.0, beta=0.5, separate_c=True)
    run_case(dev, 70, 33, 20, tin="float32", alpha=1.0, beta=-2.0,
             separate_c=True)


def test_zero_k_gives_beta_c(dev):
    for tin in ("bfloat16", "float32"):
        run_case(dev, 20, 30, 0, tin=tin, beta=0.5)
        run_case(dev, 20, 30, 0, tin=tin)
        run_case(dev, 20, 30, 0, tin=tin, epilogue=Epilogue.kBiasThenSILU)


def test_batched_strided_and_broadcast(dev):
    run_case(dev, 50, 70, 30, batch=5, pad=3)
    run_case(dev, 50, 70, 30, batch=5, pad=3, broadcast_b=True, tb=True)
    run_case(dev, 128, 128, 64, batch=16, beta=1.0)
    run_case(dev, 50, 70, 30, batch=3, pad=2, tin="float32", ta=True)


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
def test_leading_dim_padding(dev, ta, tb):
    run_case(dev, 64, 64, 48, pad=5, ta=ta, tb=tb)
    run_case(dev, 64, 64, 48, pad=5, ta=ta, tb=tb, tin="float16")


@pytest.mark.parametrize("shape,kernel", [
    ((97, 160, 72), "64x64"),
    ((1536, 1536, 72), "64x64"),
    ((2048, 12288, 40), "128x128"),
    ((4096, 4096, 40), "256x256"),
])
def test_all_tile_configs(dev, shape, kernel):
    for ta in (False, True):
        for tb in (False, True):
            m, n, k = shape
            if m > 1000 and (ta or tb) and (ta != tb):
                continue  # keep the large cases to NN and TT
            plan = run_case(dev, m, n, k, ta=ta, tb=tb,
                            beta=1.0 if m % 2 else 0.0)
            assert kernel in plan.describe()
    plan = run_case(dev, 2048, 2048, 40, tin="float32")
    assert "128x128" in plan.describe()


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
def test_interior_tile_kernel(dev, ta, tb):
    """Tile-multiple shapes run the unchecked interior-tile kernel."""
    plan = run_case(dev, 2048, 2048, 128, ta=ta, tb=tb)
    assert "gemm_fast_bf16_256x128" in plan.describe()
    plan = run_case(dev, 4096, 4096, 64, ta=ta, tb=tb, beta=1.0,
                    tin="float16")
    assert "gemm_fast_f16_256x256" in plan.describe()
    # an odd number (5) of K tiles: the loop's unpaired last tile
    plan = run_case(dev, 4096, 2048, 320, ta=ta, tb=tb)
    assert "gemm_fast_bf16" in plan.describe()
    # 256x192 tiles (384 tiles of 256x256 would be 1.5 rounds; 512 of
    # 256x192 are 2): the two-region N-contiguous B tile in NN and TN
    plan = run_case(dev, 2048, 12288, 192, ta=ta, tb=tb)
    assert "gemm_fast_bf16_256x192" in plan.describe()


def test_interior_tile_kernel_epilogues(dev):
    plan = run_case(dev, 2048, 2048, 192, tin="float16",
                    epilogue=Epilogue.kBiasThenSILUWithAux, separate_c=True,
                    beta=0.5)
    assert "gemm_fast" in plan.describe()
    plan = run_case(dev, 2048, 2048, 64, tout="float32", tb=True,
                    epilogue=Epilogue.kBiasThenGELU, alpha=0.5)
    assert "gemm_fast" in plan.describe()
    # batched with 8-element row padding (still 16-byte aligned rows)
    plan = run_case(dev, 1024, 2048, 128, batch=4, pad=8, beta=1.0)
    assert "gemm_fast" in plan.describe()
    plan = run_case(dev, 2048, 12288, 64, tin="float16",
                    epilogue=Epilogue.kBiasThenGELUWithAux, separate_c=True,
                    beta=0.25)
    assert "256x192" in plan.describe()


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
def test_interior_tile_kernel_ragged_m(dev, ta, tb):
    """M not a multiple of 256: the interior-tile kernel with a partly
    filled last M tile (A rows past M read as zeros, output rows past M not
    stored). Batched with packed batch entries, so a row written past M
    would land in the next entry's output."""
    plan = run_case(dev, 2000, 2048, 128, ta=ta, tb=tb)
    assert "gemm_fast_bf16" in plan.describe()
    plan = run_case(dev, 1000, 4096, 64, batch=4, ta=ta, tb=tb, beta=1.0,
                    tin="float16", epilogue=Epilogue.kBiasThenSILUWithAux)
    assert "gemm_fast_f16" in plan.describe()
    plan = run_case(dev, 104, 12288, 128, batch=3, ta=ta, tb=tb,
                    epilogue=Epilogue.kBiasThenGELU)
    assert "gemm_fast_bf16" in plan.describe()


def test_interior_tile_kernel_not_taken(dev):
    # rows not 16-byte aligned, K not a multiple of 64
    for kw in (dict(m=2048, n=2048, k=128, pad=3), dict(m=2048, n=2048, k=96)):
        kw = dict(kw)
        plan = run_case(dev, kw.pop("m"), kw.pop("n"), kw.pop("k"), **kw)
        assert "gemm_tile" in plan.describe()


@pytest.mark.parametrize("epilogue", [Epilogue.kReLU, Epilogue.kGELU,
                                      Epilogue.kSILU])
def test_activation_special_values(dev, epilogue):
    """K = 1 and A = 1, so the pre-activation is exactly B: the activation
    over zeros, signed zeros, saturating magnitudes, infinities and NaN, in
    f32 within 1e-5 (NaN where the quotient forms give NaN)."""
    vals = np.array([0.0, -0.0, 1e-30, -1e-30, 0.5, -0.5, 1.0, -1.0, 3.0,
                     -3.0, 20.0, -20.0, 88.0, -88.0, 100.0, -100.0, 1e20,
                     -1e20, np.inf, -np.inf, np.nan, 1e-3, -1e-3, 7.25],
                    dtype=np.float32)
    n = vals.size
    m = 3
    a = torch.ones(m, 1, dtype=torch.float32, device=dev)
    b = torch.from_numpy(vals.reshape(1, n)).to(dev)
    lay = lambda r, c: MatrixLayout("float32", r, c)
    plan = BlasLt.get_matmul_plan(
        GemmConfig(lay(m, 1), lay(1, n), lay(m, n), lay(m, n)), epilogue)
    d = torch.empty(m, n, dtype=torch.float32, device=dev)
    plan.execute_on_stream(None, MemoryArgs(a, b, None, d))
    torch.cuda.synchronize()
    _, act, _ = O.EPILOGUES[int(epilogue)]
    with np.errstate(all="ignore"):
        want = O.ACTS[act](vals.astype(np.float64))
    got = d.cpu().numpy().astype(np.float64)
    for row in got:
        same_nan = np.isnan(row) == np.isnan(want)
        assert same_nan.all(), (vals[~same_nan], row[~same_nan])
        with np.errstate(invalid="ignore"):
            ok = np.isnan(want) | (row == want) | \
                (np.abs(row - want) <= 1e-5 * (np.abs(want) + 1e-30))
        assert ok.all(), list(zip(vals[~ok], row[~ok], want[~ok]))


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
def test_split_k_kernel(dev, ta, tb):
    """Few output tiles and a long K run the split-K kernel (each wave a
    quarter of K, reduced through LDS): ragged M/N/K, all transposes."""
    plan = run_case(dev, 80, 520, 2048, ta=ta, tb=tb)
    assert "gemm_splitk4" in plan.describe()
    plan = run_case(dev, 100, 260, 1500, ta=ta, tb=tb, tin="float16",
                    beta=0.5)
    assert "gemm_splitk4" in plan.describe()


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
def test_split_k_kernel_few_rows(dev, ta, tb):
    """At most 64 rows (or columns): 32x32 tiles, eight waves over K
    (sixteen for at most 16 rows against NT weights)."""
    plan = run_case(dev, 16, 700, 2048, ta=ta, tb=tb)
    want = "gemm_splitk16" if (not ta and tb) else "gemm_splitk8"
    assert want in plan.describe()
    plan = run_case(dev, 11, 130, 1088, ta=ta, tb=tb, tin="float16",
                    epilogue=Epilogue.kBiasThenGELU, beta=0.5)
    assert want in plan.describe()
    plan = run_case(dev, 64, 512, 2048, ta=ta, tb=tb)
    assert "gemm_splitk8" in plan.describe()
    plan = run_case(dev, 61, 1030, 1024, ta=ta, tb=tb, tin="float16")
    assert "gemm_splitk8" in plan.describe()
    plan = run_case(dev, 300, 5, 1100, ta=ta, tb=tb, tin="float16",
                    epilogue=Epilogue.kBiasThenSILU)
    assert "gemm_splitk8" in plan.describe()


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
def test_fast_tiles_k_split(dev, ta, tb):
    """Few 256 x 128 tiles and more than 64 rows: the LDS-DMA tile kernel
    with K split over workgroups, partials summed in K order by the last
    workgroup of each tile (ragged M, every epilogue term, f32 output)."""
    plan = run_case(dev, 200, 1024, 8192, ta=ta, tb=tb)
    assert "gemm_fast" in plan.describe() and "_ks8" in plan.describe()
    plan = run_case(dev, 296, 512, 8192, ta=ta, tb=tb, tin="float16",
                    epilogue=Epilogue.kBiasThenSILUWithAux, separate_c=True,
                    beta=0.5, alpha=1.5, pad=8)
    assert "_ks8" in plan.describe()
    plan = run_case(dev, 72, 128, 8192, ta=ta, tb=tb, tout="float32",
                    epilogue=Epilogue.kBiasThenGELU)
    assert "_ks8" in plan.describe()
    # 64 x 64 split-K workgroups beyond one round: 384 x 4096 x 4096
    plan = run_case(dev, 384, 4096, 4096, ta=ta, tb=tb)
    assert "_ks4" in plan.describe()


def test_fast_tiles_k_split_forced_and_repeated(dev, monkeypatch):
    # uneven K ranges (32 K tiles in 3 and 5 parts), one K tile per part,
    # and the arrival counters reset for the next launch: the same plan
    # executed twice in a row on the same stream
    for split, k in (("3", 2048), ("5", 2048), ("16", 1024)):
        monkeypatch.setenv("QK_GEMM_KSPLIT", split)
        plan = run_case(dev, 130, 256, k, tb=True, seed=int(split))
        assert f"_ks{split}" in plan.describe()
        plan = run_case(dev, 130, 256, k, tb=True, seed=int(split))
    monkeypatch.setenv("QK_GEMM_KSPLIT", "0")
    plan = run_case(dev, 200, 1024, 2048)
    assert "_ks" not in plan.describe()
    monkeypatch.delenv("QK_GEMM_KSPLIT")


def test_fast_tiles_k_split_half_filled(dev):
    # 1024 x 4096 x 12288: 128 tiles of 256 x 128 would leave half the CUs
    # idle, so K is split in two; checked against a float32 torch matmul
    from qkern import blas as L
    m, n, k = 1024, 4096, 12288
    g = torch.Generator(device=dev).manual_seed(9)
    x = torch.randn(m, k, device=dev, generator=g).to(torch.bfloat16)
    w = (torch.randn(k, n, device=dev, generator=g) / 64).to(torch.bfloat16)
    bias = torch.randn(n, device=dev, generator=g).to(torch.bfloat16)
    y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
    plan = L.BlasLt.get_matmul_plan(
        L.GemmConfig(L.MatrixLayout("bfloat16", m, k),
                     L.MatrixLayout("bfloat16", k, n),
                     L.MatrixLayout("bfloat16", m, n),
                     L.MatrixLayout("bfloat16", m, n)), L.Epilogue.kBias)
    assert "_ks2" in plan.describe()
    plan.execute_on_stream(None, L.MemoryArgs(x, w, None, y, bias))
    torch.cuda.synchronize()
    ref = x.float() @ w.float() + bias.float()
    err = (y.float() - ref).abs()
    # one bf16 rounding of the output over an f32 sum
    assert (err <= 2 ** -8 * ref.abs() + 1e-3 * ref.abs().max()).all()


def test_fast_tiles_k_split_graph_replay(dev):
    # captured into a HIP graph after an eager call on the capturing stream
    # (its workspace exists), replayed three times with an eager K-split
    # GEMM of another shape on that stream between the replays, each replay
    # against the eager result
    from qkern import blas as L

    def setup(m, n, k, seed):
        g = torch.Generator(device=dev).manual_seed(seed)
        x = torch.randn(m, k, device=dev, generator=g).to(torch.bfloat16)
        w = torch.randn(k, n, device=dev, generator=g).to(torch.bfloat16)
        y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
        plan = L.BlasLt.get_matmul_plan(
            L.GemmConfig(L.MatrixLayout("bfloat16", m, k),
                         L.MatrixLayout("bfloat16", k, n),
                         L.MatrixLayout("bfloat16", m, n),
                         L.MatrixLayout("bfloat16", m, n)),
            L.Epilogue.kDefault)
        return plan, L.MemoryArgs(x, w, None, y), x, w, y

    plan, args, x, w, y = setup(200, 1024, 8192, 5)
    plan2, args2, *_ = setup(296, 512, 8192, 6)
    assert "_ks8" in plan.describe() and "_ks8" in plan2.describe()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        plan.execute_on_stream(s, args)
    torch.cuda.synchronize()
    want = y.clone()
    ref = x.float() @ w.float()
    assert ((want.float() - ref).abs() <= 2e-2 * ref.abs() + 2e-2).all()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            plan.execute_on_stream(s, args)
    torch.cuda.synchronize()
    for _ in range(3):
        y.fill_(7.0)
        with torch.cuda.stream(s):
            plan2.execute_on_stream(s, args2)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want)


@pytest.mark.parametrize("m", [1, 2, 3, 5, 8])
@pytest.mark.parametrize("k", [512, 1024, 2048])
def test_wide_gemv_few_rows(dev, m, k):
    """At most eight rows of x against NT weights with K a multiple of 512
    (the reference's wide gemv: gemv.cc:68-108 takes 2..8 vectors, K >= 512,
    NT): the bandwidth-bound gemv kernel, with ragged N and both types."""
    if m * (k // 512) > 16:  # x rows no longer fit the registers
        plan = run_case(dev, m, 77, k, tb=True)
        assert "gemv_nt" not in plan.describe()
        return
    # 7..16 rows with K >= 1024: the sixteen-wave split-K kernel instead
    want = "gemm_splitk16" if m > 6 and k >= 1024 else "gemv_nt"
    for n, tin in ((77, "bfloat16"), (1000, "float16"), (6144, "bfloat16")):
        plan = run_case(dev, m, n, k, tb=True, tin=tin, seed=m * k + n)
        assert want in plan.describe(), plan.describe()


@pytest.mark.parametrize("m", [1, 2, 3, 4])
@pytest.mark.parametrize("k", [512, 2048, 8192])
def test_gemv_nn_few_rows(dev, m, k, monkeypatch):
    """At most four rows of x against W stored [K][N] (N a multiple of
    8, K of 512): the NN gemv (one workgroup per 64 columns over all of
    K; forced here, taken by default for weights of 2^25 values or more),
    ragged last column block, both types, against the oracle."""
    monkeypatch.setenv("QK_GEMV_NN", "2")
    for n, tin in ((8, "bfloat16"), (1000, "float16"), (6144, "bfloat16")):
        plan = run_case(dev, m, n, k, tin=tin, seed=m * k + n + 1)
        assert "gemv_nn" in plan.describe(), plan.describe()


def test_gemv_nn_epilogues_batches_and_layouts(dev, monkeypatch):
    # every epilogue term, f32 output, alpha / beta with a separate C,
    # padded leading dimensions, batches with strides and a broadcast W
    monkeypatch.setenv("QK_GEMV_NN", "2")
    for epi in (Epilogue.kBiasThenSILUWithAux, Epilogue.kBiasThenGELU,
                Epilogue.kReLU, Epilogue.kBias):
        plan = run_case(dev, 4, 296, 1024, epilogue=epi, separate_c=True,
                        beta=0.5, alpha=1.5)
        assert "gemv_nn" in plan.describe()
    plan = run_case(dev, 3, 136, 512, tout="float32", pad=8, batch=3,
                    beta=1.0)
    assert "gemv_nn" in plan.describe()
    plan = run_case(dev, 3, 1000, 4096, batch=4, broadcast_b=True,
                    tin="float16", epilogue=Epilogue.kBiasThenReLU)
    assert "gemv_nn" in plan.describe()
    # off the grid (N not a multiple of 8, K of 512), or turned off: the
    # split-K kernel
    assert "gemv_nn" not in run_case(dev, 4, 700, 1024).describe()
    assert "gemv_nn" not in run_case(dev, 4, 704, 1000).describe()
    assert "gemv_nn" not in run_case(dev, 5, 704, 1024).describe()
    monkeypatch.setenv("QK_GEMV_NN", "0")
    assert "gemv_nn" not in run_case(dev, 2, 4096, 8192).describe()
    monkeypatch.delenv("QK_GEMV_NN")
    # by default from 2^25 weight values
    assert "gemv_nn" in run_case(dev, 2, 4096, 8192).describe()
    assert "gemv_nn" not in run_case(dev, 2, 4096, 4096).describe()


def test_wide_gemv_epilogues_batches_and_layouts(dev):
    # every epilogue term, f32 output, alpha / beta with a separate C,
    # padded leading dimensions, batches with strides and a broadcast B
    for epi in (Epilogue.kBiasThenSILUWithAux, Epilogue.kBiasThenGELU,
                Epilogue.kReLU, Epilogue.kBias):
        plan = run_case(dev, 4, 300, 1024, tb=True, epilogue=epi,
                        separate_c=True, beta=0.5, alpha=1.5)
        assert "gemv_nt" in plan.describe()
    plan = run_case(dev, 8, 129, 512, tb=True, tout="float32", pad=8,
                    batch=3, beta=1.0)
    assert "gemv_nt" in plan.describe()
    plan = run_case(dev, 2, 1000, 2048, tb=True, batch=4, broadcast_b=True,
                    tin="float16", epilogue=Epilogue.kBiasThenReLU)
    assert "gemv_nt" in plan.describe()
    # not NT, or K off the 512 grid: the split-K kernel as before
    plan = run_case(dev, 4, 700, 1024)
    assert "gemv_nt" not in plan.describe()
    plan = run_case(dev, 4, 700, 1000, tb=True)
    assert "gemv_nt" not in plan.describe()


def test_split_k_kernel_epilogues(dev):
    plan = run_case(dev, 32, 1000, 4096, epilogue=Epilogue.kBiasThenSILUWithAux,
                    separate_c=True, beta=1.0)
    assert "gemm_splitk8" in plan.describe()
    plan = run_case(dev, 48, 384, 1024, batch=3, pad=8, tout="float32",
                    epilogue=Epilogue.kBiasThenGELU)
    assert "gemm_splitk8" in plan.describe()
    plan = run_case(dev, 96, 384, 1024, batch=3, pad=8, tout="float32",
                    epilogue=Epilogue.kBiasThenGELU)
    assert "gemm_splitk4" in plan.describe()


def test_large_k(dev):
    run_case(dev, 64, 64, 4096, tout="float32")
    run_case(dev, 64, 64, 4096, tin="float32")


# ---------------------------------------------------------------------------
# metal_blas_lt_test.cc: every epilogue x dtype x output order x shape.


def exact_inputs(batch, m, n, k, bias_len):
    a = np.array([((i * 7) % 9) * 0.25 - 1.0 for i in range(batch * m * k)])
    b = np.array([((i * 5) % 11) * 0.25 - 1.25 for i in range(batch * k * n)])
    bias = np.array([0.5 * i - 1.0 for i in range(bias_len)])
    return a, b, bias


@pytest.mark.parametrize("epilogue", list(Epilogue))
@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("order", [Order.kRowMajor, Order.kColumnMajor])
@pytest.mark.parametrize("shape", [(5, 7, 3), (64, 96, 36)])
def test_epilogues_like_reference(dev, epilogue, dtype, order, shape):
    m, n, k = shape
    batch = 2
    bias_len = n if order == Order.kRowMajor else m
    a, b, bias = exact_inputs(batch, m, n, k, bias_len)
    has_bias, act, has_aux = O.EPILOGUES[int(epilogue)]
    out_layout = MatrixLayout(dtype, m, n, order, batch)
    cfg = GemmConfig(MatrixLayout(dtype, m, k, Order.kRowMajor, batch),
                     MatrixLayout(dtype, k, n, Order.kRowMajor, batch),
                     out_layout, out_layout)
    plan = BlasLt.get_matmul_plan(cfg, epilogue)
    da, db = to_dev(a, dtype, dev), to_dev(b, dtype, dev)
    dbias = to_dev(O.round_to(bias, dtype), dtype, dev)
    dd = torch.zeros(batch * m * n, dtype=da.dtype, device=dev)
    daux = torch.zeros_like(dd)
    plan.execute_on_stream(None, MemoryArgs(da, db, None, dd,
                                            dbias if has_bias else None,
                                            daux if has_aux else None))
    torch.cuda.synchronize()
    got, got_aux = from_dev(dd), from_dev(daux)
    tol = {"float32": 1e-5, "float16": 4e-3, "bfloat16": 2e-2}[dtype]
    ar, br = O.round_to(a, dtype), O.round_to(b, dtype)
    for bt in range(batch):
        A = ar[bt * m * k:(bt + 1) * m * k].reshape(m, k)
        B = br[bt * k * n:(bt + 1) * k * n].reshape(k, n)
        pre = A @ B
        if has_bias:
            bv = O.round_to(bias, dtype)
            pre = pre + (bv[None, :] if order == Order.kRowMajor else
                         bv[:, None])
        want = O.ACTS[act](pre)
        g = got[bt * m * n:(bt + 1) * m * n]
        g = g.reshape(m, n) if order == Order.kRowMajor else g.reshape(n, m).T
        assert np.all(np.abs(g - want) <= tol * (1 + np.abs(want))), \
            (plan.describe(), np.max(np.abs(g - want)))
        if has_aux:
            ga = got_aux[bt * m * n:(bt + 1) * m * n]
            ga = ga.reshape(m, n) if order == Order.kRowMajor else \
                ga.reshape(n, m).T
            assert np.all(np.abs(ga - pre) <= tol * (1 + np.abs(pre)))


# ---------------------------------------------------------------------------
# BASELINE configs at full size.


def test_config_f32_1024_cubed(dev):
    a, b = O.config_gemm_f32(0, 1024)
    da, db = torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev)
    d = qkern.matmul(da, db)
    torch.cuda.synchronize()
    want = a.astype(np.float64) @ b.astype(np.float64)
    err = O.rel_fro(d.cpu().numpy(), want)
    assert err <= 1e-5, err


@pytest.mark.parametrize("shape", [(4096, 4096, 4096), (2048, 12288, 4096),
                                   (2048, 4096, 12288)])
def test_config_bf16_bias_silu(dev, shape):
    # A, B ~ N(0,1)/sqrt(K) and bias ~ N(0, 0.02) from
    # numpy default_rng seeds 0, 1 and 2, rounded to bf16.
    m, n, k = shape
    a = O.bf16_round((np.random.default_rng(0).standard_normal(
        (m, k), dtype=np.float32) / np.float32(k ** 0.5)))
    b = O.bf16_round((np.random.default_rng(1).standard_normal(
        (k, n), dtype=np.float32) / np.float32(k ** 0.5)))
    bias = O.bf16_round(0.02 * np.random.default_rng(2).standard_normal(
        n, dtype=np.float32))
    d = qkern.matmul(torch.from_numpy(a).to(torch.bfloat16).to(dev),
                     torch.from_numpy(b).to(torch.bfloat16).to(dev),
                     torch.from_numpy(bias).to(torch.bfloat16).to(dev),
                     epilogue=Epilogue.kBiasThenSILU)
    torch.cuda.synchronize()
    # float64 oracle on 512 rows (the full float64 product is 137-206
    # GFLOP): the first and last 128 rows and a 256-row block across the
    # middle tile boundary.
    rows = np.r_[0:128, m // 2 - 128:m // 2 + 128, m - 128:m]
    a64 = a[rows].astype(np.float64)
    want, v = O.gemm_ref(a64, b, None, bias, act=3)
    got = d[torch.from_numpy(rows).to(dev)].float().cpu().numpy()
    assert np.all(np.isfinite(got))
    err = O.rel_fro(got, want)
    assert err <= 1e-2, err
    # elementwise: bf16 output rounding (2^-9 relative) plus f32
    # accumulation, scaled by sum_k |a||b| (SiLU' is below 1.1)
    mag = np.abs(a64) @ np.abs(b.astype(np.float64)) + np.abs(bias)
    bound = 1e-2 * np.abs(want) + 1e-3 * mag
    over = np.abs(got - want) - bound
    assert np.all(over <= 0), float(over.max())


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
def test_f32_split_kernel(dev, ta, tb):
    """f32 interior tiles run on the bf16 matrix cores with each operand
    split into three bf16 parts (gemm_f32x3.h); the product must still
    meet the f32 tolerance: 64x64 tiles (few tiles), 128x128 tiles (a full
    GPU of them), K of one and of several 32-wide tiles, batched with
    padded leading dimensions, alpha / beta and an epilogue."""
    plan = run_case(dev, 256, 192, 32, tin="float32", ta=ta, tb=tb)
    assert "gemm_f32x3_f32_64x64" in plan.describe()
    plan = run_case(dev, 2048, 2048, 96, tin="float32", ta=ta, tb=tb,
                    alpha=0.5, beta=1.0)
    assert "gemm_f32x3_f32_128x128" in plan.describe()
    plan = run_case(dev, 128, 64, 160, batch=3, pad=4, tin="float32", ta=ta,
                    tb=tb, epilogue=Epilogue.kBiasThenGELUWithAux,
                    separate_c=True, beta=0.25)
    assert "gemm_f32x3" in plan.describe()


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
def test_f32_split_kernel_ragged_m(dev, ta, tb):
    """M not a multiple of the split kernel's tile height: a partly
    filled last M tile. Batched with packed batch entries, so a row written
    past M would land in the next entry's output."""
    plan = run_case(dev, 1000, 2048, 64, tin="float32", ta=ta, tb=tb)
    assert "gemm_f32x3_f32_64x64" in plan.describe()
    plan = run_case(dev, 2000, 2048, 96, tin="float32", ta=ta, tb=tb)
    assert "gemm_f32x3_f32_128x128" in plan.describe()
    plan = run_case(dev, 100, 128, 64, batch=3, tin="float32", ta=ta, tb=tb,
                    beta=1.0, epilogue=Epilogue.kBiasThenSILUWithAux)
    assert "gemm_f32x3_f32_64x64" in plan.describe()


def test_f32_split_kernel_special_values(dev):
    """Infinities and NaNs reach the output as in an f32 product: the
    split keeps an infinite element whole in its leading part."""
    m = n = k = 64
    a = torch.ones(m, k, dtype=torch.float32, device=dev)
    b = torch.full((k, n), 0.5, dtype=torch.float32, device=dev)
    a[3, 5] = float("inf")
    a[7, 1] = float("-inf")
    b[2, 9] = float("nan")
    a[10, 0] = 3.4e38  # near the f32 maximum: the parts must stay finite
    a[11, 4] = float("nan")
    lay = lambda r, c: MatrixLayout("float32", r, c)
    plan = BlasLt.get_matmul_plan(
        GemmConfig(lay(m, k), lay(k, n), lay(m, n), lay(m, n)),
        Epilogue.kDefault)
    d = torch.empty(m, n, dtype=torch.float32, device=dev)
    plan.execute_on_stream(None, MemoryArgs(a, b, None, d))
    torch.cuda.synchronize()
    assert "gemm_f32x3" in plan.describe()
    want = a.double().cpu().numpy() @ b.double().cpu().numpy()
    got = d.cpu().numpy().astype(np.float64)
    fin = np.isfinite(want)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isposinf(got), np.isposinf(want))
    assert np.array_equal(np.isneginf(got), np.isneginf(want))
    assert np.allclose(got[fin], want[fin], rtol=1e-6, atol=0)
