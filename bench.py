#!/usr/bin/env python3
"""Benchmark of the qkern hot path on one MI355X.

Headline (`value`): int4 group-64 GEMV throughput at the Qwen3-8B decode
projection shapes (M = 1; N x K = 4096x4096, 12288x4096, 4096x12288 and the
151936x4096 lm_head), the first half of BASELINE.json's metric. One step =
one qk$qmatvec launch per shape, weights already resident in HBM. Three
copies of the weight set (1.25 GB) are rotated so that no launch reads
weights another launch left in the 256 MB Infinity Cache.

Also reported (`secondary`): bf16 GEMM + bias + SiLU TFLOP/s at the C3
shapes (the metric's second half, beside hipBLASLt), bf16 GEMM at
prefill row counts whose tiles alone would not fill the CUs (beside
hipBLASLt), f32 GEMM 1024^3, int4 M = 4 / 16 / 512 at the four Qwen3-8B
shapes, int8 affine M = 1 / 4 / 8 / 128,
RMSNorm, softmax and LayerNorm [4096, 4096], the reference's few-row GEMM
list, decode attention, the int4 embedding gather, device quantization of
a projection and device copies (the read + write ceiling); each against
its roofline. `--only PART,...` runs chosen secondary parts alone.

Timing: the W warm-up steps and the K timed steps are each captured into a
HIP graph (the launches only: outputs are preallocated, nothing is
allocated or cleared inside); the timed graph is replayed once between two
HIP events on the replaying stream, bracketed by torch.cuda.synchronize().
Wall-clock time over the same region gives `value`.

CPU baseline: the oracle's C port of the reference's _matvec_int4
(oracle/qk_oracle.c, float32, OpenMP over output rows) on the host cores,
on a bounded sample of the same workload.
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "metal-pjrt-plugin_amd"))

HBM_PEAK_GBS = 8000.0
F32_PEAK_TFLOPS = 157.3
BF16_PEAK_TFLOPS = 2500.0  # dense MFMA
QWEN3_8B = [(4096, 4096), (12288, 4096), (4096, 12288), (151936, 4096)]
GROUP = 64


def int4_bytes(m, n, k):
    """Algorithmic bytes of one int4 g64 qmatvec: codes (K/2 B per row),
    bf16 scale + bias per group, x and y in bf16, each read/written once."""
    return n * k // 2 + n * (k // GROUP) * 4 + m * k * 2 + m * n * 2


def int8_bytes(m, n, k):
    return n * k + n * (k // GROUP) * 4 + m * k * 2 + m * n * 2


def make_int4(torch, dev, n, k, gen):
    words = torch.randint(-2 ** 31, 2 ** 31 - 1, (n, k // 8), dtype=torch.int32,
                          device=dev, generator=gen)
    s = (torch.rand(n, k // GROUP, device=dev, generator=gen) * 0.019 +
         0.001).to(torch.bfloat16)
    b = (0.05 * torch.randn(n, k // GROUP, device=dev, generator=gen)).to(
        torch.bfloat16)
    return words, s, b


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles",
                               "int4_gemv_qwen3_8b_decode.md")


def profiled_traffic():
    """HBM bytes per launch of the headline kernel, from the committed
    rocprofv3 FETCH_SIZE/WRITE_SIZE summary (None when absent)."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1])
    except (OSError, ValueError):
        pass
    return None


def capture(torch, fn, iters):
    """A HIP graph of fn(0), ..., fn(iters - 1) (pure kernel launches: no
    allocation, memset or host synchronization inside). fn(0) runs once on
    the capture stream first, so that per-stream state the library keeps
    (its split-K workspace) exists before the capture."""
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn(0)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for i in range(iters):
                fn(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    return g


def timed_launches(torch, fn, iters):
    """Average device time (ms) per call of fn over `iters` back-to-back
    calls replayed from a HIP graph, from two HIP events recorded on the
    replaying stream around the replay (after one untimed replay)."""
    g = capture(torch, fn, iters)
    g.replay()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters


def gemm_vs_library(torch, ours, library, iters=20, reps=4, warm_s=0.25):
    """Median ms per launch of `ours` (graph-replayed, as timed_launches)
    and of `library` (eager: library calls may record memsets, so they are
    kept out of graphs), timed in alternating blocks after `warm_s` seconds
    of `ours`: the clocks of a long GEMM settle with the power draw, so
    both are timed in the same, settled state, and neither always first."""
    g = capture(torch, ours, iters)
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < warm_s:
        g.replay()
        torch.cuda.synchronize()

    def block(fn):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / iters

    def lib_block():
        for _ in range(iters):
            library()
    mine, lib = [], []
    for rep in range(reps):
        if rep % 2 == 0:
            mine.append(block(g.replay))
            lib.append(block(lib_block))
        else:
            lib.append(block(lib_block))
            mine.append(block(g.replay))
    return sorted(mine)[reps // 2], sorted(lib)[reps // 2]


# Secondary parts to run (bench.py --only PART[,PART]); all by default.
ONLY = None


def want(part):
    return ONLY is None or part in ONLY


def secondary(torch, qkern, dev, gen):
    out = []
    if want("gemm"):
        # bf16 GEMM + bias + SiLU (C3), NN row-major: D = silu(A @ B + bias)
        for (m, n, k) in [(4096, 4096, 4096), (2048, 12288, 4096),
                          (2048, 4096, 12288)]:
            a = (torch.randn(m, k, device=dev, generator=gen) / k ** 0.5).to(
                torch.bfloat16)
            b = (torch.randn(k, n, device=dev, generator=gen) / k ** 0.5).to(
                torch.bfloat16)
            bias = (0.02 * torch.randn(n, device=dev, generator=gen)).to(
                torch.bfloat16)
            d = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
            L = qkern.blas
            lay = lambda r, c: L.MatrixLayout("bfloat16", r, c)
            plan = L.BlasLt.get_matmul_plan(
                L.GemmConfig(lay(m, k), lay(k, n), lay(m, n), lay(m, n)),
                L.Epilogue.kBiasThenSILU)
            args = L.MemoryArgs(a, b, None, d, bias)
            for _ in range(3):
                plan.execute_on_stream(None, args)
            # hipBLASLt (torch.matmul, no epilogue) on the same operands, timed
            # alternately with it
            ms, ms_lt = gemm_vs_library(
                torch, lambda i: plan.execute_on_stream(None, args),
                lambda: torch.matmul(a, b, out=d))
            tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
            out.append({"name": f"bf16 gemm+bias+silu {m}x{n}x{k}",
                        "value": round(tf, 1), "unit": "TFLOP/s",
                        "ms": round(ms, 4), "frac": round(tf / BF16_PEAK_TFLOPS, 4),
                        "kernel": plan.describe().split("kernel=")[-1],
                        "hipblaslt_matmul_tflops": round(
                            2.0 * m * n * k / (ms_lt * 1e-3) / 1e12, 1)})
            del a, b, d
    if want("gemm_mid"):
        # bf16 GEMM D = A @ B (NN, no epilogue) at prefill row counts whose
        # 256 x 128 tiles do not fill the CUs (K split over workgroups), with
        # hipBLASLt on the same operands timed alternately
        for (m, n, k) in [(256, 12288, 4096), (512, 4096, 12288),
                          (1024, 4096, 12288), (384, 4096, 4096)]:
            a = (torch.randn(m, k, device=dev, generator=gen) / k ** 0.5).to(
                torch.bfloat16)
            b = (torch.randn(k, n, device=dev, generator=gen) / k ** 0.5).to(
                torch.bfloat16)
            d = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
            L = qkern.blas
            lay = lambda r, c: L.MatrixLayout("bfloat16", r, c)
            plan = L.BlasLt.get_matmul_plan(
                L.GemmConfig(lay(m, k), lay(k, n), lay(m, n), lay(m, n)),
                L.Epilogue.kDefault)
            args = L.MemoryArgs(a, b, None, d)
            ms, ms_lt = gemm_vs_library(
                torch, lambda i: plan.execute_on_stream(None, args),
                lambda: torch.matmul(a, b, out=d))
            tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
            out.append({"name": f"bf16 gemm {m}x{n}x{k}",
                        "value": round(tf, 1), "unit": "TFLOP/s",
                        "ms": round(ms, 4), "frac": round(tf / BF16_PEAK_TFLOPS, 4),
                        "kernel": plan.describe().split("kernel=")[-1],
                        "hipblaslt_matmul_tflops": round(
                            2.0 * m * n * k / (ms_lt * 1e-3) / 1e12, 1)})
            del a, b, d
    if want("f32"):
        # f32 GEMM C = A @ B at 1024^3 (C1), MFMA f32 peak
        n = 1024
        a = torch.randn(n, n, device=dev, generator=gen)
        b = torch.randn(n, n, device=dev, generator=gen)
        d = torch.empty(n, n, device=dev)
        L = qkern.blas
        lay = lambda r, c: L.MatrixLayout("float32", r, c)
        plan = L.BlasLt.get_matmul_plan(
            L.GemmConfig(lay(n, n), lay(n, n), lay(n, n), lay(n, n)),
            L.Epilogue.kDefault)
        args = L.MemoryArgs(a, b, None, d)
        plan.execute_on_stream(None, args)
        ms = timed_launches(torch, lambda i: plan.execute_on_stream(None, args), 20)
        tf = 2.0 * n ** 3 / (ms * 1e-3) / 1e12
        out.append({"name": "f32 gemm 1024x1024x1024", "value": round(tf, 1),
                    "unit": "TFLOP/s", "ms": round(ms, 4),
                    "frac": round(tf / F32_PEAK_TFLOPS, 4),
                    "kernel": plan.describe().split("kernel=")[-1]})
        del a, b, d
    if want("int4"):
        # int4 batched rows (decode batch / prefill), M = 4 (the top of the
        # reference's matvec range), 16 and 512 at the four Qwen3-8B shapes of the int4 config (weights rotated over at
        # least 600 MB)
        for n, k in [(12288, 4096), (4096, 4096), (4096, 12288),
                     (151936, 4096)]:
            nset = min(8, max(2, -(-(600 << 20) // (n * k // 2))))
            sets = [make_int4(torch, dev, n, k, gen) for _ in range(nset)]
            for m in (4, 16, 512):
                x = torch.randn(m, k, device=dev, generator=gen).to(
                    torch.bfloat16)
                y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
                fn = lambda i: qkern.qmatvec(x, *sets[i % nset], out=y)
                fn(0)
                ms = timed_launches(torch, fn, 16)
                gbs = int4_bytes(m, n, k) / (ms * 1e-3) / 1e9
                tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
                out.append({"name": f"int4 g64 qmatvec M={m} {n}x{k}",
                            "value": round(gbs, 1), "unit": "GB/s",
                            "tflops": round(tf, 2), "ms": round(ms, 4),
                            "frac": round(gbs / HBM_PEAK_GBS, 4)})
            del sets
    if want("int8"):
        # int8 affine GEMV (C4)
        n, k = 12288, 4096
        sets8 = []
        for _ in range(12):
            codes = torch.randint(0, 256, (n, k), dtype=torch.uint8, device=dev,
                                  generator=gen)
            s = (torch.rand(n, k // GROUP, device=dev, generator=gen) * 0.019 +
                 0.001).to(torch.bfloat16)
            b = (0.05 * torch.randn(n, k // GROUP, device=dev, generator=gen)).to(
                torch.bfloat16)
            sets8.append((codes, s, b))
        for m in (1, 4, 8, 128):
            x = torch.randn(m, k, device=dev, generator=gen).to(torch.bfloat16)
            y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
            fn = lambda i: qkern.qmatvec(x, *sets8[i % 12], out=y,
                                         packing=qkern.Packing.U8)
            fn(0)
            ms = timed_launches(torch, fn, 24)
            gbs = int8_bytes(m, n, k) / (ms * 1e-3) / 1e9
            out.append({"name": f"int8 affine g64 qmatvec M={m} {n}x{k}",
                        "value": round(gbs, 1), "unit": "GB/s", "ms": round(ms, 4),
                        "frac": round(gbs / HBM_PEAK_GBS, 4)})
        del sets8
    if want("rownorm"):
        # rownorm [4096, 4096]
        # (LayerNorm with gain and offset, eps 1e-5, beside the configured
        # RMSNorm and softmax)
        # params: "f32" gain/offset in f32, "none" without them (the
        # reference's layernorm, bench/jax_bench.py:44-46), "same" in x's
        # type
        for name, kind, dt, esz, params in [
                ("rmsnorm bf16", 0, torch.bfloat16, 2, "f32"),
                ("rmsnorm f32", 0, torch.float32, 4, "f32"),
                ("softmax f32", 2, torch.float32, 4, "f32"),
                ("layernorm bf16", 1, torch.bfloat16, 2, "none"),
                ("layernorm bf16 + bf16 gain/offset", 1, torch.bfloat16, 2,
                 "same"),
                ("layernorm bf16 + f32 gain/offset", 1, torch.bfloat16, 2,
                 "f32")]:
            xs = [torch.randn(4096, 4096, device=dev, generator=gen).to(dt)
                  for _ in range(8)]
            ys = [torch.empty_like(xs[0]) for _ in range(2)]
            g = (1 + 0.1 * torch.randn(4096, device=dev, generator=gen))
            bt = 0.1 * torch.randn(4096, device=dev, generator=gen)
            if params == "same":
                g, bt = g.to(dt), bt.to(dt)
            gain = g if kind != 2 and params != "none" else None
            beta = bt if kind == 1 and params != "none" else None
            eps = 1e-5 if kind == 1 else 1e-6
            fn = lambda i: qkern.rownorm(xs[i % 8], kind, eps=eps, gain=gain,
                                         beta=beta, out=ys[i % 2])
            fn(0)
            ms = timed_launches(torch, fn, 32)
            nbytes = (2 * 4096 * 4096 * esz + (4096 * 4 if kind != 2 else 0) +
                      (4096 * 4 if kind == 1 else 0))
            gbs = nbytes / (ms * 1e-3) / 1e9
            out.append({"name": f"{name} 4096x4096", "value": round(gbs, 1),
                        "unit": "GB/s", "ms": round(ms, 4),
                        "frac": round(gbs / HBM_PEAK_GBS, 4)})
            del xs, ys
    return out


def secondary_more(torch, qkern, dev, gen):
    """Few-row dense GEMMs, decode attention and the device copy ceiling."""
    out = []
    L = qkern.blas
    if want("fewrow"):
        # The reference's few-row list (docs/performance.md:223-242,
        # examples/llm/skinny_jax.py): 28 GEMMs x[M, 1024] @ W.T, bf16
        # W [6144, 1024] (28 distinct weights, 352 MB), one call = all 28.
        nl, kk, nn = 28, 1024, 6144
        ws = [(0.02 * torch.randn(nn, kk, device=dev, generator=gen)).to(
            torch.bfloat16) for _ in range(nl)]
        for m in (1, 2, 4, 8, 16, 32, 64):
            x = (0.01 * torch.ones(m, kk, device=dev)).to(torch.bfloat16)
            ys = [torch.empty(m, nn, dtype=torch.bfloat16, device=dev)
                  for _ in range(nl)]
            plan = L.BlasLt.get_matmul_plan(
                L.GemmConfig(L.MatrixLayout("bfloat16", m, kk),
                             L.MatrixLayout("bfloat16", kk, nn,
                                            L.Order.kColumnMajor, 1, kk, 0),
                             L.MatrixLayout("bfloat16", m, nn),
                             L.MatrixLayout("bfloat16", m, nn)),
                L.Epilogue.kDefault)

            def call(i, x=x, ys=ys, plan=plan):
                for j in range(nl):
                    plan.execute_on_stream(None, L.MemoryArgs(x, ws[j], None,
                                                              ys[j]))
            ms = timed_launches(torch, call, 4)
            nbytes = nl * (nn * kk * 2 + m * kk * 2 + m * nn * 2)
            gbs = nbytes / (ms * 1e-3) / 1e9
            out.append({"name": f"bf16 few-row gemm list 28x[{m},1024]x"
                                f"[1024,6144]^T", "value": round(gbs, 1),
                        "unit": "GB/s", "ms": round(ms, 4),
                        "frac": round(gbs / HBM_PEAK_GBS, 4),
                        "kernel": plan.describe().split("kernel=")[-1]})
        del ws
    if want("attention"):
        # Decode attention at Qwen3-8B's shape (32 query heads over 8 KV heads
        # of dim 128), one sequence, the whole cache attended: K + V read once
        for smax in (4096, 32768):
            b, kv, g, d = 1, 8, 4, 128
            nset = max(2, -(-(512 << 20) // (2 * b * kv * smax * d * 2)))
            caches = [(torch.randn(b, kv, smax, d, device=dev, generator=gen).to(
                torch.bfloat16), torch.randn(b, kv, d, smax, device=dev,
                                             generator=gen).to(torch.bfloat16))
                for _ in range(nset)]
            q = torch.randn(b, kv, g, d, device=dev, generator=gen).to(
                torch.bfloat16)
            pos = torch.tensor([smax - 1], dtype=torch.int32, device=dev)
            o = torch.empty_like(q)
            wsp = torch.empty(qkern.decode_attention_workspace_size(
                q, caches[0][0]), dtype=torch.uint8, device=dev)
            fn = lambda i: qkern.decode_attention(q, *caches[i % nset], pos,
                                                  workspace=wsp, out=o)
            fn(0)
            ms = timed_launches(torch, fn, 32)
            nbytes = 2 * b * kv * smax * d * 2 + 2 * q.numel() * 2
            gbs = nbytes / (ms * 1e-3) / 1e9
            out.append({"name": f"decode attention bf16 B=1 KV=8 G=4 D=128 "
                                f"S={smax}", "value": round(gbs, 1),
                        "unit": "GB/s", "ms": round(ms, 4),
                        "frac": round(gbs / HBM_PEAK_GBS, 4)})
            del caches
    if want("embed"):
        # Quantized token embedding (qwen3.embed) of Qwen3-8B's int4 table
        # (151936 x 4096, group 64): 2048 prefill tokens; bytes = the rows'
        # codes, scales and offsets read and the bf16 rows written
        n, k = 151936, 4096
        words, s, b = make_int4(torch, dev, n, k, gen)
        tok = torch.randint(0, n, (2048,), dtype=torch.int32, device=dev,
                            generator=gen)
        rows = torch.empty(2048, k, dtype=torch.bfloat16, device=dev)
        fn = lambda i: qkern.embed(words, tok, s, b, k=k, out=rows)
        fn(0)
        ms = timed_launches(torch, fn, 32)
        nbytes = 2048 * (k // 2 + (k // GROUP) * 4 + k * 2) + 2048 * 4
        gbs = nbytes / (ms * 1e-3) / 1e9
        out.append({"name": "int4 embed gather 2048 tokens of 151936x4096",
                    "value": round(gbs, 1), "unit": "GB/s", "ms": round(ms, 4),
                    "frac": round(gbs / HBM_PEAK_GBS, 4)})
        del words, s, b, rows
    if want("quantize"):
        # Checkpoint quantization on the device (qk_quantize): a Qwen3-8B
        # projection 12288 x 4096 bf16 to int4 u32x8 codes with f32 scales
        # and offsets; bytes = weights read + codes, scales, offsets written
        n, k = 12288, 4096
        ws = [(0.02 * torch.randn(n, k, device=dev, generator=gen)).to(
            torch.bfloat16) for _ in range(4)]
        codes = torch.empty(n, k // 8, dtype=torch.int32, device=dev)
        sc = torch.empty(n, k // GROUP, dtype=torch.float32, device=dev)
        of = torch.empty_like(sc)
        from qkern.ffi import _attrs, any_buffer, check, lib, _ref
        import ctypes
        bufs = [tuple(any_buffer(t) for t in (w, codes, sc, of)) for w in ws]
        at = _attrs(qkern.Packing.U32X8, GROUP, True)
        fn = lambda i: check(lib().qk_quantize(
            qkern.blas.stream_handle(None), *(_ref(b) for b in bufs[i % 4]),
            ctypes.byref(at)))
        fn(0)
        ms = timed_launches(torch, fn, 16)
        nbytes = n * k * 2 + n * k // 2 + 2 * n * (k // GROUP) * 4
        gbs = nbytes / (ms * 1e-3) / 1e9
        out.append({"name": "int4 quantize 12288x4096 bf16 (qk_quantize)",
                    "value": round(gbs, 1), "unit": "GB/s", "ms": round(ms, 4),
                    "frac": round(gbs / HBM_PEAK_GBS, 4)})
        del ws, codes, sc, of
    if want("copy"):
        # The practical read+write ceiling: a plain device copy of the rownorm
        # sizes (rotating over 8 sources, 537 MB or more)
        for mb, dt in ((67, torch.bfloat16), (134, torch.float32)):
            srcs = [torch.empty(4096, 4096, dtype=dt, device=dev).normal_(
                generator=gen) for _ in range(8)]
            dst = torch.empty_like(srcs[0])
            fn = lambda i: dst.copy_(srcs[i % 8])
            fn(0)
            ms = timed_launches(torch, fn, 32)
            nbytes = 2 * srcs[0].numel() * srcs[0].element_size()
            gbs = nbytes / (ms * 1e-3) / 1e9
            out.append({"name": f"device copy 4096x4096 {str(dt)[6:]} "
                                f"(read+write {2 * mb} MB)", "value": round(gbs, 1),
                        "unit": "GB/s", "ms": round(ms, 4),
                        "frac": round(gbs / HBM_PEAK_GBS, 4)})
            del srcs
    return out


def cpu_secondary(seconds=3.0):
    """CPU figures beside the GEMM and rownorm secondaries: torch's CPU
    backend running the same programs (bf16 GEMM + bias + SiLU at
    4096^3, f32 GEMM 1024^3, RMSNorm and softmax [4096, 4096]) on the host
    cores, each repeated for about `seconds`."""
    import torch
    threads = min(16, len(os.sched_getaffinity(0)))
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    res = []

    def rate(fn):
        fn()
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds:
            fn()
            n += 1
        return (time.perf_counter() - t0) / n

    a = (torch.randn(4096, 4096, generator=g) / 64).to(torch.bfloat16)
    b = (torch.randn(4096, 4096, generator=g) / 64).to(torch.bfloat16)
    bias = (0.02 * torch.randn(4096, generator=g)).to(torch.bfloat16)
    dt = rate(lambda: torch.nn.functional.silu(
        (a.float() @ b.float() + bias.float())).to(torch.bfloat16))
    res.append({"name": "bf16 gemm+bias+silu 4096x4096x4096",
                "value": round(2 * 4096 ** 3 / dt / 1e12, 3),
                "unit": "TFLOP/s"})
    a = torch.randn(1024, 1024, generator=g)
    b = torch.randn(1024, 1024, generator=g)
    dt = rate(lambda: a @ b)
    res.append({"name": "f32 gemm 1024x1024x1024",
                "value": round(2 * 1024 ** 3 / dt / 1e12, 3),
                "unit": "TFLOP/s"})
    x = torch.randn(4096, 4096, generator=g)
    w = 1 + 0.1 * torch.randn(4096, generator=g)
    xb = x.to(torch.bfloat16)
    dt = rate(lambda: (xb.float() * torch.rsqrt(
        xb.float().pow(2).mean(-1, keepdim=True) + 1e-6) * w).to(
            torch.bfloat16))
    res.append({"name": "rmsnorm bf16 4096x4096",
                "value": round(2 * 4096 * 4096 * 2 / dt / 1e9, 2),
                "unit": "GB/s"})
    dt = rate(lambda: torch.softmax(x, -1))
    res.append({"name": "softmax f32 4096x4096",
                "value": round(2 * 4096 * 4096 * 4 / dt / 1e9, 2),
                "unit": "GB/s"})
    # the host quantizer (the reference's loader quantizes in numpy,
    # examples/llm/qwen3.py:169-196): qkern.quant on a 2048 x 4096 slice
    from qkern import quant
    wq = (0.02 * torch.randn(2048, 4096, generator=g)).to(
        torch.bfloat16).float().numpy()
    dt = rate(lambda: quant.pack_u32x8(quant.quantize_int4(wq)[0]))
    res.append({"name": "int4 quantize 12288x4096 bf16 (numpy, 2048-row "
                        "slice)",
                "value": round(2048 * (4096 * 2 + 4096 // 2 + 64 * 8) / dt /
                               1e9, 2),
                "unit": "GB/s"})
    return {"impl": "torch CPU (float32 arithmetic, bf16 rounding of the "
                    "output), in place of JAX_PLATFORMS=cpu: jax is not "
                    "installed", "cores": threads, "kind": "port",
            "results": res}


def cpu_baseline(seconds=12.0):
    """The oracle's C port of _matvec_int4 on a bounded sample: repeated
    passes over the four Qwen3-8B shapes (M = 1) until `seconds` elapse."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    threads = min(16, len(os.sched_getaffinity(0)))
    rng = np.random.default_rng(0)
    data = []
    for n, k in QWEN3_8B:
        words = rng.integers(0, 2 ** 32, size=(n, k // 8), dtype=np.uint32)
        s = O.bf16_bits(rng.uniform(0.001, 0.02, (n, k // GROUP)).astype(
            np.float32))
        b = O.bf16_bits((0.05 * rng.standard_normal((n, k // GROUP))).astype(
            np.float32))
        x = O.bf16_bits(rng.standard_normal((1, k)).astype(np.float32))
        data.append((x, words, s, b, int4_bytes(1, n, k)))
    O.c_matvec_int4_u32x8(*data[0][:4], threads=threads)  # warm
    total, passes = 0, 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for x, words, s, b, nbytes in data:
            O.c_matvec_int4_u32x8(x, words, s, b, threads=threads)
            total += nbytes
        passes += 1
    dt = time.perf_counter() - t0
    return {"value": round(total / dt / 1e9, 2), "unit": "GB/s",
            "cores": O.c_threads(threads), "kind": "port",
            "sample": f"{passes} passes over the 4 Qwen3-8B int4 shapes at "
                      f"M=1 ({dt:.1f} s), oracle/qk_oracle.c float32"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default=None,
                    help="run only these secondary parts (comma list of "
                         "gemm, gemm_mid, f32, int4, int8, rownorm, fewrow, attention, "
                         "embed, copy) and print them, without the headline")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 10 plain device copies of 512 MiB (the "
                         "reference kernel for FETCH_SIZE/WRITE_SIZE scaling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(every GPU box here has one GPU). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import qkern
    import qkern.blas  # noqa: F401

    dev = torch.device("cuda:0")
    if args.copy_calibration:
        src = torch.ones(128 * 1024 * 1024, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": src.numel() * 4,
                          "copy_bytes_written": dst.numel() * 4}))
        return
    gen = torch.Generator(device=dev).manual_seed(0)
    if args.only:
        global ONLY
        ONLY = set(args.only.split(","))
        for r in (secondary(torch, qkern, dev, gen) +
                  secondary_more(torch, qkern, dev, gen)):
            print(json.dumps(r), flush=True)
        return
    rot = 3
    sets = [[make_int4(torch, dev, n, k, gen) for (n, k) in QWEN3_8B]
            for _ in range(rot)]
    xs = [torch.randn(1, k, device=dev, generator=gen).to(torch.bfloat16)
          for (n, k) in QWEN3_8B]
    ys = [torch.empty(1, n, dtype=torch.bfloat16, device=dev)
          for (n, k) in QWEN3_8B]
    step_bytes = sum(int4_bytes(1, n, k) for (n, k) in QWEN3_8B)
    per_shape_bytes = [int4_bytes(1, n, k) for (n, k) in QWEN3_8B]

    def step(i):
        ws = sets[i % rot]
        for j in range(len(QWEN3_8B)):
            qkern.qmatvec(xs[j], *ws[j], out=ys[j])

    # The K timed steps are captured into one HIP graph (so host launch
    # overhead does not leave the GPU idle between the short kernels), the
    # warm-up steps into another; both replay on one stream.
    warm = capture(torch, step, max(args.warmup, 1))
    timed = capture(torch, step, args.steps)
    warm.replay()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record()
    timed.replay()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = ev0.elapsed_time(ev1)
    value = step_bytes * args.steps / wall / 1e9
    # achieved: algorithmic bytes per launch / device time per launch, over
    # the same timed region (4 launches per step)
    achieved = step_bytes * args.steps / (gpu_ms * 1e-3) / 1e9
    del warm, timed, sets
    # per-shape breakdown: 30 back-to-back launches of one shape between two
    # events, rotating over at least 512 MB of weight copies so that no
    # launch finds its weights in the 256 MB last-level cache
    shapes = []
    for j, (n, k) in enumerate(QWEN3_8B):
        copies = max(2, -(-(512 << 20) // per_shape_bytes[j]))
        wset = [make_int4(torch, dev, n, k, gen) for _ in range(copies)]
        ms = timed_launches(
            torch, lambda i: qkern.qmatvec(xs[j], *wset[i % copies],
                                           out=ys[j]), 30)
        shapes.append({"n": n, "k": k, "us": round(ms * 1e3, 2),
                       "gbs": round(per_shape_bytes[j] / (ms * 1e-3) / 1e9,
                                    1)})
        del wset

    result = {
        "metric": "int4 GEMV HBM GB/s (% of peak); bf16 GEMM TFLOP/s "
                  "(% MFMA peak)",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "gpu_ms_per_step": round(gpu_ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4xbf16->f32",
        "data": "synthetic (uniform int4 codes, bf16 scale U(0.001,0.02) "
                "and bias N(0,0.05) per group of 64, x ~ N(0,1) bf16)",
        "config": {"workload": "int4 g64 u32x8 qmatvec, Qwen3-8B decode "
                               "projections at M=1: 4096x4096, 12288x4096, "
                               "4096x12288, 151936x4096 (one launch each "
                               "per step, 3 rotated weight sets)",
                   "bytes_per_step": step_bytes,
                   "per_shape": shapes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic(),
                     "traffic_unit": "bytes per launch (profiles/"
                                     "int4_gemv_qwen3_8b_decode.md)",
                     "kernel": "qmv_m1_kernel (algorithmic bytes / "
                               "device time, over the 4 launches of each "
                               "timed step)"},
    }
    if not args.no_secondary:
        result["secondary"] = (secondary(torch, qkern, dev, gen) +
                               secondary_more(torch, qkern, dev, gen))
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline()
        if not args.no_secondary:
            result["cpu_secondary"] = cpu_secondary()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
