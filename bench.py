"""Benchmark of the hot path on one MI355X; prints ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]

Headline workload (``value``): the TinyLlama-1.1B-shaped prefill block,
512 tokens, fp16 -- RMSNorm(2048, eps 1e-5) -> QKV 2048->2560 -> O 2048->2048
-> fused gate/up 2048->11264 with SiLU-mul -> down 5632->2048 -- as TFLOP/s
of GEMM work over the whole block (inputs resident in HBM, HIP events around
exactly K steps).  ``roofline`` reports the block's dominant kernel (the
gate/up SiLU-mul GEMM) against the fp16 MFMA peak.

Secondary lines in the same JSON object (``secondary``): the 1024^3 and
4096^3 fp16 GEMMs, the Qwen2.5-0.5B decode GEMVs (fp16 and int8
weight-only, rotating weight copies past the 256 MB Infinity Cache), a
whole 24-layer decode step, RMSNorm, softmax and the ViT-B/16 block.

``cpu_baseline`` times the oracle (numpy fp32, the reference's CPU-path
semantics) on the host cores for a bounded sample of the same block.
"""
from __future__ import annotations

import argparse
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_FP16_TFLOPS = 2516.6  # 256 CU x 4096 FLOP/clk x 2.4 GHz, dense
PEAK_HBM_GBS = 8000.0

TL_M, TL_H, TL_QKV, TL_I = 512, 2048, 2560, 5632


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def tinyllama_flops() -> dict:
    f = {
        "qkv": 2 * TL_M * TL_H * TL_QKV,
        "o": 2 * TL_M * TL_H * TL_H,
        "gate_up": 2 * TL_M * TL_H * 2 * TL_I,
        "down": 2 * TL_M * TL_I * TL_H,
    }
    f["total"] = sum(f.values())
    return f


class Timer:
    """HIP events on the stream the kernels are launched on (torch's current
    stream: the C ABI is handed torch.cuda.current_stream())."""

    def __init__(self, torch, warm_ms: float = 100.0):
        self.torch = torch
        self.warm_ms = warm_ms

    def _warm(self, fn) -> None:
        """Back-to-back calls for warm_ms of wall time (steady-state clocks)."""
        t_end = time.perf_counter() + self.warm_ms * 1e-3
        while time.perf_counter() < t_end:
            for i in range(10):
                fn(i)
            self.torch.cuda.synchronize()

    def per_iter_ms(self, fn, iters: int, warmup: int = 3) -> float:
        """Eager launches (host launch cost included when it dominates)."""
        torch = self.torch
        for _ in range(warmup):
            fn(0)
        self._warm(fn)
        torch.cuda.synchronize()
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        for i in range(iters):
            fn(i)
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / iters

    def capture(self, fn, n: int):
        """HIP graph of fn(0) .. fn(n-1), captured after eager warm-up."""
        torch = self.torch
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for i in range(min(n, 3)):
                fn(i)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(n):
                fn(i)
        return g

    def graph_ms(self, fn, n: int, replays: int = 3) -> float:
        """Per-call time of fn from replays of a graph of n back-to-back calls
        (launch cost reduced to the GPU's own dispatch), HIP events on the
        stream the replays run on."""
        torch = self.torch
        g = self.capture(fn, n)
        t_end = time.perf_counter() + self.warm_ms * 1e-3
        while time.perf_counter() < t_end:
            g.replay()
            torch.cuda.synchronize()
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(replays):
            g.replay()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / (n * replays)


def make_block(pkg, torch, dev):
    g = torch.Generator().manual_seed(0)
    x = torch.randn(TL_M, TL_H, generator=g).half().to(dev)
    gn = (1 + 0.02 * torch.randn(TL_H, generator=g)).half().to(dev)
    wqkv = (torch.randn(TL_QKV, TL_H, generator=g) * 0.02).half().to(dev)
    wo = (torch.randn(TL_H, TL_H, generator=g) * 0.02).half().to(dev)
    wg = (torch.randn(TL_I, TL_H, generator=g) * 0.02).half().to(dev)
    wu = (torch.randn(TL_I, TL_H, generator=g) * 0.02).half().to(dev)
    wgu = pkg.pack_gate_up(wg, wu)
    wd = (torch.randn(TL_H, TL_I, generator=g) * 0.02).half().to(dev)
    xa = torch.randn(TL_M, TL_H, generator=g).half().to(dev)  # attention output stand-in
    # RMSNorm weight folded into the two projections that consume the
    # normalised rows (a load-time transform, like the gate/up packing)
    wqkv_f = pkg.fold_rms_weight(wqkv, gn)
    wgu_f = pkg.fold_rms_weight(wgu, gn)
    buf = {
        "rs": torch.empty(TL_M, dtype=torch.float32, device=dev),
        "xn": torch.empty(TL_M, TL_H, dtype=torch.float16, device=dev),
        "qkv": torch.empty(TL_M, TL_QKV, dtype=torch.float16, device=dev),
        "o": torch.empty(TL_M, TL_H, dtype=torch.float16, device=dev),
        "h": torch.empty(TL_M, TL_I, dtype=torch.float16, device=dev),
        "d": torch.empty(TL_M, TL_H, dtype=torch.float16, device=dev),
    }

    def step(_i=0):
        # QKV takes the row statistics of x and publishes the row scales;
        # gate/up applies them (both with the folded norm weight)
        pkg.rms_norm_linear(x, wqkv_f, 1e-5, out=buf["qkv"], rscale_out=buf["rs"])
        pkg.gemm(xa, wo, b_layout="nt", out=buf["o"])
        pkg.rms_norm_linear(x, wgu_f, 1e-5, epilogue="silu_mul", out=buf["h"], rscale_in=buf["rs"])
        pkg.gemm(buf["h"], wd, b_layout="nt", out=buf["d"])

    def step_unfused(_i=0):
        pkg.rms_norm(x, gn, 1e-5, out=buf["xn"])
        pkg.gemm(buf["xn"], wqkv, b_layout="nt", out=buf["qkv"])
        pkg.gemm(xa, wo, b_layout="nt", out=buf["o"])
        pkg.gemm(buf["xn"], wgu, b_layout="nt", epilogue="silu_mul", out=buf["h"])
        pkg.gemm(buf["h"], wd, b_layout="nt", out=buf["d"])

    def gate_up(_i=0):
        pkg.rms_norm_linear(x, wgu_f, 1e-5, epilogue="silu_mul", out=buf["h"], rscale_in=buf["rs"])

    tensors = dict(x=x, gn=gn, wqkv=wqkv, wo=wo, wg=wg, wu=wu, wd=wd, xa=xa, step_unfused=step_unfused)
    return step, gate_up, tensors, buf


def bench_gemm(pkg, torch, dev, timer, M, N, K, layout, iters):
    g = torch.Generator().manual_seed(1)
    a = (torch.rand(M, K, generator=g) * 2 - 1).half().to(dev)
    b = (torch.rand(K, N, generator=g) * 2 - 1).half().to(dev) if layout == "nn" else \
        (torch.rand(N, K, generator=g) * 2 - 1).half().to(dev)
    c = torch.empty(M, N, dtype=torch.float16, device=dev)
    ms = timer.graph_ms(lambda i: pkg.gemm(a, b, b_layout=layout, out=c), iters)
    tf = 2 * M * N * K / (ms * 1e-3) / 1e12
    return {"ms": round(ms, 5), "tflops": round(tf, 1), "frac_mfma_peak": round(tf / PEAK_FP16_TFLOPS, 4)}


def bench_gemv(pkg, torch, dev, timer, M, K, N, int8, iters, min_bytes=768 << 20):
    """GB/s of one decode linear with enough distinct weight copies in the
    rotation that no copy is still cached when it is read again."""
    g = torch.Generator().manual_seed(2)
    wbytes = N * K * (1 if int8 else 2)
    copies = max(2, -(-min_bytes // wbytes))
    copies = min(copies, 64)
    x = torch.randn(M, K, generator=g).half().to(dev)
    y = torch.empty(M, N, dtype=torch.float16, device=dev)
    if int8:
        ws = [torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev) for _ in range(copies)]
        s = (torch.rand(N, generator=g) * 9e-3 + 1e-3).half().to(dev)
        fn = lambda i: pkg.w8a16_linear(x, ws[i % copies], s, out=y)  # noqa: E731
        algo = N * K + 2 * N + 2 * M * K + 2 * M * N
    else:
        ws = [torch.empty(N, K, dtype=torch.float16, device=dev).normal_(0, 0.02) for _ in range(copies)]
        fn = lambda i: pkg.gemv(x, ws[i % copies], out=y)  # noqa: E731
        algo = 2 * (N * K + M * K + M * N)
    ms = timer.graph_ms(fn, max(iters, 2 * copies))
    gbs = algo / (ms * 1e-3) / 1e9
    del ws
    return {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1), "frac_hbm_peak": round(gbs / PEAK_HBM_GBS, 4),
            "bytes": algo, "weight_copies": copies}


def bench_decode_step(pkg, torch, dev, timer, iters):
    """One Qwen2.5-0.5B decode step at M=1: 24 layers of distinct weights +
    lm_head, ~0.99 GB streamed.  Projections that read the same input share
    one weight matrix (q|k|v 896->1152, gate|up 896->9728), as decoders
    pack them, so a layer is 4 GEMV launches."""
    H, KV, I, V, L = 896, 128, 4864, 151936, 24
    g = torch.Generator().manual_seed(3)
    x = torch.randn(1, H, generator=g).half().to(dev)
    shapes = [(H + 2 * KV, H), (H, H), (2 * I, H), (H, I)]
    layers = [[torch.empty(n, k, dtype=torch.float16, device=dev).normal_(0, 0.02) for n, k in shapes]
              for _ in range(L)]
    lm = torch.empty(V, H, dtype=torch.float16, device=dev).normal_(0, 0.02)
    outs = {n: torch.empty(1, n, dtype=torch.float16, device=dev) for n in (H, H + 2 * KV, 2 * I, V)}
    xi = torch.randn(1, I, generator=g).half().to(dev)

    def step(_i=0):
        for ws in layers:
            for w in ws:
                inp = xi if w.shape[1] == I else x
                pkg.gemv(inp, w, out=outs[w.shape[0]])
        pkg.gemv(x, lm, out=outs[V])

    nbytes = sum(2 * (w.numel() + w.shape[1] + w.shape[0]) for ws in layers for w in ws) + 2 * (lm.numel() + H + V)
    ms = timer.graph_ms(step, iters)
    gbs = nbytes / (ms * 1e-3) / 1e9
    del layers, lm
    return {"us": round(ms * 1e3, 1), "GB/s": round(gbs, 1), "frac_hbm_peak": round(gbs / PEAK_HBM_GBS, 4),
            "bytes": nbytes, "launches": L * len(shapes) + 1}


def bench_rows(pkg, torch, dev, timer, iters):
    out = {}
    g = torch.Generator().manual_seed(4)
    rows, cols = 512, 2048
    copies = 64
    xs = [torch.randn(rows, cols, generator=g).half().to(dev) for _ in range(copies)]
    w = torch.ones(cols, dtype=torch.float16, device=dev)
    y = torch.empty(rows, cols, dtype=torch.float16, device=dev)
    ms = timer.graph_ms(lambda i: pkg.rms_norm(xs[i % copies], w, 1e-5, out=y), iters)
    nb = 2 * (2 * rows * cols + cols)
    out["rmsnorm_512x2048"] = {"us": round(ms * 1e3, 2), "GB/s": round(nb / (ms * 1e-3) / 1e9, 1)}
    s = torch.randn(96 * 197, 197, generator=g).half().to(dev)
    p = torch.empty_like(s)
    ms = timer.graph_ms(lambda i: pkg.softmax(s, 0.125, out=p), iters)
    nb = 2 * 2 * s.numel()
    out["softmax_18912x197"] = {"us": round(ms * 1e3, 2), "GB/s": round(nb / (ms * 1e-3) / 1e9, 1),
                                "frac_hbm_peak": round(nb / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
    return out


def bench_vit(pkg, torch, dev, timer, iters):
    g = torch.Generator().manual_seed(5)
    B, S, Hh, D, E, F = 8, 197, 12, 64, 768, 3072
    q = torch.randn(B * Hh, S, D, generator=g).half().to(dev)
    k = torch.randn(B * Hh, S, D, generator=g).half().to(dev)
    v = torch.randn(B * Hh, S, D, generator=g).half().to(dev)
    x = torch.randn(B * S, E, generator=g).half().to(dev)
    w1 = (torch.randn(F, E, generator=g) * 0.02).half().to(dev)
    b1 = (torch.randn(F, generator=g) * 0.02).half().to(dev)
    w2 = (torch.randn(E, F, generator=g) * 0.02).half().to(dev)
    b2 = (torch.randn(E, generator=g) * 0.02).half().to(dev)

    def step(_i=0):
        pkg.attention(q, k, v, 0.125)
        h = pkg.linear(x, w1, b1, epilogue="gelu_tanh")
        pkg.linear(h, w2, b2)

    ms = timer.graph_ms(step, iters)
    flops = 2 * (2 * B * Hh * S * S * D) + 2 * (2 * B * S * E * F)
    att_ms = timer.graph_ms(lambda _i=0: pkg.attention(q, k, v, 0.125), iters)
    att_flops = 2 * (2 * B * Hh * S * S * D)
    att_bytes = 4 * B * Hh * S * D * 2  # Q, K, V read once, O written once
    return {"us": round(ms * 1e3, 1), "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
            "attention_us": round(att_ms * 1e3, 2), "attention_tflops": round(att_flops / (att_ms * 1e-3) / 1e12, 1),
            "attention_gbs": round(att_bytes / (att_ms * 1e-3) / 1e9, 1)}


def cpu_baseline(budget_s: float = 12.0) -> dict:
    """The oracle (numpy fp32) running the same prefill block on host cores,
    repeated until about budget_s seconds of CPU work."""
    import numpy as np

    from oracle import hot_path as ref

    try:
        from threadpoolctl import threadpool_info

        threads = max((i.get("num_threads", 1) for i in threadpool_info()), default=1)
    except Exception:  # pragma: no cover - threadpoolctl is optional
        threads = os.cpu_count() or 1
    r = np.random.default_rng(0)
    x = r.standard_normal((TL_M, TL_H)).astype(np.float16)
    gn = (1 + 0.02 * r.standard_normal(TL_H)).astype(np.float16)
    wqkv = (0.02 * r.standard_normal((TL_QKV, TL_H))).astype(np.float16)
    wo = (0.02 * r.standard_normal((TL_H, TL_H))).astype(np.float16)
    wg = (0.02 * r.standard_normal((TL_I, TL_H))).astype(np.float16)
    wu = (0.02 * r.standard_normal((TL_I, TL_H))).astype(np.float16)
    wd = (0.02 * r.standard_normal((TL_H, TL_I))).astype(np.float16)
    xa = r.standard_normal((TL_M, TL_H)).astype(np.float16)

    def block():
        xn = ref.rms_norm(x, gn, 1e-5).astype(np.float16)
        ref.linear(xn, wqkv)
        ref.linear(xa, wo)
        h = ref.silu_mul_linear(xn, wg, wu).astype(np.float16)
        ref.linear(h, wd)

    block()
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s or n < 2:
        block()
        n += 1
    dt = (time.perf_counter() - t0) / n
    tf = tinyllama_flops()["total"] / dt / 1e12
    return {"value": round(tf, 4), "unit": "TFLOP/s", "cores": int(threads), "kind": "port",
            "sample": f"{n} passes of the full 512-token TinyLlama block (fp32 numpy oracle), {dt * 1e3:.1f} ms each"}


def profile_suite(pkg, torch, dev, timer) -> None:
    """Launches for counter runs: 4096^3 NT GEMM and the Qwen2.5-0.5B lm_head
    GEMVs, each warmed up by time, then 5 launches (weights rotate over
    copies so none is cache-resident), then five 256 MiB copies."""
    g = torch.Generator().manual_seed(1)
    a = (torch.rand(4096, 4096, generator=g) * 2 - 1).half().to(dev)
    b = (torch.rand(4096, 4096, generator=g) * 2 - 1).half().to(dev)
    c = torch.empty(4096, 4096, dtype=torch.float16, device=dev)
    gemm = lambda i=0: pkg.gemm(a, b, b_layout="nt", out=c)
    timer._warm(gemm)
    for _ in range(5):
        gemm()
    H, V = 896, 151936
    ws = [torch.empty(V, H, dtype=torch.float16, device=dev).normal_(0, 0.02) for _ in range(3)]
    qs = [torch.randint(-127, 128, (V, H), dtype=torch.int8, device=dev) for _ in range(3)]
    sc = (torch.rand(V, generator=g) * 9e-3 + 1e-3).half().to(dev)
    for M in (1, 16):
        x = torch.randn(M, H, generator=g).half().to(dev)
        y = torch.empty(M, V, dtype=torch.float16, device=dev)
        gemv = lambda i=0: pkg.gemv(x, ws[i % 3], out=y)
        timer._warm(gemv)
        for i in range(5):
            gemv(i)
    for M in (1, 16):
        x = torch.randn(M, H, generator=g).half().to(dev)
        y = torch.empty(M, V, dtype=torch.float16, device=dev)
        w8 = lambda i=0: pkg.w8a16_linear(x, qs[i % 3], sc, out=y)
        timer._warm(w8)
        for i in range(5):
            w8(i)
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    log("[bench] profile suite: 4096^3 GEMM, lm_head GEMV fp16 M=1/16, int8 M=1/16, 5 x 256 MiB copies")


def traffic_from_profiles():
    """HBM bytes per launch of the dominant kernel from the committed rocprof
    PMC summary (FETCH_SIZE + WRITE_SIZE, copy-kernel calibrated), if present."""
    p = ROOT / "profiles" / "gate_up_silu_gemm_traffic.json"
    if p.exists():
        try:
            return json.loads(p.read_text()).get("bytes_per_launch")
        except Exception:
            return None
    return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--warmup-ms", type=float, default=300.0,
                    help="minimum wall time of back-to-back warm-up steps before the timed region")
    ap.add_argument("--quick", action="store_true", help="skip the secondary measurements")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--profile", action="store_true",
                    help="for rocprofv3: run only the dominant kernel (gate/up SiLU-mul GEMM) --steps times, then a "
                         "256 MiB device copy 5 times (calibrates FETCH_SIZE/WRITE_SIZE), and exit")
    ap.add_argument("--profile-suite", action="store_true",
                    help="for rocprofv3 counter runs: the 4096^3 fp16 NT GEMM and the lm_head decode GEMVs (fp16 "
                         "M=1 and M=16, int8 M=1), each warmed up and then launched 5 times, then the 256 MiB copy "
                         "calibration, and exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: hexagon-mlir_amd has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        return 2

    import torch

    import __graft_entry__

    pkg = __graft_entry__.load_package()
    pkg.load_library()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    timer = Timer(torch)

    if args.profile_suite:
        profile_suite(pkg, torch, dev, timer)
        return 0
    step, gate_up, block_tensors, _ = make_block(pkg, torch, dev)
    fl = tinyllama_flops()
    if args.profile:
        step()
        for _ in range(args.steps):
            gate_up()
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] profile mode: {args.steps} gate/up launches, 5 x 256 MiB copies")
        return 0
    # One step = the block's kernels launched eagerly on torch's current
    # stream (each kernel outlasts its host launch, so launches queue ahead of
    # the GPU); HIP events bracket exactly K steps after W warm-up steps.
    # Warm-up: at least W steps, and at least --warmup-ms of back-to-back
    # steps, so the timed steps run at the clocks the GPU settles at under
    # sustained load (MI355X ramps its clock over tens of milliseconds).
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t_end = time.perf_counter() + args.warmup_ms * 1e-3
    while time.perf_counter() < t_end:
        for _ in range(20):
            step()
        torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(args.steps):
        step()
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / args.steps
    value = fl["total"] / (ms * 1e-3) / 1e12
    log(f"[bench] tinyllama block {ms * 1e3:.1f} us/step, {value:.1f} TFLOP/s")
    graph_step_ms = timer.graph_ms(step, 10)
    log(f"[bench] tinyllama block as a HIP graph (10 steps per graph) {graph_step_ms * 1e3:.1f} us/step")

    # the dominant kernel alone, back to back on the same stream: its average
    # launch duration (rocprofv3 kernel-trace of this command agrees)
    gu_ms = timer.per_iter_ms(gate_up, max(args.steps, 20))
    gu_tf = fl["gate_up"] / (gu_ms * 1e-3) / 1e12
    log(f"[bench] gate/up SiLU-mul GEMM {gu_ms * 1e3:.2f} us, {gu_tf:.1f} TFLOP/s")

    # the same block with RMSNorm as its own kernel writing the normalised x
    unfused_ms = timer.per_iter_ms(block_tensors["step_unfused"], args.steps)
    log(f"[bench] tinyllama block, separate RMSNorm kernel {unfused_ms * 1e3:.1f} us/step")
    secondary = {"tinyllama_block_hip_graph": {"us": round(graph_step_ms * 1e3, 1),
                                               "tflops": round(fl["total"] / (graph_step_ms * 1e-3) / 1e12, 1)},
                 "tinyllama_block_separate_rmsnorm": {"us": round(unfused_ms * 1e3, 1),
                                                      "tflops": round(fl["total"] / (unfused_ms * 1e-3) / 1e12, 1)}}
    if not args.quick:
        secondary["gemm_1024_nn"] = bench_gemm(pkg, torch, dev, timer, 1024, 1024, 1024, "nn", 200)
        secondary["gemm_4096_nn"] = bench_gemm(pkg, torch, dev, timer, 4096, 4096, 4096, "nn", 30)
        secondary["gemm_4096_nt"] = bench_gemm(pkg, torch, dev, timer, 4096, 4096, 4096, "nt", 30)
        log(f"[bench] gemm {json.dumps(secondary)}")
        gv = {}
        for (K, N) in [(896, 896), (896, 128), (896, 4864), (4864, 896), (896, 151936)]:
            for M in (1, 4, 16):
                gv[f"M{M}_{K}x{N}"] = bench_gemv(pkg, torch, dev, timer, M, K, N, False, 50)
        secondary["decode_gemv_fp16"] = gv
        log(f"[bench] gemv lm_head M1 {gv['M1_896x151936']}")
        w8 = {}
        for (K, N) in [(896, 896), (896, 4864), (4864, 896), (896, 151936)]:
            for M in (1, 16, 256):
                w8[f"M{M}_{K}x{N}"] = bench_gemv(pkg, torch, dev, timer, M, K, N, True, 50)
        secondary["w8a16"] = w8
        log(f"[bench] w8a16 lm_head M1 {w8['M1_896x151936']}")
        secondary["decode_step_qwen_m1"] = bench_decode_step(pkg, torch, dev, timer, 10)
        log(f"[bench] decode step {secondary['decode_step_qwen_m1']}")
        secondary.update(bench_rows(pkg, torch, dev, timer, 100))
        secondary["vit_b16_block_b8"] = bench_vit(pkg, torch, dev, timer, 20)
        log(f"[bench] rows/vit done")

    cpu = None if args.no_cpu else cpu_baseline()
    if cpu:
        log(f"[bench] cpu baseline {cpu}")

    line = {
        "metric": "GEMM TFLOP/s & % fp16 MFMA peak; decode GEMV GB/s & % HBM peak",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 (fp32 accumulate)",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights)",
        "config": {"workload": "TinyLlama-1.1B prefill block, 512 tokens, fp16: RMSNorm 2048 -> QKV 2048x2560 -> "
                               "O 2048x2048 -> gate/up 2048x11264 + SiLU-mul -> down 5632x2048 (RMSNorm statistics "
                               "taken in the QKV GEMM, row scales applied in the QKV and gate/up GEMMs)",
                   "tokens": TL_M, "hidden": TL_H, "gemm_flop_per_step": fl["total"]},
        "roofline": {"kernel": "gemm_mfma, gate/up + RMSNorm row scale + SiLU-mul epilogue (M=512, N=11264, K=2048)",
                     "bound": "mfma", "achieved": round(gu_tf, 2), "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(gu_tf / PEAK_FP16_TFLOPS, 4), "traffic": traffic_from_profiles(),
                     "algorithmic_flop_per_launch": fl["gate_up"], "avg_launch_us": round(gu_ms * 1e3, 3)},
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
