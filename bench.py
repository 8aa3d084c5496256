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

``cpu_baseline`` times the reference's own CPU path (PyTorch CPU ops in
fp32) on the same block, on the host's allowed threads and on one thread.
"""
from __future__ import annotations

import argparse
import dataclasses
import gc
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

ROOFLINE = json.loads((ROOT / "config" / "roofline.json").read_text())
PEAK_FP16_TFLOPS = ROOFLINE["peak_fp16_tflops"]  # 256 CU x 4096 FLOP/clk x 2.4 GHz, dense
PEAK_HBM_GBS = ROOFLINE["peak_hbm_gbs"]

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

    tensors = dict(x=x, gn=gn, wqkv=wqkv, wo=wo, wg=wg, wu=wu, wd=wd, xa=xa, wqkv_f=wqkv_f, wgu_f=wgu_f,
                   step_unfused=step_unfused)
    return step, gate_up, tensors, buf


def check_block(torch, t, buf, tol: float = 1e-2) -> dict:
    """One TinyLlama block step's outputs against a plain torch fp32
    computation of the same block on the GPU (RMSNorm in fp32 with the folded
    weights, fp32 matmuls, SiLU-mul, the down projection of the kernel's own
    fp16 h): max relative error per output, floor 1e-3 of its RMS."""
    f = lambda v: v.float()  # noqa: E731
    xn = f(t["x"]) * torch.rsqrt(f(t["x"]).pow(2).mean(-1, keepdim=True) + 1e-5)
    exp = {"qkv": xn @ f(t["wqkv_f"]).t(), "o": f(t["xa"]) @ f(t["wo"]).t()}
    gu = xn @ f(t["wgu_f"]).t()  # packed columns: [32q, 32q+16) gate, [32q+16, 32q+32) up
    gu = gu.reshape(gu.shape[0], -1, 2, 16)
    exp["h"] = (torch.nn.functional.silu(gu[:, :, 0]) * gu[:, :, 1]).reshape(gu.shape[0], -1)
    exp["d"] = f(buf["h"]) @ f(t["wd"]).t()
    return {k: rel_err(torch, buf[k], v) for k, v in exp.items()}


def rel_err(torch, out, exp, vs_scale: bool = False) -> float:
    """max |out - exp| / max(|exp|, 1e-3 * rms(exp)), on the device; with
    vs_scale, max |out - exp| / max |exp| (for attention, whose fp16
    probabilities leave ~1e-4 absolute noise at outputs that average to ~0)."""
    out, exp = out.float(), exp.float()
    if not bool(torch.isfinite(out).all()):
        return float("inf")
    if vs_scale:
        return float((out - exp).abs().max() / exp.abs().max().clamp_min(1e-30))
    floor = max(1e-3 * float(exp.pow(2).mean().sqrt()), 1e-30)
    return float(((out - exp).abs() / exp.abs().clamp_min(floor)).max())


VIT_B, VIT_S, VIT_H, VIT_D, VIT_E, VIT_F = 8, 197, 12, 64, 768, 3072


def make_vit(pkg, torch, dev):
    """ViT-B/16-shaped attention + MLP, batch 8, fp16: Q/K/V [96, 197, 64] ~
    N(0,1), SDPA with scale 1/8; x [1576, 768] ~ N(0,1) -> fc1 768->3072 +
    bias + tanh-GELU -> fc2 3072->768 + bias, weights and biases N(0,0.02)."""
    g = torch.Generator().manual_seed(5)
    B, S, Hh, D, E, F = VIT_B, VIT_S, VIT_H, VIT_D, VIT_E, VIT_F
    t = {
        "q": torch.randn(B * Hh, S, D, generator=g).half().to(dev),
        "k": torch.randn(B * Hh, S, D, generator=g).half().to(dev),
        "v": torch.randn(B * Hh, S, D, generator=g).half().to(dev),
        "x": torch.randn(B * S, E, generator=g).half().to(dev),
        "w1": (torch.randn(F, E, generator=g) * 0.02).half().to(dev),
        "b1": (torch.randn(F, generator=g) * 0.02).half().to(dev),
        "w2": (torch.randn(E, F, generator=g) * 0.02).half().to(dev),
        "b2": (torch.randn(E, generator=g) * 0.02).half().to(dev),
    }
    buf = {"attn": torch.empty(B * Hh, S, D, dtype=torch.float16, device=dev),
           "h": torch.empty(B * S, F, dtype=torch.float16, device=dev),
           "y": torch.empty(B * S, E, dtype=torch.float16, device=dev)}

    def attention(_i=0):
        pkg.attention(t["q"], t["k"], t["v"], 0.125, out=buf["attn"])

    def step(_i=0):
        attention()
        pkg.linear(t["x"], t["w1"], t["b1"], epilogue="gelu_tanh", out=buf["h"])
        pkg.linear(buf["h"], t["w2"], t["b2"], out=buf["y"])

    return step, attention, t, buf


def check_vit(torch, t, buf) -> dict:
    """The ViT step's outputs against torch fp32 on the GPU: SDPA in fp32,
    fc1 + bias + tanh-GELU, fc2 + bias of the kernel's own fp16 h."""
    f = lambda v: v.float()  # noqa: E731
    s = torch.bmm(f(t["q"]), f(t["k"]).transpose(1, 2).contiguous()) * 0.125
    exp = {"attn": torch.bmm(torch.softmax(s, -1), f(t["v"]))}
    exp["h"] = torch.nn.functional.gelu(f(t["x"]) @ f(t["w1"]).t() + f(t["b1"]), approximate="tanh")
    exp["y"] = f(buf["h"]) @ f(t["w2"]).t() + f(t["b2"])
    return {k: rel_err(torch, buf[k], v, vs_scale=(k == "attn")) for k, v in exp.items()}


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
    """One decode linear, rotating over enough distinct weight copies (>= 768
    MB in all, three times the 256 MB Infinity Cache) that no copy is still
    cached when it is read again; each graph replay reads every copy once.
    GB/s against the HBM peak; for M > 16 (near the ridge) also TFLOP/s
    against min(MFMA peak, arithmetic intensity x HBM peak)."""
    g = torch.Generator().manual_seed(2)
    wbytes = N * K * (1 if int8 else 2)
    copies = max(2, -(-min_bytes // wbytes))
    x = torch.randn(M, K, generator=g).half().to(dev)
    y = torch.empty(M, N, dtype=torch.float16, device=dev)
    if int8:
        ws = torch.randint(-127, 128, (copies, N, K), dtype=torch.int8, device=dev)
        s = (torch.rand(N, generator=g) * 9e-3 + 1e-3).half().to(dev)
        fn = lambda i: pkg.w8a16_linear(x, ws[i % copies], s, out=y)  # noqa: E731
        algo = N * K + 2 * N + 2 * M * K + 2 * M * N
    else:
        ws = torch.empty(copies, N, K, dtype=torch.float16, device=dev).normal_(0, 0.02)
        fn = lambda i: pkg.gemv(x, ws[i % copies], out=y)  # noqa: E731
        algo = 2 * (N * K + M * K + M * N)
    ms = timer.graph_ms(fn, max(iters, copies))
    gbs = algo / (ms * 1e-3) / 1e9
    del ws
    out = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1), "frac_hbm_peak": round(gbs / PEAK_HBM_GBS, 4),
           "bytes": algo, "weight_copies": copies}
    if M > 16:
        flop = 2 * M * N * K
        tf = flop / (ms * 1e-3) / 1e12
        bound = min(PEAK_FP16_TFLOPS, flop / algo * PEAK_HBM_GBS / 1e3)
        out.update({"tflops": round(tf, 1), "roofline_tflops": round(bound, 1), "frac_roofline": round(tf / bound, 4)})
    return out


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


def bench_decode_full(pkg, torch, dev, timer, iters):
    """The whole one-token Qwen2.5-0.5B forward at position 0 (what the
    reference's Qwen run computes: RMSNorms, q|k|v with bias, attention over
    the one key, o + residual, gate|up, SiLU-mul, down + residual, final norm,
    lm_head), 0.99 GB of fp16 weights: as the persistent decode kernel (one
    launch + the lm_head GEMV) and as the same step from separate library
    launches (RMSNorm, GEMV, torch elementwise glue), both in HIP graphs; the
    persistent kernel also with each layer's o projection folded onto the
    normalised layer input (DecoderStack.fold_o: three dependent phases a
    layer instead of four; the folding is weight preparation, done before
    the timed region).  The outputs are compared before anything is timed."""
    H, KV, I, V, L, heads, kvh = 896, 128, 4864, 151936, 24, 14, 2
    g = torch.Generator(device=dev).manual_seed(11)
    rnd = lambda *s, std=0.02, mean=0.0: (torch.randn(*s, generator=g, device=dev) * std + mean).half()
    st = pkg.hxmi.DecoderStack(
        w_qkv=rnd(L, H + 2 * KV, H), b_qkv=rnd(L, H + 2 * KV, std=0.1), w_o=rnd(L, H, H), w_gu=rnd(L, 2 * I, H),
        w_down=rnd(L, H, I), g_attn=rnd(L, H, std=0.1, mean=1.0), g_mlp=rnd(L, H, std=0.1, mean=1.0),
        g_final=rnd(H, std=0.1, mean=1.0), heads=heads, kv_heads=kvh, eps=1e-6, w_lm=rnd(V, H))
    x = torch.randn(H, generator=g, device=dev).half()
    grp, hd = heads // kvh, H // heads

    def chained(_i=0):
        xs = x.view(1, H)
        for l in range(L):
            h = pkg.rms_norm(xs, st.g_attn[l], st.eps)
            qkv = pkg.gemv(h, st.w_qkv[l], st.b_qkv[l])
            att = qkv[:, H + KV:].view(kvh, hd).repeat_interleave(grp, dim=0).reshape(1, H)
            xs = xs + pkg.gemv(att, st.w_o[l])
            h = pkg.rms_norm(xs, st.g_mlp[l], st.eps)
            gu = pkg.gemv(h, st.w_gu[l])
            a = torch.nn.functional.silu(gu[:, :I]) * gu[:, I:]
            xs = xs + pkg.gemv(a, st.w_down[l])
        return pkg.gemv(pkg.rms_norm(xs, st.g_final, st.eps), st.w_lm)

    stf = dataclasses.replace(st).fold_o()
    out = pkg.hxmi.decode_step(x, st)
    outf = pkg.hxmi.decode_step(x, stf)
    ref_logits = chained()
    torch.cuda.synchronize()
    status = pkg.hxmi.decode_status()
    err = ((out["logits"].float() - ref_logits[0].float()).abs().max() / ref_logits.float().abs().max()).item()
    errf = ((outf["logits"].float() - ref_logits[0].float()).abs().max() / ref_logits.float().abs().max()).item()
    if status != 0 or not err < 1e-2 or not errf < 1e-2:
        raise SystemExit(f"[bench] decode step check failed: status {status}, logits rel err {err} / folded {errf}")
    nbytes = 2 * sum(t.numel() for t in (st.w_qkv, st.b_qkv, st.w_o, st.w_gu, st.w_down, st.g_attn, st.g_mlp,
                                         st.g_final, st.w_lm))
    res = {"bytes": nbytes, "logits_rel_err_vs_chained": round(err, 5),
           "folded_o_logits_rel_err_vs_chained": round(errf, 5)}
    for name, fn in (("persistent", lambda i: pkg.hxmi.decode_step(x, st)),
                     ("persistent_folded_o", lambda i: pkg.hxmi.decode_step(x, stf)), ("chained_launches", chained)):
        ms = timer.graph_ms(fn, iters)
        gbs = nbytes / (ms * 1e-3) / 1e9
        res[name] = {"us": round(ms * 1e3, 1), "GB/s": round(gbs, 1), "frac_hbm_peak": round(gbs / PEAK_HBM_GBS, 4)}
    # the timed replays' own waits: an expired one voids the timing
    torch.cuda.synchronize()
    status = pkg.hxmi.decode_status()
    if status != 0:
        raise SystemExit(f"[bench] decode step: a wait expired during the timed graph replays (status {status})")
    res["status_after_replays"] = status
    del st, stf
    return res


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
    step, attention, t, buf = make_vit(pkg, torch, dev)
    B, S, Hh, D, E, F = VIT_B, VIT_S, VIT_H, VIT_D, VIT_E, VIT_F
    step()
    torch.cuda.synchronize()
    errs = check_vit(torch, t, buf)
    log(f"[bench] ViT check vs torch fp32: {errs}")
    if max(errs.values()) > 1e-2:
        raise SystemExit("[bench] FAILED: the ViT block's outputs differ from the fp32 reference by more than 1e-2")
    ms = timer.graph_ms(step, iters)
    flops = 2 * (2 * B * Hh * S * S * D) + 2 * (2 * B * S * E * F)
    att_ms = timer.graph_ms(attention, iters)
    att_flops = 2 * (2 * B * Hh * S * S * D)
    att_bytes = 4 * B * Hh * S * D * 2  # Q, K, V read once, O written once
    return {"us": round(ms * 1e3, 1), "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
            "attention_us": round(att_ms * 1e3, 2), "attention_tflops": round(att_flops / (att_ms * 1e-3) / 1e12, 1),
            "attention_gbs": round(att_bytes / (att_ms * 1e-3) / 1e9, 1),
            "attention_frac_hbm_peak": round(att_bytes / (att_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _host_cpu_info() -> dict:
    """What lscpu reports (model name, sockets, cores per socket, threads per
    core), the physical cores (distinct (package, core) pairs in
    /proc/cpuinfo) and the logical CPUs this process may run on."""
    import subprocess

    info = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            key = key.strip()
            if key in ("Model name", "Socket(s)", "Core(s) per socket", "Thread(s) per core", "CPU(s)"):
                info["lscpu_" + key.lower().replace("(s)", "s").replace(" ", "_")] = val.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    cores, pkg_id = set(), "0"
    try:
        for line in open("/proc/cpuinfo"):
            key, _, val = line.partition(":")
            key = key.strip()
            if key == "physical id":
                pkg_id = val.strip()
            elif key == "core id":
                cores.add((pkg_id, val.strip()))
    except OSError:
        pass
    info["physical_cores"] = len(cores) or None
    info["allowed_cpus"] = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    return info


def cpu_baseline(runs: int = 7) -> dict:
    """The reference's CPU path for the headline block: PyTorch CPU ops in
    fp32 (the x86 forward its benchmarks compare against,
    benchmark_models/run_tinyllama.py:204-205,
    micro_bench/test_matmul_benchmark.py:91) -- RMSNorm, the QKV, O, gate,
    up and down linears and SiLU-mul of the 512-token TinyLlama block on the
    same-shaped seeded inputs -- timed on this host with every thread torch
    is allowed (OMP_NUM_THREADS) and with one thread: median of `runs` blocks
    after one warm-up block each."""
    import torch
    import torch.nn.functional as F

    g = torch.Generator().manual_seed(0)
    x = torch.randn(TL_M, TL_H, generator=g)
    gn = 1 + 0.02 * torch.randn(TL_H, generator=g)
    wqkv = 0.02 * torch.randn(TL_QKV, TL_H, generator=g)
    wo = 0.02 * torch.randn(TL_H, TL_H, generator=g)
    wg = 0.02 * torch.randn(TL_I, TL_H, generator=g)
    wu = 0.02 * torch.randn(TL_I, TL_H, generator=g)
    wd = 0.02 * torch.randn(TL_H, TL_I, generator=g)
    xa = torch.randn(TL_M, TL_H, generator=g)

    def block():
        xn = F.rms_norm(x, (TL_H,), gn, 1e-5)
        F.linear(xn, wqkv)
        F.linear(xa, wo)
        h = F.silu(F.linear(xn, wg)) * F.linear(xn, wu)
        F.linear(h, wd)

    def median_ms(threads: int) -> float:
        torch.set_num_threads(threads)
        times = []
        with torch.no_grad():
            block()
            for _ in range(runs):
                t0 = time.perf_counter()
                block()
                times.append(time.perf_counter() - t0)
        return sorted(times)[len(times) // 2] * 1e3

    all_threads = torch.get_num_threads()
    ms_all = median_ms(all_threads)
    ms_one = median_ms(1)
    torch.set_num_threads(all_threads)
    flop = tinyllama_flops()["total"]
    tf = lambda ms: round(flop / (ms * 1e-3) / 1e12, 4)  # noqa: E731
    return {"value": tf(ms_all), "unit": "TFLOP/s", "cores": int(all_threads), "kind": "reference",
            "sample": f"the reference's CPU path: torch {torch.__version__} CPU fp32 ops of the full 512-token "
                      f"TinyLlama block (RMSNorm, QKV, O, gate/up + SiLU-mul, down), median of {runs} blocks "
                      f"after a warm-up, {ms_all:.1f} ms each on {all_threads} threads",
            "median_ms": round(ms_all, 2), "single_thread": {"value": tf(ms_one), "median_ms": round(ms_one, 2)},
            "cpu_model": _cpu_model(), "host_cpus": os.cpu_count(), **_host_cpu_info(), "torch": torch.__version__}


def profile_suite(pkg, torch, dev, timer) -> None:
    """Launches for counter runs, each warmed up by time, then 5 launches:
    4096^3 NT and NN GEMMs, the 1024^3 NN GEMM, the Qwen2.5-0.5B lm_head fp16 / int8 GEMVs (M = 1, 16)
    and the int8 GEMM at M = 256 (weights rotate over copies so none is
    cache-resident), the ViT-B/16 batch-8 fused attention, fc1 and fc2,
    softmax [18912, 197], RMSNorm [512, 2048]; then five 256 MiB copies."""
    g = torch.Generator().manual_seed(1)
    a = (torch.rand(4096, 4096, generator=g) * 2 - 1).half().to(dev)
    b = (torch.rand(4096, 4096, generator=g) * 2 - 1).half().to(dev)
    c = torch.empty(4096, 4096, dtype=torch.float16, device=dev)
    gemm = lambda i=0: pkg.gemm(a, b, b_layout="nt", out=c)
    timer._warm(gemm)
    for _ in range(5):
        gemm()
    gemm_nn = lambda i=0: pkg.gemm(a, b, b_layout="nn", out=c)
    timer._warm(gemm_nn)
    for _ in range(5):
        gemm_nn()
    # the 1024^3 NN GEMM (C = A . B, uniform [-1, 1] operands)
    a1 = (torch.rand(1024, 1024, generator=g) * 2 - 1).half().to(dev)
    b1k = (torch.rand(1024, 1024, generator=g) * 2 - 1).half().to(dev)
    c1 = torch.empty(1024, 1024, dtype=torch.float16, device=dev)
    g1024 = lambda i=0: pkg.gemm(a1, b1k, b_layout="nn", out=c1)
    timer._warm(g1024)
    for _ in range(5):
        g1024()
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
    # int8 lm_head at M = 256 (the MFMA GEMM with int8 B), three weight copies
    x = torch.randn(256, H, generator=g).half().to(dev)
    y = torch.empty(256, V, dtype=torch.float16, device=dev)
    w8g = lambda i=0: pkg.w8a16_linear(x, qs[i % 3], sc, out=y)
    timer._warm(w8g)
    for i in range(5):
        w8g(i)
    del ws, qs
    # ViT-B/16 batch 8: fused attention, fc1 (+bias, tanh-GELU), fc2 (+bias)
    B, S, Hh, D, E, F = VIT_B, VIT_S, VIT_H, VIT_D, VIT_E, VIT_F
    q, k, v = (torch.randn(B, Hh, S, D, generator=g).half().to(dev) for _ in range(3))
    o = torch.empty_like(q)
    xv = torch.randn(B * S, E, generator=g).half().to(dev)
    w1 = (torch.randn(F, E, generator=g) * 0.02).half().to(dev)
    b1 = (torch.randn(F, generator=g) * 0.02).half().to(dev)
    w2 = (torch.randn(E, F, generator=g) * 0.02).half().to(dev)
    b2 = (torch.randn(E, generator=g) * 0.02).half().to(dev)
    h1 = torch.empty(B * S, F, dtype=torch.float16, device=dev)
    h2 = torch.empty(B * S, E, dtype=torch.float16, device=dev)
    att = lambda i=0: pkg.attention(q, k, v, D ** -0.5, out=o)
    fc1 = lambda i=0: pkg.linear(xv, w1, b1, epilogue="gelu_tanh", out=h1)
    fc2 = lambda i=0: pkg.linear(h1, w2, b2, out=h2)
    # row kernels: softmax [18912, 197] (scale 0.125), RMSNorm [512, 2048]
    sm_x = torch.randn(B * Hh * S, S, generator=g).half().to(dev)
    sm_y = torch.empty_like(sm_x)
    rn_x = torch.randn(512, 2048, generator=g).half().to(dev)
    rn_w = torch.ones(2048, dtype=torch.float16, device=dev)
    rn_y = torch.empty_like(rn_x)
    smx = lambda i=0: pkg.softmax(sm_x, 0.125, out=sm_y)
    rms = lambda i=0: pkg.rms_norm(rn_x, rn_w, 1e-5, out=rn_y)
    for fn in (att, fc1, fc2, smx, rms):
        timer._warm(fn)
        for _ in range(5):
            fn()
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    log("[bench] profile suite: 4096^3 GEMM NT / NN, 1024^3 GEMM NN, lm_head GEMV fp16 M=1/16, int8 M=1/16/256, ViT-B/16 attention / fc1 / "
        "fc2, softmax [18912, 197], RMSNorm [512, 2048], 5 x 256 MiB copies")


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


def teardown(torch, pkg) -> None:
    """Finish the GPU work and release the library's cached workspaces and
    torch's cached blocks before the interpreter exits, so that no device
    memory the kernels used is still held while the runtime unloads."""
    torch.cuda.synchronize()
    pkg.hxmi.release_workspaces()
    gc.collect()
    torch.cuda.empty_cache()
    torch.cuda.synchronize()


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
                    help="for rocprofv3 counter runs: the 4096^3 fp16 NT and NN GEMMs, the 1024^3 NN GEMM, the "
                         "lm_head decode GEMVs (fp16 M=1 and M=16, int8 M=1/16) and int8 GEMM (M=256), the ViT-B/16 "
                         "attention / fc1 / fc2, softmax and RMSNorm, each warmed up and then launched 5 times, then "
                         "the 256 MiB copy calibration, and exit")
    ap.add_argument("--profile-decode", action="store_true",
                    help="for rocprofv3: the full Qwen2.5-0.5B one-token forward, as the persistent decode kernel "
                         "and as separate launches, checked against each other and timed, and exit")
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
    try:
        return run(args, pkg, torch, dev, timer)
    finally:
        teardown(torch, pkg)


def run(args, pkg, torch, dev, timer) -> int:
    if args.profile_suite:
        profile_suite(pkg, torch, dev, timer)
        return 0
    if args.profile_decode:
        log(f"[bench] full decode forward {bench_decode_full(pkg, torch, dev, timer, 5)}")
        return 0
    step, gate_up, block_tensors, block_buf = make_block(pkg, torch, dev)
    fl = tinyllama_flops()
    # one step checked against torch fp32 before anything is timed
    step()
    torch.cuda.synchronize()
    errs = check_block(torch, block_tensors, block_buf)
    log(f"[bench] block check vs torch fp32 (max rel err): {errs}")
    if max(errs.values()) > 1e-2:
        log("[bench] FAILED: the block's outputs differ from the fp32 reference by more than 1e-2")
        return 3
    if args.profile:
        # gate/up back to back for --warmup-ms (steady clocks), then --steps
        # launches timed with HIP events on the launch stream: the trace's
        # last --steps dispatches are the ones the printed average covers
        step()
        t_end = time.perf_counter() + args.warmup_ms * 1e-3
        while time.perf_counter() < t_end:
            for _ in range(10):
                gate_up()
            torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(args.steps):
            gate_up()
        e.record()
        torch.cuda.synchronize()
        us = s.elapsed_time(e) * 1e3 / args.steps
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] profile mode: {args.steps} gate/up launches after {args.warmup_ms:.0f} ms of warm-up, "
            f"{us:.2f} us each (HIP events), then 5 x 256 MiB copies")
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
        secondary["decode_forward_qwen_m1"] = bench_decode_full(pkg, torch, dev, timer, 5)
        log(f"[bench] full decode forward {secondary['decode_forward_qwen_m1']}")
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
