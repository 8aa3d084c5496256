"""Persistent one-token decode step (hxmi_decode_step_f16, and
hxmi_decode_step_ov_f16 with the o projection folded onto the normalised
layer input, fold=True) against the oracle.

The oracle (oracle.decode_step, pinned against transformers' Qwen2 forward in
tests/test_decode_oracle.py) runs on the CPU from the same fp16 weights.  The
kernel rounds to fp16 where the HF fp16 forward does, so it is compared with
the oracle's fp16-rounding mode: per-element fp16 results can differ by an
ulp where the fp32 sums of a dot product differ in order, and such a
difference travels through the residual stream, so the bound is a relative
one over the vector (max |diff| / max |ref|).  The fp32 forward bounds the
same outputs within the 1e-2 relative error fp16 outputs are held to.
"""
import numpy as np
import pytest
import torch

from oracle import hot_path as ref

pytestmark = pytest.mark.gpu

QWEN = dict(layers=24, hidden=896, heads=14, kv_heads=2, inter=4864, vocab=151936, bias=True, eps=1e-6)
TINYLLAMA = dict(layers=3, hidden=2048, heads=32, kv_heads=4, inter=5632, vocab=0, bias=False, eps=1e-5)


def make_stack(pkg, dev, layers, hidden, heads, kv_heads, inter, vocab, bias, eps, seed=0):
    """Random stack on the GPU (weights N(0, 0.02), norm weights 1 + N(0, 0.1),
    biases N(0, 0.1)) and its numpy copy for the oracle."""
    g = torch.Generator(device=dev).manual_seed(seed)
    kv = hidden // heads * kv_heads
    rnd = lambda *shape, std=0.02, mean=0.0: (torch.randn(*shape, generator=g, device=dev) * std + mean).half()
    st = pkg.hxmi.DecoderStack(
        w_qkv=rnd(layers, hidden + 2 * kv, hidden), b_qkv=rnd(layers, hidden + 2 * kv, std=0.1) if bias else None,
        w_o=rnd(layers, hidden, hidden), w_gu=rnd(layers, 2 * inter, hidden), w_down=rnd(layers, hidden, inter),
        g_attn=rnd(layers, hidden, std=0.1, mean=1.0), g_mlp=rnd(layers, hidden, std=0.1, mean=1.0),
        g_final=rnd(hidden, std=0.1, mean=1.0), heads=heads, kv_heads=kv_heads, eps=eps,
        w_lm=rnd(vocab, hidden) if vocab else None)
    x = torch.randn(hidden, generator=g, device=dev).half()
    np_w = {k: (None if getattr(st, k) is None else getattr(st, k).cpu().numpy())
            for k in ("w_qkv", "b_qkv", "w_o", "w_gu", "w_down", "g_attn", "g_mlp", "g_final", "w_lm")}
    return st, x, np_w


@pytest.fixture(params=[False, True], ids=["o", "folded_o"])
def fold(request):
    return request.param


def stack_for(pkg, dev, fold, **kw):
    st, x, np_w = make_stack(pkg, dev, **kw)
    if fold:
        st.fold_o()
    return st, x, np_w


def oracle(x, st, np_w, fp16=True):
    return ref.decode_step(x.cpu().numpy(), heads=st.heads, kv_heads=st.kv_heads, eps=st.eps, fp16=fp16, **np_w)


def rel(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-6))


def check(out, want, want32, tag, tol16=4e-3, tol32=1e-2):
    errs = {k: rel(out[k].float().cpu().numpy(), want[k]) for k in ("h", "x", "qkv")}
    if out["logits"] is not None:
        errs["logits"] = rel(out["logits"].float().cpu().numpy(), want["logits"])
    errs32 = {k: rel(out[k].float().cpu().numpy(), want32[k]) for k in ("h", "x")}
    print(f"[decode {tag}] rel err vs fp16 oracle {errs}, vs fp32 {errs32}", flush=True)
    assert all(v < tol16 for v in errs.values()), errs
    assert all(v < tol32 for v in errs32.values()), errs32


def test_decode_step_qwen05b_matches_oracle(pkg, dev, fold):
    st, x, np_w = stack_for(pkg, dev, fold, **QWEN, seed=1)
    out = pkg.hxmi.decode_step(x, st, out_qkv=True)
    torch.cuda.synchronize()
    assert pkg.hxmi.decode_status() == 0
    check(out, oracle(x, st, np_w), oracle(x, st, np_w, fp16=False), "qwen2.5-0.5b")


def test_decode_step_tinyllama_dims(pkg, dev, fold):
    st, x, np_w = stack_for(pkg, dev, fold, **TINYLLAMA, seed=2)
    out = pkg.hxmi.decode_step(x, st, out_qkv=True)
    torch.cuda.synchronize()
    assert pkg.hxmi.decode_status() == 0
    check(out, oracle(x, st, np_w), oracle(x, st, np_w, fp16=False), "tinyllama")


@pytest.mark.parametrize("dims", [
    dict(layers=2, hidden=64, heads=2, kv_heads=1, inter=40, vocab=96, bias=True, eps=1e-6),  # most CUs own no row
    dict(layers=5, hidden=520, heads=13, kv_heads=1, inter=1000, vocab=0, bias=False, eps=1e-6),  # ragged rows, 13 q heads per kv head
])
def test_decode_step_small_and_ragged(pkg, dev, fold, dims):
    st, x, np_w = stack_for(pkg, dev, fold, **dims, seed=3)
    out = pkg.hxmi.decode_step(x, st, out_qkv=True)
    torch.cuda.synchronize()
    assert pkg.hxmi.decode_status() == 0
    check(out, oracle(x, st, np_w), oracle(x, st, np_w, fp16=False), f"H{dims['hidden']}")


def test_decode_step_repeats_exactly_with_fresh_inputs(pkg, dev, fold):
    # every launch publishes under new tags: a launch never reads the previous one's vectors
    st, x, np_w = stack_for(pkg, dev, fold, layers=4, hidden=896, heads=14, kv_heads=2, inter=4864, vocab=0, bias=True,
                             eps=1e-6, seed=4)
    x2 = torch.randn(896, generator=torch.Generator(device=dev).manual_seed(9), device=dev).half()
    a = pkg.hxmi.decode_step(x, st)
    b = pkg.hxmi.decode_step(x2, st)
    c = pkg.hxmi.decode_step(x, st)
    torch.cuda.synchronize()
    assert pkg.hxmi.decode_status() == 0
    assert torch.equal(a["h"], c["h"]) and torch.equal(a["x"], c["x"])
    assert rel(b["h"].float().cpu().numpy(), oracle(x2, st, np_w)["h"]) < 4e-3
    assert not torch.equal(a["h"], b["h"])


def test_decode_step_expired_wait_is_reported_and_recovered(pkg, dev, fold):
    # a 1 us bound on every wait: the launch gives up early (every wave still
    # leaves), the error word says so, and the next launch is correct
    st, x, np_w = stack_for(pkg, dev, fold, layers=4, hidden=896, heads=14, kv_heads=2, inter=4864, vocab=0, bias=True,
                             eps=1e-6, seed=5)
    pkg.hxmi.decode_step(x, st, timeout_us=1)
    torch.cuda.synchronize()
    assert pkg.hxmi.decode_status(clear=True) == 1
    assert pkg.hxmi.decode_status() == 0
    out = pkg.hxmi.decode_step(x, st)
    torch.cuda.synchronize()
    assert pkg.hxmi.decode_status() == 0
    assert rel(out["h"].float().cpu().numpy(), oracle(x, st, np_w)["h"]) < 4e-3


def test_decode_step_is_the_chain_of_library_ops(pkg, dev):
    # the same step from separate launches (RMSNorm, GEMV, elementwise) agrees
    st, x, np_w = make_stack(pkg, dev, layers=2, hidden=896, heads=14, kv_heads=2, inter=4864, vocab=1024,
                             bias=True, eps=1e-6, seed=6)
    out = pkg.hxmi.decode_step(x, st)
    H, kv, I = 896, 128, 4864
    xs = x.view(1, H)
    for l in range(2):
        h = pkg.rms_norm(xs, st.g_attn[l], st.eps)
        qkv = pkg.gemv(h, st.w_qkv[l], st.b_qkv[l])
        v = qkv[:, H + kv:].view(2, 64)
        att = v.repeat_interleave(7, dim=0).reshape(1, H).contiguous()
        xs = xs + pkg.gemv(att, st.w_o[l])
        h = pkg.rms_norm(xs, st.g_mlp[l], st.eps)
        gu = pkg.gemv(h, st.w_gu[l])
        a = (torch.nn.functional.silu(gu[:, :I]) * gu[:, I:]).contiguous()
        xs = xs + pkg.gemv(a, st.w_down[l])
    h = pkg.rms_norm(xs, st.g_final, st.eps)
    logits = pkg.gemv(h, st.w_lm)
    torch.cuda.synchronize()
    assert rel(out["h"].float().cpu().numpy(), h[0].float().cpu().numpy()) < 4e-3
    assert rel(out["logits"].float().cpu().numpy(), logits[0].float().cpu().numpy()) < 1e-2


def test_fold_o_weights(pkg, dev):
    """w_ov = w_o E w_v and b_ov = w_o E b_v per layer (E copies key/value head
    j to the query heads of its group), against float64 on the CPU."""
    st, x, np_w = make_stack(pkg, dev, layers=2, hidden=896, heads=14, kv_heads=2, inter=64, vocab=0, bias=True,
                             eps=1e-6, seed=7)
    st.fold_o()
    H, kv, hd, grp = 896, 128, 64, 7
    i = np.arange(H)
    vrow = H + kv + (i // hd // grp) * hd + i % hd
    for l in range(2):
        wv = np_w["w_qkv"][l].astype(np.float64)[vrow]
        want = np_w["w_o"][l].astype(np.float64) @ wv
        got = st.w_ov[l].float().cpu().numpy()
        assert ref.max_rel_err(got, want) <= 1e-2
        wantb = np_w["w_o"][l].astype(np.float64) @ np_w["b_qkv"][l].astype(np.float64)[vrow]
        assert ref.max_rel_err(st.b_ov[l].float().cpu().numpy(), wantb) <= 1e-2
    # without biases there is no b_ov
    st2, _, _ = make_stack(pkg, dev, layers=1, hidden=64, heads=2, kv_heads=1, inter=40, vocab=0, bias=False,
                           eps=1e-6, seed=8)
    assert st2.fold_o().b_ov is None
