"""GPU parity of the fused attention kernel (hxmi_attention_f16) against the
oracle's SDPA (the reference's tm_tensor.attention lowering,
LowerTmTensor.cpp:91-250: bmm(Q, K^T) * scale -> softmax -> bmm(P, V))."""
import math

import numpy as np
import pytest
import torch

from gpu_util import TOL, normal, np32, uniform
from oracle import hot_path as ref

pytestmark = pytest.mark.gpu


def _attn(pkg, q, k, v, scale):
    return pkg.attention(q.cuda(), k.cuda(), v.cuda(), scale=scale).cpu()


def _check(out, q, k, v, scale):
    exp = ref.sdpa(np32(q), np32(k), np32(v), scale)
    o = np32(out)
    # fp16 probabilities feed P.V, so outputs that average to ~0 carry ~1e-4
    # absolute noise: the bar is relative to the output's scale, plus an RMS bound
    assert ref.max_err_vs_scale(o, exp) <= TOL
    assert np.sqrt(np.mean((o - exp) ** 2)) <= 2e-3 * np.sqrt(np.mean(exp**2)) + 1e-6


@pytest.mark.parametrize(
    "bh,s,skv,d",
    [
        (12, 197, 197, 64),  # ViT-B/16 self-attention, 12 heads
        (4, 300, 300, 128),
        (3, 1, 1, 64),
        (2, 77, 300, 128),  # cross-attention, ragged lengths
        (2, 129, 33, 64),
        (1, 256, 512, 64),
    ],
)
def test_attention_vs_oracle(pkg, dev, bh, s, skv, d):
    q = uniform((bh, s, d), 1)
    k = uniform((bh, skv, d), 2)
    v = uniform((bh, skv, d), 3)
    scale = 1.0 / math.sqrt(d)
    _check(_attn(pkg, q, k, v, scale), q, k, v, scale)


@pytest.mark.parametrize("d", [64, 128])
def test_attention_one_hot_is_exact(pkg, dev, d):
    """Q[q] = alpha * K[t(q)] makes key t(q) win by > 20 nats, so softmax is
    one-hot to far below fp16 resolution and O[q] must equal V[t(q)] bit for
    bit: any wrong key, head-dim or query index shows up."""
    bh, s, skv = 3, 150, 260
    scale = 1.0 / math.sqrt(d)
    k = uniform((bh, skv, d), 11)
    v = uniform((bh, skv, d), 12)
    t = torch.randint(0, skv, (bh, s), generator=torch.Generator().manual_seed(13))
    alpha = 200.0 / (scale * d / 3)  # scaled winning score ~ 200: |K_t|^2 ~ d / 3 for uniform [-1, 1]
    q = (alpha * torch.gather(k.float(), 1, t[..., None].expand(bh, s, d))).half()
    exp = ref.sdpa(np32(q), np32(k), np32(v), scale)
    sc = np.einsum("bqd,bkd->bqk", np32(q), np32(k)) * scale
    srt = np.sort(sc, axis=-1)
    assert (srt[..., -1] - srt[..., -2]).min() > 20  # the premise of the test
    assert np.array_equal(np.argmax(sc, -1), t.numpy())
    want = torch.gather(v, 1, t[..., None].expand(bh, s, d))
    assert np.abs(exp - np32(want)).max() < 1e-6
    out = _attn(pkg, q, k, v, scale)
    assert torch.equal(out, want)


def test_attention_constant_v_is_exact(pkg, dev):
    """A V with identical rows comes back unchanged: softmax weights sum to one
    (the kernel normalises by the sum of the same fp16 weights it multiplies)."""
    bh, s, skv, d = 2, 100, 333, 64
    q = uniform((bh, s, d), 21)
    k = uniform((bh, skv, d), 22)
    row = uniform((bh, 1, d), 23)
    v = row.expand(bh, skv, d).contiguous()
    out = _attn(pkg, q, k, v, 0.125)
    want = row.expand(bh, s, d)
    # exact up to fp32 accumulation of <= 333 weighted terms
    assert np.abs(np32(out) - np32(want)).max() <= 2e-3 * np.abs(np32(row)).max()


def test_attention_strided_views(pkg, dev):
    """q, k, v as column slices of one packed [bh, S, 3D] buffer (row stride 3D)."""
    bh, s, d = 6, 197, 64
    qkv = uniform((bh, s, 3 * d), 31).cuda()
    q, k, v = qkv[..., :d], qkv[..., d : 2 * d], qkv[..., 2 * d :]
    assert q.stride(1) == 3 * d
    out = pkg.attention(q, k, v, scale=0.125).cpu()
    _check(out, q.cpu(), k.cpu(), v.cpu(), 0.125)


def test_attention_4d_heads(pkg, dev):
    """[B, H, S, D] inputs, the layout torch's scaled_dot_product_attention takes."""
    b, h, s, d = 2, 3, 65, 128
    q = uniform((b, h, s, d), 41)
    k = uniform((b, h, s, d), 42)
    v = uniform((b, h, s, d), 43)
    out = _attn(pkg, q, k, v, None)
    assert out.shape == (b, h, s, d)
    _check(out.reshape(-1, s, d), q.reshape(-1, s, d), k.reshape(-1, s, d), v.reshape(-1, s, d), d**-0.5)


def test_attention_rejects_bad_head_dim_through_abi(pkg, dev):
    lib = pkg.hxmi.load_library()
    x = torch.zeros(4, 96, dtype=torch.float16, device="cuda")
    rc = lib.hxmi_attention_f16(x.data_ptr(), x.data_ptr(), x.data_ptr(), x.data_ptr(), 1, 4, 4, 96, 96, 96, 96, 96,
                                0, 0, 0, 0, 1.0, None)
    assert rc == 1 and b"head dim" in lib.hxmi_last_error()


# ---- mask operand, causal rules, grouped K/V heads ---------------------------------------------------

CFGS_64 = [41, 22, 14, 21, 12, 42, 24]  # query waves * 10 + key-split waves
CFGS_128 = [41, 22, 14, 21, 12]


def _check_nan(out, exp):
    """As _check, where rows whose every key is masked must be NaN in both."""
    o = np32(out)
    nan_e = np.isnan(exp).all(-1)
    assert np.array_equal(np.isnan(o).all(-1), nan_e) and not np.isnan(o[~nan_e]).any()
    o, exp = o[~nan_e], exp[~nan_e]
    assert ref.max_err_vs_scale(o, exp) <= TOL
    assert np.sqrt(np.mean((o - exp) ** 2)) <= 2e-3 * np.sqrt(np.mean(exp**2)) + 1e-6


@pytest.mark.parametrize(
    "b,h,s,skv,d,mshape",
    [
        (2, 3, 197, 197, 64, "b1"),  # HF-style [B, 1, S, S_kv] mask shared by the heads
        (1, 4, 77, 300, 128, "bh"),  # one mask slice per head
        (2, 2, 100, 256, 64, "ss"),  # one [S, S_kv] mask for every slice (aligned rows: 8-byte loads)
        (1, 3, 33, 45, 128, "ss"),
    ],
)
def test_attention_additive_mask(pkg, dev, b, h, s, skv, d, mshape):
    q, k, v = uniform((b, h, s, d), 51), uniform((b, h, skv, d), 52), uniform((b, h, skv, d), 53)
    shape = {"b1": (b, 1, s, skv), "bh": (b, h, s, skv), "ss": (s, skv)}[mshape]
    m = normal(shape, 54)
    drop = torch.rand(shape, generator=torch.Generator().manual_seed(55)) < 0.2
    m = m.masked_fill(drop, float("-inf"))
    m[..., 0] = 0.0  # every query keeps key 0
    scale = d**-0.5
    out = pkg.attention(q.cuda(), k.cuda(), v.cuda(), scale, mask=m.cuda()).cpu()
    exp = ref.sdpa(np32(q), np32(k), np32(v), scale, mask=np32(m))
    _check_nan(out, exp)


def test_attention_bool_mask(pkg, dev):
    b, h, s, d = 2, 2, 130, 64
    q, k, v = uniform((b, h, s, d), 61), uniform((b, h, s, d), 62), uniform((b, h, s, d), 63)
    keep = torch.rand((b, 1, s, s), generator=torch.Generator().manual_seed(64)) > 0.5
    keep[..., 7] = True
    out = pkg.attention(q.cuda(), k.cuda(), v.cuda(), mask=keep.cuda()).cpu()
    add = np.where(keep.numpy(), 0.0, -np.inf).astype(np.float32)
    _check_nan(out, ref.sdpa(np32(q), np32(k), np32(v), d**-0.5, mask=add))


@pytest.mark.parametrize(
    "bh,s,skv,d,causal",
    [
        (4, 300, 300, 64, 1),
        (2, 512, 512, 128, 1),  # TinyLlama-sized causal prefill head pair
        (3, 100, 300, 128, 2),  # bottom-right: queries are the last 100 positions
        (2, 300, 100, 64, 2),  # S > S_kv: the first 200 queries see no key (NaN rows)
        (2, 45, 197, 64, 1),
    ],
)
def test_attention_causal(pkg, dev, bh, s, skv, d, causal):
    q, k, v = uniform((bh, s, d), 71), uniform((bh, skv, d), 72), uniform((bh, skv, d), 73)
    out = pkg.attention(q.cuda(), k.cuda(), v.cuda(), 0.1, causal=causal).cpu()
    _check_nan(out, ref.sdpa(np32(q), np32(k), np32(v), 0.1, causal=causal))


def test_attention_causal_with_mask_and_gqa(pkg, dev):
    """TinyLlama's attention shape: 32 query heads over 4 K/V heads, causal, plus a padding mask."""
    b, hq, hkv, s, d = 1, 32, 4, 256, 64
    q, k, v = uniform((b, hq, s, d), 81), uniform((b, hkv, s, d), 82), uniform((b, hkv, s, d), 83)
    m = torch.zeros((b, 1, s, s), dtype=torch.float16)
    m[..., 200:] = float("-inf")  # padded keys
    out = pkg.attention(q.cuda(), k.cuda(), v.cuda(), mask=m.cuda(), causal=1).cpu()
    exp = ref.sdpa(np32(q), np32(k), np32(v), d**-0.5, mask=np32(m), causal=1, kv_group=hq // hkv)
    _check_nan(out, exp)


@pytest.mark.parametrize("hq,hkv,d", [(8, 2, 64), (6, 1, 128), (4, 4, 64)])
def test_attention_gqa(pkg, dev, hq, hkv, d):
    b, s = 2, 129
    q, k, v = uniform((b, hq, s, d), 91), uniform((b, hkv, s, d), 92), uniform((b, hkv, s, d), 93)
    out = pkg.attention(q.cuda(), k.cuda(), v.cuda()).cpu()
    _check_nan(out, ref.sdpa(np32(q), np32(k), np32(v), d**-0.5, kv_group=hq // hkv))


def test_attention_mask_picks_key_exactly(pkg, dev):
    """mask[q, t(q)] = +200 makes key t(q) win by far more than fp16 resolves
    (scores of uniform [-1, 1] inputs stay below 8), so O[q] = V[t(q)] bit for
    bit: a mask read at a wrong (slice, query, key) shows up.  The mask is
    [B, 1, S, S_kv], one slice per batch row shared by its heads."""
    b, h, s, skv, d = 3, 4, 150, 260, 64
    q, k, v = uniform((b, h, s, d), 101), uniform((b, h, skv, d), 102), uniform((b, h, skv, d), 103)
    t = torch.randint(0, skv, (b, s), generator=torch.Generator().manual_seed(104))
    m = torch.zeros((b, 1, s, skv), dtype=torch.float16)
    m.scatter_(3, t[:, None, :, None], 200.0)
    out = pkg.attention(q.cuda(), k.cuda(), v.cuda(), 0.125, mask=m.cuda()).cpu()
    want = torch.gather(v, 2, t[:, None, :, None].expand(b, h, s, d))
    assert torch.equal(out, want)


@pytest.mark.parametrize("cfg", CFGS_64)
def test_attention_launch_shapes_d64(pkg, dev, knobs, cfg):
    """Every workgroup shape (query waves x key-split waves) on the ViT-B/16
    head shape, unmasked and with a causal padding mask."""
    knobs(attn_cfg=cfg)
    bh, s, d = 12, 197, 64
    q, k, v = uniform((bh, s, d), 111), uniform((bh, s, d), 112), uniform((bh, s, d), 113)
    out = pkg.attention(q.cuda(), k.cuda(), v.cuda(), 0.125).cpu()
    _check(out, q, k, v, 0.125)
    m = torch.zeros((s, s), dtype=torch.float16)
    m[:, 150:] = float("-inf")
    out = pkg.attention(q.cuda(), k.cuda(), v.cuda(), 0.125, mask=m.cuda(), causal=1).cpu()
    _check_nan(out, ref.sdpa(np32(q), np32(k), np32(v), 0.125, mask=np32(m), causal=1))


@pytest.mark.parametrize("cfg", CFGS_128)
def test_attention_launch_shapes_d128(pkg, dev, knobs, cfg):
    knobs(attn_cfg=cfg)
    bh, s, skv, d = 5, 300, 333, 128
    q, k, v = uniform((bh, s, d), 121), uniform((bh, skv, d), 122), uniform((bh, skv, d), 123)
    out = pkg.attention(q.cuda(), k.cuda(), v.cuda(), 0.09).cpu()
    _check(out, q, k, v, 0.09)
    out = pkg.attention(q.cuda(), k.cuda(), v.cuda(), 0.09, causal=2).cpu()
    _check_nan(out, ref.sdpa(np32(q), np32(k), np32(v), 0.09, causal=2))


def test_attention_ex_rejects_bad_arguments(pkg, dev):
    lib = pkg.hxmi.load_library()
    x = torch.zeros(4, 64, dtype=torch.float16, device="cuda")
    args = [x.data_ptr()] * 4 + [2, 4, 4, 64, 64, 64, 64, 64, 256, 256, 256, 256]
    rc = lib.hxmi_attention_ex_f16(*args, 3, None, 0, 0, 1, 0, 1.0, None)  # kv_group 3 does not divide bh 2
    assert rc == 1 and b"kv_group" in lib.hxmi_last_error()
    rc = lib.hxmi_attention_ex_f16(*args, 1, None, 0, 0, 1, 3, 1.0, None)
    assert rc == 1 and b"causal" in lib.hxmi_last_error()
    rc = lib.hxmi_attention_ex_f16(*args, 1, None, 0, 0, 1, 0, -1.0, None)
    assert rc == 1 and b"scale" in lib.hxmi_last_error()
    rc = lib.hxmi_attention_ex_f16(*args, 1, x.data_ptr(), 2, 0, 1, 0, 1.0, None)  # ldm below s_kv
    assert rc == 1 and b"mask row stride" in lib.hxmi_last_error()


# ---- the three-step path with the mask operand (any head dim, bf16) ---------------------------------


def _check_nan_tol(out, exp, rms):
    """_check_nan with the RMS bound given: bf16 rounds S and P to 8 mantissa
    bits against fp16's 11, so its RMS bar is 8x fp16's (the max-error bar
    relative to the output's scale stays 1e-2)."""
    o = np32(out)
    nan_e = np.isnan(exp).all(-1)
    assert np.array_equal(np.isnan(o).all(-1), nan_e) and not np.isnan(o[~nan_e]).any()
    o, exp = o[~nan_e], exp[~nan_e]
    assert ref.max_err_vs_scale(o, exp) <= TOL
    assert np.sqrt(np.mean((o - exp) ** 2)) <= rms * np.sqrt(np.mean(exp**2)) + 1e-6


RMS = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize(
    "b,h,s,skv,d,mshape",
    [
        (2, 3, 197, 197, 80, "b1"),  # head dim 80: not a fused-kernel shape
        (1, 4, 77, 130, 32, "bh"),
        (2, 2, 100, 256, 96, "ss"),
        (1, 2, 33, 45, 64, "ss"),  # head dim 64: bf16 takes the three steps, fp16 the fused kernel
    ],
)
def test_attention_three_step_masked(pkg, dev, dtype, b, h, s, skv, d, mshape):
    q, k, v = (uniform(sh, 150 + i, dtype=dtype) for i, sh in enumerate([(b, h, s, d), (b, h, skv, d), (b, h, skv, d)]))
    shape = {"b1": (b, 1, s, skv), "bh": (b, h, s, skv), "ss": (s, skv)}[mshape]
    m = normal(shape, 154)
    drop = torch.rand(shape, generator=torch.Generator().manual_seed(155)) < 0.2
    m = m.masked_fill(drop, float("-inf"))
    m[..., 0] = 0.0
    out = pkg.attention(q.cuda(), k.cuda(), v.cuda(), d**-0.5, mask=m.cuda()).cpu()
    assert out.dtype == dtype
    _check_nan_tol(out, ref.sdpa(np32(q), np32(k), np32(v), d**-0.5, mask=np32(m)), RMS[dtype])


@pytest.mark.parametrize(
    "bh,s,skv,d,causal,dtype",
    [
        (4, 300, 300, 80, 1, torch.float16),
        (3, 100, 300, 32, 2, torch.float16),  # bottom-right: queries are the last 100 positions
        (2, 300, 100, 80, 2, torch.float16),  # S > S_kv: the first 200 queries see no key (NaN rows)
        (2, 129, 129, 64, 1, torch.bfloat16),
        (2, 64, 200, 128, 2, torch.bfloat16),
    ],
)
def test_attention_three_step_causal(pkg, dev, bh, s, skv, d, causal, dtype):
    q, k, v = uniform((bh, s, d), 171, dtype=dtype), uniform((bh, skv, d), 172, dtype=dtype), \
        uniform((bh, skv, d), 173, dtype=dtype)
    out = pkg.attention(q.cuda(), k.cuda(), v.cuda(), 0.1, causal=causal).cpu()
    _check_nan_tol(out, ref.sdpa(np32(q), np32(k), np32(v), 0.1, causal=causal), RMS[dtype])


@pytest.mark.parametrize("dtype,d", [(torch.float16, 80), (torch.bfloat16, 64), (torch.bfloat16, 128)])
def test_attention_three_step_gqa_mask_causal(pkg, dev, dtype, d):
    """Grouped K/V heads (8 query heads over 2) with a padding mask and the
    causal rule: the query heads of one K/V head are one GEMM batch entry."""
    b, hq, hkv, s = 2, 8, 2, 150
    q, k, v = uniform((b, hq, s, d), 181, dtype=dtype), uniform((b, hkv, s, d), 182, dtype=dtype), \
        uniform((b, hkv, s, d), 183, dtype=dtype)
    m = torch.zeros((b, 1, s, s), dtype=torch.float16)
    m[1, ..., 120:] = float("-inf")  # padded keys of the second batch row
    out = pkg.attention(q.cuda(), k.cuda(), v.cuda(), mask=m.cuda(), causal=1).cpu()
    exp = ref.sdpa(np32(q), np32(k), np32(v), d**-0.5, mask=np32(m), causal=1, kv_group=hq // hkv)
    _check_nan_tol(out, exp, RMS[dtype])


def test_attention_three_step_negative_scale(pkg, dev):
    """scale <= 0 is outside the fused kernel's range: the three steps take it."""
    q, k, v = uniform((3, 90, 64), 191), uniform((3, 70, 64), 192), uniform((3, 70, 64), 193)
    out = pkg.attention(q.cuda(), k.cuda(), v.cuda(), -0.125, causal=2).cpu()
    _check_nan_tol(out, ref.sdpa(np32(q), np32(k), np32(v), -0.125, causal=2), RMS[torch.float16])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_softmax_masked_through_abi(pkg, dev, dtype):
    """hxmi_softmax_masked_*: scores [slices, s_q, s_kv] in padded rows, scale,
    a mask shared by groups of two slices, causal = 2, in place and out of
    place; every element against the oracle's masked softmax."""
    lib = pkg.load_library()
    fn = lib.hxmi_softmax_masked_f16 if dtype == torch.float16 else lib.hxmi_softmax_masked_bf16
    slices, sq, skv, ld = 6, 37, 53, 56
    x = normal((slices, sq, ld), 201, 3.0, dtype=dtype)
    m = normal((3, sq, skv), 202)
    m = m.masked_fill(torch.rand((3, sq, skv), generator=torch.Generator().manual_seed(203)) < 0.3, float("-inf"))
    scale = 0.7
    z = np32(x)[..., :skv] * np.float32(scale) + np.repeat(np32(m), 2, axis=0)
    z = np.where(np.arange(skv)[None, :] > np.arange(sq)[:, None] + (skv - sq), np.float32(-np.inf), z)
    with np.errstate(invalid="ignore"):
        e = np.exp(z - z.max(-1, keepdims=True))
        want = e / e.sum(-1, keepdims=True)
    xd, md = x.cuda(), m.cuda()
    y = torch.full((slices, sq, skv), float("nan"), dtype=dtype, device=dev)
    rc = fn(xd.data_ptr(), y.data_ptr(), slices, sq, skv, ld, sq * ld, skv, sq * skv, md.data_ptr(), skv, sq * skv,
            2, 2, scale, None)
    assert rc == 0, lib.hxmi_last_error()
    rc = fn(xd.data_ptr(), xd.data_ptr(), slices, sq, skv, ld, sq * ld, ld, sq * ld, md.data_ptr(), skv, sq * skv,
            2, 2, scale, None)
    assert rc == 0, lib.hxmi_last_error()
    torch.cuda.synchronize()
    tol = 1e-2 if dtype == torch.bfloat16 else 2e-3
    for got in (np32(y.cpu()), np32(xd.cpu())[..., :skv]):
        assert np.array_equal(np.isnan(got), np.isnan(want))
        ok = ~np.isnan(want)
        assert np.abs(got[ok] - want[ok]).max() <= tol
    # argument checks before any launch
    assert fn(xd.data_ptr(), y.data_ptr(), slices, sq, skv, ld, sq * ld, skv, sq * skv, md.data_ptr(), skv, 0, 0, 1,
              1.0, None) == 1  # mask_group 0
    assert fn(xd.data_ptr(), y.data_ptr(), slices, sq, skv, ld, 1, skv, sq * skv, None, 0, 0, 1, 0, 1.0, None) == 1
