"""GPU parity of the fused attention kernel (hxmi_attention_f16) against the
oracle's SDPA (the reference's tm_tensor.attention lowering,
LowerTmTensor.cpp:91-250: bmm(Q, K^T) * scale -> softmax -> bmm(P, V))."""
import math

import numpy as np
import pytest
import torch

from gpu_util import TOL, np32, uniform
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
