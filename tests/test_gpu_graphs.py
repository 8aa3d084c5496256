"""Workspaces under HIP graph capture.

The split-K GEMM and the persistent decode step keep state in a workspace
that must start from zero (arrival counters; the decode step's tag base,
done / abort words and tagged vectors).  torch captures every graph on one
shared capture stream, so workspaces are keyed by capture: each graph gets
its own, cleared by a fill node it recorded itself.  Two graphs captured one
after the other, the second replayed before the first, must both match the
oracle and each other's eager results.
"""
import pytest
import torch

from oracle import hot_path as ref
from gpu_util import TOL, normal, np32
from test_gpu_decode import check, make_stack, oracle

pytestmark = pytest.mark.gpu


def test_two_captures_replayed_out_of_order(pkg, dev):
    # graph 1: the 512-token TinyLlama down projection 512x2048x5632, which
    # the dispatcher splits over K by default (a split-K workspace)
    assert pkg.load_library().hxmi_gemm_workspace_bytes(512, 2048, 5632, 1, 0) > 0
    x = normal((512, 5632), 70).to(dev)
    w = normal((2048, 5632), 71, 0.02).to(dev)
    y = torch.empty((512, 2048), dtype=torch.float16, device=dev)
    # graph 2: a 2-layer decode step (a decode workspace)
    st, xd, np_w = make_stack(pkg, dev, layers=2, hidden=256, heads=4, kv_heads=2, inter=512, vocab=1000,
                              bias=True, eps=1e-6, seed=5)
    torch.cuda.synchronize()

    g1, g2 = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.graph(g1):
        pkg.gemm(x, w, b_layout="nt", out=y)
    with torch.cuda.graph(g2):
        out = pkg.hxmi.decode_step(xd, st, out_qkv=True)
    # both captures ran on torch's one capture stream; nothing replayed yet
    want_y = ref.linear(x.cpu().numpy(), w.cpu().numpy())
    want, want32 = oracle(xd, st, np_w), oracle(xd, st, np_w, fp16=False)
    first_y = None
    for rep in range(3):
        for t in (out["h"], out["x"], out["qkv"], out["logits"]):
            t.fill_(float("nan"))
        g2.replay()
        torch.cuda.synchronize()
        print(f"[graphs] replay {rep}: decode graph", flush=True)
        assert pkg.hxmi.decode_status() == 0
        check(out, want, want32, f"graph replay {rep}")
        y.fill_(float("nan"))
        g1.replay()
        torch.cuda.synchronize()
        print(f"[graphs] replay {rep}: split-K graph", flush=True)
        assert ref.max_rel_err(np32(y.cpu()), want_y) <= TOL
        first_y = y.clone() if first_y is None else first_y
        assert torch.equal(y, first_y)  # the fix-up adds slices in order: bit-identical
        # eager calls of both between replays, on the current stream's own workspaces
        ye = pkg.gemm(x, w, b_layout="nt")
        oe = pkg.hxmi.decode_step(xd, st, out_qkv=True)
        torch.cuda.synchronize()
        assert pkg.hxmi.decode_status() == 0
        assert torch.equal(ye, first_y)
        check(oe, want, want32, f"eager call after replay {rep}")
