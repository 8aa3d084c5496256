"""Graph planner: rewrites the aten graph of an exported PyTorch program so
its hot-path ops run on the hxmi HIP kernels.

This is the GPU counterpart of what the reference's pipeline does to the
torch-mlir linalg module (LinalgToLLVMPass.cpp:80-405): matmuls become the
MFMA GEMM, the elementwise generics after them are fused into its epilogue
(the reference's HexagonFusionPass stops at the matmul, FusionPass.cpp
:161-179), the RMSNorm and softmax reductions become the row kernels, and
tm_tensor.attention (LowerTmTensor.cpp:52-250) becomes one attention kernel.

Patterns (fp16 / bf16 values only, decided from the export's shape/dtype
metadata; everything else stays a torch op on the GPU and is listed as such
in the plan):
  rms_norm       aten.rms_norm, or the HF LlamaRMSNorm chain
                 to(f32) -> pow 2 -> mean(-1) -> add eps -> rsqrt -> mul ->
                 to(dtype) -> mul weight
  rms_linear     an fp16 RMSNorm whose every user is a linear layer (q/k/v,
                 with or without bias) or a fused gate/up: the norm weight is
                 folded into each weight, the first projection takes the row
                 statistics inside its GEMM and publishes the row scales, the
                 others reuse them (no RMSNorm kernel, the normalised
                 activations never go to memory)
  silu_mul       mul(silu(linear(h, Wg)), linear(h, Wu)) -> one GEMM over the
                 packed gate/up weight with the SiLU-mul epilogue
  linear_gelu    gelu(linear(x, W, b), approximate="tanh") -> GEMM + epilogue
  attention      matmul(softmax(matmul(q, k^T) * s), v) and
                 scaled_dot_product_attention (additive or boolean mask,
                 is_causal, grouped K/V heads; no dropout)
  linear, matmul, bmm, mm, addmm, softmax(-1) -> GEMM / row kernels
"""
from __future__ import annotations

import math
import operator
from dataclasses import dataclass, field
from typing import Any, Optional

import torch
from torch import fx

aten = torch.ops.aten
_HALF = (torch.float16, torch.bfloat16)


def _pkg():
    import hexagon_mlir_amd as pkg

    return pkg


# ---- runtime ops (targets of the rewritten call_function nodes) ----------------


def hx_rms_norm(x, weight, eps):
    return _pkg().rms_norm(x, weight, eps)


def hx_linear(x, w, b=None, act=None):
    return _pkg().linear(x, w, b, epilogue=act)


def hx_silu_mul_linear(x, w_packed):
    return _pkg().linear(x, w_packed, epilogue="silu_mul")


def hx_rms_linear_group(x, eps, specs):
    """The projections of one RMSNorm: specs = ((w_folded, bias, epilogue), ...).
    The first takes the row statistics and publishes the row scales; the
    others apply them.  Returns one output per spec."""
    pkg = _pkg()
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1])
    rs = torch.empty(x2.shape[0], dtype=torch.float32, device=x.device)
    outs = []
    for i, (w, b, epi) in enumerate(specs):
        rsk = {"rscale_out": rs} if i == 0 else {"rscale_in": rs}
        y = pkg.rms_norm_linear(x2, w, eps, epilogue=epi, bias=b, **rsk)
        outs.append(y.reshape(*lead, y.shape[-1]))
    return tuple(outs)


def _as_nt(b):
    """b viewed as [..., N, K] with unit stride in K, if it is a transposed view."""
    if b.dim() >= 2 and b.stride(-2) == 1 and b.size(-2) > 1:
        return b.transpose(-1, -2)
    return None


def hx_matmul(a, b, alpha=1.0):
    pkg = _pkg()
    if a.dim() == 2 and b.dim() == 2:
        bt = _as_nt(b)
        if bt is not None:
            return pkg.gemm(a.contiguous(), bt, b_layout="nt", alpha=alpha)
        return pkg.gemm(a.contiguous(), b.contiguous(), b_layout="nn", alpha=alpha)
    lead = torch.broadcast_shapes(a.shape[:-2], b.shape[:-2])
    a3 = a.expand(*lead, *a.shape[-2:]).reshape(-1, *a.shape[-2:])
    bt = _as_nt(b)
    if bt is not None:
        b3 = bt.expand(*lead, *bt.shape[-2:]).reshape(-1, *bt.shape[-2:])
        out = pkg.bgemm(a3.contiguous(), b3.contiguous(), b_layout="nt", alpha=alpha)
    else:
        b3 = b.expand(*lead, *b.shape[-2:]).reshape(-1, *b.shape[-2:])
        out = pkg.bgemm(a3.contiguous(), b3.contiguous(), b_layout="nn", alpha=alpha)
    return out.reshape(*lead, out.shape[-2], out.shape[-1])


def hx_addmm(bias, a, b):
    bt = _as_nt(b)
    if bt is not None:
        return _pkg().gemm(a.contiguous(), bt, b_layout="nt", epilogue="bias", bias=bias)
    return _pkg().gemm(a.contiguous(), b.contiguous(), b_layout="nn", epilogue="bias", bias=bias)


def hx_softmax(x):
    return _pkg().softmax(x.contiguous())


def hx_attention(q, k, v, scale, mask=None, causal=0):
    return _pkg().attention(q.contiguous(), k.contiguous(), v.contiguous(), scale, mask=mask, causal=causal)


# ---- planning -------------------------------------------------------------------------


@dataclass
class Plan:
    """The rewritten module plus a human-readable record of what runs where."""

    module: fx.GraphModule
    kernels: list = field(default_factory=list)  # (pattern, node name)
    torch_ops: list = field(default_factory=list)  # aten ops left to torch
    gemm_tile: Optional[int] = None  # GEMM tile forced for this plan's runs (tileSizes), else the picker's

    def __call__(self, *args):
        """Run the planned module.  A forced tile steers only the GEMMs of this
        run (a thread-local override, restored afterwards), as the
        reference's tileSizes option applies to one compilation."""
        if self.gemm_tile is None:
            return self.module(*args)
        with _pkg().tuning(gemm_tile=self.gemm_tile):
            return self.module(*args)

    def summary(self) -> str:
        lines = [f"hxmi kernels: {len(self.kernels)}"]
        lines += [f"  {pat:12s} {name}" for pat, name in self.kernels]
        lines.append(f"torch ops: {len(self.torch_ops)}")
        lines += [f"  {name}" for name in self.torch_ops]
        return "\n".join(lines)


def _val(n) -> Optional[torch.Tensor]:
    v = n.meta.get("val") if isinstance(n, fx.Node) else None
    return v if isinstance(v, torch.Tensor) else None


def _is_half(n) -> bool:
    v = _val(n)
    return v is not None and v.dtype in _HALF


def _is(n, *targets) -> bool:
    return isinstance(n, fx.Node) and n.op == "call_function" and n.target in targets


def _single_user(n) -> bool:
    return len(n.users) == 1


class _Planner:
    def __init__(self, gm: fx.GraphModule, fusion: bool):
        self.gm = gm
        self.g = gm.graph
        self.fusion = fusion
        self.plan = Plan(gm)
        self._packed = 0
        self._entry = {}  # rewritten node -> its index in plan.kernels
        self._dropped = set()  # plan.kernels entries whose kernel a later fusion removed

    def replace(self, old: fx.Node, fn, args, pattern: str):
        with self.g.inserting_before(old):
            new = self.g.call_function(fn, tuple(args))
        new.meta.update(old.meta)
        old.replace_all_uses_with(new)
        self.g.erase_node(old)  # some ops (e.g. SDPA) are not removed by dead-code elimination
        self._entry[new] = len(self.plan.kernels)
        self.plan.kernels.append((pattern, old.name))
        return new

    def _buffer(self, t: torch.Tensor, stem: str) -> str:
        name = f"_hxmi_{stem}_{self._packed}"
        self._packed += 1
        self.gm.register_buffer(name, t)
        return name

    # -- patterns ----------------------------------------------------------------------

    def rms_norm_chains(self):
        for rs in list(self.g.nodes):
            if not _is(rs, aten.rsqrt.default):
                continue
            add = rs.args[0]
            if not (_is(add, aten.add.Tensor) and isinstance(add.args[1], (int, float))):
                continue
            mean = add.args[0]
            if not (_is(mean, aten.mean.dim) and list(mean.args[1]) in ([-1],) and
                    (mean.args[2] if len(mean.args) > 2 else mean.kwargs.get("keepdim", False))):
                continue
            pw = mean.args[0]
            if not (_is(pw, aten.pow.Tensor_Scalar) and pw.args[1] == 2):
                continue
            x32 = pw.args[0]
            if not (_is(x32, aten.to.dtype, aten._to_copy.default) and _is_half(x32.args[0])):
                continue
            x = x32.args[0]
            muls = [u for u in rs.users if _is(u, aten.mul.Tensor) and set(u.args) == {x32, rs}]
            if len(muls) != 1 or not _single_user(muls[0]):
                continue
            to16 = next(iter(muls[0].users))
            if not (_is(to16, aten.to.dtype) and to16.args[1] == _val(x).dtype and _single_user(to16)):
                continue
            out = next(iter(to16.users))
            if not _is(out, aten.mul.Tensor):
                continue
            w = out.args[0] if out.args[1] is to16 else out.args[1]
            wv = _val(w)
            if wv is None or wv.dim() != 1 or wv.dtype != _val(x).dtype or wv.numel() != _val(x).shape[-1]:
                continue
            self.replace(out, hx_rms_norm, (x, w, float(add.args[1])), "rms_norm")

    def rms_norm_ops(self):
        for n in list(self.g.nodes):
            if _is(n, aten.rms_norm.default) and _is_half(n.args[0]):
                w = n.args[2] if len(n.args) > 2 else n.kwargs.get("weight")
                eps = n.args[3] if len(n.args) > 3 else n.kwargs.get("eps")
                if w is None or eps is None or len(n.args[1]) != 1:
                    continue
                self.replace(n, hx_rms_norm, (n.args[0], w, float(eps)), "rms_norm")

    def _attr(self, n) -> Optional[torch.Tensor]:
        if isinstance(n, fx.Node) and n.op == "get_attr":
            obj = self.gm
            for part in n.target.split("."):
                obj = getattr(obj, part)
            return obj
        return None

    def silu_mul(self):
        for m in list(self.g.nodes):
            if not _is(m, aten.mul.Tensor) or len(m.args) != 2:
                continue
            a, b = m.args
            for s, u in ((a, b), (b, a)):
                if not (_is(s, aten.silu.default) and _single_user(s)):
                    continue
                g = s.args[0]
                if not (_is(g, aten.linear.default, ) and _is(u, aten.linear.default) and _single_user(g)
                        and _single_user(u)):
                    continue
                if len(g.args) > 2 and g.args[2] is not None or len(u.args) > 2 and u.args[2] is not None:
                    continue
                if g.args[0] is not u.args[0] or not _is_half(g.args[0]):
                    continue
                wg, wu = self._attr(g.args[1]), self._attr(u.args[1])
                if wg is None or wu is None or wg.shape != wu.shape or wg.shape[0] % 16:
                    continue
                packed = _pkg().pack_gate_up(wg.detach(), wu.detach())
                name = f"_hxmi_gate_up_{self._packed}"
                self._packed += 1
                self.gm.register_buffer(name, packed)
                with self.g.inserting_before(m):
                    pw = self.g.get_attr(name)
                self.replace(m, hx_silu_mul_linear, (g.args[0], pw), "silu_mul")
                break

    def rms_linear(self):
        for rn in list(self.g.nodes):
            if not (rn.op == "call_function" and rn.target is hx_rms_norm):
                continue
            x, gw, eps = rn.args
            g = self._attr(gw)
            if g is None or _val(x) is None or _val(x).dtype != torch.float16 or not rn.users:
                continue
            specs = []  # (consumer, weight, bias, epilogue)
            for u in rn.users:
                if u.op == "call_function" and u.target is hx_silu_mul_linear and u.args[0] is rn:
                    specs.append((u, self._attr(u.args[1]), None, "silu_mul"))
                elif _is(u, aten.linear.default) and u.args[0] is rn and _is_half(u):
                    b = u.args[2] if len(u.args) > 2 else None
                    bt = None if b is None else self._attr(b)
                    if b is not None and bt is None:
                        break
                    specs.append((u, self._attr(u.args[1]), bt, None))
                else:
                    break
                if specs[-1][1] is None:
                    break
            else:
                order = {n: i for i, n in enumerate(self.g.nodes)}
                specs.sort(key=lambda sp: order[sp[0]])
                first = specs[0][0]
                with self.g.inserting_before(first):
                    args = []
                    for _, w, bt, epi in specs:
                        wf = self.g.get_attr(self._buffer(_pkg().fold_rms_weight(w.detach(), g.detach()), "rmsfold"))
                        bn = None if bt is None else self.g.get_attr(self._buffer(bt.detach().clone(), "bias"))
                        args.append((wf, bn, epi))
                    grp = self.g.call_function(hx_rms_linear_group, (x, float(eps), tuple(args)))
                for i, (u, _, _, epi) in enumerate(specs):
                    with self.g.inserting_before(u):
                        item = self.g.call_function(operator.getitem, (grp, i))
                    item.meta.update(u.meta)
                    u.replace_all_uses_with(item)
                    if u in self._entry:
                        self._dropped.add(self._entry[u])
                    self.g.erase_node(u)
                    self.plan.kernels.append(("rms_linear" if epi is None else "rms_silu_mul", u.name))
                if rn in self._entry:
                    self._dropped.add(self._entry[rn])
                self.g.erase_node(rn)

    def linear_gelu(self):
        for ge in list(self.g.nodes):
            if not _is(ge, aten.gelu.default):
                continue
            approx = ge.kwargs.get("approximate", ge.args[1] if len(ge.args) > 1 else "none")
            lin = ge.args[0]
            if approx != "tanh" or not (_is(lin, aten.linear.default) and _single_user(lin) and _is_half(lin)):
                continue
            b = lin.args[2] if len(lin.args) > 2 else None
            self.replace(ge, hx_linear, (lin.args[0], lin.args[1], b, "gelu_tanh"), "linear_gelu")

    def attention(self):
        for out in list(self.g.nodes):
            if not (_is(out, aten.matmul.default) and _is_half(out)):
                continue
            sm, v = out.args
            if not (_is(sm, aten.softmax.int, aten._softmax.default) and _single_user(sm)):
                continue
            if sm.args[1] not in (-1, _val(sm).dim() - 1):
                continue
            z = sm.args[0]
            scale = 1.0
            if _is(z, aten.mul.Tensor, aten.div.Tensor) and isinstance(z.args[1], (int, float)) and _single_user(z):
                scale = float(z.args[1]) if z.target is aten.mul.Tensor else 1.0 / float(z.args[1])
                z = z.args[0]
            if not (_is(z, aten.matmul.default) and _single_user(z)):
                continue
            q, kt = z.args
            if not (_is(kt, aten.transpose.int) and sorted(kt.args[1:3]) == sorted([-1, -2])):
                continue
            if _val(q).dim() < 3:
                continue
            self.replace(out, hx_attention, (q, kt.args[0], v, scale), "attention")
        for n in list(self.g.nodes):
            if not (_is(n, aten.scaled_dot_product_attention.default) and _is_half(n)):
                continue
            arg = lambda i, name, dflt: n.kwargs.get(name, n.args[i] if len(n.args) > i else dflt)  # noqa: E731
            mask, causal = arg(3, "attn_mask", None), bool(arg(5, "is_causal", False))
            if arg(4, "dropout_p", 0.0):
                continue
            q, k, v = (_val(x) for x in n.args[:3])
            scale = arg(6, "scale", None) or 1.0 / math.sqrt(q.shape[-1])
            gqa = k.shape[-3] != q.shape[-3]
            # (hx_attention takes every head dim and fp16 / bf16: the fused kernel where it applies, else the
            # three steps with the masked softmax)
            if gqa and not arg(7, "enable_gqa", False):
                continue
            if mask is not None and _val(mask).dtype not in (torch.bool, torch.float16, torch.bfloat16):
                continue
            self.replace(n, hx_attention, (n.args[0], n.args[1], n.args[2], float(scale), mask, int(causal)),
                         "attention")

    def single_ops(self):
        for n in list(self.g.nodes):
            if not _is_half(n):
                continue
            if _is(n, aten.linear.default):
                b = n.args[2] if len(n.args) > 2 else None
                self.replace(n, hx_linear, (n.args[0], n.args[1], b, None), "linear")
            elif _is(n, aten.matmul.default, aten.mm.default, aten.bmm.default):
                self.replace(n, hx_matmul, (n.args[0], n.args[1]), "matmul")
            elif _is(n, aten.addmm.default) and not n.kwargs and len(n.args) == 3 and _val(n.args[0]).dim() == 1:
                self.replace(n, hx_addmm, n.args, "addmm")
            elif _is(n, aten.softmax.int, aten._softmax.default) and n.args[1] in (-1, _val(n).dim() - 1):
                if len(n.args) > 2 and n.args[2] not in (None, False, _val(n).dtype):
                    continue
                self.replace(n, hx_softmax, (n.args[0],), "softmax")

    def run(self) -> Plan:
        for n in list(self.g.nodes):
            if _is(n, aten._assert_tensor_metadata.default):
                self.g.erase_node(n)
        if self.fusion:
            self.rms_norm_chains()
            self.silu_mul()
            self.linear_gelu()
            self.attention()
            self.g.eliminate_dead_code()  # drop what the fused patterns replaced
            self.rms_norm_ops()
            self.rms_linear()
        self.rms_norm_ops()
        self.single_ops()
        self.g.eliminate_dead_code()
        self.g.lint()
        self.gm.recompile()
        self.plan.kernels = [k for i, k in enumerate(self.plan.kernels) if i not in self._dropped]
        self.plan.torch_ops = [f"{n.name}: {n.target}" for n in self.g.nodes
                               if n.op == "call_function" and isinstance(n.target, torch._ops.OpOverload)]
        return self.plan


def plan_program(program: Any, device: torch.device, fusion: bool = True, gemm_tile: Optional[int] = None) -> Plan:
    """Plan an ExportedProgram (or a GraphModule) for execution on `device`;
    gemm_tile forces the GEMM tile (TileId) of the plan's runs."""
    gm = program.module() if hasattr(program, "module") else program
    gm = gm.to(device)
    plan = _Planner(gm, fusion).run()
    plan.gemm_tile = gemm_tile
    return plan
