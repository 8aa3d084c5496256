"""Drop-in launcher for PyTorch programs, with the reference's entry point
``TorchMLIRHexagonLauncher().run_torch_mlir(...)``
(qcom_hexagon_backend/backend/torch_mlir_hexagon_launcher.py:258-306).

Reference flow: model -> torch-mlir linalg bytecode file -> compile to a
Hexagon .so -> run on the DSP over adb -> output files -> CPU tensors.
Here: model -> ``export_program`` / ``write_program_to_file`` (a
torch.export program file takes the place of the linalg bytecode) ->
``compile_torch_mlir`` plans the graph onto the hxmi kernels
(backend/graph.py) -> run in-process on the GPU -> CPU tensors.  Same
arguments, same return value (one CPU tensor per returned tensor), same
Test_Info report and timestamped artifact folder.
"""
from __future__ import annotations

import os
import shutil
import time
from typing import Optional, Sequence

import torch
from torch import Tensor

from .graph import Plan, plan_program
from .hexagon_launcher_base import HexagonLauncherBase, create_timestamped_folder
from .hexagon_options import HexagonOptions, options_from_dict
from .utils import write_output_tensor


def export_program(model: torch.nn.Module, inputs: Sequence, func_name: str = "main"):
    """Export `model` for `inputs` (the place of the reference scripts'
    ``fx_mlir.export_and_import(..., output_type="linalg-on-tensors")``,
    e.g. benchmark_models/run_tinyllama.py:70-88)."""
    del func_name  # the program file has one entry, named by the caller at run time
    model = model.eval()
    return torch.export.export(model, tuple(inputs))


def write_program_to_file(program, filename: str) -> None:
    """Save an exported program (the place of writing the MLIR bytecode file,
    benchmark_models/micro_bench/test_matmul_benchmark.py:43-47)."""
    torch.export.save(program, filename)


def _flatten(out):
    if isinstance(out, torch.Tensor):
        return [out]
    if isinstance(out, (list, tuple)):
        res = []
        for o in out:
            res += _flatten(o)
        return res
    return []


class TorchMLIRHexagonLauncher(HexagonLauncherBase):
    def __init__(self, device: Optional[torch.device] = None):
        self.device = device or torch.device("cuda", torch.cuda.current_device() if torch.cuda.is_available() else 0)
        self.last_plan: Optional[Plan] = None

    def compile_torch_mlir(self, local_dir: str, mlir_bytecode_path: str, func_name: str, options: dict) -> Plan:
        """Load the program file and plan it onto the GPU kernels; the plan
        summary is written to <func_name>.plan.txt in the artifact folder."""
        opts = options_from_dict(options)
        program = torch.export.load(mlir_bytecode_path)
        tile = _tile_id(opts.tileSizes) if opts.tileSizes else None
        plan = plan_program(program, self.device, fusion=opts.fusion, gemm_tile=tile)
        if opts.lowerConstantsInSeparateSharedObjects:
            self._constants_artifact(plan, local_dir, func_name)
        with open(os.path.join(local_dir, f"{func_name}.plan.txt"), "w") as f:
            f.write(plan.summary() + "\n")
        self.last_plan = plan
        return plan

    def run_torch_mlir(
        self,
        mlir_bytecode_path: str,
        inputs: list[Tensor],
        func_name: str,
        base_dir_for_artifacts: Optional[str] = None,
        iterations: int = 1,
        options: dict = None,
        enable_etm=False,
    ) -> list[Tensor]:
        if options is None:
            options = HexagonOptions().__dict__
        opts = options_from_dict(options)
        if enable_etm:
            raise NotImplementedError("ETM tracing has no MI355X equivalent; profile with rocprofv3")
        local_dir = create_timestamped_folder(func_name, base_dir_for_artifacts)
        shutil.copy(mlir_bytecode_path, os.path.join(local_dir, os.path.basename(mlir_bytecode_path)))

        start = time.time()
        plan = self.compile_torch_mlir(local_dir, mlir_bytecode_path, func_name, options)
        print(f"Compilation from program file to GPU plan took {time.time() - start:.4f} seconds", flush=True)
        return self.execute_kernel(plan, inputs, func_name, local_dir, iterations, opts.enableLWP)

    def _constants_artifact(self, plan: Plan, local_dir: str, func_name: str) -> str:
        """The plan's constants (weights after folding and packing) written to
        <func_name>.constants.safetensors, an artifact of their own as the
        reference's split-constants mode produces
        (triton_qcom_hexagon_backend_api.cc:196-214); the module's constants
        are then overwritten with the values read back from that file, so the
        run uses what the artifact holds."""
        from safetensors.torch import load_file, save_file

        path = os.path.join(local_dir, f"{func_name}.constants.safetensors")
        named = dict(plan.module.named_parameters())
        named.update(plan.module.named_buffers())
        save_file({k: v.detach().to("cpu").clone().contiguous() for k, v in named.items()}, path,
                  metadata={"format": "hxmi-constants", "func": func_name})
        loaded = load_file(path, device=str(self.device))
        with torch.no_grad():
            for k, v in named.items():
                v.copy_(loaded[k])
        return path

    def execute_kernel(self, plan: Plan, inputs: list, func_name: str, local_dir: str, iterations: int = 1,
                       lwp: bool = False) -> list[Tensor]:
        """Run the plan on the GPU: one untimed run, `iterations` timed runs
        (HIP events), the Test_Info report, outputs as CPU tensors (also
        written to <func_name>_o<i>.raw in the reference's output format)."""
        args = [x.to(self.device) if isinstance(x, torch.Tensor) else x for x in inputs]
        with torch.no_grad():
            outs = plan(*args)
            torch.cuda.synchronize(self.device)
            iters = max(int(iterations), 1)
            s = torch.cuda.Event(enable_timing=True)
            e = torch.cuda.Event(enable_timing=True)
            s.record()
            for _ in range(iters):
                outs = plan(*args)
            e.record()
            torch.cuda.synchronize(self.device)
        self.report(local_dir, "_mlir_ciface_" + func_name, s.elapsed_time(e) * 1e3 / iters)
        if lwp:
            self._per_op_timing(plan, args, local_dir)
        results = [o.detach().cpu() for o in _flatten(outs)]
        for i, r in enumerate(results):
            try:
                write_output_tensor(os.path.join(local_dir, f"_mlir_ciface_{func_name}_o{i}.raw"), r)
            except ValueError:
                pass  # dtype without a raw-file id (e.g. bool): returned, not written
        return results

    def _per_op_timing(self, plan: Plan, args: list, local_dir: str) -> None:
        """Region timing of one run in the reference's LWP files: region 0 is
        the whole function, region i >= 1 the i-th op of the planned graph;
        begin and end markers on the GPU stream bracket each region's kernels
        (lwp.json), and lwp_infodump.txt maps each id to the op's position in
        the graph and its name."""
        from torch.fx import Interpreter

        from .lwp import LwpRecorder, write_lwp

        ops = [n for n in plan.module.graph.nodes if n.op in ("call_function", "call_module")]
        ids = {n: i + 1 for i, n in enumerate(ops)}
        positions = {n: i for i, n in enumerate(plan.module.graph.nodes)}
        rec = LwpRecorder(self.device, capacity=2 * len(ops) + 2)

        class Marked(Interpreter):
            def run_node(self, n):
                if n not in ids:
                    return super().run_node(n)
                rec.mark(ids[n])
                r = super().run_node(n)
                rec.mark(ids[n])
                return r

        with torch.no_grad():
            ctx = self._tile_scope(plan)
            with ctx:
                rec.mark(0)
                Marked(plan.module).run(*args)
                rec.mark(0)
        regions = [(0, [0], ["func"])]
        regions += [(ids[n], [positions[n]], [n.name + ": " + getattr(n.target, "__name__", str(n.target))])
                    for n in ops]
        write_lwp(os.path.join(local_dir, "lwp.json"), os.path.join(local_dir, "lwp_infodump.txt"), rec.entries(),
                  rec.clock_hz(), regions)

    @staticmethod
    def _tile_scope(plan: Plan):
        import contextlib

        if plan.gemm_tile is None:
            return contextlib.nullcontext()
        from .. import hxmi

        return hxmi.tuning(gemm_tile=plan.gemm_tile)


def _tile_id(tile_sizes: str) -> int:
    """'BM,BN' -> the GEMM tile id with that shape."""
    shapes = {(256, 256): 8, (128, 256): 1, (256, 128): 2, (128, 128): 3, (64, 128): 4, (128, 64): 5, (64, 64): 6}
    try:
        bm, bn = (int(v) for v in tile_sizes.replace("x", ",").split(",")[:2])
        return shapes[(bm, bn)]
    except (ValueError, KeyError):
        raise ValueError(f"tileSizes {tile_sizes!r}: expected 'BM,BN' among {sorted(shapes)}") from None
