"""Artifact folders and the Test_Info performance report of the reference
launcher (qcom_hexagon_backend/backend/hexagon_launcher_base.py:388-422,
test/utils/dsp/include/test_report.h:43-50)."""
from __future__ import annotations

import os
from datetime import datetime
from typing import Optional


def create_timestamped_folder(model_name: str, optional_base_dir: Optional[str] = None) -> str:
    """<base>/<model_name>-YYYY-mm-dd_HH-MM-SS-ffffff, where base is the
    argument, else $HEXAGON_MLIR_DUMP_DIR, else /tmp; asserts base exists."""
    if optional_base_dir is not None:
        base_dir, reason = optional_base_dir, "(as requested by the --output-dir argument provided)"
    elif os.getenv("HEXAGON_MLIR_DUMP_DIR") is not None:
        base_dir, reason = os.getenv("HEXAGON_MLIR_DUMP_DIR"), "(as specified by the env variable HEXAGON_MLIR_DUMP_DIR)"
    else:
        base_dir, reason = "/tmp", "(as default location)"
    assert os.path.isdir(base_dir), f"The base directory {base_dir} ({reason}) isn't a valid directory"
    folder_name = datetime.now().strftime(model_name + "-%Y-%m-%d_%H-%M-%S-%f")
    full_path = os.path.join(base_dir, folder_name)
    os.makedirs(full_path)
    print(f"==> Folder '{folder_name}' created successfully inside of", base_dir, reason)
    return full_path


def format_test_info(name: str, perf: float, units: str = "us", result: str = "Pass") -> str:
    """The Test_Info block callers regex-parse for Perf and Units
    (benchmark_models/micro_bench/test_matmul_benchmark.py:84-88)."""
    return f"Test_Info: {{\n\tName:{name}\n\tResult:{result}\n\tPerf:{perf:f}\n\tUnits:{units}\n}}\n"


class HexagonLauncherBase:
    """Common launcher plumbing: the report is printed and saved as perf.txt
    in the run's artifact folder, as the generated main() does."""

    @staticmethod
    def report(local_dir: str, name: str, perf_us: float, result: str = "Pass") -> str:
        text = format_test_info(name, perf_us, "us", result)
        print(text, end="", flush=True)
        with open(os.path.join(local_dir, "perf.txt"), "w") as f:
            f.write(text)
        return text
