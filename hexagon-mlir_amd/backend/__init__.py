"""The reference's Python surface (qcom_hexagon_backend/backend/) on top of
the hxmi kernels: options, launcher, artifact/report helpers, raw tensor I/O."""
from .graph import Plan, plan_program
from .hexagon_launcher_base import HexagonLauncherBase, create_timestamped_folder, format_test_info
from .hexagon_options import HexagonOptions, options_from_dict
from .torch_mlir_hexagon_launcher import TorchMLIRHexagonLauncher, export_program, write_program_to_file
from .utils import DTYPE_IDS, read_output_tensor, to_torch_type, write_input_tensor, write_output_tensor

__all__ = [
    "DTYPE_IDS",
    "HexagonLauncherBase",
    "HexagonOptions",
    "Plan",
    "TorchMLIRHexagonLauncher",
    "create_timestamped_folder",
    "export_program",
    "format_test_info",
    "options_from_dict",
    "plan_program",
    "read_output_tensor",
    "to_torch_type",
    "write_input_tensor",
    "write_output_tensor",
    "write_program_to_file",
]
