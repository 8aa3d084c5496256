"""CPU checks of the C ABI boundary: the library loads, exports exactly what
include/hxmi.h declares, and rejects invalid arguments before any launch."""
import ctypes
import re

import pytest
import torch

from conftest import ROOT

HEADER = ROOT / "include" / "hxmi.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_abi():
    names = declared_functions()
    for n in ["hxmi_gemm_f16", "hxmi_bgemm_f16", "hxmi_gemv_f16", "hxmi_gemv_w8a16", "hxmi_rmsnorm_f16",
              "hxmi_softmax_f16", "hexkl_matmul_f16f16_f32", "hxmi_last_error"]:
        assert n in names


def test_library_exports_every_declared_symbol(pkg):
    lib = pkg.load_library()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert set(declared_functions()) == set(pkg.hxmi.SIGNATURES)


def test_version(pkg):
    assert pkg.load_library().hxmi_version() >= 100


def test_header_compiles_as_c(tmp_path):
    import subprocess

    src = tmp_path / "t.c"
    src.write_text('#include "hxmi.h"\nint main(void){return hxmi_version() > 0 ? 0 : 1;}\n')
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-c", str(src), "-I", str(ROOT / "include"), "-o",
                        str(tmp_path / "t.o")], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


@pytest.mark.parametrize(
    "args, msg",
    [
        ((None, None, None, None, -1, 8, 8, 8, 8, 8, 1, 0, 1.0, None, 0, None), "negative size"),
        ((1, 1, 1, None, 8, 8, 8, 8, 8, 8, 2, 0, 1.0, None, 0, None), "b_is_nt"),
        ((1, 1, 1, None, 8, 8, 8, 8, 8, 8, 1, 9, 1.0, None, 0, None), "unknown epilogue"),
        ((1, 1, 1, None, 8, 48, 8, 8, 8, 48, 1, 2, 1.0, None, 0, None), "SiLU-mul"),
        ((None, 1, 1, None, 8, 8, 8, 8, 8, 8, 1, 0, 1.0, None, 0, None), "null"),
        ((1, 1, 1, None, 8, 8, 8, 8, 8, 8, 1, 1, 1.0, None, 0, None), "bias"),
        ((1, 1, 1, None, 8, 8, 16, 8, 16, 8, 1, 0, 1.0, None, 0, None), "leading dimension"),
    ],
)
def test_gemm_rejects_invalid_arguments(pkg, args, msg):
    lib = pkg.load_library()
    rc = lib.hxmi_gemm_f16(*args)
    assert rc == 1
    assert msg in lib.hxmi_last_error().decode()


def test_empty_problems_are_noops(pkg):
    lib = pkg.load_library()
    assert lib.hxmi_gemm_f16(None, None, None, None, 0, 8, 8, 8, 8, 8, 1, 0, 1.0, None, 0, None) == 0
    assert lib.hxmi_last_error() == b""
    assert lib.hxmi_gemv_f16(None, None, None, None, 0, 8, 8, 8, 8, 8, None, 0, None) == 0
    assert lib.hxmi_rmsnorm_f16(None, None, None, 0, 16, 16, 16, 1e-5, None) == 0
    assert lib.hxmi_softmax_f16(None, None, 4, 0, 0, 0, 1.0, None) == 0


def test_row_ops_reject_invalid(pkg):
    lib = pkg.load_library()
    assert lib.hxmi_rmsnorm_f16(1, None, 1, 4, 16, 16, 16, 1e-5, None) == 1  # no weight
    assert lib.hxmi_softmax_f16(1, 1, 4, 16, 8, 16, 1.0, None) == 1  # ldx < cols
    assert "leading dimension" in lib.hxmi_last_error().decode()


def test_masked_softmax_validates_before_launch(pkg):
    lib = pkg.load_library()
    for fn in (lib.hxmi_softmax_masked_f16, lib.hxmi_softmax_masked_bf16):
        # empty problems are no-ops (no pointer is touched)
        assert fn(None, None, 0, 4, 4, 4, 16, 4, 16, None, 0, 0, 1, 0, 1.0, None) == 0
        assert fn(None, None, 2, 4, 0, 4, 16, 4, 16, None, 0, 0, 1, 0, 1.0, None) == 0
        assert fn(None, None, 2, 4, 4, 4, 16, 4, 16, None, 0, 0, 1, 0, 1.0, None) == 1  # null x / y
        assert fn(16, 16, 2, 4, 8, 4, 16, 8, 32, None, 0, 0, 1, 0, 1.0, None) == 1  # ldx < s_kv
        assert "row stride" in lib.hxmi_last_error().decode()
        assert fn(16, 16, 2, 4, 4, 4, 8, 4, 16, None, 0, 0, 1, 0, 1.0, None) == 1  # slices overlap
        assert fn(16, 16, 2, 4, 4, 4, 16, 4, 16, None, 0, 0, 1, 3, 1.0, None) == 1  # causal 3
        assert "causal" in lib.hxmi_last_error().decode()
        assert fn(16, 16, 2, 4, 4, 4, 16, 4, 16, 16, 4, 16, 0, 0, 1.0, None) == 1  # mask_group 0
        assert fn(16, 16, 2, 4, 4, 4, 16, 4, 16, 17, 4, 16, 1, 0, 1.0, None) == 1  # odd mask address


def test_w8a16_rejects_unaligned_k(pkg):
    lib = pkg.load_library()
    assert lib.hxmi_gemv_w8a16(16, 16, 16, None, 16, 1, 8, 24, 24, 32, 8, None, 0, None) == 1
    assert "K % 16" in lib.hxmi_last_error().decode()


def test_python_ops_refuse_cpu_tensors(pkg):
    a = torch.zeros(8, 8, dtype=torch.float16)
    with pytest.raises(pkg.HxmiError, match="GPU"):
        pkg.gemm(a, a)
    with pytest.raises(pkg.HxmiError, match="GPU"):
        pkg.rms_norm(a, torch.ones(8, dtype=torch.float16))


def test_error_is_thread_local(pkg):
    import threading

    lib = pkg.load_library()
    lib.hxmi_gemm_f16(None, None, None, None, -1, 8, 8, 8, 8, 8, 1, 0, 1.0, None, 0, None)
    seen = []
    t = threading.Thread(target=lambda: seen.append(lib.hxmi_last_error()))
    t.start()
    t.join()
    assert seen == [b""]
    assert lib.hxmi_last_error() != b""


def test_workspace_queries(pkg):
    lib = pkg.load_library()
    # TinyLlama down projection: 64 tiles of 128x128 -> split K
    need = lib.hxmi_gemm_workspace_bytes(512, 2048, 5632, 1, 0)
    assert need > 2 * 512 * 2048 * 4  # >= 2 fp32 partial outputs + arrival counters
    # 4096^3 fills the GPU without splitting; batched / short-K never split
    assert lib.hxmi_gemm_workspace_bytes(4096, 4096, 4096, 1, 0) == 0
    assert lib.hxmi_gemm_workspace_bytes(512, 2048, 512, 1, 0) == 0
    # decode GEMV: long K on 2560 rows splits K over workgroups; down
    # projections (<= 2048 rows) split K inside one workgroup per row tile,
    # wide outputs and the lm_head never split
    assert lib.hxmi_w8a16_workspace_bytes(16, 2560, 8192) > 0
    assert lib.hxmi_gemv_workspace_bytes(1, 2560, 8192) > 0
    assert lib.hxmi_gemv_workspace_bytes(1, 896, 4864) == 0
    assert lib.hxmi_w8a16_workspace_bytes(16, 896, 4864) == 0
    assert lib.hxmi_gemv_workspace_bytes(1, 4864, 896) == 0
    assert lib.hxmi_gemv_workspace_bytes(1, 151936, 896) == 0
    assert lib.hxmi_gemv_workspace_bytes(17, 896, 4864) == 0  # the GEMM's case
    assert lib.hxmi_w8a16_workspace_bytes(256, 896, 4864) > 0


@pytest.mark.parametrize(
    "args, msg",
    [
        ((16, 16, 16, -1, 8, 8, 8, None), "negative size"),
        ((None, 16, 16, 4, 8, 8, 8, None), "null"),
        ((16, 16, 16, 4, 12, 12, 12, None), "multiples of 8"),
        ((16, 16, 16, 4, 16, 8, 16, None), "leading dimension"),
        ((24, 16, 16, 4, 8, 8, 8, None), "aligned"),
    ],
)
def test_quantizer_rejects_invalid_arguments(pkg, args, msg):
    lib = pkg.load_library()
    assert lib.hxmi_quantize_int8_rows_f16(*args) == 1
    assert msg in lib.hxmi_last_error().decode()
    assert lib.hxmi_quantize_int8_rows_f16(None, None, None, 0, 8, 8, 8, None) == 0


def test_tuning_overrides_are_per_thread_and_restorable(pkg):
    """hxmi_set_tuning: per-thread launch-shape overrides, each call returning
    the previous one so a scope can restore it (no GPU work involved)."""
    import threading

    assert pkg.set_tuning("gemm_tile", 3) is None
    assert pkg.set_tuning("gemm_tile", 5) == 3
    other = []
    t = threading.Thread(target=lambda: other.append(pkg.set_tuning("gemm_tile", None)))
    t.start()
    t.join()
    assert other == [None]  # another thread does not see this thread's override
    assert pkg.set_tuning("gemm_tile", None) == 5
    with pkg.tuning(splitk=4, gemv_path="ksplit"):
        assert pkg.set_tuning("splitk", 4) == 4
        assert pkg.set_tuning("gemv_path", 3) == 3
    assert pkg.set_tuning("splitk", None) is None and pkg.set_tuning("gemv_path", None) is None
    with pytest.raises(pkg.HxmiError, match="unknown knob"):
        pkg.set_tuning("no_such_knob", 1)


def test_plan_tile_applies_to_its_own_runs_only(pkg):
    from hexagon_mlir_amd.backend.graph import Plan

    seen = []

    class Probe:
        def __call__(self, *args):
            prev = pkg.set_tuning("gemm_tile", None)
            seen.append(prev)
            pkg.set_tuning("gemm_tile", prev)
            return args

    Plan(module=Probe(), gemm_tile=6)(1)
    Plan(module=Probe())(1)
    assert seen == [6, None]
    assert pkg.set_tuning("gemm_tile", None) is None


def test_noalloc_gemm_rejects_partials_beyond_its_scratch(pkg):
    """A forced 4-way K split of 1216 x 2560 x 8192 needs ~50 MB of partials,
    more than the 32 MiB scratch: rejected before any launch."""
    lib = pkg.load_library()
    fake = 1 << 12  # aligned, never dereferenced: the call fails its size check first
    with pkg.tuning(splitk=4):
        rc = lib.hxmi_gemm_f16_noalloc(fake, fake, fake, None, 1216, 2560, 8192, 8192, 8192, 2560, 1, 0, 1.0, None)
        msg = lib.hxmi_last_error()  # (the next successful call clears it)
    assert rc == 1
    assert b"device scratch" in msg


def test_decode_step_rejects_before_launch(pkg):
    lib = pkg.load_library()
    need = lib.hxmi_decode_workspace_bytes(896, 128, 4864)
    assert need == 4 * (64 + 2 * (2 * 896 + 128 + 4864))  # control words + 2 copies of the vectors
    assert lib.hxmi_decode_workspace_bytes(0, 128, 4864) == 0
    P = 4096  # 256-byte aligned stand-in addresses: every call below fails before touching them

    def call(layers=24, hidden=896, heads=14, kv_heads=2, head_dim=64, inter=4864, ws_bytes=need, ptr=P, ws=P,
             w_lm=None, logits=None, vocab=0):
        return lib.hxmi_decode_step_f16(ptr, P, None, P, P, P, P, P, P, w_lm, None, None, P, logits, layers,
                                        hidden, heads, kv_heads, head_dim, inter, vocab, 1e-6, 0, ws, ws_bytes,
                                        None)

    assert call(layers=0) == 1 and "positive" in lib.hxmi_last_error().decode()
    assert call(ptr=None) == 1 and "null" in lib.hxmi_last_error().decode()
    assert call(ws_bytes=need - 4) == 1 and "workspace" in lib.hxmi_last_error().decode()
    assert call(ws=P + 16) == 1 and "256-byte" in lib.hxmi_last_error().decode()
    assert call(w_lm=P) == 1 and "w_lm" in lib.hxmi_last_error().decode()
    assert call(ptr=P + 2) == 1 and "16-byte" in lib.hxmi_last_error().decode()
    # shapes outside the kernel's limits: heads * head_dim != hidden, hidden > 2048, intermediate > 6144
    assert call(heads=13) == 2
    assert call(hidden=4096, heads=64, ws_bytes=1 << 20) == 2
    assert call(inter=8192, ws_bytes=1 << 20) == 2
    assert "unsupported shape" in lib.hxmi_last_error().decode()

    # the folded-o entry point checks the same way, and needs w_ov
    def call_ov(w_ov=P, b_ov=None, layers=24, ptr=P):
        return lib.hxmi_decode_step_ov_f16(ptr, P, None, w_ov, b_ov, P, P, P, P, P, None, None, None, P, None,
                                           layers, 896, 14, 2, 64, 4864, 0, 1e-6, 0, P, need, None)

    assert call_ov(w_ov=None) == 1 and "null" in lib.hxmi_last_error().decode()
    assert call_ov(layers=0) == 1 and "positive" in lib.hxmi_last_error().decode()
    assert call_ov(b_ov=P + 1) == 1 and "b_ov" in lib.hxmi_last_error().decode()
    assert call_ov(w_ov=P + 2) == 1 and "16-byte" in lib.hxmi_last_error().decode()
