"""CPU-side checks of the drop-in boundary: the C-ABI library loads and exports every entry point
include/axis_hip.h declares (no compute call: there is no GPU here)."""
import ctypes
import os
import subprocess

import pytest

from axis_amd import hip


def test_header_declares_the_hot_path_surface():
    names = set(hip.header_functions())
    for required in ["axis_matmul", "axis_matmul_left_backward", "axis_matmul_right_backward",
                     "axis_unfold", "axis_unfold_backward", "axis_grouped", "axis_grouped_minimum",
                     "axis_mask_gradient", "axis_relu_backward", "axis_categorical_cross_entropy",
                     "axis_categorical_cross_entropy_backward", "axis_adam", "axis_adam_multi",
                     "axis_sum_squares", "axis_inverse_sqrt", "axis_multiply_scalar"]:
        assert required in names, required


def test_library_exports_every_declared_symbol():
    lib = hip.load()
    missing = [name for name in hip.header_functions() if not hasattr(lib, name)]
    assert not missing, missing
    assert b"gfx950" in lib.axis_version()


def test_integration_binding_covers_every_entry():
    # the reference-side Rust extern block must bind every entry point the header declares
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    text = open(os.path.join(root, "INTEGRATION.md")).read()
    missing = [name for name in hip.header_functions() if f"pub fn {name}(" not in text]
    assert not missing, missing


def test_library_is_built_for_gfx950_only(tmp_path):
    build = os.path.join(os.path.dirname(hip.LIB_PATH), "_build")
    objs = [os.path.join(build, f) for f in os.listdir(build) if f.endswith(".o")
            and not f.startswith("host_")] if os.path.isdir(build) else []
    if not objs:
        pytest.skip("no build objects to inspect")
    for obj in objs:
        fatbin = str(tmp_path / (os.path.basename(obj) + ".fatbin"))
        subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", obj, fatbin],
                       check=True)
        out = subprocess.run(["/opt/rocm/llvm/bin/clang-offload-bundler", "--list", "--type=o",
                              f"--input={fatbin}"], capture_output=True, text=True)
        targets = [t for t in out.stdout.split() if "amdgcn" in t]
        assert targets and all(t.endswith("gfx950") for t in targets), (obj, out.stdout)


def test_errors_are_reported_without_a_device():
    lib = hip.load()
    # a null handle is rejected before any HIP call
    assert lib.axis_matmul(None, None, None, None, 1, 1, 1, 1) == 1
    assert b"null axis_device" in lib.axis_last_error()


def test_unfold_spec_layout_matches_the_oracle_struct():
    from oracle import oracle
    assert ctypes.sizeof(hip.UnfoldSpec) == ctypes.sizeof(oracle.UnfoldSpec)
    for (name, _), (oname, _) in zip(hip.UnfoldSpec._fields_, oracle.UnfoldSpec._fields_):
        assert name == oname
        assert getattr(hip.UnfoldSpec, name).offset == getattr(oracle.UnfoldSpec, oname).offset
