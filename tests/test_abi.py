"""CPU-side checks of the drop-in boundary: the C-ABI library loads and exports every entry point
include/axis_hip.h declares (no compute call: there is no GPU here)."""
import ctypes
import os
import re
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


ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
RUST_SYS = os.path.join(ROOT, "ffi", "axis-hip-sys", "src", "lib.rs")
_C_BASE = {"int": "c_int", "int32_t": "i32", "int64_t": "i64", "uint8_t": "u8", "float": "f32",
           "double": "f64", "size_t": "usize", "char": "c_char", "void": "c_void",
           "axis_device": "axis_device", "axis_plan": "axis_plan", "axis_unfold_spec": "axis_unfold_spec",
           "axis_adam_tensor": "axis_adam_tensor"}


def _c_type(decl):
    """A C parameter or field declaration (name included) as the Rust type that binds it:
    `const T *x` -> `*const T`, `T *x` / `T x[n]` (a parameter) -> `*mut T` / `*const T`."""
    decl = " ".join(decl.split())
    array = re.search(r"\[\d*\]$", decl)
    decl = re.sub(r"\s*\[\d*\]$", "", decl)
    m = re.fullmatch(r"(const )?(\w+)\s*(\**)\s*\w+", decl)
    assert m, decl
    const, base, stars = m.group(1), _C_BASE[m.group(2)], len(m.group(3)) + (1 if array else 0)
    if stars == 0:
        return base
    inner = ("*const " if const else "*mut ") + base
    return "*mut " * (stars - 1) + inner


def _strip_c(text):
    return re.sub(r"//[^\n]*", "", re.sub(r"/\*.*?\*/", "", text, flags=re.S))


def c_prototypes():
    text = _strip_c(open(hip.HEADER).read())
    out = {}
    for ret, name, params in re.findall(r"(int|const char \*)\s*(axis_\w+)\s*\(([^)]*)\)\s*;", text, re.S):
        args = [] if params.strip() == "void" else [_c_type(p) for p in params.split(",")]
        out[name] = ("c_int" if ret == "int" else "*const c_char", args)
    return out


def c_structs():
    text = _strip_c(open(hip.HEADER).read())
    out = {}
    for body, name in re.findall(r"typedef struct \{(.*?)\}\s*(\w+)\s*;", text, re.S):
        fields = []
        for decl in body.split(";"):
            decl = " ".join(decl.split())
            if not decl:
                continue
            array = re.search(r"\[(\d+)\]$", decl)
            if array:   # a struct member array is a value, not a pointer
                base = _c_type(re.sub(r"\s*\[\d+\]$", "", decl))
                fields.append(f"[{base}; {array.group(1)}]")
            else:
                fields.append(_c_type(decl))
        out[name] = fields
    return out


def rust_declarations():
    text = re.sub(r"//[^\n]*", "", open(RUST_SYS).read())
    fns = {}
    for name, params, ret in re.findall(r"pub fn (axis_\w+)\(([^)]*)\)\s*->\s*([^;]+);", text, re.S):
        args = [" ".join(p.split(":", 1)[1].split()) for p in params.split(",") if p.strip()]
        fns[name] = (" ".join(ret.split()), args)
    structs = {}
    for name, body in re.findall(r"#\[repr\(C\)\]\s*pub struct (\w+)\s*\{([^{}]*)\}", text):
        if name.endswith("_s"):   # the opaque handle types
            continue
        structs[name] = [" ".join(f.split(":", 1)[1].split()) for f in body.split(",") if ":" in f]
    return fns, structs


def test_rust_sys_crate_matches_the_header_argument_by_argument():
    # ffi/axis-hip-sys binds every prototype of include/axis_hip.h with the same argument count,
    # order and types, the same return type, and the same struct layouts, and nothing else
    c_fns, c_st = c_prototypes(), c_structs()
    rust_fns, rust_st = rust_declarations()
    assert sorted(c_fns) == hip.header_functions()
    assert sorted(rust_fns) == sorted(c_fns), set(rust_fns) ^ set(c_fns)
    for name, (ret, args) in c_fns.items():
        assert rust_fns[name] == (ret, args), (name, rust_fns[name], (ret, args))
    assert rust_st == c_st, (rust_st, c_st)


def test_signature_parsers_catch_a_swapped_argument():
    # the comparison above is sensitive: swapping two differently typed arguments, dropping const
    # or changing an integer width in the Rust text all change the parsed signature
    fns, _ = rust_declarations()
    ret, args = fns["axis_adam"]
    assert args[1] == "*const f32" and args[6] == "i64" and args[7] == "f32"
    assert _c_type("const float *a") == "*const f32" and _c_type("float *a") == "*mut f32"
    assert _c_type("void **stream") == "*mut *mut c_void" and _c_type("const int32_t kernel[2]") == "*const i32"
    assert _c_type("int64_t len") == "i64" and _c_type("int n") == "c_int"


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
