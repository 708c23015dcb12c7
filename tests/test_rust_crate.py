"""The Rust crate's FFI declarations (crates/iris-hip/src/ffi.rs) against
include/iris_hip.h (no GPU, no Rust toolchain): every function the header
declares is declared in the crate's extern block with the same parameter
and return types, and nothing else is; the first five keep the reference's
own extern block (crates/inference/kernels/src/gpu.rs:45-62); the
IrisModelDesc struct has the header's fields in the header's order.

The crate itself is not compiled here (this image has no cargo/rustc)."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "iris_hip.h")
FFI = os.path.join(ROOT, "crates", "iris-hip", "src", "ffi.rs")

C_SCALARS = {"int": "c_int", "char": "c_char", "void": "c_void", "double": "f64", "int8_t": "i8", "uint8_t": "u8",
             "int32_t": "i32", "uint32_t": "u32", "int64_t": "i64", "uint64_t": "u64"}


def _strip_c_comments(text):
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.sub(r"//[^\n]*", "", text)


def _c_type_to_rust(t: str) -> str:
    t = " ".join(t.replace("*", " * ").split())
    # split into base and pointer levels, each with its own const
    tokens = t.split()
    base_const = False
    i = 0
    if tokens[i] == "const":
        base_const = True
        i += 1
    base = tokens[i]
    i += 1
    levels = []  # const-ness of each pointer level, innermost first
    pending_const = base_const
    while i < len(tokens):
        if tokens[i] == "*":
            levels.append(pending_const)
            pending_const = False
        elif tokens[i] == "const":
            pending_const = True
        i += 1
    rust = C_SCALARS.get(base, base)
    for const in levels:
        rust = ("*const " if const else "*mut ") + rust
    return rust


def header_decls():
    text = _strip_c_comments(open(HEADER).read())
    decls = {}
    for m in re.finditer(r"([A-Za-z_][A-Za-z0-9_ \*]*?)\b([a-z][a-z0-9_]*)\s*\(([^;{)]*)\)\s*;", text):
        ret, name, params = m.group(1).strip(), m.group(2), m.group(3).strip()
        if ret.startswith("typedef") or not ret:
            continue
        args = []
        if params and params != "void":
            for p in params.split(","):
                p = " ".join(p.split())
                pm = re.match(r"(.*?)([A-Za-z_][A-Za-z0-9_]*)$", p)
                args.append(_c_type_to_rust(pm.group(1).strip()))
        rret = None if ret == "void" else _c_type_to_rust(ret)
        decls[name] = (rret, args)
    return decls


def rust_decls():
    text = re.sub(r"//[^\n]*", "", open(FFI).read())
    block = re.search(r'extern "C" \{(.*)\n\}', text, flags=re.S).group(1)
    decls = {}
    for m in re.finditer(r"pub fn ([a-z0-9_]+)\s*\((.*?)\)\s*(->\s*([^;]+))?;", block, flags=re.S):
        name, params, ret = m.group(1), m.group(2), m.group(4)
        args = []
        for p in [p for p in params.split(",") if p.strip()]:
            args.append(" ".join(p.split(":", 1)[1].split()))
        decls[name] = (" ".join(ret.split()) if ret else None, args)
    return decls


def test_every_header_function_is_declared_with_the_same_types():
    c, r = header_decls(), rust_decls()
    assert len(c) >= 30
    assert sorted(c) == sorted(r), (set(c) ^ set(r))
    for name in c:
        assert c[name] == r[name], (name, c[name], r[name])


def test_the_reference_extern_block_is_kept():
    r = rust_decls()
    # crates/inference/kernels/src/gpu.rs:45-62 (its DeviceMatrix is our Q8GpuMatrix)
    assert r["q8gpu_error"] == ("*const c_char", ["c_int"])
    assert r["q8gpu_init"] == ("c_int", [])
    assert r["q8gpu_upload"] == ("c_int", ["*const i8", "*const i64", "u32", "u32", "*mut *mut Q8GpuMatrix"])
    assert r["q8gpu_free"] == (None, ["*mut Q8GpuMatrix"])
    assert r["q8gpu_product"] == ("c_int", ["*const Q8GpuMatrix", "*const i32", "u32", "*mut i32"])


def test_model_desc_fields_match():
    c = _strip_c_comments(open(HEADER).read())
    body = re.search(r"typedef struct IrisModelDesc \{(.*?)\} IrisModelDesc;", c, flags=re.S).group(1)
    c_fields = []
    for decl in body.split(";"):
        decl = " ".join(decl.split())
        if not decl:
            continue
        m = re.match(r"(const \w+\*|\w+) (.*)", decl)
        ctype = m.group(1)
        for n in m.group(2).split(","):
            c_fields.append((n.strip(), _c_type_to_rust(ctype)))
    r = re.sub(r"//[^\n]*", "", open(FFI).read())
    rbody = re.search(r"pub struct IrisModelDesc \{(.*?)\n\}", r, flags=re.S).group(1)
    r_fields = [(m.group(1), " ".join(m.group(2).split())) for m in re.finditer(r"pub (\w+): ([^,]+),", rbody)]
    assert c_fields == r_fields


def test_python_bindings_match_the_header_too():
    # iris_amd.direct.ModelDesc is the same struct on the Python side.
    from iris_amd.direct import ModelDesc
    names = [f[0] for f in ModelDesc._fields_]
    r = re.sub(r"//[^\n]*", "", open(FFI).read())
    rbody = re.search(r"pub struct IrisModelDesc \{(.*?)\n\}", r, flags=re.S).group(1)
    assert names == [m.group(1) for m in re.finditer(r"pub (\w+):", rbody)]
