"""The Rust -sys crate (mini-rust-inference_amd/rust/mri-sys) against the C
headers it declares (include/mri_qmatmul.h, include/mri_llama.h): every
function with the same name, argument types in the same order and the same
return type; the enum values, the #define and the two structs' fields.
No Rust toolchain is needed: both sides are parsed as text, and the C types
are mapped to the Rust types the crate must use (size_t -> usize,
int -> c_int, T * -> *mut T, const T * -> *const T, enums -> c_int)."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", "mri_qmatmul.h"),
           os.path.join(ROOT, "include", "mri_llama.h")]
CRATE = os.path.join(ROOT, "mini-rust-inference_amd", "rust", "mri-sys")
LIB_RS = os.path.join(CRATE, "src", "lib.rs")

BASE = {"int8_t": "i8", "uint8_t": "u8", "int32_t": "i32", "uint32_t": "u32",
        "size_t": "usize", "float": "f32", "int": "c_int", "void": "c_void",
        "char": "c_char"}


def c_source():
    src = "\n".join(open(h).read() for h in HEADERS)
    return re.sub(r"/\*.*?\*/", "", src, flags=re.S)


def c_type(t):
    """A C type (without the parameter name) as the crate must spell it."""
    t = " ".join(t.replace("*", " * ").split())
    stars = t.count("*")
    words = [w for w in t.split() if w != "*"]
    const = words[0] == "const"
    base = words[-1]
    rust = BASE.get(base, base)
    if stars == 0:
        return rust
    out = f"*{'const' if const else 'mut'} {rust}"
    for _ in range(stars - 1):
        out = f"*mut {out}"
    return out


def c_param(p):
    p = " ".join(p.split())
    if p == "void":
        return None
    m = re.match(r"(.*?)\s*\b([A-Za-z_][A-Za-z0-9_]*)\s*(\[\s*\d*\s*\])?$", p)
    typ, arr = m.group(1), m.group(3)
    if arr:  # an array parameter is a pointer
        typ += " *"
    return c_type(typ)


def c_functions():
    src = re.sub(r"#[^\n]*", "", c_source())
    fns = {}
    for m in re.finditer(r"([A-Za-z_][A-Za-z0-9_ \*]*?)\b(mri_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;",
                         src):
        ret, name, params = m.group(1).strip(), m.group(2), m.group(3)
        args = [a for a in (c_param(p) for p in params.split(",")) if a is not None]
        fns[name] = (args, None if ret == "void" else c_type(ret))
    return fns


def c_constants():
    src = c_source()
    consts = {}
    for body in re.findall(r"typedef\s+enum\s*\w*\s*\{(.*?)\}", src, flags=re.S):
        for name, val in re.findall(r"(MRI_[A-Z0-9_]+)\s*=\s*(\d+)", body):
            consts[name] = int(val)
    for name, a, b in re.findall(r"#define\s+(MRI_[A-Z0-9_]+)\s+\((\d+)\s*<<\s*(\d+)\)", src):
        consts[name] = int(a) << int(b)
    return consts


def c_structs():
    src = c_source()
    out = {}
    for body, name in re.findall(r"typedef\s+struct\s+\w+\s*\{(.*?)\}\s*(\w+)\s*;", src,
                                 flags=re.S):
        fields = []
        for decl in body.split(";"):
            decl = " ".join(decl.split())
            if decl:
                fields.append((re.search(r"(\w+)$", decl).group(1), c_param(decl)))
        out[name] = fields
    return out


def rust_source():
    return re.sub(r"//[^\n]*", "", open(LIB_RS).read())


def rust_norm(t):
    """One spelling per Rust type: `*const T`, `*mut *mut T`, single spaces."""
    return " ".join(t.replace("*", " *").split()).replace("* ", "*").strip()


def rust_functions(src=None):
    src = rust_source() if src is None else src
    hip = src.index("pub mod hip")
    src = src[:hip]  # the HIP runtime declarations are not part of the headers
    fns = {}
    for block in re.findall(r'extern\s+"C"\s*\{(.*?)\n\}', src, flags=re.S):
        for m in re.finditer(r"pub fn (mri_[a-z0-9_]+)\s*\((.*?)\)\s*(->\s*([^;]+))?;", block,
                             flags=re.S):
            name, params, ret = m.group(1), m.group(2), m.group(4)
            args = []
            for p in [p.strip() for p in params.split(",") if p.strip()]:
                args.append(rust_norm(p.split(":", 1)[1]))
            fns[name] = (args, rust_norm(ret) if ret else None)
    return fns


def test_crate_files_exist():
    for f in ("Cargo.toml", "build.rs", os.path.join("src", "lib.rs")):
        assert os.path.isfile(os.path.join(CRATE, f)), f
    toml = open(os.path.join(CRATE, "Cargo.toml")).read()
    assert 'links = "mri_qmatmul"' in toml
    assert "rustc-link-lib=dylib=mri_qmatmul" in open(os.path.join(CRATE, "build.rs")).read()


def differences(c, r):
    """Every way the crate's functions r differ from the headers' c."""
    out = [f"missing in the crate: {n}" for n in sorted(set(c) - set(r))]
    out += [f"not in the headers: {n}" for n in sorted(set(r) - set(c))]
    for name in sorted(set(c) & set(r)):
        (cargs, cret), (rargs, rret) = c[name], r[name]
        want = [rust_norm(a) for a in cargs]
        if rargs != want:
            out.append(f"{name}: arguments {rargs} != {want}")
        if rret != (rust_norm(cret) if cret else None):
            out.append(f"{name}: returns {rret} != {cret}")
    return out


def test_every_function_declared_with_the_same_signature():
    c, r = c_functions(), rust_functions()
    assert len(c) > 40
    assert differences(c, r) == []


def test_constants_match():
    src = rust_source()
    rust = {n: v for n, v in re.findall(r"pub const (MRI_[A-Z0-9_]+):[^=]+=\s*([^;]+);", src)}
    c = c_constants()
    assert sorted(c) == sorted(rust), (sorted(set(c) - set(rust)), sorted(set(rust) - set(c)))
    for name, val in c.items():
        assert eval(rust[name].strip()) == val, (name, rust[name], val)


@pytest.mark.parametrize("name", ["mri_llama_config", "mri_weight_ref"])
def test_struct_fields_match(name):
    src = rust_source()
    m = re.search(r"pub struct " + name + r"\s*\{(.*?)\}", src, flags=re.S)
    assert m, name
    rust = [(f.split(":")[0].replace("pub", "").strip(), rust_norm(f.split(":", 1)[1]))
            for f in m.group(1).split(",") if f.strip()]
    c = [(n, rust_norm(t)) for n, t in c_structs()[name]]
    assert rust == c, (rust, c)
    assert re.search(r"#\[repr\(C\)\]\s*(#\[derive[^\]]*\]\s*)?pub struct " + name, src)


def test_parser_catches_a_mismatch():
    """The check is not vacuous: the C side parses to the expected Rust
    spellings, and a wrong type, two swapped arguments or a missing function
    planted in a copy of the crate's text are each reported."""
    c = c_functions()
    args, _ = c["mri_matmul_int8"]
    assert args == ["*const i8", "usize", "f32", "*const mri_qmatrix", "usize", "*mut f32",
                    "*mut i32", "*mut c_void"]
    assert c["mri_llama_set_layer"][0][-1] == "*const mri_weight_ref"
    assert c["mri_qmatrix_create"][0][-1] == "*mut *mut mri_qmatrix"
    assert c["mri_last_error"] == ([], "*const c_char")
    assert c["mri_qmatrix_destroy"][1] is None
    src = rust_source()
    wrong_type = src.replace("        act_scale: f32,", "        act_scale: f64,", 1)
    swapped = src.replace("        m: usize,\n        k: usize,", "        k: usize,\n        m: f32,", 1)
    missing = src.replace("pub fn mri_argmax(", "pub fn mri_argmax_gone(", 1)
    for planted in (wrong_type, swapped, missing):
        assert planted != src
        assert differences(c, rust_functions(planted)), "planted mistake not seen"
