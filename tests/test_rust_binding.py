"""The Rust side of the boundary against the C header.

integration/rust/prism-ffi/src/hip.rs is the extern block a maintainer adds
to prism-ffi (prism-ffi/src/lib.rs:28-90 is where the crate's own C ABI
lives).  No Rust toolchain is available here, so instead of compiling it this
test parses both files and checks that every function of include/prism_hip.h
is declared once in Rust with the same argument and return types (C types
mapped to their Rust FFI equivalents), that the error codes and the model
config struct agree, and that INTEGRATION.md shows the file's text.
"""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "prism_hip.h")
RUST = os.path.join(ROOT, "integration", "rust", "prism-ffi", "src", "hip.rs")

C_BASE = {"uint8_t": "u8", "uint16_t": "u16", "uint32_t": "u32", "int64_t": "i64", "size_t": "usize",
          "int": "c_int", "float": "f32", "char": "c_char", "void": "c_void"}


def _strip_c_comments(s):
    return re.sub(r"/\*.*?\*/", " ", re.sub(r"//[^\n]*", " ", s), flags=re.S)


def c_type_to_rust(t):
    t = " ".join(t.replace("*", " * ").split())
    ptr = t.count("*")
    const = t.startswith("const ")
    base = t.replace("const ", "").replace("*", "").strip()
    rb = C_BASE.get(base, base)
    if ptr == 0:
        return "" if base == "void" else rb
    assert ptr == 1, t
    return ("*const " if const else "*mut ") + rb


def header_functions():
    src = _strip_c_comments(open(HEADER).read())
    out = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(prism_hip_\w+)\s*\(([^;{]*?)\)\s*;", src):
        ret, name, params = m.group(1), m.group(2), m.group(3)
        ret = ret.replace("extern", "").strip()
        if ret.startswith("typedef"):
            continue
        args = []
        if params.strip() != "void":
            for p in params.split(","):
                p = " ".join(p.split())
                pm = re.match(r"(.*?)(\w+)$", p)
                args.append(c_type_to_rust(pm.group(1)))
        out[name] = (args, c_type_to_rust(ret))
    return out


def rust_functions(text):
    body = text[text.index('extern "C" {'):]
    body = body[:body.index("\n}\n")]
    body = re.sub(r"//[^\n]*", " ", body)
    out = {}
    for m in re.finditer(r"pub fn (prism_hip_\w+)\s*\((.*?)\)\s*(->\s*([^;]+))?;", body, re.S):
        name, params, ret = m.group(1), m.group(2), m.group(4)
        args = []
        for p in [p for p in params.split(",") if p.strip()]:
            ty = p.split(":", 1)[1]
            args.append(" ".join(ty.split()))
        assert name not in out, f"{name} declared twice"
        out[name] = (args, " ".join(ret.split()) if ret else "")
    return out


def test_every_header_function_is_bound_with_the_same_types():
    h = header_functions()
    r = rust_functions(open(RUST).read())
    assert len(h) >= 40
    assert set(h) == set(r), f"only in header: {sorted(set(h) - set(r))}; only in Rust: {sorted(set(r) - set(h))}"
    for name, (args, ret) in h.items():
        rargs, rret = r[name]
        assert rargs == args, f"{name}: Rust {rargs} vs C {args}"
        assert rret == ret, f"{name}: Rust returns {rret!r}, C {ret!r}"


def test_error_codes_match():
    src = open(HEADER).read()
    c = {m.group(1): int(m.group(2)) for m in re.finditer(r"#define (PRISM_HIP_\w+)\s+\(?(-?\d+)\)?", src)}
    rs = open(RUST).read()
    r = {m.group(1): int(m.group(2)) for m in re.finditer(r"pub const (PRISM_HIP_\w+): c_int = (-?\d+);", rs)}
    codes = {k: v for k, v in c.items() if k.startswith("PRISM_HIP_OK") or k.startswith("PRISM_HIP_ERR_")}
    assert codes and codes == r


def test_model_config_fields_match():
    src = _strip_c_comments(open(HEADER).read())
    m = re.search(r"typedef struct prism_hip_model_config \{(.*?)\} prism_hip_model_config;", src, re.S)
    cfields = []
    for decl in m.group(1).split(";"):
        decl = " ".join(decl.split())
        if not decl:
            continue
        ty, names = decl.split(" ", 1)
        for n in names.split(","):
            cfields.append((n.strip(), C_BASE[ty]))
    rs = open(RUST).read()
    rm = re.search(r"pub struct prism_hip_model_config \{(.*?)\}", rs, re.S)
    rfields = [(a.strip(), b.strip()) for a, b in re.findall(r"pub (\w+):\s*(\w+)", rm.group(1))]
    assert cfields == rfields


@pytest.mark.parametrize("path", [RUST, os.path.join(ROOT, "integration", "rust", "src", "backend", "hip.rs"),
                                  os.path.join(ROOT, "integration", "rust", "src", "lut", "plan_hip.rs")])
def test_integration_md_shows_the_files(path):
    md = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    blocks = re.findall(r"```rust\n(.*?)```", md, re.S)
    text = open(path).read()
    assert any(b.strip() == text.strip() for b in blocks), f"INTEGRATION.md's block differs from {path}"


def test_backend_calls_only_bound_functions():
    """Every prism_hip_* call in the HipBackend file is declared in hip.rs."""
    bound = set(rust_functions(open(RUST).read()))
    text = open(os.path.join(ROOT, "integration", "rust", "src", "backend", "hip.rs")).read()
    called = set(re.findall(r"\b(prism_hip_\w+)\s*\(", text))
    assert called and called <= bound, sorted(called - bound)
