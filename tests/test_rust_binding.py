"""The Rust FFI crate (rust/grout-hip-sys) against the C header it binds.

There is no Rust toolchain on this image, so the crate is never compiled
here; this test keeps its declarations from drifting from
include/grout_attn_hip.h:

* every function the header declares is in the crate's extern "C" block and
  nothing else is, with the same argument names and types in the same order
  and the same return type (C types mapped to their Rust FFI equivalents);
* every struct the header defines has a #[repr(C)] struct with the same
  fields in the same order and of the same types;
* the status codes, limits and dtype constants have the same values;
* the library exports every function the crate declares.
"""
from __future__ import annotations

import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "grout_attn_hip.h")
CRATE = os.path.join(ROOT, "rust", "grout-hip-sys")
LIB_RS = os.path.join(CRATE, "src", "lib.rs")

# C struct / handle names -> Rust names.
STRUCTS = {"grout_decode_layer": "GroutDecodeLayer", "grout_qwen3_layer": "GroutQwen3Layer",
           "grout_qwen3_model": "GroutQwen3Model", "grout_graph": "GroutGraph",
           "grout_decode_runner": "GroutDecodeRunner", "grout_qwen3_runner": "GroutQwen3Runner"}
SCALARS = {"int32_t": "i32", "int64_t": "i64", "uint32_t": "u32", "uint16_t": "u16",
           "float": "f32", "void": "c_void", "char": "c_char", **STRUCTS}


def c_to_rust(ctype: str) -> str:
    """A C parameter/field/return type as the crate spells it."""
    t = " ".join(ctype.replace("*", " * ").split())
    if t == "grout_stream_t":
        return "HipStream"
    stars = t.count("*")
    base = t.replace("*", "").strip()
    const = base.startswith("const ")
    base = base[len("const "):] if const else base
    rust = SCALARS[base.strip()]
    if stars == 0:
        return rust
    # The outermost pointer of `T**` is mutable; `const` binds to the pointee.
    out = ("*const " if const else "*mut ") + rust
    for _ in range(stars - 1):
        out = "*mut " + out
    return out


def _strip_c_comments(text: str) -> str:
    return re.sub(r"/\*.*?\*/", "", text, flags=re.S)


def header_functions() -> dict:
    text = _strip_c_comments(open(HEADER).read())
    funcs = {}
    for m in re.finditer(r"\n((?:const\s+)?(?:int32_t|int64_t|char)\s*\**)\s*(grout_\w+)\s*\(([^)]*)\);",
                         text):
        ret, name, args = m.group(1), m.group(2), " ".join(m.group(3).split())
        params = []
        for a in ([] if args in ("", "void") else args.split(",")):
            a = a.strip()
            pm = re.match(r"(.*?)(\w+)$", a)
            params.append((pm.group(2), c_to_rust(pm.group(1).strip())))
        funcs[name] = (c_to_rust(ret.strip()), params)
    return funcs


def header_structs() -> dict:
    text = _strip_c_comments(open(HEADER).read())
    out = {}
    for m in re.finditer(r"typedef struct (\w+) \{(.*?)\} (\w+);", text, flags=re.S):
        fields = []
        for line in m.group(2).split(";"):
            line = " ".join(line.split())
            if not line:
                continue
            fm = re.match(r"(.*?)(\w+)$", line)
            fields.append((fm.group(2), c_to_rust(fm.group(1).strip())))
        out[STRUCTS[m.group(1)]] = fields
    return out


def header_constants() -> dict:
    text = _strip_c_comments(open(HEADER).read())
    consts = {m.group(1): int(m.group(2)) for m in
              re.finditer(r"#define (GROUT_[A-Z0-9_]+) (-?\d+)", text)}
    enum = re.search(r"enum \{(.*?)\};", text, flags=re.S).group(1)
    consts.update({m.group(1): int(m.group(2)) for m in
                   re.finditer(r"(GROUT_\w+) = (-?\d+)", enum)})
    return consts


def _strip_rust_comments(text: str) -> str:
    return re.sub(r"//[^\n]*", "", text)


def crate_functions() -> dict:
    text = _strip_rust_comments(open(LIB_RS).read())
    block = re.search(r'extern "C" \{(.*?)\n\}', text, flags=re.S).group(1)
    funcs = {}
    for m in re.finditer(r"pub fn (\w+)\s*\((.*?)\)\s*->\s*([^;]+);", block, flags=re.S):
        name, args, ret = m.group(1), " ".join(m.group(2).split()), m.group(3).strip()
        params = []
        for a in args.split(","):
            a = a.strip()
            if not a:
                continue
            pn, pt = a.split(":", 1)
            params.append((pn.strip(), " ".join(pt.split())))
        funcs[name] = (" ".join(ret.split()), params)
    return funcs


def crate_structs() -> dict:
    text = _strip_rust_comments(open(LIB_RS).read())
    out = {}
    for m in re.finditer(r"#\[repr\(C\)\]\s*(?:#\[derive\([^)]*\)\]\s*)?pub struct (\w+) \{(.*?)\}",
                         text, flags=re.S):
        fields = []
        for fm in re.finditer(r"(\w+)\s*:\s*([^,]+),", m.group(2)):
            fields.append((fm.group(1).replace("pub ", ""), " ".join(fm.group(2).split())))
        out[m.group(1)] = fields
    return out


def crate_constants() -> dict:
    text = _strip_rust_comments(open(LIB_RS).read())
    return {m.group(1): int(m.group(2)) for m in
            re.finditer(r"pub const (GROUT_\w+): i32 = (-?\d+);", text)}


def test_crate_files_present():
    for rel in ("Cargo.toml", "build.rs", os.path.join("src", "lib.rs")):
        assert os.path.isfile(os.path.join(CRATE, rel)), rel
    cargo = open(os.path.join(CRATE, "Cargo.toml")).read()
    assert 'name = "grout-hip-sys"' in cargo
    build = open(os.path.join(CRATE, "build.rs")).read()
    assert "rustc-link-lib=dylib=grout_attn_hip" in build


def test_type_mapping_examples():
    assert c_to_rust("const uint16_t*") == "*const u16"
    assert c_to_rust("uint16_t*") == "*mut u16"
    assert c_to_rust("grout_graph**") == "*mut *mut GroutGraph"
    assert c_to_rust("const grout_decode_layer*") == "*const GroutDecodeLayer"
    assert c_to_rust("const void*") == "*const c_void"
    assert c_to_rust("uint16_t") == "u16"


def test_every_function_declared_with_same_signature():
    hdr, crate = header_functions(), crate_functions()
    assert len(hdr) >= 40, "header parse found too few functions"
    assert sorted(hdr) == sorted(crate), (
        f"only in header: {sorted(set(hdr) - set(crate))}; "
        f"only in crate: {sorted(set(crate) - set(hdr))}")
    for name, (ret, params) in hdr.items():
        cret, cparams = crate[name]
        assert cret == ret, f"{name}: return {cret} != {ret}"
        assert len(cparams) == len(params), f"{name}: arity {len(cparams)} != {len(params)}"
        for i, ((hn, ht), (cn, ct)) in enumerate(zip(params, cparams)):
            assert (cn, ct) == (hn, ht), f"{name} argument {i}: crate {cn}: {ct}, header {hn}: {ht}"


def test_every_struct_has_same_fields_in_order():
    hdr, crate = header_structs(), crate_structs()
    assert set(hdr) == {"GroutDecodeLayer", "GroutQwen3Layer", "GroutQwen3Model"}
    for name, fields in hdr.items():
        assert name in crate, f"no #[repr(C)] struct {name}"
        assert crate[name] == fields, f"{name}: crate {crate[name]} != header {fields}"
    for handle in ("GroutGraph", "GroutDecodeRunner", "GroutQwen3Runner"):
        assert crate.get(handle) == [("_opaque", "[u8; 0]")], f"opaque handle {handle}"


def test_constants_match():
    hdr, crate = header_constants(), crate_constants()
    assert hdr, "no constants parsed"
    for k, v in hdr.items():
        assert crate.get(k) == v, f"{k}: crate {crate.get(k)} != header {v}"


def test_library_exports_every_crate_function():
    try:
        import grout_amd

        L = grout_amd.lib()
    except Exception as e:  # the library is built by __graft_entry__.build()
        pytest.fail(f"library not loadable: {e}")
    missing = [n for n in crate_functions() if not hasattr(L, n)]
    assert not missing, f"not exported: {missing}"
