"""The Rust binding printed in the repository's integration guide against the C
ABI it binds.

No Rust toolchain exists here, so the `hip` module cannot be compiled.  This
test parses its `extern "C"` block and its `#[repr(C)]` config struct and
checks them against `include/edgebert_hip.h`: every declared function exists,
with the same return type and the same parameter types in the same order, and
the struct has the same fields in the same order.  A change to the header that
the binding text does not follow fails here.
"""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# Rust base types -> C base types (after pointer levels are stripped).
RUST_BASE = {
    "f32": "float", "f64": "double", "u32": "uint32_t", "i32": "int32_t", "i64": "int64_t",
    "c_int": "int32_t", "c_char": "char", "c_float": "float", "c_void": "void", "usize": "size_t",
    "EbhModel": "ebh_model", "EbhTokenizer": "ebh_tokenizer", "EbhConfig": "ebh_config",
}
C_BASE = {"int": "int32_t", "int32_t": "int32_t"}


def canon_rust(t):
    """`*const *const c_char` -> ('char', ('const', 'const'))."""
    t = t.strip()
    quals = []
    while t.startswith("*"):
        m = re.match(r"\*(const|mut)\s+(.*)", t)
        assert m, f"unparsed Rust type {t!r}"
        quals.append(m.group(1))
        t = m.group(2).strip()
    return RUST_BASE.get(t, t), tuple(q == "const" for q in reversed(quals))


def canon_c(t):
    """`const char* const*` -> ('char', (True, True)): constness of each pointee level,
    innermost first (matching canon_rust's order)."""
    t = re.sub(r"\s+", " ", t.strip())
    parts = [p.strip() for p in t.split("*")]
    base = parts[0].split()
    const_base = "const" in base
    base = [w for w in base if w != "const" and w != "struct"][-1]
    # parts[1:] are what follows each '*': 'const' there qualifies the pointer itself.
    levels = []
    pointee_const = const_base
    for p in parts[1:]:
        levels.append(pointee_const)
        pointee_const = "const" in p.split()
    return C_BASE.get(base, base), tuple(levels)


def rust_block():
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    sec = text[text.index("## 2. FFI module"):text.index("## 3.")]
    return re.sub(r"//[^\n]*", "", sec)


def rust_externs():
    block = rust_block()
    body = block[block.index('extern "C" {'):]
    body = body[:body.index("\n}")]
    out = {}
    for m in re.finditer(r"fn\s+(\w+)\s*\(([^)]*)\)\s*(->\s*([^;]+))?;", body, re.S):
        name, params, ret = m.group(1), m.group(2), m.group(4)
        types = []
        for p in [p for p in params.split(",") if p.strip()]:
            types.append(canon_rust(p.split(":", 1)[1]))
        out[name] = (canon_rust(ret) if ret else ("void", ()), types)
    return out


def c_decls():
    text = open(os.path.join(ROOT, "include", "edgebert_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    out = {}
    for m in re.finditer(r"EBH_API\s+([^;(]+?)\s*(\bebh_\w+)\s*\(([^)]*)\)\s*;", text, re.S):
        ret, name, params = m.group(1), m.group(2), m.group(3)
        types = []
        for p in [p for p in params.split(",") if p.strip() and p.strip() != "void"]:
            p = re.sub(r"\s+", " ", p.strip())
            # drop the parameter name (the last identifier not followed by '*')
            mm = re.match(r"(.*?[\s*])(\w+)$", p)
            types.append(canon_c(mm.group(1)))
        out[name] = (canon_c(ret), types)
    return out


def test_every_rust_extern_matches_the_header():
    rust, c = rust_externs(), c_decls()
    assert len(rust) >= 12, sorted(rust)
    for name, (ret, params) in rust.items():
        assert name in c, f"{name} is not declared in include/edgebert_hip.h"
        cret, cparams = c[name]
        assert ret == cret, f"{name}: Rust returns {ret}, C returns {cret}"
        assert len(params) == len(cparams), f"{name}: {len(params)} Rust parameters, {len(cparams)} in C"
        for i, (a, b) in enumerate(zip(params, cparams)):
            assert a == b, f"{name} parameter {i}: Rust {a} against C {b}"


def test_config_struct_matches_the_header():
    block = rust_block()
    m = re.search(r"pub struct EbhConfig\s*\{(.*?)\}", block, re.S)
    fields = [(f.split(":")[0].replace("pub", "").strip(), canon_rust(f.split(":")[1]))
              for f in m.group(1).split(",") if f.strip()]
    text = open(os.path.join(ROOT, "include", "edgebert_hip.h")).read()
    cm = re.search(r"typedef struct ebh_config\s*\{(.*?)\}\s*ebh_config;", text, re.S)
    cfields = []
    for line in cm.group(1).split(";"):
        line = re.sub(r"//[^\n]*", "", line).strip()
        if line:
            t, n = line.rsplit(None, 1)
            cfields.append((n, canon_c(t)))
    assert fields == cfields


@pytest.mark.parametrize("rust_t,c_t", [
    ("*const *const c_char", "const char* const*"), ("*mut *mut EbhModel", "ebh_model**"),
    ("*const f32", "const float*"), ("i32", "int32_t"), ("c_int", "int")])
def test_type_mapping(rust_t, c_t):
    assert canon_rust(rust_t) == canon_c(c_t)


def test_a_changed_signature_is_caught():
    """A planted mismatch (one parameter dropped from a Rust declaration) fails."""
    rust, c = rust_externs(), c_decls()
    ret, params = rust["ebh_encode"]
    assert len(params[:-1]) != len(c["ebh_encode"][1])


REF = "/root/reference/src"


@pytest.mark.skipif(not os.path.isdir(REF), reason="reference sources not present on this machine")
def test_reference_items_the_binding_uses_exist():
    """Every ModelWeights method and Config field the binding calls exists in
    the reference crate with the types the binding assumes (weights.rs
    accessors returning Result<Array1/Array2<f32>>, Result<f32>, bool;
    Config's usize fields and f32 layer_norm_eps)."""
    block = rust_block()
    weights_src = open(os.path.join(REF, "weights.rs")).read()
    lib_src = open(os.path.join(REF, "lib.rs")).read()
    assert re.search(r"^\s*(pub\s+)?mod weights\s*;", lib_src, re.M), "lib.rs has no `mod weights;`"
    want_ret = {"get_array1": r"Result<Array1<f32>>", "get_array2": r"Result<Array2<f32>>",
                "get_scalar": r"Result<f32>", "is_cross_encoder": r"bool"}
    used = set(re.findall(r"weights\.(\w+)\(", block))
    assert used == set(want_ret), used
    for name in used:
        assert re.search(rf"pub fn {name}\(&self[^)]*\)\s*->\s*{re.escape(want_ret[name])}", weights_src), name
    cfg = re.search(r"pub struct Config\s*\{(.*?)\}", lib_src, re.S).group(1)
    types = dict((f.strip().replace("pub ", "").split(":")[0].strip(), f.split(":")[1].strip())
                 for f in cfg.split(",") if ":" in f)
    for field in set(re.findall(r"\bc\.(\w+)", block)):
        assert field in types, f"Config has no field {field}"
        assert types[field] == ("f32" if field == "layer_norm_eps" else "usize"), (field, types[field])
