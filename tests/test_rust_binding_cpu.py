"""The Rust binding a maintainer adds to exllamav3-rs (the ```rust blocks of INTEGRATION.md: the
src/ffi.rs externs that replace src/ffi.rs:43-65, 114-127 and the #[repr(C)] Exl3rRopeDesc) checked
mechanically against the C header include/exl3r/rowops.h, since no Rust toolchain is here to compile it:

- every `fn exl3r_*` extern names a header function, with the same parameter names in the same order and
  the same C type for each (`*const c_void` is `const void*`, `i64` is `int64_t`, ...), and the same
  return type; every header function but the version query has an extern;
- `Exl3rRopeDesc` has exl3r_rope_desc's fields in the header's order with the same types, and the offsets
  a #[repr(C)] layout gives them (computed with ctypes from the Rust types) are the ones gcc prints for
  the C struct;
- the HIP runtime externs of src/hip.rs have the arity and argument classes (pointer, 32/64-bit integer,
  size) of their declarations in the installed hip_runtime_api.h.

A drifted argument (an i32 where the header has int64_t, two swapped strides, a field moved) fails here.
"""
import ctypes
import os
import re
import subprocess
import tempfile

import pytest

from exl3r import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INTEGRATION = os.path.join(ROOT, "INTEGRATION.md")
HIP_API = "/opt/rocm/include/hip/hip_runtime_api.h"


# --- type model: scalars are names, pointers ("ptr", pointee_is_const, pointee) ---------------------

RUST_SCALARS = {"i32": "i32", "i64": "i64", "u32": "u32", "usize": "usize", "f32": "f32", "c_void": "void",
                "c_char": "char", "std::os::raw::c_char": "char", "Exl3rRopeDesc": "exl3r_rope_desc",
                "HipStream": ("ptr", False, "void"), "HipGraph": ("ptr", False, "void"),
                "HipGraphExec": ("ptr", False, "void")}
C_SCALARS = {"int": "i32", "int32_t": "i32", "int64_t": "i64", "uint32_t": "u32", "unsigned": "u32",
             "unsigned int": "u32", "size_t": "usize", "float": "f32", "void": "void", "char": "char",
             "exl3r_rope_desc": "exl3r_rope_desc"}


def rust_type(t):
    t = t.strip()
    m = re.match(r"^\*(const|mut)\s+(.*)$", t)
    if m:
        return ("ptr", m.group(1) == "const", rust_type(m.group(2)))
    assert t in RUST_SCALARS, f"unknown Rust type {t!r}"
    return RUST_SCALARS[t]


def c_type(t):
    """A C type as written in the header ('const void* const*', 'int64_t', ...)."""
    toks = re.findall(r"\*|[A-Za-z_][A-Za-z_0-9]*", t)
    const = False
    base = []
    i = 0
    while i < len(toks) and toks[i] != "*":
        if toks[i] == "const":
            const = True
        else:
            base.append(toks[i])
        i += 1
    name = " ".join(base)
    assert name in C_SCALARS, f"unknown C type {name!r} in {t!r}"
    cur, cur_const = C_SCALARS[name], const
    while i < len(toks):
        assert toks[i] == "*", t
        cur, cur_const = ("ptr", cur_const, cur), False
        i += 1
        if i < len(toks) and toks[i] == "const":
            cur_const = True
            i += 1
    return cur


# --- parsers ------------------------------------------------------------------------------------------

def rust_blocks():
    text = open(INTEGRATION).read()
    return re.findall(r"```rust\n(.*?)```", text, re.S)


def rust_externs():
    """{name: (ret, [(param, type)])} of the fns inside every `extern "C" { ... }` of the rust blocks."""
    out = {}
    for block in rust_blocks():
        for body in re.findall(r'extern "C"\s*\{(.*?)\n\}', block, re.S):
            for m in re.finditer(r"fn\s+(\w+)\s*\((.*?)\)\s*(?:->\s*([^;]+))?;", body, re.S):
                name, params, ret = m.group(1), m.group(2), m.group(3)
                ps = []
                for p in [p for p in (s.strip() for s in params.split(",")) if p]:
                    pn, pt = p.split(":", 1)
                    ps.append((pn.strip(), rust_type(pt)))
                out[name] = (rust_type(ret) if ret else "void", ps)
    return out


def strip_c_comments(s):
    s = re.sub(r"/\*.*?\*/", " ", s, flags=re.S)
    return re.sub(r"//[^\n]*", " ", s)


def split_decl(d):
    """'const void* const* pre_scales' -> ('const void* const*', 'pre_scales')."""
    m = re.match(r"^(.*?)([A-Za-z_]\w*)\s*$", d.strip(), re.S)
    return m.group(1).strip(), m.group(2)


def header_functions():
    text = strip_c_comments(open(_lib.HEADER_PATH).read())
    out = {}
    for m in re.finditer(r"EXL3R_API\s+([^;()]*?)\b(exl3r_\w+)\s*\(([^)]*)\)\s*;", text, re.S):
        ret, name, params = m.group(1), m.group(2), m.group(3).strip()
        ps = []
        if params and params != "void":
            for p in params.split(","):
                t, n = split_decl(p)
                ps.append((n, c_type(t)))
        out[name] = (c_type(ret), ps)
    return out


def header_desc_fields():
    text = strip_c_comments(open(_lib.HEADER_PATH).read())
    body = re.search(r"typedef\s+struct\s+exl3r_rope_desc\s*\{(.*?)\}\s*exl3r_rope_desc\s*;", text, re.S).group(1)
    fields = []
    for decl in (d.strip() for d in body.split(";")):
        if not decl:
            continue
        parts = [p.strip() for p in decl.split(",")]
        base, first = split_decl(parts[0])
        fields.append((first, c_type(base)))
        for p in parts[1:]:
            stars = p.count("*")
            fields.append((p.replace("*", "").strip(), c_type(base + "*" * stars)))
    return fields


def rust_desc_fields():
    for block in rust_blocks():
        m = re.search(r"#\[repr\(C\)\][^\n]*\n(?:#\[[^\n]*\]\n)*pub struct Exl3rRopeDesc\s*\{(.*?)\n\}", block, re.S)
        if m:
            return [(n, rust_type(t)) for n, t in re.findall(r"pub\s+(\w+)\s*:\s*([^,\n]+?)\s*,", m.group(1))]
    raise AssertionError("no #[repr(C)] Exl3rRopeDesc in INTEGRATION.md")


# --- checks -------------------------------------------------------------------------------------------

def test_parsers_see_the_declarations():
    """The parsers find what the files hold (a parser that matched nothing would pass every check)."""
    hdr, rs = header_functions(), rust_externs()
    assert len(hdr) == open(_lib.HEADER_PATH).read().count("EXL3R_API int") + \
        open(_lib.HEADER_PATH).read().count("EXL3R_API size_t") + open(_lib.HEADER_PATH).read().count("EXL3R_API const")
    assert len([n for n in rs if n.startswith("exl3r_")]) >= 30
    assert len(header_desc_fields()) >= 40
    # the type model itself: the forms the binding uses
    assert c_type("const void* const*") == rust_type("*const *const c_void")
    assert c_type("void* const*") == rust_type("*const *mut c_void")
    assert c_type("void*") != rust_type("*const c_void")
    assert c_type("int64_t") != rust_type("i32")


def test_every_extern_matches_the_header():
    hdr, rs = header_functions(), rust_externs()
    bad = []
    for name, (ret, params) in sorted(rs.items()):
        if not name.startswith("exl3r_"):
            continue
        if name not in hdr:
            bad.append(f"{name}: not in the header")
            continue
        hret, hparams = hdr[name]
        if ret != hret:
            bad.append(f"{name}: returns {ret}, the header {hret}")
        if len(params) != len(hparams):
            bad.append(f"{name}: {len(params)} parameters, the header {len(hparams)}")
            continue
        for i, ((rn, rt), (cn, ct)) in enumerate(zip(params, hparams)):
            if rn != cn:
                bad.append(f"{name} arg {i}: named {rn}, the header {cn}")
            if rt != ct:
                bad.append(f"{name} arg {i} ({cn}): {rt} vs the header's {ct}")
    assert not bad, "\n".join(bad)


def test_every_header_function_has_an_extern():
    unbound = set(header_functions()) - set(rust_externs())
    assert unbound <= {"exl3r_version"}, sorted(unbound)


def test_rope_desc_fields_match_the_header():
    rs, hs = rust_desc_fields(), header_desc_fields()
    assert [n for n, _ in rs] == [n for n, _ in hs]
    for (n, rt), (_, ct) in zip(rs, hs):
        assert rt == ct, n


CTYPES = {"i32": ctypes.c_int32, "i64": ctypes.c_int64, "u32": ctypes.c_uint32, "usize": ctypes.c_size_t,
          "f32": ctypes.c_float}


def test_rope_desc_repr_c_offsets_match_gcc():
    fields = rust_desc_fields()
    RustDesc = type("RustDesc", (ctypes.Structure,),
                    {"_fields_": [(n, ctypes.c_void_p if isinstance(t, tuple) else CTYPES[t]) for n, t in fields]})
    src = "#include <stddef.h>\n#include <stdio.h>\n#include \"exl3r/rowops.h\"\nint main(void) {\n"
    src += '  printf("size %zu\\n", sizeof(exl3r_rope_desc));\n'
    for n, _ in fields:
        src += f'  printf("{n} %zu\\n", offsetof(exl3r_rope_desc, {n}));\n'
    src += "  return 0;\n}\n"
    inc = os.path.dirname(os.path.dirname(_lib.HEADER_PATH))
    with tempfile.TemporaryDirectory() as d:
        c, exe = os.path.join(d, "layout.c"), os.path.join(d, "layout")
        open(c, "w").write(src)
        subprocess.run(["gcc", "-std=c11", "-I", inc, c, "-o", exe], check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    lay = {k: int(v) for k, v in (line.split() for line in out.strip().splitlines())}
    assert lay.pop("size") == ctypes.sizeof(RustDesc)
    for n, off in lay.items():
        assert getattr(RustDesc, n).offset == off, n


# HIP's own types by the argument class they pass as.
HIP_CLASSES = {"hipStream_t": "ptr", "hipGraph_t": "ptr", "hipGraphExec_t": "ptr", "hipError_t": "i32",
               "hipMemcpyKind": "i32", "hipStreamCaptureMode": "i32", "int": "i32", "unsigned int": "u32",
               "size_t": "usize", "const char": "ptr"}


def hip_class(t):
    t = re.sub(r"\s+", " ", t.replace("const ", "const ")).strip()
    if "*" in t:
        return "ptr"
    t = t.replace("const ", "")
    assert t in HIP_CLASSES, f"unknown HIP type {t!r}"
    return HIP_CLASSES[t]


def rust_class(t):
    return "ptr" if isinstance(t, tuple) else t


@pytest.mark.skipif(not os.path.exists(HIP_API), reason="no HIP runtime header")
def test_hip_externs_match_the_runtime_header():
    text = strip_c_comments(open(HIP_API).read())
    text = re.sub(r"__dparm\([^)]*\)", "", text)
    bad = []
    hip = {n: v for n, v in rust_externs().items() if n.startswith("hip")}
    assert len(hip) >= 10
    for name, (ret, params) in sorted(hip.items()):
        m = re.search(r"\b(hipError_t|const char\s*\*)\s+" + name + r"\s*\(([^)]*)\)\s*;", text)
        if not m:
            bad.append(f"{name}: no C declaration in hip_runtime_api.h")
            continue
        cps = [split_decl(p)[0] for p in m.group(2).split(",") if p.strip()]
        if len(cps) != len(params):
            bad.append(f"{name}: {len(params)} parameters, HIP {len(cps)}")
            continue
        if rust_class(ret) != hip_class(m.group(1)):
            bad.append(f"{name}: returns {ret}, HIP {m.group(1)}")
        for i, ((pn, pt), ct) in enumerate(zip(params, cps)):
            if rust_class(pt) != hip_class(ct):
                bad.append(f"{name} arg {i} ({pn}): {pt} vs HIP's {ct}")
    assert not bad, "\n".join(bad)


def test_every_header_constant_has_a_rust_const():
    """Each integer #define EXL3R_<NAME> of the header has `pub const EXL3R_<NAME>: i32 = <same value>;` in the
    binding (status codes, dtype codes, activations, rotary styles, the exact-Hadamard flag)."""
    text = strip_c_comments(open(_lib.HEADER_PATH).read())
    hdr = {n: int(v) for n, v in re.findall(r"#define\s+(EXL3R_[A-Z0-9_]+)\s+\(?(-?\d+)\)?\s*$", text, re.M)}
    assert {"EXL3R_F16", "EXL3R_EINVAL", "EXL3R_ACT_GELU", "EXL3R_HAD_EXACT", "EXL3R_ROPE_NEOX"} <= set(hdr)
    rs = {}
    for block in rust_blocks():
        rs.update({n: int(v) for n, v in re.findall(r"pub const (EXL3R_[A-Z0-9_]+):\s*i32\s*=\s*(-?\d+)\s*;", block)})
    bad = [f"{n}: header {v}, binding {rs.get(n)}" for n, v in sorted(hdr.items()) if rs.get(n) != v]
    assert not bad, "\n".join(bad)
