"""The Rust FFI crate (rust/nemotron-hip-sys) against include/nemotron_hip.h.

No Rust toolchain is needed: the crate's source is parsed and compared with the
header declaration by declaration (name, order, argument names and types,
return type), enum constant by constant, and struct field by field, with the C
offsets taken from gcc's offsetof and the Rust ones from a ctypes layout of the
Rust field types (the repr(C) rules are the C ones).  The compile-time asserts
in the crate are checked against the same gcc figures."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.join(os.path.dirname(__file__), "..")
HEADER = os.path.join(ROOT, "include", "nemotron_hip.h")
SYS_RS = os.path.join(ROOT, "rust", "nemotron-hip-sys", "src", "lib.rs")

C_TO_RUST = {"size_t": "usize", "int": "c_int", "float": "f32", "uint32_t": "u32", "uint64_t": "u64",
             "int32_t": "i32", "int8_t": "i8", "uint8_t": "u8", "char": "c_char", "void": "c_void",
             "nh_context": "nh_context", "nh_stream": "nh_stream", "nh_dtype": "nh_dtype",
             "nh_status": "nh_status", "nh_error": "nh_error", "nh_tensor_info": "nh_tensor_info",
             "nh_moe_biases": "nh_moe_biases"}


def c_source():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", " ", src, flags=re.S)
    return "\n".join(l for l in src.splitlines() if not l.strip().startswith("#"))


def c_type_to_rust(t):
    """A C parameter type as the Rust FFI spells it: const T * -> *const T,
    T * -> *mut T, pointer to pointer innermost-first."""
    t = " ".join(t.split())
    const = t.startswith("const ")
    base = t[6:] if const else t
    stars = base.count("*")
    r = C_TO_RUST[base.replace("*", "").strip()]
    for i in range(stars):
        r = ("*const " if const and i == 0 else "*mut ") + r
    return r


def header_functions():
    src = c_source()
    body = src[src.index('extern "C" {') + len('extern "C" {'):src.rindex("}")]
    body = re.sub(r"typedef\s+(enum|struct)\s+\w+\s*\{.*?\}\s*\w+\s*;", "", body, flags=re.S)
    body = re.sub(r"typedef[^;]*;", "", body)
    out = []
    for d in body.split(";"):
        d = " ".join(d.split())
        if "(" not in d:
            continue
        m = re.match(r"(.+?)\s*\b(nh_\w+)\s*\((.*)\)$", d)
        assert m, d
        ret, name, args = m.group(1).strip(), m.group(2), m.group(3).strip()
        params = []
        if args != "void":
            for a in args.split(","):
                am = re.match(r"(.+?)\s*(\w+)\s*(\[\d+\])?$", a.strip())
                ty = am.group(1) + ("*" if am.group(3) else "")  # an array parameter is a pointer
                params.append((am.group(2), c_type_to_rust(ty)))
        out.append((name, params, None if ret == "void" else c_type_to_rust(ret)))
    return out


def rust_functions():
    src = open(SYS_RS).read()
    src = re.sub(r"//[^\n]*", "", src)
    block = src[src.index('extern "C" {') + len('extern "C" {'):src.rindex("}")]
    out = []
    for m in re.finditer(r"pub fn (\w+)\s*\((.*?)\)\s*(->\s*([^;]+))?;", block, flags=re.S):
        params = []
        for p in [p.strip() for p in m.group(2).split(",") if p.strip()]:
            n, t = p.split(":", 1)
            params.append((n.strip(), " ".join(t.split())))
        out.append((m.group(1), params, " ".join(m.group(4).split()) if m.group(4) else None))
    return out


def test_every_declaration_bound_once_in_header_order():
    h = [f[0] for f in header_functions()]
    r = [f[0] for f in rust_functions()]
    assert len(h) > 60 and len(set(r)) == len(r)
    assert r == h


@pytest.mark.parametrize("fn", [f[0] for f in header_functions()])
def test_signature_matches_header(fn):
    h = {f[0]: f for f in header_functions()}[fn]
    r = {f[0]: f for f in rust_functions()}[fn]
    assert len(r[1]) == len(h[1]), f"{fn}: {len(r[1])} Rust arguments, {len(h[1])} in C"
    for (hn, ht), (rn, rt) in zip(h[1], r[1]):
        assert rn == hn, f"{fn}: argument {rn} where the header has {hn}"
        assert rt == ht, f"{fn}({hn}): Rust {rt}, C maps to {ht}"
    assert r[2] == h[2], f"{fn}: returns {r[2]} in Rust, {h[2]} in C"


def test_status_and_dtype_constants_match_header_enums():
    src = c_source()
    rs = open(SYS_RS).read()
    consts = dict((n, int(v)) for n, v in re.findall(r"pub const (\w+): Self = Self\((\d+)\);", rs))
    status = re.search(r"typedef enum nh_status \{(.*?)\} nh_status;", src, flags=re.S).group(1)
    pairs = re.findall(r"NH_(\w+)\s*=\s*(\d+)", status)
    assert len(pairs) == 12
    for name, v in pairs:
        assert consts[name] == int(v), name
    dtype = re.search(r"typedef enum nh_dtype \{(.*?)\} nh_dtype;", src, flags=re.S).group(1)
    for name, v in re.findall(r"NH_(\w+)\s*=\s*(\d+)", dtype):
        assert consts[name] == int(v), name
    assert re.search(r"#\[repr\(transparent\)\]\s*#\[derive[^\]]*\]\s*pub struct nh_status\(pub c_int\);", rs)
    assert re.search(r"#\[repr\(transparent\)\]\s*#\[derive[^\]]*\]\s*pub struct nh_dtype\(pub c_int\);", rs)


RUST_CTYPES = {"u64": ctypes.c_uint64, "u32": ctypes.c_uint32, "f32": ctypes.c_float, "c_int": ctypes.c_int,
               "c_char": ctypes.c_char, "*const c_char": ctypes.c_void_p, "*const f32": ctypes.c_void_p}


def rust_struct(name):
    rs = open(SYS_RS).read()
    m = re.search(r"#\[repr\(C\)\]\s*(#\[derive[^\]]*\]\s*)?pub struct %s \{(.*?)\n\}" % name, rs, flags=re.S)
    assert m, name
    fields = []
    for line in m.group(2).splitlines():
        line = line.split("//")[0].strip()
        fm = re.match(r"pub (\w+): (.+),$", line)
        if fm:
            fields.append((fm.group(1), fm.group(2).strip()))
    return fields


def ctypes_layout(fields):
    spec = []
    for n, t in fields:
        am = re.match(r"\[(.+); (\d+)\]$", t)
        spec.append((n, RUST_CTYPES[am.group(1)] * int(am.group(2)) if am else RUST_CTYPES[t]))
    S = type("S", (ctypes.Structure,), {"_fields_": spec})
    return ctypes.sizeof(S), {n: getattr(S, n).offset for n, _ in fields}


def gcc_layout(tmp_path, struct, fields):
    prog = tmp_path / "layout.c"
    prog.write_text("#include <stdio.h>\n#include <stddef.h>\n#include \"nemotron_hip.h\"\nint main(void) {\n"
                    f"  printf(\"%zu\\n\", sizeof({struct}));\n"
                    + "".join(f"  printf(\"%zu\\n\", offsetof({struct}, {n}));\n" for n, _ in fields)
                    + "  return 0;\n}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), "-o", str(exe), str(prog)], check=True)
    vals = [int(v) for v in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]
    return vals[0], dict(zip([n for n, _ in fields], vals[1:]))


@pytest.mark.parametrize("struct", ["nh_error", "nh_tensor_info", "nh_moe_biases"])
def test_struct_layout_matches_c(tmp_path, struct):
    fields = rust_struct(struct)
    src = c_source()
    cbody = re.search(r"typedef struct %s \{(.*?)\} %s;" % (struct, struct), src, flags=re.S).group(1)
    cnames = re.findall(r"(\w+)\s*(?:\[\d+\])?\s*;", cbody)
    assert [n for n, _ in fields] == cnames, "field names or order differ"
    csize, coff = gcc_layout(tmp_path, struct, fields)
    rsize, roff = ctypes_layout(fields)
    assert rsize == csize and roff == coff
    # the crate's compile-time asserts state the same figures
    rs = open(SYS_RS).read()
    assert re.search(r"size_of::<%s>\(\) == %d" % (struct, csize), rs)
    for n, off in coff.items():
        assert re.search(r"offset_of!\(%s, %s\) == %d\)" % (struct, n, off), rs), n


def test_nh_error_byte_payload_is_u32():
    # Int4OutOfRange carries a u8, but the C field is uint32_t: a u8 here
    # would shift `message` and lose every error text
    assert dict(rust_struct("nh_error"))["byte"] == "u32"


def split_top_level(args):
    out, depth, cur = [], 0, ""
    for ch in args:
        if ch in "([{":
            depth += 1
        elif ch in ")]}":
            depth -= 1
        if ch == "," and depth == 0:
            out.append(cur)
            cur = ""
        else:
            cur += ch
    if cur.strip():
        out.append(cur)
    return [a.strip() for a in out if a.strip()]


def test_safe_crate_calls_bound_functions_with_their_arity():
    """Every sys::nh_* call of rust/nemotron-hip names a declaration of the
    sys crate and passes exactly its number of arguments."""
    arity = {f[0]: len(f[1]) for f in rust_functions()}
    src_dir = os.path.join(ROOT, "rust", "nemotron-hip", "src")
    calls = 0
    for fn in sorted(os.listdir(src_dir)):
        src = re.sub(r"//[^\n]*", "", open(os.path.join(src_dir, fn)).read())
        for m in re.finditer(r"sys::(nh_\w+)\(", src):
            name = m.group(1)
            assert name in arity, f"{fn}: {name} is not bound"
            depth, i = 1, m.end()
            while depth:
                depth += {"(": 1, ")": -1}.get(src[i], 0)
                i += 1
            args = split_top_level(src[m.end():i - 1])
            assert len(args) == arity[name], f"{fn}: {name} called with {len(args)} arguments, takes {arity[name]}"
            calls += 1
    assert calls >= 15
