"""The Rust binding (integration/rust/bramha-hip-sys/src/lib.rs) against the C header.

This image has no Rust toolchain, so the crate is not compiled here. The test parses both
sides and checks that the extern "C" block declares exactly the header's functions, each with
the same argument count, the argument and return types the C types map to, and that the
#[repr(C)] config struct has the header's fields in order with the same types.
"""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "bramha_hip.h")
SYS_RS = os.path.join(ROOT, "integration", "rust", "bramha-hip-sys", "src", "lib.rs")
BACKEND_RS = os.path.join(ROOT, "integration", "rust", "hip_backend.rs")

_SCALARS = {"int": "c_int", "float": "f32", "double": "f64", "size_t": "usize", "char": "c_char", "void": "c_void",
            "int8_t": "i8", "uint8_t": "u8", "int32_t": "i32", "uint32_t": "u32", "int64_t": "i64",
            "uint64_t": "u64", "uint16_t": "u16", "bh_ctx": "bh_ctx", "bh_weight": "bh_weight",
            "bh_model": "bh_model", "bh_model_config": "bh_model_config"}


def C2RUST(ctype):
    """Rust FFI type of a C type: pointers keep their constness, T** becomes *mut *mut T."""
    t = ctype.strip()
    stars = t.count("*")
    base = t.replace("*", " ").split()
    const = base[0] == "const"
    if const:
        base = base[1:]
    assert len(base) == 1, ctype
    r = _SCALARS[base[0]]
    if stars == 0:
        return r
    r = ("*const " if const else "*mut ") + r
    for _ in range(stars - 1):
        r = "*mut " + r
    return r


def _strip_comments(text):
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return re.sub(r"//[^\n]*", " ", text)


def parse_c_header(text):
    """[(name, return type, [(arg type, arg name)])] of every function prototype."""
    out = []
    for stmt in _strip_comments(text).split(";"):
        m = re.search(r"((?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\**)\s*(bh_[a-z0-9_]+)\s*\(([^()]*)\)\s*$", stmt)
        if not m:
            continue
        ret, name, args = " ".join(m.group(1).split()), m.group(2), m.group(3).strip()
        if ret.startswith(("typedef", "return")):
            continue
        al = []
        if args and args != "void":
            for a in args.split(","):
                a = " ".join(a.split())
                am = re.match(r"(.*?)([A-Za-z_][A-Za-z0-9_]*)$", a)
                al.append((am.group(1).strip(), am.group(2)))
        out.append((name, ret, al))
    return out


def parse_c_struct(text, name):
    body = _strip_comments(text)
    m = re.search(r"typedef struct\s*\{(.*?)\}\s*" + name + r"\s*;", body, flags=re.S)
    fields = []
    for decl in m.group(1).split(";"):
        decl = " ".join(decl.split())
        if not decl:
            continue
        ctype, names = decl.split(" ", 1)
        for n in names.split(","):
            fields.append((n.strip(), _SCALARS[ctype]))
    return fields


def parse_rust_extern(text):
    """{name: (return type, [arg types])} of the `extern "C"` block's fns."""
    body = re.sub(r"//[^\n]*", " ", text)
    blk = re.search(r'extern "C"\s*\{(.*?)\n\}', body, flags=re.S).group(1)
    out = {}
    for m in re.finditer(r"pub fn (bh_[a-z0-9_]+)\s*\((.*?)\)\s*(?:->\s*([^;]+))?;", blk, flags=re.S):
        name, args, ret = m.group(1), m.group(2), (m.group(3) or "void").strip()
        types = [" ".join(a.split(":", 1)[1].split()) for a in args.split(",") if a.strip()]
        out[name] = (ret, types)
    return out


def parse_rust_struct(text, name):
    m = re.search(r"pub struct " + name + r"\s*\{(.*?)\}", text, flags=re.S)
    fields = []
    for f in re.sub(r"//[^\n]*", " ", m.group(1)).split(","):
        f = " ".join(f.split())
        if f:
            n, t = f.replace("pub ", "").split(":")
            fields.append((n.strip(), t.strip()))
    return fields


def test_extern_block_matches_header():
    protos = parse_c_header(open(HEADER).read())
    assert len(protos) >= 45
    rs = parse_rust_extern(open(SYS_RS).read())
    assert sorted(rs) == sorted(p[0] for p in protos)
    for name, ret, args in protos:
        rret, rtypes = rs[name]
        assert rret == ("void" if ret == "void" else C2RUST(ret)), name
        assert len(rtypes) == len(args), name
        for (ctype, cname), rtype in zip(args, rtypes):
            assert rtype == C2RUST(ctype), (name, cname, ctype, rtype)


def test_config_struct_matches_header():
    c = parse_c_struct(open(HEADER).read(), "bh_model_config")
    r = parse_rust_struct(open(SYS_RS).read(), "bh_model_config")
    assert [n for n, _ in r] == [n for n, _ in c]
    assert [t for _, t in r] == [t for _, t in c]


def test_backend_calls_only_declared_functions():
    used = set(re.findall(r"sys::(bh_[a-z0-9_]+)\s*\(", open(BACKEND_RS).read()))
    declared = {p[0] for p in parse_c_header(open(HEADER).read())}
    assert used and used <= declared
    for seam in ("bh_matvec_mul", "bh_matvec_mul_int8", "bh_matvec_mul_int4", "bh_clear_persistent_buffers",
                 "bh_init"):
        assert seam in used, seam
