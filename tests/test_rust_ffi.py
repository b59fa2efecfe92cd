"""The Rust FFI crate (crates/hip_sampling) declares every function of include/gbs_sample.h with the same parameters
and return type (C types mapped to their Rust equivalents), and its #[repr(C)] records match the C structs. No Rust
toolchain is in this image, so the crate is checked here against the header text, parameter by parameter."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gbs_sample.h")
CRATE = os.path.join(ROOT, "crates", "hip_sampling", "src", "lib.rs")

C_TO_RUST = {
    "int": "i32", "size_t": "usize", "void*": "*mut c_void", "const void*": "*const c_void", "int*": "*mut i32",
    "const int*": "*const i32", "float*": "*mut f32", "const float*": "*const f32", "const int32_t*": "*const i32",
    "const uint32_t*": "*const u32", "unsigned long long": "u64", "double": "f64", "const char*": "*const c_char",
    "const GbsKeyedRow*": "*const KeyedRow", "const GbsRowParams*": "*const RowParams", "int64_t": "i64",
}


def header_functions():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"^\s*((?:const\s+)?[A-Za-z_][\w ]*?\**)\s*\b((?:gb|gbs)_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.M | re.S):
        ret, name, params = m.group(1).strip(), m.group(2), m.group(3)
        types = []
        for prm in params.split(","):
            prm = " ".join(prm.split())
            if not prm or prm == "void":
                continue
            t = re.sub(r"\s*\b\w+$", "", prm).replace(" *", "*")
            types.append(t)
        out[name] = (ret.replace(" *", "*"), types)
    return out


def rust_functions():
    text = open(CRATE).read()
    block = text[text.index('extern "C" {'):]
    block = block[:block.index("\n    }\n")]
    out = {}
    for m in re.finditer(r"pub fn ((?:gb|gbs)_\w+)\(([^)]*)\)\s*(?:->\s*([^;]+))?;", block, flags=re.S):
        name, params, ret = m.group(1), m.group(2), (m.group(3) or "()").strip()
        types = [" ".join(p.split(":", 1)[1].split()) for p in params.split(",") if p.strip()]
        out[name] = (ret, types)
    return out


def test_every_header_function_is_declared_in_the_crate_with_the_same_signature():
    h, r = header_functions(), rust_functions()
    assert len(h) >= 30
    assert set(h) == set(r), (set(h) ^ set(r))
    for name, (ret, types) in h.items():
        rret, rtypes = r[name]
        assert C_TO_RUST[ret] == rret, (name, ret, rret)
        assert [C_TO_RUST[t] for t in types] == rtypes, (name, types, rtypes)


def test_records_match_the_c_structs():
    text = open(CRATE).read()
    def fields(rust_name):
        body = re.search(r"pub struct " + rust_name + r" \{(.*?)\}", text, flags=re.S).group(1)
        return [tuple(x.strip().rstrip(",").replace("pub ", "").split(": ")) for x in body.strip().splitlines()]
    hdr = open(HEADER).read()
    def cfields(c_name):
        body = re.search(r"typedef struct " + c_name + r" \{(.*?)\}", hdr, flags=re.S).group(1)
        return [tuple(x.strip().rstrip(";").split()) for x in body.strip().splitlines()]
    cmap = {"uint64_t": "u64", "double": "f64", "float": "f32", "int32_t": "i32"}
    for rname, cname in (("KeyedRow", "GbsKeyedRow"), ("RowParams", "GbsRowParams")):
        assert [(n, t) for n, t in fields(rname)] == [(n, cmap[t]) for t, n in cfields(cname)], rname


def test_constants_match_the_header():
    text, hdr = open(CRATE).read(), open(HEADER).read()
    for rust, c in (("ROW_NAN_LOGIT", "GBS_ROW_NAN_LOGIT"), ("DTYPE_F16", "GBS_DTYPE_F16"), ("MAX_COUNT", "GBS_MAX_COUNT")):
        rv = re.search(r"pub const " + rust + r": \w+ = ([\d_]+);", text).group(1).replace("_", "")
        cv = re.search(r"#define " + c + r" (\d+)", hdr).group(1)
        assert rv == cv, rust
    assert re.search(r"pub const KMAX_MIXED: i32 = -1;", text) and "#define GBS_KMAX_MIXED (-1)" in hdr
    assert "pub const NOALLOC_SCRATCH_BYTES: usize = 32 << 20;" in text and "((size_t)32 << 20)" in hdr
