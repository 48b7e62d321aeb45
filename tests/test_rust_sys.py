"""The Rust declarations crate (rust/cpb-moe-sys/src/lib.rs) matches the C
headers it binds, checked without cargo (absent here): every function of
include/cpb_moe.h and include/cpb_gguf.h with its parameter count, every
constant with its value, and every #[repr(C)] struct field for field, with
offsets computed from the Rust field types and compared with the ctypes
mirror of the C structs."""
import ctypes as C
import re
from pathlib import Path

from cpubrrr_amd import _lib as L

ROOT = Path(__file__).resolve().parent.parent
RS = (ROOT / "rust" / "cpb-moe-sys" / "src" / "lib.rs").read_text()
HEADERS = [(ROOT / "include" / h).read_text() for h in ("cpb_moe.h", "cpb_gguf.h", "cpb_head.h", "cpb_attn.h")]


def c_functions():
    out = {}
    for h in HEADERS:
        body = re.sub(r"/\*.*?\*/", "", h, flags=re.S)
        for m in re.finditer(r"^\s*[A-Za-z_][\w\s\*]*?\b(cpb_\w+)\s*\(([^)]*)\)\s*;", body, re.M):
            args = m.group(2).strip()
            out[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def rust_functions():
    out = {}
    for m in re.finditer(r"pub fn (cpb_\w+)\(([^)]*)\)", RS, re.S):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if not args else args.count(",") + 1
    return out


def test_every_function_declared_with_arity():
    c, r = c_functions(), rust_functions()
    assert "cpb_moe_forward" in c and "cpb_moe_load_gguf_layer" in c
    assert set(c) == set(r), (set(c) ^ set(r))
    for name in c:
        assert c[name] == r[name], (name, c[name], r[name])


def test_constants():
    cdefs = {}
    for h in HEADERS:
        for m in re.finditer(r"#define\s+(CPB_\w+)\s+(-?\d+)", h):
            cdefs[m.group(1)] = int(m.group(2))
    rdefs = {m.group(1): int(m.group(2)) for m in re.finditer(r"pub const (CPB_\w+): c_int = (-?\d+);", RS)}
    assert cdefs == rdefs


_RUST_SIZE = {"c_int": 4, "f32": 4, "i32": 4, "u32": 4, "i64": 8, "u64": 8, "f64": 8}


def _rust_layout(struct):
    m = re.search(r"pub struct %s \{(.*?)\n\}" % struct, RS, re.S)
    fields = re.findall(r"pub (\w+): ([^,]+),", m.group(1))
    out, off = [], 0
    for name, ty in fields:
        ty = ty.strip()
        if ty.startswith("*"):
            size = align = 8
        elif ty.startswith("["):
            el, n = re.match(r"\[(\w+); (\d+)\]", ty).groups()
            align = 1 if el == "c_char" else _RUST_SIZE[el]
            size = (1 if el == "c_char" else _RUST_SIZE[el]) * int(n)
        else:
            size = align = _RUST_SIZE[ty]
        off = (off + align - 1) // align * align
        out.append((name.rstrip("_"), off))
        off += size
    return out


def test_struct_layouts():
    for rust, cty in (("cpb_moe_cfg", L.MoeCfg), ("cpb_moe_trace", L.MoeTrace),
                      ("cpb_gguf_tensor", L.GgufTensor), ("cpb_gguf_hparams", L.GgufHparams),
                      ("cpb_head_cfg", L.HeadCfg), ("cpb_head_trace", L.HeadTrace),
                      ("cpb_attn_cfg", L.AttnCfg), ("cpb_attn_trace", L.AttnTrace)):
        want = [(name, getattr(cty, name).offset) for name, _ in cty._fields_]
        assert _rust_layout(rust) == want, rust


def test_ctypes_mirrors_follow_the_headers():
    # the ctypes structs (used above as the C layout) list the header's fields in order
    for h, name, cty in ((HEADERS[0], "cpb_moe_cfg", L.MoeCfg), (HEADERS[0], "cpb_moe_trace", L.MoeTrace),
                         (HEADERS[1], "cpb_gguf_tensor", L.GgufTensor), (HEADERS[1], "cpb_gguf_hparams", L.GgufHparams),
                         (HEADERS[2], "cpb_head_cfg", L.HeadCfg), (HEADERS[2], "cpb_head_trace", L.HeadTrace),
                         (HEADERS[3], "cpb_attn_cfg", L.AttnCfg), (HEADERS[3], "cpb_attn_trace", L.AttnTrace)):
        body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (name, name), h, re.S).group(1)
        body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
        names = []
        for decl in body.split(";"):
            decl = decl.strip()
            if not decl:
                continue
            decl = re.sub(r"\bconst\b", "", decl)
            rest = re.match(r"\s*\w+[\s\*]+(.*)$", decl, re.S).group(1)   # drop the one-word type
            names += [re.sub(r"\[.*\]", "", t).strip("* \n") for t in rest.split(",")]
        assert names == [n for n, _ in cty._fields_], (name, names)
