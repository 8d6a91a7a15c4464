"""A small parser for include/huncho_rocm.h (function prototypes, #define constants, typedef'd
structs) and the C -> Rust type mapping the FFI crate (rust/huncho-rocm-sys) must follow. Used
by tests/test_rust_binding.py to check the crate's declarations against the header."""
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "huncho_rocm.h"
RUST_LIB = ROOT / "rust" / "huncho-rocm-sys" / "src" / "lib.rs"

SCALARS = {"int": "c_int", "long": "c_long", "size_t": "usize", "float": "f32", "double": "f64",
           "uint64_t": "u64", "int32_t": "i32", "uint16_t": "u16", "char": "c_char", "void": "c_void"}


def strip_comments(text: str) -> str:
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.sub(r"//[^\n]*", "", text)


def c_to_rust(ctype: str) -> str:
    """'const int32_t*' -> '*const i32'; 'hk_ctx**' -> '*mut *mut hk_ctx'; 'int' -> 'c_int'."""
    t = ctype.strip()
    stars = t.count("*")
    base = t.replace("*", " ").split()
    const = base[0] == "const"
    base = [b for b in base if b != "const"]
    name = " ".join(base)
    rust = SCALARS.get(name, name)
    for i in range(stars):
        rust = ("*const " if (const and i == 0) else "*mut ") + rust
    return rust


def split_param(p: str):
    """'const int32_t* cu_seqlens_dev' -> ('const int32_t*', 'cu_seqlens_dev')."""
    p = " ".join(p.split())
    m = re.match(r"^(.*?)([A-Za-z_][A-Za-z0-9_]*)$", p)
    ctype, name = m.group(1).strip(), m.group(2)
    return ctype, name


def header_prototypes():
    """name -> (rust return type, [rust parameter types])"""
    text = strip_comments(HEADER.read_text())
    out = {}
    for m in re.finditer(r"([A-Za-z_][A-Za-z0-9_ ]*?\**)\s*\b(hk_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        ret, name, params = m.group(1), m.group(2), m.group(3).strip()
        ps = [] if params in ("", "void") else [c_to_rust(split_param(p)[0]) for p in params.split(",")]
        out[name] = (c_to_rust(ret), ps)
    return out


def header_defines():
    return {m.group(1): int(m.group(2)) for m in re.finditer(r"#define\s+(HK_[A-Z0-9_]+)\s+(-?\d+)",
                                                             HEADER.read_text())}


def header_structs():
    """typedef struct { ... } name; -> name -> [(field, rust type)] in order."""
    text = strip_comments(HEADER.read_text())
    out = {}
    for m in re.finditer(r"typedef\s+struct\s*\{(.*?)\}\s*([A-Za-z_0-9]+)\s*;", text, flags=re.S):
        fields = []
        for decl in m.group(1).split(";"):
            decl = " ".join(decl.split())
            if not decl:
                continue
            arr = re.match(r"^(.*?)([A-Za-z_0-9]+)\[(\d+)\]$", decl)
            if arr:
                fields.append((arr.group(2), f"[{c_to_rust(arr.group(1))}; {arr.group(3)}]"))
                continue
            # 'const void *a, *b' and 'int a, b, c'
            first, *rest = [x.strip() for x in decl.split(",")]
            ctype, name = split_param(first.replace("*", "* ").replace("  ", " "))
            base = ctype.replace("*", "").strip()
            fields.append((name, c_to_rust(ctype)))
            for r in rest:
                stars = r.count("*")
                rname = r.replace("*", "").strip()
                fields.append((rname, c_to_rust(base + "*" * stars)))
        out[m.group(2)] = fields
    return out


def rust_externs():
    """name -> (return type, [parameter types]) from the crate's extern "C" block."""
    text = RUST_LIB.read_text()
    block = re.search(r'extern "C" \{(.*?)\n\}', text, flags=re.S).group(1)
    block = re.sub(r"//[^\n]*", "", block)
    out = {}
    for m in re.finditer(r"pub fn (hk_[a-z0-9_]+)\s*\((.*?)\)\s*(?:->\s*([^;]+))?;", block, flags=re.S):
        params = [p.strip() for p in m.group(2).split(",") if p.strip()]
        types = [" ".join(p.split(":", 1)[1].split()) for p in params]
        out[m.group(1)] = (" ".join((m.group(3) or "()").split()), types)
    return out


def rust_structs():
    text = RUST_LIB.read_text()
    out = {}
    for m in re.finditer(r"#\[repr\(C\)\]\s*(?:#\[derive\([^)]*\)\]\s*)?pub struct ([A-Za-z_0-9]+)\s*\{(.*?)\n\}", text,
                         flags=re.S):
        fields = []
        for line in m.group(2).split(","):
            line = re.sub(r"//[^\n]*", "", line).strip()
            if not line:
                continue
            fm = re.match(r"pub ([A-Za-z_0-9]+):\s*(.+)$", line, flags=re.S)
            if fm:
                fields.append((fm.group(1), " ".join(fm.group(2).split())))
        out[m.group(1)] = fields
    return out


def rust_consts():
    return {m.group(1): int(m.group(2)) for m in re.finditer(r"pub const (HK_[A-Z0-9_]+): c_int = (-?\d+);",
                                                             RUST_LIB.read_text())}
