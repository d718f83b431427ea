"""Generate src/lib.rs (the raw FFI declarations of libvelox_hip.so) from
include/velox_hip.h, the one source of truth for the C ABI.

    python velox-hip-sys/gen_lib.py          # rewrite src/lib.rs
    python velox-hip-sys/gen_lib.py --check  # fail if src/lib.rs is stale

The header's C subset is small and regular: typedef'd enums and structs
(fields of scalar, pointer or struct type, and function-pointer fields),
one #define constant, and function prototypes.
"""
from __future__ import annotations

import os
import re
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
HEADER = os.path.join(HERE, "..", "include", "velox_hip.h")
OUT = os.path.join(HERE, "src", "lib.rs")

SCALARS = {"int": "c_int", "int64_t": "i64", "uint64_t": "u64", "int32_t": "i32", "uint32_t": "u32",
           "uint16_t": "u16", "size_t": "usize", "float": "f32", "double": "f64", "char": "c_char",
           "void": "c_void"}


def strip_comments(text: str) -> str:
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return re.sub(r"//[^\n]*", " ", text)


def rust_type(ctype: str) -> str:
    """C type (without the name) -> Rust FFI type."""
    t = " ".join(ctype.replace("*", " * ").split())
    # pointer levels from the right: 'const uint32_t * const *'
    parts = t.split(" * ")
    if "*" not in t:
        base = t.replace("const ", "").strip()
        return SCALARS.get(base, base)
    toks = t.split()
    stars = [i for i, x in enumerate(toks) if x == "*"]
    base_toks = toks[: stars[0]]
    const_base = "const" in base_toks
    base = " ".join(x for x in base_toks if x != "const")
    out = SCALARS.get(base, base)
    prev_const = const_base
    for si, pos in enumerate(stars):
        nxt = toks[pos + 1] if pos + 1 < len(toks) else ""
        out = ("*const " if prev_const else "*mut ") + out
        prev_const = nxt == "const"
    return out


def split_args(arglist: str):
    arglist = arglist.strip()
    if arglist in ("", "void"):
        return []
    args, depth, cur = [], 0, ""
    for ch in arglist:
        if ch == "(":
            depth += 1
        elif ch == ")":
            depth -= 1
        if ch == "," and depth == 0:
            args.append(cur.strip())
            cur = ""
        else:
            cur += ch
    args.append(cur.strip())
    return args


def split_decl(decl: str):
    """'const uint32_t *const *prompts' -> (type, name)."""
    m = re.match(r"^(.*?)([A-Za-z_][A-Za-z0-9_]*)$", decl.strip())
    return m.group(1).strip(), m.group(2)


RUST_KEYWORDS = {"type", "ref", "fn", "in", "match", "move", "mod", "loop", "use", "impl", "self", "box", "where"}


def rname(n: str) -> str:
    return "r#" + n if n in RUST_KEYWORDS else n


def parse(text: str):
    body = strip_comments(text)
    consts = []
    for m in re.finditer(r"#define\s+(VX_[A-Z0-9_]+)\s+\(\(size_t\)\((\d+)u\s*<<\s*(\d+)\)\s*\+\s*(\d+)u\)", body):
        consts.append((m.group(1), "usize", f"({m.group(2)} << {m.group(3)}) + {m.group(4)}"))
    enums = []
    for m in re.finditer(r"typedef\s+enum\s*\{(.*?)\}\s*(\w+)\s*;", body, re.S):
        for item in m.group(1).split(","):
            if "=" in item:
                k, v = item.split("=")
                enums.append((k.strip(), int(v.strip())))
    structs, opaque = [], []
    for m in re.finditer(r"typedef\s+struct\s+(\w+)\s+(\w+)\s*;", body):
        opaque.append(m.group(2))
    for m in re.finditer(r"typedef\s+struct\s*\{(.*?)\}\s*(\w+)\s*;", body, re.S):
        fields = []
        for decl in [d.strip() for d in m.group(1).split(";") if d.strip()]:
            fp = re.match(r"^(.*?)\(\s*\*\s*(\w+)\s*\)\s*\((.*)\)$", decl, re.S)
            if fp:  # function pointer field
                ret = rust_type(fp.group(1).strip())
                args = [rust_type(split_decl(a)[0]) for a in split_args(fp.group(3))]
                sig = "unsafe extern \"C\" fn(" + ", ".join(args) + ")" + ("" if ret == "c_void" else f" -> {ret}")
                fields.append((fp.group(2), f"Option<{sig}>"))
                continue
            base, names = decl.split(None, 1) if not decl.startswith("const") else (None, None)
            # 'int64_t a, b, c' / 'const uint16_t *ln1, *ln2' / 'double x[3]'
            head = re.match(r"^((?:const\s+)?\w+)\s+(.*)$", decl, re.S)
            btype, rest = head.group(1), head.group(2)
            for nm in [x.strip() for x in rest.split(",")]:
                arr = re.match(r"^(\**)\s*(\w+)\s*\[(\d+)\]$", nm)
                if arr:
                    fields.append((arr.group(2), f"[{rust_type(btype + ' ' + arr.group(1))}; {arr.group(3)}]"))
                    continue
                stars = len(nm) - len(nm.lstrip("*"))
                fields.append((nm.lstrip("*").strip(), rust_type(btype + " " + "*" * stars)))
        structs.append((m.group(2), fields))
    funcs = []
    for m in re.finditer(r"(?:(?<=[;}])|^)\s*((?:const\s+)?[\w]+\s*\**\s*)(vx_\w+)\s*\(([^;{}]*?)\)\s*;", body,
                         re.S | re.M):
        ret = rust_type(m.group(1).strip())
        args = [split_decl(a) for a in split_args(m.group(3))]
        funcs.append((m.group(2), ret, [(n, rust_type(t)) for t, n in args]))
    return consts, enums, opaque, structs, funcs


def render(text: str) -> str:
    consts, enums, opaque, structs, funcs = parse(text)
    out = ["// Generated by gen_lib.py from include/velox_hip.h: do not edit by hand.",
           "//! Raw FFI bindings of libvelox_hip.so, the MI355X (gfx950) speculative-decoding",
           "//! verify path. Every item mirrors a declaration of include/velox_hip.h with the",
           "//! same name, field order and argument order; see that header for semantics.",
           "#![allow(non_camel_case_types, non_upper_case_globals, clippy::missing_safety_doc)]",
           "", "use std::ffi::{c_char, c_int, c_void};", ""]
    for k, v in enums:
        out.append(f"pub const {k}: c_int = {v};")
    for k, t, v in consts:
        out.append(f"pub const {k}: {t} = {v};")
    out.append("")
    for name in opaque:
        out.append(f"#[repr(C)]\npub struct {name} {{\n    _opaque: [u8; 0],\n}}\n")
    for name, fields in structs:
        out.append("#[repr(C)]\n#[derive(Copy, Clone)]\npub struct " + name + " {")
        for fname, ftype in fields:
            out.append(f"    pub {rname(fname)}: {ftype},")
        out.append("}\n")
    out.append('#[link(name = "velox_hip")]\nextern "C" {')
    for name, ret, args in funcs:
        a = ", ".join(f"{rname(n)}: {t}" for n, t in args)
        r = "" if ret == "c_void" else f" -> {ret}"
        out.append(f"    pub fn {name}({a}){r};")
    out.append("}\n")
    return "\n".join(out)


def main() -> int:
    text = open(HEADER).read()
    want = render(text)
    if "--check" in sys.argv:
        have = open(OUT).read() if os.path.exists(OUT) else ""
        if have != want:
            print("src/lib.rs is stale: run python velox-hip-sys/gen_lib.py", file=sys.stderr)
            return 1
        return 0
    with open(OUT, "w") as f:
        f.write(want)
    return 0


if __name__ == "__main__":
    sys.exit(main())
