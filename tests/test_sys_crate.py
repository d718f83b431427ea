"""The Rust -sys crate (velox-hip-sys/) matches the C ABI of
include/velox_hip.h.  No Rust toolchain is in this image, so the crate is
checked by parsing: src/lib.rs must be what velox-hip-sys/gen_lib.py makes of
the current header, and, read with a parser of its own (Rust syntax, not the
generator's C parser), its extern block must declare every header function
with the same argument count, and its #[repr(C)] structs the header's fields
in the header's order."""
import os
import re
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "velox_hip.h")
LIB_RS = os.path.join(ROOT, "velox-hip-sys", "src", "lib.rs")


def c_functions():
    body = re.sub(r"/\*.*?\*/", " ", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"\b(vx_\w+)\s*\(([^;{}()]*(?:\([^()]*\)[^;{}()]*)*)\)\s*;", body):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def c_struct_fields():
    body = re.sub(r"/\*.*?\*/", " ", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"typedef\s+struct\s*\{(.*?)\}\s*(\w+)\s*;", body, re.S):
        names = []
        for decl in [d.strip() for d in m.group(1).split(";") if d.strip()]:
            fp = re.search(r"\(\s*\*\s*(\w+)\s*\)", decl)
            if fp:
                names.append(fp.group(1))
                continue
            rest = re.match(r"^(?:const\s+)?\w+\s+(.*)$", decl, re.S).group(1)
            names += [re.sub(r"\[.*\]", "", x).strip(" *") for x in rest.split(",")]
        out[m.group(2)] = names
    return out


def rust_functions():
    text = open(LIB_RS).read()
    block = text[text.index('extern "C" {'):]
    out = {}
    for m in re.finditer(r"pub fn (vx_\w+)\((.*?)\)\s*(?:->\s*[^;]+)?;", block, re.S):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if not args else len(re.findall(r"\b[\w#]+\s*:", args))
    return out


def rust_struct_fields():
    text = open(LIB_RS).read()
    out = {}
    for m in re.finditer(r"pub struct (\w+)\s*\{(.*?)\n\}", text, re.S):
        out[m.group(1)] = re.findall(r"pub (?:r#)?(\w+)\s*:", m.group(2))
    return out


def test_lib_rs_is_generated_from_the_current_header():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "velox-hip-sys", "gen_lib.py"), "--check"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_every_header_function_is_bound_with_its_argument_count():
    c, rs = c_functions(), rust_functions()
    assert len(c) >= 55
    assert set(c) == set(rs), (sorted(set(c) - set(rs)), sorted(set(rs) - set(c)))
    bad = {n: (c[n], rs[n]) for n in c if c[n] != rs[n]}
    assert not bad, bad


def test_structs_keep_the_header_field_order():
    c, rs = c_struct_fields(), rust_struct_fields()
    for name, fields in c.items():
        assert rs.get(name) == fields, (name, fields, rs.get(name))


def test_build_script_links_the_library():
    text = open(os.path.join(ROOT, "velox-hip-sys", "build.rs")).read()
    assert "rustc-link-lib=dylib=velox_hip" in text and "rustc-link-lib=dylib=amdhip64" in text
    cargo = open(os.path.join(ROOT, "velox-hip-sys", "Cargo.toml")).read()
    assert 'links = "velox_hip"' in cargo
